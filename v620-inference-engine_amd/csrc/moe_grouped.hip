// Grouped q4 expert GEMMs for prefill chunks (reference role:
// gpu::moe_experts_T, src/kernels/moe_experts.hip:17-171, which dequantises
// the expert's q4 weights into an fp16 LDS tile and multiplies gathered
// token rows).
//
// Work is the (expert, tile) list written by the routing kernel
// (qw_moe_route with tile_m = GROUPED_TILE_M = -64: mixed tiles of 256, 128
// and 64 slots); slots of one expert are contiguous (offsets[e] ..), slot p
// carries token pair_tok[p]. A tile's height follows from its start and the
// expert's slot count (tile_rows). Each block runs the shared q4 MFMA GEMM
// core (q4_gemm_core.cuh) at that height on one list entry and 256 weight
// rows (64- and 128-slot tiles: its register-dequant form, gemm_tile_rd):
//   gate/up  A = the tile's gathered token rows of x (fp16 copy in the
//            workspace), weight rows = 128 gate rows and the same 128 up rows,
//            interleaved by 32 (32-row groups alternate gate, up); epilogue
//            h = silu(g) * u in fp16 (saturated), the reference's fp16
//            intermediate.
//   down     A = the tile's h rows (contiguous slots), 256 down rows, fp32 yp.
// Blocks past the list's length (n_tiles, known only on the device) exit at
// once; the grid is sized for the largest possible list.
#include "q4_gemm_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

constexpr int GROUPED_TILE_M = -64;

int moe_grouped_tile_m() { return GROUPED_TILE_M; }

size_t moe_grouped_workspace_bytes(int T, int, int, int H, int) { return gemm_workspace_bytes(T, H); }

static __device__ __forceinline__ uint16_t f32_to_f16_sat(float v) {
    return __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(v));
}

static __device__ __forceinline__ float silu_mul(float g, float u) { return silu_ref(g) * u; }

struct GateUpTile {
    const uint32_t *gw, *uw;
    const uint16_t *gs, *gz, *us, *uz;
    const int32_t *pair_tok;
    const uint16_t *xh;
    int H, F;
    uint16_t *h;
};

// One gate/up tile of BM slot rows (M of them real) starting at slot base.
template <int BM, bool HAS_Z>
__device__ __forceinline__ void gate_up_tile(const GateUpTile &a, int e, int base, int M, int j0) {
    using Sh = GemmShape<BM>;
    const int tid = threadIdx.x, wave = tid / WAVE;
    if constexpr (BM == 128) {
        // register-dequant core, wave w: all 128 rows x 32 weight rows (group
        // w: gate when even, up when odd, columns j0 + 32 (w / 2) ..)
        const int r = wave * 32 + tid % 32, col = (r / 64) * 32 + r % 32;
        const bool up = (r % 64) >= 32;
        const int64_t wrow = int64_t(e) * a.F + min(j0 + col, a.F - 1);
        const BRow b = up ? BRow(a.uw, a.us, a.uz, wrow, a.H / QGROUP) : BRow(a.gw, a.gs, a.gz, wrow, a.H / QGROUP);
        const int lr = wave * 8 + (tid % WAVE) / 8;
        const uint16_t *const arow[2] = {a.xh + int64_t(a.pair_tok[base + min(lr, M - 1)]) * a.H,
                                         a.xh + int64_t(a.pair_tok[base + min(64 + lr, M - 1)]) * a.H};
        f32x16 acc[4][1];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][0] = f32x16{};
        gemm_tile_rd<128, HAS_Z, 3>(arow, b, a.H, acc);
        // the up wave of each pair hands its accumulators over through LDS
        // (lds_a1 for pairs 0-1, lds_b1 for 2-3: free after the core)
        const int pr = wave / 2, lane = tid % WAVE;
        float *xbuf = reinterpret_cast<float *>(pr < 2 ? lds_a1 : lds_b1) + (pr % 2) * (4 * 16 * WAVE);
        if (wave & 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int q = 0; q < 16; ++q) xbuf[(i * 16 + q) * WAVE + lane] = acc[i][0][q];
        }
        __syncthreads();
        if (!(wave & 1)) {
            auto cvt = [](float v, int, int) { return f32_to_f16_sat(v); };
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                f32x16 hv[2][1];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int q = 0; q < 16; ++q)
                        hv[i][0][q] = silu_mul(acc[2 * hh + i][0][q], xbuf[((2 * hh + i) * 16 + q) * WAVE + lane]);
                emit_tile<1, 2>(epi_slot(wave), hv, cvt, [&](int tr, int c, uint4 v) {
                    const int m = hh * 64 + tr, j = j0 + pr * 32 + c;
                    if (m < M && j < a.F) *reinterpret_cast<uint4 *>(a.h + int64_t(base + m) * a.F + j) = v;
                });
            }
        }
        return;
    }
    // weight tile row r = b_tile_row(): 32-row group r / 32 is gate when even,
    // up when odd, for columns j0 + 32 (r / 64) + r % 32 (wave-uniform choice)
    // (64-row tiles: the row this lane multiplies, 32 wave + lane % 32, the
    // tile row the register-dequant core gives it)
    const int r = BM == 64 ? wave * 32 + tid % 32 : b_tile_row(), col = (r / 64) * 32 + r % 32;
    const bool up = (r % 64) >= 32;
    const int64_t wrow = int64_t(e) * a.F + min(j0 + col, a.F - 1);
    const BRow b = up ? BRow(a.uw, a.us, a.uz, wrow, a.H / QGROUP) : BRow(a.gw, a.gs, a.gz, wrow, a.H / QGROUP);
    f32x16 acc[2][Sh::NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < Sh::NJ; ++j) acc[i][j] = f32x16{};
    if constexpr (BM == 64) {
        const uint16_t *const arow[1] = {a.xh + int64_t(a.pair_tok[base + min(wave * 8 + (tid % WAVE) / 8, M - 1)]) * a.H};
        gemm_tile_rd<64, HAS_Z, 0>(arow, b, a.H, acc);
    } else {
        const uint16_t *ap[BM / 32];
#pragma unroll
        for (int j = 0; j < BM / 32; ++j) ap[j] = a.xh + int64_t(a.pair_tok[base + min(a_load_row(j), M - 1)]) * a.H;
        gemm_tile<BM, HAS_Z>(ap, b, a.H, acc);
    }

    const int wm = wave / Sh::NWN, wn2 = wave % Sh::NWN;
    auto store = [&](int cbase) {
        return [&, cbase](int tr, int c, uint4 v) {
            const int m = wm * 64 + tr, j = j0 + cbase + c;
            if (m < M && j < a.F) *reinterpret_cast<uint4 *>(a.h + int64_t(base + m) * a.F + j) = v;
        };
    };
    auto cvt = [](float v, int, int) { return f32_to_f16_sat(v); };
    if constexpr (Sh::NJ >= 2) {
        // the wave's 32-row groups 2p (gate) and 2p + 1 (up) hold the same
        // 32 columns, wn2 * WNR / 2 + 32 p ..
        f32x16 hv[2][Sh::NJ / 2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < Sh::NJ / 2; ++p)
#pragma unroll
                for (int q = 0; q < 16; ++q) hv[i][p][q] = silu_mul(acc[i][2 * p][q], acc[i][2 * p + 1][q]);
        emit_tile<Sh::NJ / 2, 2>(epi_slot(wave), hv, cvt, store(wn2 * (Sh::WNR / 2)));
    } else {
        // one 32-row group per wave: wave 2p holds gate, 2p + 1 up of columns
        // 32 p ..; the up wave hands its accumulators over through LDS
        // (lds_a1, free after gemm_tile; same lane layout in both waves)
        float *xbuf = reinterpret_cast<float *>(lds_a1) + (wave / 2) * (2 * 16 * WAVE);
        const int lane = tid % WAVE;
        if (wave & 1) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int q = 0; q < 16; ++q) xbuf[(i * 16 + q) * WAVE + lane] = acc[i][0][q];
        }
        __syncthreads();
        if (!(wave & 1)) {
            f32x16 hv[2][1];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int q = 0; q < 16; ++q) hv[i][0][q] = silu_mul(acc[i][0][q], xbuf[(i * 16 + q) * WAVE + lane]);
            emit_tile<1, 2>(epi_slot(wave), hv, cvt, store((wave / 2) * 32));
        }
    }
}

template <bool HAS_Z>
__global__ __launch_bounds__(G_THREADS) void moe_gate_up_gemm_kernel(GateUpTile a, const int32_t *__restrict__ offsets,
                                                                     const int32_t *__restrict__ tile_e,
                                                                     const int32_t *__restrict__ tile_m0,
                                                                     const int32_t *__restrict__ n_tiles) {
    const int tile = blockIdx.y;
    if (tile >= *n_tiles) return;
    const int e = tile_e[tile], m0 = tile_m0[tile], rem = offsets[e + 1] - offsets[e] - m0;
    const int base = offsets[e] + m0, rows = tile_rows(rem, GROUPED_TILE_M), M = min(rows, rem);
    const int j0 = blockIdx.x * 128;
    if (rows == 256) gate_up_tile<256, HAS_Z>(a, e, base, M, j0);
    else if (rows == 128) gate_up_tile<128, HAS_Z>(a, e, base, M, j0);
    else gate_up_tile<64, HAS_Z>(a, e, base, M, j0);
}

// One down tile of BM slot rows (M real) starting at slot base.
// yp rows fp32 (YP16 false) or fp16 (finite values beyond +-65504 saturate,
// as the reference keeps yp, src/kernels/moe.hpp:20-25).
template <int BM, bool HAS_Z, bool YP16>
__device__ __forceinline__ void down_tile(const uint32_t *dw, const uint16_t *ds, const uint16_t *dz, int e,
                                          int base, int M, const uint16_t *h, int H, int F, void *yp) {
    using Sh = GemmShape<BM>;
    const int tid = threadIdx.x, wave = tid / WAVE;
    const int n0 = blockIdx.x * GB_N;
    constexpr int YB = YP16 ? 2 : 4;
    if constexpr (BM == 128) {
        // register-dequant core, wave w: all 128 rows x down rows n0 + 32 w ..
        const BRow b(dw, ds, dz, int64_t(e) * H + min(n0 + wave * 32 + tid % 32, H - 1), F / QGROUP);
        const int lr = wave * 8 + (tid % WAVE) / 8;
        const uint16_t *const arow[2] = {h + int64_t(base + min(lr, M - 1)) * F, h + int64_t(base + min(64 + lr, M - 1)) * F};
        f32x16 acc[4][1];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][0] = f32x16{};
        gemm_tile_rd<128, HAS_Z, 5 + YP16>(arow, b, F, acc);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
            emit_tile<1, YB>(
                epi_slot(wave), *reinterpret_cast<const f32x16(*)[2][1]>(&acc[2 * hh][0]),
                [](float v, int, int) { return f32_to_f16_sat(v); },
                [&](int tr, int c, uint4 v) {
                    const int m = hh * 64 + tr, n = n0 + wave * 32 + c;
                    if (m < M && n < H)
                        *reinterpret_cast<uint4 *>(static_cast<unsigned char *>(yp) + (int64_t(base + m) * H + n) * YB) = v;
                });
        return;
    }
    const int r = BM == 64 ? wave * 32 + tid % 32 : b_tile_row();  // (as in gate_up_tile)
    const BRow b(dw, ds, dz, int64_t(e) * H + min(n0 + r, H - 1), F / QGROUP);
    f32x16 acc[2][Sh::NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < Sh::NJ; ++j) acc[i][j] = f32x16{};
    if constexpr (BM == 64) {
        const uint16_t *const arow[1] = {h + int64_t(base + min(wave * 8 + (tid % WAVE) / 8, M - 1)) * F};
        gemm_tile_rd<64, HAS_Z, 1 + YP16>(arow, b, F, acc);
    } else {
        const uint16_t *ap[BM / 32];
#pragma unroll
        for (int j = 0; j < BM / 32; ++j) ap[j] = h + int64_t(base + min(a_load_row(j), M - 1)) * F;
        gemm_tile<BM, HAS_Z>(ap, b, F, acc);
    }

    const int wm = wave / Sh::NWN, wn2 = wave % Sh::NWN;
    emit_tile<Sh::NJ, YB>(
        epi_slot(wave), acc, [](float v, int, int) { return f32_to_f16_sat(v); },
        [&](int tr, int c, uint4 v) {
            const int m = wm * 64 + tr, n = n0 + wn2 * Sh::WNR + c;
            if (m < M && n < H)
                *reinterpret_cast<uint4 *>(static_cast<unsigned char *>(yp) + (int64_t(base + m) * H + n) * YB) = v;
        });
}

template <bool HAS_Z, bool YP16>
__global__ __launch_bounds__(G_THREADS) void moe_down_gemm_kernel(
    const uint32_t *__restrict__ dw, const uint16_t *__restrict__ ds, const uint16_t *__restrict__ dz,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ tile_e, const int32_t *__restrict__ tile_m0,
    const int32_t *__restrict__ n_tiles, const uint16_t *__restrict__ h, int H, int F, void *__restrict__ yp) {
    const int tile = blockIdx.y;
    if (tile >= *n_tiles) return;
    const int e = tile_e[tile], m0 = tile_m0[tile], rem = offsets[e + 1] - offsets[e] - m0;
    const int base = offsets[e] + m0, rows = tile_rows(rem, GROUPED_TILE_M), M = min(rows, rem);
    if (rows == 256) down_tile<256, HAS_Z, YP16>(dw, ds, dz, e, base, M, h, H, F, yp);
    else if (rows == 128) down_tile<128, HAS_Z, YP16>(dw, ds, dz, e, base, M, h, H, F, yp);
    else down_tile<64, HAS_Z, YP16>(dw, ds, dz, e, base, M, h, H, F, yp);
}

void launch_moe_grouped(const MoeGroupedArgs &a, hipStream_t s) {
    // bf16 rows through the fp16 pre-pass into the workspace; fp16 rows as they are
    const uint16_t *xh = a.x;
    if (!a.x_f16) {
        uint16_t *w = static_cast<uint16_t *>(a.ws);
        launch_x_to_f16(a.x, a.H, a.T, a.H, w, s);
        xh = w;
    }
    const int max_tiles = a.T * a.topk / -GROUPED_TILE_M + a.E;
    const dim3 g1(unsigned((a.F + 127) / 128), unsigned(max_tiles)),
        g2(unsigned((a.H + GB_N - 1) / GB_N), unsigned(max_tiles));
    const GateUpTile gu{a.gw, a.uw, a.gs, a.gz, a.us, a.uz, a.pair_tok, xh, a.H, a.F, a.h};
    if (a.gz) moe_gate_up_gemm_kernel<true><<<g1, G_THREADS, 0, s>>>(gu, a.offsets, a.tile_e, a.tile_m0, a.n_tiles);
    else moe_gate_up_gemm_kernel<false><<<g1, G_THREADS, 0, s>>>(gu, a.offsets, a.tile_e, a.tile_m0, a.n_tiles);
    auto down = [&](auto kern) {
        kern<<<g2, G_THREADS, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.tile_e, a.tile_m0, a.n_tiles, a.h, a.H, a.F, a.yp);
    };
    if (a.dz) {
        if (a.yp_f16) down(moe_down_gemm_kernel<true, true>);
        else down(moe_down_gemm_kernel<true, false>);
    } else {
        if (a.yp_f16) down(moe_down_gemm_kernel<false, true>);
        else down(moe_down_gemm_kernel<false, false>);
    }
}

}  // namespace qwq4
