// Grouped q4 expert GEMMs for prefill chunks (reference role:
// gpu::moe_experts_T, src/kernels/moe_experts.hip:17-171, which dequantises
// the expert's q4 weights into an fp16 LDS tile and multiplies gathered
// token rows).
//
// Work is the (expert, tile) list written by the routing kernel
// (qw_moe_route with tile_m = GROUPED_TILE_M = -32: mixed tiles of 32 to 160
// slots); slots of one expert are contiguous (offsets[e] ..), slot p
// carries token pair_tok[p]. A tile's height follows from its start and the
// expert's slot count (tile_rows). Each block runs the register-dequant MFMA
// core (gemm_tile_rd2, q4_gemm_core.cuh) at that height on one list entry
// and 512 weight rows:
//   gate/up  A = the tile's gathered token rows of x (fp16 copy in the
//            workspace); wave w holds the gate and the up rows of the same 32
//            columns j0 + 32 w .., so h = silu(g) * u (fp16, saturated, the
//            reference's fp16 intermediate) is formed in the wave.
//   down     A = the tile's h rows (contiguous slots), 512 down rows; yp fp32
//            or fp16.
// Blocks past the list's length (n_tiles, known only on the device) exit at
// once; the grid is sized for the largest possible list (they are dispatched
// after every real tile).
#include "q4_gemm_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

// 32 to 160 slots. Before the 96- and 160-slot tiles (128, 64 or 32 slots):
// same box, config 5, 1.82-1.86 ms per chunk against
// 1.96 with tiles of 256 (role-split core), 128 and 64 (one 32-row weight
// group per wave); the finer remainders cut the padded rows from 1.25 to 1.12
// of the real ones, and each A fragment feeds two MFMAs.
constexpr int GROUPED_TILE_M = -32;

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

// ---- a tile of 32 to 160 slots by 512 weight rows (gemm_tile_rd2)
// gate/up: wave w holds gate and up rows of the same 32 columns j0 + 32 w ..
// (group 0 gate, group 1 up), so h = silu(g) * u is formed in the wave.
template <int BM, bool HAS_Z>
__device__ __forceinline__ void gate_up_tile(const GateUpTile &a, int e, int base, int M, int j0) {
    constexpr int NI = BM / 32, NA = (BM + 63) / 64;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int64_t wrow = int64_t(e) * a.F + min(j0 + wave * 32 + lane % 32, a.F - 1);
    const int G = a.H / QGROUP;
    const BRow bg(a.gw, a.gs, a.gz, wrow, G), bu(a.uw, a.us, a.uz, wrow, G);
    const uint16_t *arow[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) arow[j] = a.xh + int64_t(a.pair_tok[base + min(64 * j + wave * 8 + lane / 8, M - 1)]) * a.H;
    f32x16 acc[NI][2];
#pragma unroll
    for (int i = 0; i < NI; ++i) acc[i][0] = acc[i][1] = f32x16{};
    gemm_tile_rd2<BM, HAS_Z, 0>(arow, bg, bu, a.H, acc);
    auto cvt = [](float v, int, int) { return f32_to_f16_sat(v); };
#pragma unroll
    for (int hh = 0; hh < (NI + 1) / 2; ++hh) {
        f32x16 hv[2][1];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q)
                hv[i][0][q] = 2 * hh + i < NI ? silu_mul(acc[min(2 * hh + i, NI - 1)][0][q], acc[min(2 * hh + i, NI - 1)][1][q]) : 0.f;
        emit_tile<1, 2>(epi_slot(wave), hv, cvt, [&](int tr, int c, uint4 v) {
            const int m = hh * 64 + tr, j = j0 + wave * 32 + c;
            if (m < M && j < a.F) *reinterpret_cast<uint4 *>(a.h + int64_t(base + m) * a.F + j) = v;
        });
    }
}

template <int BM, bool HAS_Z, bool YP16>
__device__ __forceinline__ void down_tile(const uint32_t *dw, const uint16_t *ds, const uint16_t *dz, int e, int base,
                                           int M, const uint16_t *h, int H, int F, void *yp) {
    constexpr int NI = BM / 32, NA = (BM + 63) / 64, YB = YP16 ? 2 : 4;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int n0 = blockIdx.x * 512 + wave * 64;
    const int G = F / QGROUP;
    const BRow b0(dw, ds, dz, int64_t(e) * H + min(n0 + lane % 32, H - 1), G),
        b1(dw, ds, dz, int64_t(e) * H + min(n0 + 32 + lane % 32, H - 1), G);
    const uint16_t *arow[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) arow[j] = h + int64_t(base + min(64 * j + wave * 8 + lane / 8, M - 1)) * F;
    f32x16 acc[NI][2];
#pragma unroll
    for (int i = 0; i < NI; ++i) acc[i][0] = acc[i][1] = f32x16{};
    gemm_tile_rd2<BM, HAS_Z, 1 + YP16>(arow, b0, b1, F, acc);
#pragma unroll
    for (int hh = 0; hh < (NI + 1) / 2; ++hh) {
        f32x16 o[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) o[i][j] = 2 * hh + i < NI ? acc[min(2 * hh + i, NI - 1)][j] : f32x16{};
        emit_tile<2, YB>(
            epi_slot(wave), o, [](float v, int, int) { return f32_to_f16_sat(v); },
            [&](int tr, int c, uint4 v) {
                const int m = hh * 64 + tr, n = n0 + c;
                if (m < M && n < H)
                    *reinterpret_cast<uint4 *>(static_cast<unsigned char *>(yp) + (int64_t(base + m) * H + n) * YB) = v;
            });
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
    const int j0 = blockIdx.x * 256;
    if (rows == 160) gate_up_tile<160, HAS_Z>(a, e, base, M, j0);
    else if (rows == 128) gate_up_tile<128, HAS_Z>(a, e, base, M, j0);
    else if (rows == 96) gate_up_tile<96, HAS_Z>(a, e, base, M, j0);
    else if (rows == 64) gate_up_tile<64, HAS_Z>(a, e, base, M, j0);
    else gate_up_tile<32, HAS_Z>(a, e, base, M, j0);
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
    if (rows == 160) down_tile<160, HAS_Z, YP16>(dw, ds, dz, e, base, M, h, H, F, yp);
    else if (rows == 128) down_tile<128, HAS_Z, YP16>(dw, ds, dz, e, base, M, h, H, F, yp);
    else if (rows == 96) down_tile<96, HAS_Z, YP16>(dw, ds, dz, e, base, M, h, H, F, yp);
    else if (rows == 64) down_tile<64, HAS_Z, YP16>(dw, ds, dz, e, base, M, h, H, F, yp);
    else down_tile<32, HAS_Z, YP16>(dw, ds, dz, e, base, M, h, H, F, yp);
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
    const dim3 g1(unsigned((a.F + 255) / 256), unsigned(max_tiles)), g2(unsigned((a.H + 511) / 512), unsigned(max_tiles));
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
