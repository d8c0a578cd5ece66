// Grouped q4 expert GEMMs for prefill chunks (reference role:
// gpu::moe_experts_T, src/kernels/moe_experts.hip:17-171, which dequantises
// the expert's q4 weights into an fp16 LDS tile and multiplies gathered
// token rows).
//
// Work is the (expert, tile of GROUPED_TILE_M slots) list written by the
// routing kernel (qw_moe_route with tile_m = GROUPED_TILE_M); slots of one
// expert are contiguous (offsets[e] ..), slot p carries token pair_tok[p].
// Each block runs the shared q4 MFMA GEMM core (q4_gemm_core.cuh) on one
// list entry and 256 weight rows:
//   gate/up  A = the tile's gathered token rows of x (fp16 copy in the
//            workspace), weight rows = 128 gate rows and the same 128 up rows,
//            interleaved by 32 so each wave holds gate and up of the same
//            columns; epilogue h = silu(g) * u in fp16 (saturated), the
//            reference's fp16 intermediate.
//   down     A = the tile's h rows (contiguous slots), 256 down rows, fp32 yp.
// Blocks past the list's length (n_tiles, known only on the device) exit at
// once; the grid is sized for the largest possible list.
#include "q4_gemm_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

constexpr int GROUPED_TILE_M = 128;

int moe_grouped_tile_m() { return GROUPED_TILE_M; }

size_t moe_grouped_workspace_bytes(int T, int, int, int H, int) { return gemm_workspace_bytes(T, H); }

static __device__ __forceinline__ uint16_t f32_to_f16_sat(float v) {
    v = fminf(fmaxf(v, -65504.f), 65504.f);
    return __builtin_bit_cast(uint16_t, _Float16(v));
}

template <bool HAS_Z>
__global__ __launch_bounds__(G_THREADS) void moe_gate_up_gemm_kernel(
    const uint32_t *__restrict__ gw, const uint16_t *__restrict__ gs, const uint16_t *__restrict__ gz,
    const uint32_t *__restrict__ uw, const uint16_t *__restrict__ us, const uint16_t *__restrict__ uz,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ pair_tok, const int32_t *__restrict__ tile_e,
    const int32_t *__restrict__ tile_m0, const int32_t *__restrict__ n_tiles, const uint16_t *__restrict__ xh, int H,
    int F, uint16_t *__restrict__ h) {
    constexpr int BM = GROUPED_TILE_M;
    using Sh = GemmShape<BM>;
    static_assert(Sh::NJ == 2, "gate/up pairing assumes two 32-row MFMA tiles per wave");
    const int tile = blockIdx.y;
    if (tile >= *n_tiles) return;
    const int e = tile_e[tile], m0 = tile_m0[tile];
    const int base = offsets[e] + m0, M = min(BM, offsets[e + 1] - offsets[e] - m0);
    const int tid = threadIdx.x, wave = tid / WAVE;
    const int j0 = blockIdx.x * 128;
    // tile row r = b_tile_row(): 64-row band r / 64 covers columns j0 + 32 (r / 64)
    // .. + 32; inside it rows 0-31 are gate, 32-63 up (wave-uniform choice)
    const int r = b_tile_row(), col = (r / 64) * 32 + r % 32;
    const bool up = (r % 64) >= 32;
    const int64_t wrow = int64_t(e) * F + min(j0 + col, F - 1);
    const BRow b = up ? BRow(uw, us, uz, wrow, H / QGROUP) : BRow(gw, gs, gz, wrow, H / QGROUP);
    const uint16_t *ap[BM / 32];
#pragma unroll
    for (int j = 0; j < BM / 32; ++j) ap[j] = xh + int64_t(pair_tok[base + min(a_load_row(j), M - 1)]) * H;
    f32x16 acc[2][Sh::NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < Sh::NJ; ++j) acc[i][j] = f32x16{};
    unsigned char *ep = gemm_tile<BM, HAS_Z>(ap, b, H, acc);

    // acc[i][0] (gate) and acc[i][1] (up) hold the same 32 columns
    f32x16 hv[2][1];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const float g = acc[i][0][q], u = acc[i][1][q];
            hv[i][0][q] = g / (1.f + __expf(-g)) * u;
        }
    const int wm = wave / Sh::NWN, wn2 = wave % Sh::NWN;
    emit_tile<1, 2>(
        ep + wave * 64 * 32 * 2, hv, [](float v, int, int) { return f32_to_f16_sat(v); },
        [&](int tr, int c, uint4 v) {
            const int m = wm * 64 + tr, j = j0 + wn2 * 32 + c;
            if (m < M && j < F) *reinterpret_cast<uint4 *>(h + int64_t(base + m) * F + j) = v;
        });
}

template <bool HAS_Z>
__global__ __launch_bounds__(G_THREADS) void moe_down_gemm_kernel(
    const uint32_t *__restrict__ dw, const uint16_t *__restrict__ ds, const uint16_t *__restrict__ dz,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ tile_e, const int32_t *__restrict__ tile_m0,
    const int32_t *__restrict__ n_tiles, const uint16_t *__restrict__ h, int H, int F, float *__restrict__ yp) {
    constexpr int BM = GROUPED_TILE_M;
    using Sh = GemmShape<BM>;
    const int tile = blockIdx.y;
    if (tile >= *n_tiles) return;
    const int e = tile_e[tile], m0 = tile_m0[tile];
    const int base = offsets[e] + m0, M = min(BM, offsets[e + 1] - offsets[e] - m0);
    const int tid = threadIdx.x, wave = tid / WAVE;
    const int n0 = blockIdx.x * GB_N;
    const BRow b(dw, ds, dz, int64_t(e) * H + min(n0 + b_tile_row(), H - 1), F / QGROUP);
    const uint16_t *ap[BM / 32];
#pragma unroll
    for (int j = 0; j < BM / 32; ++j) ap[j] = h + int64_t(base + min(a_load_row(j), M - 1)) * F;
    f32x16 acc[2][Sh::NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < Sh::NJ; ++j) acc[i][j] = f32x16{};
    unsigned char *ep = gemm_tile<BM, HAS_Z>(ap, b, F, acc);

    const int wm = wave / Sh::NWN, wn2 = wave % Sh::NWN;
    emit_tile<Sh::NJ, 4>(
        ep + wave * 64 * 32 * 4, acc, [](float, int, int) { return uint16_t(0); },
        [&](int tr, int c, uint4 v) {
            const int m = wm * 64 + tr, n = n0 + wn2 * Sh::WNR + c;
            if (m < M && n < H) *reinterpret_cast<uint4 *>(yp + int64_t(base + m) * H + n) = v;
        });
}

void launch_moe_grouped(const MoeGroupedArgs &a, hipStream_t s) {
    uint16_t *xh = static_cast<uint16_t *>(a.ws);
    launch_x_to_f16(a.x, a.H, a.T, a.H, xh, s);
    const int max_tiles = a.T * a.topk / GROUPED_TILE_M + a.E;
    const dim3 g1(unsigned((a.F + 127) / 128), unsigned(max_tiles)),
        g2(unsigned((a.H + GB_N - 1) / GB_N), unsigned(max_tiles));
    if (a.gz) {
        moe_gate_up_gemm_kernel<true><<<g1, G_THREADS, 0, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets,
                                                                      a.pair_tok, a.tile_e, a.tile_m0, a.n_tiles, xh,
                                                                      a.H, a.F, a.h);
    } else {
        moe_gate_up_gemm_kernel<false><<<g1, G_THREADS, 0, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets,
                                                                       a.pair_tok, a.tile_e, a.tile_m0, a.n_tiles, xh,
                                                                       a.H, a.F, a.h);
    }
    if (a.dz) {
        moe_down_gemm_kernel<true><<<g2, G_THREADS, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.tile_e, a.tile_m0,
                                                                   a.n_tiles, a.h, a.H, a.F, a.yp);
    } else {
        moe_down_gemm_kernel<false><<<g2, G_THREADS, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.tile_e, a.tile_m0,
                                                                    a.n_tiles, a.h, a.H, a.F, a.yp);
    }
}

}  // namespace qwq4
