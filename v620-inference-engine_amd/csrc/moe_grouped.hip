// Grouped q4 expert GEMMs for prefill chunks (reference role:
// gpu::moe_experts_T, src/kernels/moe_experts.hip:17-171).
//
// Work is the (expert, 32-token tile) list written by the routing kernel
// (qw_moe_route with tile_m = 32). This first version runs each tile through
// the GEMV wave core: every wave owns 16 weight rows and the tile's 32 tokens.
#include "q4_kernels.hpp"
#include "q4_wave.cuh"

namespace qwq4 {

constexpr int GROUPED_TILE_M = 32;

size_t moe_grouped_workspace_bytes(int, int, int, int, int) { return 0; }

template <bool HAS_Z>
__global__ __launch_bounds__(512) void moe_gate_up_tile_kernel(
    const uint32_t *__restrict__ gw, const uint16_t *__restrict__ gs, const uint16_t *__restrict__ gz,
    const uint32_t *__restrict__ uw, const uint16_t *__restrict__ us, const uint16_t *__restrict__ uz,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ pair_tok, const int32_t *__restrict__ tile_e,
    const int32_t *__restrict__ tile_m0, const int32_t *__restrict__ n_tiles, const uint16_t *__restrict__ x, int H,
    int F, uint16_t *__restrict__ h) {
    const int tile = blockIdx.y;
    if (tile >= *n_tiles) return;
    const int e = tile_e[tile], m0 = tile_m0[tile];
    const int base = offsets[e] + m0, M = min(GROUPED_TILE_M, offsets[e + 1] - offsets[e] - m0);
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16, n = lane % 16;
    const int G = H / QGROUP, fsub = F / 16, lsub = blockIdx.x * 8 + wave;
    const int64_t sub = int64_t(e) * fsub + min(lsub, fsub - 1);
    const Q4Tile wt[2] = {Q4Tile(gw, gs, gz, sub, G), Q4Tile(uw, us, uz, sub, G)};
    const uint16_t *arow[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) arow[mb] = x + int64_t(pair_tok[base + min(mb * 16 + n, M - 1)]) * H;
    f32x4 acc[2][2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) acc[mb][0] = acc[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    q4_groups<BF16, 2, 2, HAS_Z, 2>(wt, arow, 0, G, lane, acc);
    if (lsub >= fsub) return;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m < M) h[int64_t(base + m) * F + lsub * 16 + n] = silu_mul_f16(acc[mb][0][r], acc[mb][1][r]);
        }
}

template <bool HAS_Z>
__global__ __launch_bounds__(512) void moe_down_tile_kernel(const uint32_t *__restrict__ dw,
                                                            const uint16_t *__restrict__ ds,
                                                            const uint16_t *__restrict__ dz,
                                                            const int32_t *__restrict__ offsets,
                                                            const int32_t *__restrict__ tile_e,
                                                            const int32_t *__restrict__ tile_m0,
                                                            const int32_t *__restrict__ n_tiles,
                                                            const uint16_t *__restrict__ h, int H, int F,
                                                            float *__restrict__ yp) {
    const int tile = blockIdx.y;
    if (tile >= *n_tiles) return;
    const int e = tile_e[tile], m0 = tile_m0[tile];
    const int base = offsets[e] + m0, M = min(GROUPED_TILE_M, offsets[e + 1] - offsets[e] - m0);
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16, n = lane % 16;
    const int G = F / QGROUP, hsub = H / 16, lsub = blockIdx.x * 8 + wave;
    const int64_t sub = int64_t(e) * hsub + min(lsub, hsub - 1);
    const Q4Tile wt[1] = {Q4Tile(dw, ds, dz, sub, G)};
    const uint16_t *arow[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) arow[mb] = h + int64_t(base + min(mb * 16 + n, M - 1)) * F;
    f32x4 acc[2][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}, {f32x4{0.f, 0.f, 0.f, 0.f}}};
    q4_groups<F16, 2, 1, HAS_Z, 4>(wt, arow, 0, G, lane, acc);
    if (lsub >= hsub) return;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m < M) yp[int64_t(base + m) * H + lsub * 16 + n] = acc[mb][0][r];
        }
}

int moe_grouped_tile_m() { return GROUPED_TILE_M; }

void launch_moe_grouped(const MoeGroupedArgs &a, hipStream_t s) {
    const int max_tiles = a.T * a.topk / GROUPED_TILE_M + a.E;
    const dim3 g1(unsigned((a.F + 127) / 128), unsigned(max_tiles)), g2(unsigned((a.H + 127) / 128), unsigned(max_tiles));
    if (a.gz)
        moe_gate_up_tile_kernel<true><<<g1, 512, 0, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets, a.pair_tok,
                                                         a.tile_e, a.tile_m0, a.n_tiles, a.x, a.H, a.F, a.h);
    else
        moe_gate_up_tile_kernel<false><<<g1, 512, 0, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets, a.pair_tok,
                                                          a.tile_e, a.tile_m0, a.n_tiles, a.x, a.H, a.F, a.h);
    if (a.dz)
        moe_down_tile_kernel<true><<<g2, 512, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.tile_e, a.tile_m0, a.n_tiles,
                                                      a.h, a.H, a.F, a.yp);
    else
        moe_down_tile_kernel<false><<<g2, 512, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.tile_e, a.tile_m0, a.n_tiles,
                                                       a.h, a.H, a.F, a.yp);
}

}  // namespace qwq4
