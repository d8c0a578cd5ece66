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

__global__ __launch_bounds__(512) void moe_gate_up_tile_kernel(
    const uint32_t *__restrict__ gw, const uint16_t *__restrict__ gs, const uint32_t *__restrict__ gz,
    const uint32_t *__restrict__ uw, const uint16_t *__restrict__ us, const uint32_t *__restrict__ uz,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ pair_tok, const int32_t *__restrict__ tile_e,
    const int32_t *__restrict__ tile_m0, const int32_t *__restrict__ n_tiles, const uint16_t *__restrict__ x, int H,
    int F, uint16_t *__restrict__ h) {
    const int tile = blockIdx.y;
    if (tile >= *n_tiles) return;
    const int e = tile_e[tile], m0 = tile_m0[tile];
    const int base = offsets[e] + m0, M = min(GROUPED_TILE_M, offsets[e + 1] - offsets[e] - m0);
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16;
    const int G = H / QGROUP, zw = (G + 7) / 8;
    const int n = (blockIdx.x * 8 + wave) * 16 + lane % 16;
    const int64_t row = int64_t(e) * F + (n < F ? n : F - 1);
    const uint32_t *wrow[2] = {gw + row * (H / 8), uw + row * (H / 8)};
    const uint16_t *srow[2] = {gs + row * G, us + row * G};
    const uint32_t *zrow[2] = {gz ? gz + row * zw : nullptr, uz ? uz + row * zw : nullptr};
    const uint16_t *arow[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const int m = mb * 16 + lane % 16;
        arow[mb] = m < M ? x + int64_t(pair_tok[base + m]) * H : nullptr;
    }
    f32x4 acc[2][2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) acc[mb][0] = acc[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    q4_groups<BF16, 2, 2, false>(wrow, srow, zrow, arow, 0, G, q, acc);
    if (n >= F) return;
    const int col = (n & ~7) + op_pos(n & 7);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m >= M) continue;
            const float g = acc[mb][0][r], u = acc[mb][1][r];
            float v = g / (1.f + __expf(-g)) * u;
            v = fminf(fmaxf(v, -65504.f), 65504.f);
            h[int64_t(base + m) * F + col] = __builtin_bit_cast(uint16_t, _Float16(v));
        }
}

__global__ __launch_bounds__(512) void moe_down_tile_kernel(const uint32_t *__restrict__ dw,
                                                            const uint16_t *__restrict__ ds,
                                                            const uint32_t *__restrict__ dz,
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
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16;
    const int G = F / QGROUP, zw = (G + 7) / 8;
    const int n = (blockIdx.x * 8 + wave) * 16 + lane % 16;
    const int64_t row = int64_t(e) * H + (n < H ? n : H - 1);
    const uint32_t *wrow[1] = {dw + row * (F / 8)};
    const uint16_t *srow[1] = {ds + row * G};
    const uint32_t *zrow[1] = {dz ? dz + row * zw : nullptr};
    const uint16_t *arow[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const int m = mb * 16 + lane % 16;
        arow[mb] = m < M ? h + int64_t(base + m) * F : nullptr;
    }
    f32x4 acc[2][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}, {f32x4{0.f, 0.f, 0.f, 0.f}}};
    q4_groups<F16, 2, 1, true>(wrow, srow, zrow, arow, 0, G, q, acc);
    if (n >= H) return;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m < M) yp[int64_t(base + m) * H + n] = acc[mb][0][r];
        }
}

int moe_grouped_tile_m() { return GROUPED_TILE_M; }

void launch_moe_grouped(const MoeGroupedArgs &a, hipStream_t s) {
    const int max_tiles = a.T * a.topk / GROUPED_TILE_M + a.E;
    const dim3 g1(unsigned((a.F + 127) / 128), unsigned(max_tiles)), g2(unsigned((a.H + 127) / 128), unsigned(max_tiles));
    moe_gate_up_tile_kernel<<<g1, 512, 0, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets, a.pair_tok, a.tile_e,
                                               a.tile_m0, a.n_tiles, a.x, a.H, a.F, a.h);
    moe_down_tile_kernel<<<g2, 512, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.tile_e, a.tile_m0, a.n_tiles, a.h, a.H,
                                            a.F, a.yp);
}

}  // namespace qwq4
