// q4 GEMV for decode rows (M <= 32) and the gathered per-expert GEMV of routed
// MoE tokens, on the gfx950 16x16x32 MFMA.
//
// Reference roles: gpu::gemv_rows (src/kernels/gemv.hip:7-42, decode
// projections and LM head, fp16 weights there) and gpu::moe_experts_P
// (src/kernels/moe_experts.hip:189-245). The arithmetic is
// ref::Model::expert_linear (src/ref/ref_model.cpp:100-119) with a per-group
// zero point.
//
// Work split. A wave owns a 16-row subtile of W and a contiguous range of the
// 128-wide K groups; KS waves of a 512-thread block share one subtile (a K
// split, reduced through LDS in a fixed order), so small N still fills the
// chip. Lane l serves weight row n = l % 16 and K-quarter q = l / 16 of every
// group: one 16-byte load per lane per group, 1 KB per wave-instruction, the
// row's nibbles unpacked in registers (q4_common.cuh). The MFMA's other
// operand is the activations: lane l feeds token row m = l % 16 (zero beyond
// M), so the 16x16 result holds every (token, row) pair; each lane ends with
// one weight row n and four token rows 4(l/16) + r, so the group scale and
// zero are one value per lane.
#include "q4_wave.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

// ------------------------------------------------------------ dense GEMV
template <int KS, int MB>
__global__ __launch_bounds__(512) void q4_gemv_kernel(const uint32_t *__restrict__ W, const uint16_t *__restrict__ S,
                                                      const uint32_t *__restrict__ Z, const uint16_t *__restrict__ x,
                                                      int xs, void *__restrict__ y, int ys, int y_bf16, int N, int K,
                                                      int M, int accumulate) {
    constexpr int SUB = 8 / KS;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16;
    const int sub = blockIdx.x * SUB + wave / KS, kp = wave % KS;
    const int G = K / QGROUP, zw = (G + 7) / 8, gpk = G / KS;
    const int n = sub * 16 + lane % 16;
    const int64_t row = n < N ? n : N - 1;
    const uint32_t *wrow[1] = {W + row * (K / 8)};
    const uint16_t *srow[1] = {S + row * G};
    const uint32_t *zrow[1] = {Z ? Z + row * zw : nullptr};
    const uint16_t *arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = mb * 16 + lane % 16;
        arow[mb] = m < M ? x + int64_t(m) * xs : nullptr;
    }
    f32x4 acc[MB][1];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    q4_groups<BF16, MB, 1, false>(wrow, srow, zrow, arow, kp * gpk, kp * gpk + gpk, q, acc);
    ksplit_reduce<MB, 1, KS>(acc, wave, kp, lane);
    if (kp != 0 || n >= N) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m >= M) continue;
            const int64_t o = int64_t(m) * ys + n;
            float v = acc[mb][0][r];
            if (y_bf16) {
                uint16_t *yb = static_cast<uint16_t *>(y);
                if (accumulate) v += bf16_bits_to_f32(yb[o]);
                yb[o] = f32_to_bf16_rne(v);
            } else {
                float *yf = static_cast<float *>(y);
                if (accumulate) v += yf[o];
                yf[o] = v;
            }
        }
}

// Smallest power-of-two K split (<= 8, dividing the group count) that gives
// at least `want` waves.
static int pick_ks(int64_t subtiles, int G, int64_t want) {
    int ks = 1;
    while (ks < 8 && subtiles * ks < want && G % (ks * 2) == 0) ks *= 2;
    return ks;
}

template <int KS>
static void launch_gemv_ks(const GemvArgs &a, hipStream_t s) {
    const int64_t subtiles = (a.N + 15) / 16;
    const dim3 grid(unsigned((subtiles + (8 / KS) - 1) / (8 / KS))), block(512);
    if (a.M <= 16)
        q4_gemv_kernel<KS, 1><<<grid, block, 0, s>>>(a.W, a.S, a.Z, a.x, a.xs, a.y, a.ys, a.y_bf16, a.N, a.K, a.M,
                                                     a.accumulate);
    else
        q4_gemv_kernel<KS, 2><<<grid, block, 0, s>>>(a.W, a.S, a.Z, a.x, a.xs, a.y, a.ys, a.y_bf16, a.N, a.K, a.M,
                                                     a.accumulate);
}

void launch_gemv(const GemvArgs &a, hipStream_t s) {
    const int ks = pick_ks((a.N + 15) / 16, a.K / QGROUP, 2048);
    switch (ks) {
        case 1: launch_gemv_ks<1>(a, s); break;
        case 2: launch_gemv_ks<2>(a, s); break;
        case 4: launch_gemv_ks<4>(a, s); break;
        default: launch_gemv_ks<8>(a, s); break;
    }
}

// ------------------------------------------------ routed-expert GEMVs
// grid (row blocks of one expert, max active experts). Block y serves the
// y-th expert with tokens (active[] ascending); its M tokens are the slots
// offsets[e] .. offsets[e+1]-1.

// gate/up fused with SiLU * up: h[slot][F] (fp16, operand order within each
// 8-chunk, the layout the down GEMV reads).
template <int KS, int MB>
__global__ __launch_bounds__(512) void moe_gate_up_gemv_kernel(
    const uint32_t *__restrict__ gw, const uint16_t *__restrict__ gs, const uint32_t *__restrict__ gz,
    const uint32_t *__restrict__ uw, const uint16_t *__restrict__ us, const uint32_t *__restrict__ uz,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ active, const int32_t *__restrict__ n_active,
    const int32_t *__restrict__ pair_tok, const uint16_t *__restrict__ x, int H, int F, uint16_t *__restrict__ h) {
    if (int(blockIdx.y) >= *n_active) return;
    constexpr int SUB = 8 / KS;
    const int e = active[blockIdx.y];
    const int base = offsets[e], M = offsets[e + 1] - base;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16;
    const int sub = blockIdx.x * SUB + wave / KS, kp = wave % KS;
    const int G = H / QGROUP, zw = (G + 7) / 8, gpk = G / KS;
    const int n = sub * 16 + lane % 16;
    const int64_t row = int64_t(e) * F + (n < F ? n : F - 1);
    const uint32_t *wrow[2] = {gw + row * (H / 8), uw + row * (H / 8)};
    const uint16_t *srow[2] = {gs + row * G, us + row * G};
    const uint32_t *zrow[2] = {gz ? gz + row * zw : nullptr, uz ? uz + row * zw : nullptr};
    const uint16_t *arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = mb * 16 + lane % 16;
        arow[mb] = m < M ? x + int64_t(pair_tok[base + m]) * H : nullptr;
    }
    f32x4 acc[MB][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb][0] = acc[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    q4_groups<BF16, MB, 2, false>(wrow, srow, zrow, arow, kp * gpk, kp * gpk + gpk, q, acc);
    ksplit_reduce<MB, 2, KS>(acc, wave, kp, lane);
    if (kp != 0 || n >= F) return;
    const int col = (n & ~7) + op_pos(n & 7);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m >= M) continue;
            const float g = acc[mb][0][r], u = acc[mb][1][r];
            float v = g / (1.f + __expf(-g)) * u;
            v = fminf(fmaxf(v, -65504.f), 65504.f);  // fp16 range, saturating
            h[int64_t(base + m) * F + col] = __builtin_bit_cast(uint16_t, _Float16(v));
        }
}

// down: yp[slot][H] (fp32) = D_e h[slot].
template <int KS, int MB>
__global__ __launch_bounds__(512) void moe_down_gemv_kernel(const uint32_t *__restrict__ dw,
                                                            const uint16_t *__restrict__ ds,
                                                            const uint32_t *__restrict__ dz,
                                                            const int32_t *__restrict__ offsets,
                                                            const int32_t *__restrict__ active,
                                                            const int32_t *__restrict__ n_active,
                                                            const uint16_t *__restrict__ h, int H, int F,
                                                            float *__restrict__ yp) {
    if (int(blockIdx.y) >= *n_active) return;
    constexpr int SUB = 8 / KS;
    const int e = active[blockIdx.y];
    const int base = offsets[e], M = offsets[e + 1] - base;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16;
    const int sub = blockIdx.x * SUB + wave / KS, kp = wave % KS;
    const int G = F / QGROUP, zw = (G + 7) / 8, gpk = G / KS;
    const int n = sub * 16 + lane % 16;
    const int64_t row = int64_t(e) * H + (n < H ? n : H - 1);
    const uint32_t *wrow[1] = {dw + row * (F / 8)};
    const uint16_t *srow[1] = {ds + row * G};
    const uint32_t *zrow[1] = {dz ? dz + row * zw : nullptr};
    const uint16_t *arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = mb * 16 + lane % 16;
        arow[mb] = m < M ? h + int64_t(base + m) * F : nullptr;
    }
    f32x4 acc[MB][1];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    q4_groups<F16, MB, 1, true>(wrow, srow, zrow, arow, kp * gpk, kp * gpk + gpk, q, acc);
    ksplit_reduce<MB, 1, KS>(acc, wave, kp, lane);
    if (kp != 0 || n >= H) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m < M) yp[int64_t(base + m) * H + n] = acc[mb][0][r];
        }
}

template <int KS>
static void launch_moe_gemv_ks(const MoeGemvArgs &a, int max_active, bool down, hipStream_t s) {
    const int rows = down ? a.H : a.F;
    const int64_t subtiles = (rows + 15) / 16;
    const dim3 grid(unsigned((subtiles + (8 / KS) - 1) / (8 / KS)), unsigned(max_active)), block(512);
    const bool mb2 = a.T > 16;
    if (!down) {
        if (mb2)
            moe_gate_up_gemv_kernel<KS, 2><<<grid, block, 0, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets,
                                                                  a.active, a.n_active, a.pair_tok, a.x, a.H, a.F, a.h);
        else
            moe_gate_up_gemv_kernel<KS, 1><<<grid, block, 0, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets,
                                                                  a.active, a.n_active, a.pair_tok, a.x, a.H, a.F, a.h);
    } else {
        if (mb2)
            moe_down_gemv_kernel<KS, 2><<<grid, block, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.active, a.n_active, a.h,
                                                               a.H, a.F, a.yp);
        else
            moe_down_gemv_kernel<KS, 1><<<grid, block, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.active, a.n_active, a.h,
                                                               a.H, a.F, a.yp);
    }
}

static void launch_moe_one(const MoeGemvArgs &a, bool down, hipStream_t s) {
    const int max_active = a.T * a.topk < a.E ? a.T * a.topk : a.E;
    const int rows = down ? a.H : a.F, G = (down ? a.F : a.H) / QGROUP;
    // the K split is sized for the expected number of distinct experts
    // E (1 - (1 - k/E)^T) of T tokens routed uniformly
    double miss = 1.0;
    for (int t = 0; t < a.T; ++t) miss *= 1.0 - double(a.topk) / a.E;
    const int64_t expect = int64_t(a.E * (1.0 - miss)) > a.topk ? int64_t(a.E * (1.0 - miss)) : a.topk;
    const int ks = pick_ks(int64_t((rows + 15) / 16) * expect, G, 2048);
    switch (ks) {
        case 1: launch_moe_gemv_ks<1>(a, max_active, down, s); break;
        case 2: launch_moe_gemv_ks<2>(a, max_active, down, s); break;
        case 4: launch_moe_gemv_ks<4>(a, max_active, down, s); break;
        default: launch_moe_gemv_ks<8>(a, max_active, down, s); break;
    }
}

void launch_moe_gemv(const MoeGemvArgs &a, hipStream_t s) {
    launch_moe_one(a, false, s);
    launch_moe_one(a, true, s);
}

}  // namespace qwq4
