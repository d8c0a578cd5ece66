// q4-dequant prefill GEMM: Y[t][n] = sum_k X[t][k] * W[n][k] for a chunk of
// T tokens (reference role: gpu::gemm, src/kernels/gemm.hip:10-18, which
// calls rocBLAS on fp16 weights; here the weights stay q4 in HBM and are
// unpacked on the fly for the bf16 MFMA).
//
// This first version computes each 16-row x 32-token tile with the GEMV wave
// core (q4_wave.cuh): correct, MFMA-based, but it re-reads weight rows from
// L2 for every 32 tokens.
#include "q4_kernels.hpp"
#include "q4_wave.cuh"

namespace qwq4 {

size_t gemm_workspace_bytes(int T, int K) {
    const size_t xp = size_t(T) * K * 2, xs = size_t(T) * (K / QGROUP) * 4;
    return ((xp + 255) & ~size_t(255)) + ((xs + 255) & ~size_t(255));
}

template <bool HAS_Z>
__global__ __launch_bounds__(512) void q4_gemm_simple_kernel(const uint32_t *__restrict__ W,
                                                             const uint16_t *__restrict__ S,
                                                             const uint16_t *__restrict__ Z,
                                                             const uint16_t *__restrict__ X, int ldx, int T,
                                                             void *__restrict__ Y, int ldy, int y_bf16, int N, int K) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16, n = lane % 16;
    const int nsub = N / 16, lsub = blockIdx.x * 8 + wave;
    const int t0 = blockIdx.y * 32;
    const int G = K / QGROUP;
    const Q4Tile tile[1] = {Q4Tile(W, S, Z, min(lsub, nsub - 1), G)};
    const uint16_t *arow[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) arow[mb] = X + int64_t(min(t0 + mb * 16 + n, T - 1)) * ldx;
    f32x4 acc[2][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}, {f32x4{0.f, 0.f, 0.f, 0.f}}};
    q4_groups<BF16, 2, 1, HAS_Z, 4>(tile, arow, 0, G, lane, acc);
    if (lsub >= nsub) return;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + mb * 16 + 4 * q + r;
            if (t >= T) continue;
            const int64_t o = int64_t(t) * ldy + lsub * 16 + n;
            if (y_bf16)
                static_cast<uint16_t *>(Y)[o] = f32_to_bf16_rne(acc[mb][0][r]);
            else
                static_cast<float *>(Y)[o] = acc[mb][0][r];
        }
}

void launch_gemm(const GemmArgs &a, hipStream_t s) {
    const int nsub = a.N / 16;
    const dim3 grid(unsigned((nsub + 7) / 8), unsigned((a.T + 31) / 32)), block(512);
    if (a.Z)
        q4_gemm_simple_kernel<true><<<grid, block, 0, s>>>(a.W, a.S, a.Z, a.X, a.ldx, a.T, a.Y, a.ldy, a.y_bf16, a.N,
                                                           a.K);
    else
        q4_gemm_simple_kernel<false><<<grid, block, 0, s>>>(a.W, a.S, a.Z, a.X, a.ldx, a.T, a.Y, a.ldy, a.y_bf16, a.N,
                                                            a.K);
}

}  // namespace qwq4
