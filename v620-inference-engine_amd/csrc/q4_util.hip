// Format kernels: nibble unpack, exact dequantisation and conversion from the
// reference engine's repacked word order. These are the bit-exact parity
// surface of the q4 format (reference: src/ref/ref_model.cpp:108-114,
// src/engine/weight_convert.cpp:61-71).
#include "q4_common.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

// out[n][8c+i] = (W[n][c] >> 4i) & 0xf; one thread per word, 8 bytes out.
__global__ void unpack_kernel(const uint32_t *__restrict__ W, int64_t n_words, uint8_t *__restrict__ out) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n_words) return;
    const uint32_t w = W[i];
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    uint2 r;
    r.x = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // e0 e1 e2 e3
    r.y = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // e4 e5 e6 e7
    *reinterpret_cast<uint2 *>(out + i * 8) = r;
}

// out[n][k] = float(q - z) * float(s), one thread per word.
__global__ void dequant_kernel(const uint32_t *__restrict__ W, const uint16_t *__restrict__ S,
                               const uint32_t *__restrict__ Z, int64_t N, int64_t K, float *__restrict__ out) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t wpr = K / 8;
    if (i >= N * wpr) return;
    const int64_t n = i / wpr, c = i % wpr;
    const int G = int(K / QGROUP), g = int(c * 8 / QGROUP);
    const float s = f16_bits_to_f32(S[n * G + g]);
    const int z = group_zero(Z, n, (G + 7) / 8, g);
    const uint32_t w = W[i];
    float4 a, b;
    a.x = float(int(w & 0xfu) - z) * s;
    a.y = float(int((w >> 4) & 0xfu) - z) * s;
    a.z = float(int((w >> 8) & 0xfu) - z) * s;
    a.w = float(int((w >> 12) & 0xfu) - z) * s;
    b.x = float(int((w >> 16) & 0xfu) - z) * s;
    b.y = float(int((w >> 20) & 0xfu) - z) * s;
    b.z = float(int((w >> 24) & 0xfu) - z) * s;
    b.w = float(int((w >> 28) & 0xfu) - z) * s;
    float4 *o = reinterpret_cast<float4 *>(out + i * 8);
    o[0] = a;
    o[1] = b;
}

// Engine order (element 2m at bits 4m, element 2m+1 at bits 16+4m) back to
// the checkpoint order (element i at bits 4i).
__global__ void from_engine_kernel(const uint32_t *__restrict__ in, uint32_t *__restrict__ out, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t w = in[i];
    uint32_t r = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        r |= ((w >> (4 * m)) & 0xfu) << (8 * m);
        r |= ((w >> (16 + 4 * m)) & 0xfu) << (8 * m + 4);
    }
    out[i] = r;
}

static unsigned blocks(int64_t n, int b) { return unsigned((n + b - 1) / b); }

void launch_unpack(const uint32_t *W, int64_t N, int64_t K, uint8_t *out, hipStream_t s) {
    const int64_t n = N * (K / 8);
    unpack_kernel<<<blocks(n, 256), 256, 0, s>>>(W, n, out);
}

void launch_dequant(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, float *out,
                    hipStream_t s) {
    dequant_kernel<<<blocks(N * (K / 8), 256), 256, 0, s>>>(W, S, Z, N, K, out);
}

void launch_from_engine_order(const uint32_t *in, uint32_t *out, int64_t n, hipStream_t s) {
    from_engine_kernel<<<blocks(n, 256), 256, 0, s>>>(in, out, n);
}

}  // namespace qwq4
