// The q4 MFMA wave core shared by the GEMV-shaped kernels: a wave owns a
// 16-row weight subtile and a range of 128-wide K groups (see q4_gemv.hip).
#pragma once

#include "q4_common.cuh"

namespace qwq4 {

// Per-group contribution for NB weight subtiles that share their activations
// (NB = 2 for the fused gate/up), over MB blocks of 16 token rows.
//   wrow[nb]  lane's weight row (uint32 words), srow[nb] its scales, zrow[nb]
//             its zero words (null: z = 8)
//   arow[mb]  lane's activation row (16-bit elements), null if the lane's
//             token row is beyond M
//   OPORDER   activations already stored in operand order
template <typename T, int MB, int NB, bool OPORDER>
__device__ __forceinline__ void q4_groups(const uint32_t *const (&wrow)[NB], const uint16_t *const (&srow)[NB],
                                          const uint32_t *const (&zrow)[NB], const uint16_t *const (&arow)[MB], int g0,
                                          int g1, int q, f32x4 (&acc)[MB][NB]) {
    const uint4 negb = make_uint4(T::NEG_BIAS, T::NEG_BIAS, T::NEG_BIAS, T::NEG_BIAS);

    for (int g = g0; g < g1; ++g) {
        uint4 wv[NB];
        float s[NB];
        uint32_t zb[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            wv[nb] = *reinterpret_cast<const uint4 *>(wrow[nb] + g * 16 + q * 4);
            s[nb] = f16_bits_to_f32(srow[nb][g]);
            zb[nb] = zero_bytes(zrow[nb] ? (zrow[nb][g >> 3] >> (4 * (g & 7))) & 0xfu : 8u);
        }
        uint4 a[MB][4];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            if (arow[mb]) {
                const uint4 *src = reinterpret_cast<const uint4 *>(arow[mb] + g * QGROUP + q * 32);
#pragma unroll
                for (int t = 0; t < 4; ++t) a[mb][t] = OPORDER ? src[t] : act_perm(src[t]);
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) a[mb][t] = make_uint4(0, 0, 0, 0);
            }
        }
        f32x4 xsn[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            xsn[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) xsn[mb] = mfma16<T>(a[mb][t], negb, xsn[mb]);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            uint4 b[4];
            b[0] = unpack8<T>(wv[nb].x, zb[nb]);
            b[1] = unpack8<T>(wv[nb].y, zb[nb]);
            b[2] = unpack8<T>(wv[nb].z, zb[nb]);
            b[3] = unpack8<T>(wv[nb].w, zb[nb]);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                f32x4 p = xsn[mb];
#pragma unroll
                for (int t = 0; t < 4; ++t) p = mfma16<T>(a[mb][t], b[t], p);
                acc[mb][nb] += s[nb] * p;
            }
        }
    }
}

// Sums the KS partial results of a subtile in k-part order (deterministic).
// All waves of the block must call it.
template <int MB, int NB, int KS>
__device__ __forceinline__ void ksplit_reduce(f32x4 (&acc)[MB][NB], int wave, int kp, int lane) {
    if constexpr (KS > 1) {
        __shared__ f32x4 red[8][MB * NB][WAVE];
        if (kp != 0) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) red[wave][mb * NB + nb][lane] = acc[mb][nb];
        }
        __syncthreads();
        if (kp == 0) {
#pragma unroll
            for (int j = 1; j < KS; ++j)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] += red[wave + j][mb * NB + nb][lane];
        }
    }
}

}  // namespace qwq4
