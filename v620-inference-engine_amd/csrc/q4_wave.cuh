// The q4 MFMA wave core shared by the GEMV-shaped kernels (routed-expert
// GEMVs, the grouped expert GEMM): a wave owns a 16-row weight subtile and a
// range of 128-wide K groups.
//
// Lane l serves weight row n = l % 16 and K quarter q = l / 16 of every
// group; the MFMA's other operand is the activations, lane l feeding token
// row m = l % 16 (+16 per row block). Lanes whose token row is past M read a
// valid row anyway: rows of the product do not mix, so those outputs are
// simply not stored. Nothing on the load path is under a divergent branch.
#pragma once

#include "q4_common.cuh"

namespace qwq4 {

// Accumulates sum over groups [g0, g1) of s_g * (x . (q - z)) into acc for NB
// weight subtiles sharing their activations (NB = 2: fused gate/up) and MB
// blocks of 16 token rows.
//   tile[nb]  the subtiles, arow[mb] the lane's activation row (T elements)
// Groups are processed in chunks of CH; the weights of the next chunk are
// requested before the current one is computed.
template <typename T, int MB, int NB, bool HAS_Z, int CH>
__device__ __forceinline__ void q4_groups(const Q4Tile (&tile)[NB], const uint16_t *const (&arow)[MB], int g0, int g1,
                                          int lane, f32x4 (&acc)[MB][NB]) {
    if (g0 >= g1) return;
    const int q = lane / 16, n = lane % 16;
    const uint4 negb = make_uint4(T::NEG_BIAS, T::NEG_BIAS, T::NEG_BIAS, T::NEG_BIAS);
    uint4 wc[CH][NB];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) wc[c][nb] = tile[nb].word4(min(g0 + c, g1 - 1), lane);
    for (int gb = g0; gb < g1; gb += CH) {
        uint4 wn[CH][NB];
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) wn[c][nb] = tile[nb].word4(min(gb + CH + c, g1 - 1), lane);
        uint32_t sraw[CH][NB], zraw[CH][NB];
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int g = min(gb + c, g1 - 1);
                sraw[c][nb] = tile[nb].scale(g, n);
                if constexpr (HAS_Z) zraw[c][nb] = tile[nb].zero_word(g, n);
            }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int g = gb + c;
            if (g >= g1) break;
            uint4 a[MB][4];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const uint4 *src = reinterpret_cast<const uint4 *>(arow[mb] + g * QGROUP + q * 32);
#pragma unroll
                for (int t = 0; t < 4; ++t) a[mb][t] = src[t];
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
                const uint32_t zb = zero_bytes(HAS_Z ? Q4Tile::zero_of(zraw[c][nb], g) : 8u);
                const float s = f16_bits_to_f32(uint16_t(sraw[c][nb]));
                uint4 b[4];
                b[0] = unpack8<T>(wc[c][nb].x, zb);
                b[1] = unpack8<T>(wc[c][nb].y, zb);
                b[2] = unpack8<T>(wc[c][nb].z, zb);
                b[3] = unpack8<T>(wc[c][nb].w, zb);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    f32x4 p = xsn[mb];
#pragma unroll
                    for (int t = 0; t < 4; ++t) p = mfma16<T>(a[mb][t], b[t], p);
                    acc[mb][nb] += s * p;
                }
            }
        }
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) wc[c][nb] = wn[c][nb];
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

// silu(g) * u, saturated to the fp16 range, as fp16 bits.
__device__ __forceinline__ uint16_t silu_mul_f16(float g, float u) {
    float v = g / (1.f + __expf(-g)) * u;
    v = fminf(fmaxf(v, -65504.f), 65504.f);
    return __builtin_bit_cast(uint16_t, _Float16(v));
}

}  // namespace qwq4
