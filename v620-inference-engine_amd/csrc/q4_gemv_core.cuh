// Wave-level pieces of the q4 GEMVs (dense decode rows and routed experts).
//
// A wave owns a 16-row subtile of the tiled weights and a range of the
// 128-wide K groups. Lane l serves weight row n = l % 16 and K quarter
// q = l / 16 of every group: one 16-byte load per lane per group, 1 KB of
// contiguous HBM per wave instruction, nibbles unpacked in registers
// (q4_common.cuh). The MFMA's other operand is the activations, staged in
// LDS: lane l feeds token row m = l % 16, so the 16x16 result holds every
// (token, row) pair; each lane ends with one weight row n and four token rows
// 4(l/16) + r, so the group scale and zero are one value per lane.
#pragma once

#include "q4_common.cuh"

namespace qwq4 {

// LDS-only barrier: orders this block's LDS traffic without draining the
// global-memory loads in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 16-byte pieces of M activation rows of K elements, rounded to whole waves.
__host__ __device__ inline int x_pieces(int M, int K) { return (M * (K / 8) + WAVE - 1) / WAVE * WAVE; }

// Rows 0..M-1 (row m starts at row(m)) of K 16-bit elements -> LDS [M][K]
// with direct global->LDS loads (no registers; 1 KB per wave instruction).
// Issued before the weight loads; the barrier that follows those waits for
// both, so activations (L2) and weights (HBM) are requested before anything
// waits.
template <class RowFn>
__device__ __forceinline__ void stage_rows_issue(RowFn row, int M, int K, uint4 *xl) {
    const int kc = K / 8, total = M * kc, wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int nw = blockDim.x / WAVE;
    for (int base = wave * WAVE; base < total; base += nw * WAVE) {
        const int i = min(base + lane, total - 1), m = i / kc, c = i - m * kc;
        __builtin_amdgcn_global_load_lds(row(m) + c * 8, xl + base, 16, 0, 0);
    }
}

// One group of one subtile: acc[mb] += s * (x . (q - z)) for the lane's rows.
// xr[mb] points at the lane's activation row (LDS) at K quarter q.
template <typename T, int MB>
__device__ __forceinline__ void dense_group(const uint4 &w, uint32_t zb, float s, const uint4 *const (&xr)[MB], int g,
                                            f32x4 (&acc)[MB]) {
    const uint4 negb = make_uint4(T::NEG_BIAS, T::NEG_BIAS, T::NEG_BIAS, T::NEG_BIAS);
    uint4 b[4];
    b[0] = unpack8<T>(w.x, zb);
    b[1] = unpack8<T>(w.y, zb);
    b[2] = unpack8<T>(w.z, zb);
    b[3] = unpack8<T>(w.w, zb);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        uint4 a[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t] = xr[mb][g * 16 + t];
        f32x4 p = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) p = mfma16<T>(a[t], negb, p);
#pragma unroll
        for (int t = 0; t < 4; ++t) p = mfma16<T>(a[t], b[t], p);
        acc[mb] += s * p;
    }
}

// A wave's whole K range of one subtile (groups g0 .. g0 + n - 1, n <= GW),
// requested up front into registers.
template <int GW, bool HAS_Z>
struct WaveRange {
    uint4 w[GW];
    uint32_t sv[GW], zv[GW];
    int g0, n;
    __device__ __forceinline__ void fetch(const Q4Tile &t, int g0_, int n_, int lane) {
        g0 = g0_;
        n = n_;
        const int r = lane % 16;
#pragma unroll
        for (int c = 0; c < GW; ++c) {
            const int g = g0 + min(c, n - 1);
            w[c] = t.word4(g, lane);
            sv[c] = t.scale(g, r);
            if constexpr (HAS_Z) zv[c] = t.zero_word(g, r);
        }
    }
    template <typename T, int MB>
    __device__ __forceinline__ void compute(const uint4 *const (&xr)[MB], f32x4 (&acc)[MB]) const {
#pragma unroll
        for (int c = 0; c < GW; ++c) {
            if (c < n) {
                const int g = g0 + c;
                const uint32_t zb = zero_bytes(HAS_Z ? Q4Tile::zero_of(zv[c], g) : 8u);
                dense_group<T, MB>(w[c], zb, f16_bits_to_f32(uint16_t(sv[c])), xr, g, acc);
            }
        }
    }
};

__device__ __forceinline__ void store_y(void *y, int64_t o, float v, int y_bf16, int accumulate) {
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

}  // namespace qwq4
