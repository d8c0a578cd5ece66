// Routing pieces shared by the routing kernels (moe_route.hip) and the
// decode experts that route their own tokens (moe_gemv.hip): the C library's
// expf evaluated on the device, wave-wide DPP reductions and scans, and the
// top-k of one token by one wave.
//
// Reference: the math of ref::Model::moe (src/ref/ref_model.cpp:412-431).
#pragma once

#include "q4_common.cuh"

namespace qwq4 {

// ---- glibc's expf (glibc 2.28 and later; the algorithm of ARM's
// optimized-routines expf): with N = 32, x * N / ln 2 = k + r, |r| <= 1/2,
// exp(x) = 2^(k/N) * 2^(r/N), 2^(k/N) from a table of 2^(i/N) (i = k mod N,
// the integer part of k / N added to the exponent bits), 2^(r/N) by the
// cubic 1 + C2 r + C1 r^2 + C0 r^3, all in double, rounded to float once.
// Table entry i is the double nearest 2^(i/32) with i << 47 subtracted from
// its bits (so adding k << 47 scales it by 2^(k div 32)). The result equals
// the C library's expf on every float in [-4, 0) and on a sample below (a
// test compares them); for x below ln(2^-150) it is 0, as there.
static __device__ const uint64_t kExp2Tab32[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

struct ExpfGlibc {
    uint32_t lo, hi;  // this lane's table entry, lane % 32
    __device__ __forceinline__ void load(int lane) {
        const uint64_t t = kExp2Tab32[lane & 31];
        lo = uint32_t(t);
        hi = uint32_t(t >> 32);
    }
    // every lane of the wave must call it (the table lookup is a cross-lane
    // permute)
    __device__ __forceinline__ float operator()(float x) const {
#pragma clang fp contract(off)
        constexpr double InvLn2N = 0x1.71547652b82fep+0 * 32, Shift = 0x1.8p+52;
        constexpr double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                         C2 = 0x1.62e42ff0c52d6p-1 / 32;
        const double z = InvLn2N * double(x);
        double kd = z + Shift;
        const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
        kd -= Shift;
        const double r = z - kd;
        const int src = int(ki & 31) * 4;
        const uint64_t t = ((uint64_t(uint32_t(__builtin_amdgcn_ds_bpermute(src, int(hi)))) << 32) |
                            uint32_t(__builtin_amdgcn_ds_bpermute(src, int(lo)))) +
                           (ki << 47);
        const double sc = __builtin_bit_cast(double, t);
        const double zz = __builtin_fma(C0, r, C1), r2 = r * r;
        const double y = __builtin_fma(zz, r2, __builtin_fma(C2, r, 1.0)) * sc;
        return x < -0x1.9fe368p6f ? 0.f : float(y);
    }
};


// ---- wave-wide reductions and scans on DPP (row-local lane permutes, no
// LDS traffic) plus readlane across the four 16-lane rows
#define QW_DPP(v, ctrl, rm, bm, bc) \
    uint32_t(__builtin_amdgcn_update_dpp(0, int(v), ctrl, rm, bm, bc))

constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <-> 7 - i within 8
constexpr int DPP_MIRROR = 0x140;       // lane i <-> 15 - i within 16
constexpr int DPP_BCAST15 = 0x142;      // lane 15 of each row into the next row
constexpr int DPP_BCAST31 = 0x143;      // lane 31 into rows 2 and 3


// Wave maximum of a 32-bit unsigned value (lane 63's result, read to every
// lane): each step's DPP move fuses into the max instruction.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#define QW_UMAX_STEP(ctrl, rm) v = max(v, QW_DPP(v, ctrl, rm, 0xf, false));
    QW_UMAX_STEP(DPP_XOR1, 0xf)
    QW_UMAX_STEP(DPP_XOR2, 0xf)
    QW_UMAX_STEP(DPP_HALF_MIRROR, 0xf)
    QW_UMAX_STEP(DPP_MIRROR, 0xf)
    QW_UMAX_STEP(DPP_BCAST15, 0xa)
    QW_UMAX_STEP(DPP_BCAST31, 0xc)
#undef QW_UMAX_STEP
    return uint32_t(__builtin_amdgcn_readlane(int(v), 63));
}

// The wave maximum of 64-bit keys as two 32-bit maxima: the high words',
// then the low words' among the lanes whose high word is that maximum (the
// same order as comparing whole keys).
__device__ __forceinline__ uint64_t wave_max_key(uint64_t v) {
    const uint32_t hi = uint32_t(v >> 32), mh = wave_max_u32(hi);
    const uint64_t at = __ballot(hi == mh);
    // one lane holds the largest high word (the usual case: no two equal
    // probabilities): its key is the maximum, no second reduction
    if ((at & (at - 1)) == 0ull) return (uint64_t(mh) << 32) | uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v)), __builtin_ctzll(at)));
    const uint32_t ml = wave_max_u32(hi == mh ? uint32_t(v) : 0u);
    return (uint64_t(mh) << 32) | ml;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#define QW_FMAX_STEP(ctrl) v = fmaxf(v, __builtin_bit_cast(float, QW_DPP(__builtin_bit_cast(uint32_t, v), ctrl, 0xf, 0xf, false)));
    QW_FMAX_STEP(DPP_XOR1)
    QW_FMAX_STEP(DPP_XOR2)
    QW_FMAX_STEP(DPP_HALF_MIRROR)
    QW_FMAX_STEP(DPP_MIRROR)
#undef QW_FMAX_STEP
    // as in wave_max_u32 (masked-off lanes read 0 and may end wrong; only
    // lane 63, in both masks, is read)
#define QW_FMAX_STEP_RM(ctrl, rm) \
    v = fmaxf(v, __builtin_bit_cast(float, QW_DPP(__builtin_bit_cast(uint32_t, v), ctrl, rm, 0xf, false)));
    QW_FMAX_STEP_RM(DPP_BCAST15, 0xa)
    QW_FMAX_STEP_RM(DPP_BCAST31, 0xc)
#undef QW_FMAX_STEP_RM
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Inclusive prefix sum over the wave's 64 lanes (the GCN row_shr /
// row_bcast sequence).
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t x) {
    uint32_t s = x + QW_DPP(x, 0x111, 0xf, 0xf, true);   // row_shr:1
    s += QW_DPP(x, 0x112, 0xf, 0xf, true);               // row_shr:2
    s += QW_DPP(x, 0x113, 0xf, 0xf, true);               // row_shr:3
    s += QW_DPP(s, 0x114, 0xf, 0xe, true);               // row_shr:4, banks 1-3
    s += QW_DPP(s, 0x118, 0xf, 0xc, true);               // row_shr:8, banks 2-3
    s += QW_DPP(s, 0x142, 0xa, 0xf, false);              // row_bcast:15 into rows 1, 3
    s += QW_DPP(s, 0x143, 0xc, 0xf, false);              // row_bcast:31 into rows 2, 3
    return s;
}

// One wave routes one token; the wave's lanes hold PER logits each (expert
// lane + 64 i). A selection key packs the probability's bits (p >= 0, so
// they order like p) over the complement of the expert index, so one 64-bit
// maximum picks the largest p and, among equal p, the lowest index. Lane
// j < k ends with the j-th selection.
// ex: the lane's expf table entry, loaded by the caller at kernel start (its
// memory latency then overlaps the logits' instead of following them).
template <int PER, class LogitFn>
__device__ __forceinline__ void topk_wave(const ExpfGlibc &ex, LogitFn logit, int E, int k, int lane, int32_t *te,
                                          float *tw) {
    float v[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int idx = lane + WAVE * i;
        v[i] = idx < E ? logit(idx) : -INFINITY;
        mx = fmaxf(mx, v[i]);
    }
    mx = wave_max_f32(mx);
    uint64_t key[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int idx = lane + WAVE * i;
        const float p = ex(v[i] - mx);
        key[i] = idx < E ? (uint64_t(__builtin_bit_cast(uint32_t, p)) << 32) | uint32_t(~uint32_t(idx)) : 0ull;
    }
    // the lane's keys in descending order (insertion network), so that its
    // best untaken key is always key[0]
#pragma unroll
    for (int i = 1; i < PER; ++i)
#pragma unroll
        for (int j = i; j > 0; --j) {
            const uint64_t a = key[j - 1], b = key[j];
            key[j - 1] = a > b ? a : b;
            key[j] = a > b ? b : a;
        }
    double top = 0.0;
    int my_e = 0;
    float my_p = 0.f;
    for (int j = 0; j < k; ++j) {
        const uint64_t w = wave_max_key(key[0]);
        if (key[0] == w) {  // taken (keys are distinct: one lane): its next key moves up
#pragma unroll
            for (int i = 0; i + 1 < PER; ++i) key[i] = key[i + 1];
            key[PER - 1] = 0ull;
        }
        const float p = __builtin_bit_cast(float, uint32_t(w >> 32));
        top += double(p);
        if (lane == j) {
            my_e = int(~uint32_t(w));
            my_p = p;
        }
    }
    if (lane < k) {
        te[lane] = my_e;
        tw[lane] = float(double(my_p) / top);
    }
}

}  // namespace qwq4
