// Block bodies of the 16-bit GEMVs (w16_gemv.hip): each takes its row tile
// (bx) as an argument, so a kernel that also runs other work in the same
// grid (the fused MoE decode block's launches) can call it for a part of its
// blocks. Blocks are W16_MAX_KS waves when K allows (K / 32 >= 8).
#pragma once

#include "q4_gemv_core.cuh"

namespace qwq4 {

constexpr int W16_MAX_KS = 8;  // waves per block

// WS: 32-element MFMA steps a wave keeps in flight (8 or 16: 32 or 64 VGPRs),
// the smallest that holds its range where one does (the shared expert's down
// projection, 6 steps per wave: 16 held 81-97 VGPRs, 4-5 waves per SIMD;
// 8 make it 10% faster per layer)
template <typename XT, int MB, int MR, int XPT, int WS, bool TILED>
__device__ __forceinline__ void w16_gemv_block(const uint16_t *W, int ldw, const uint16_t *x, int xs, int M, int K, int N,
                                               void *__restrict__ y, int ys, int y_bf16, int accumulate, int n_lo,
                                               int bx) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int KS = blockDim.x / WAVE;
    const int tid = threadIdx.x, kp = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE, q = lane / 16,
              n = lane % 16;
    const int steps = K / 32, spw = (steps + KS - 1) / KS, s0 = kp * spw, ns = min(spw, steps - s0);
    const int kc = x_row_stride(K);
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    float *red = reinterpret_cast<float *>(xl + x_pieces(M, K));
    XRegs xv;
    if constexpr (XPT > 0) stage_regs_issue<XPT>(x, xs, M, K, xv);
    else stage_x_issue(x, xs, M, K, xl);
    __builtin_amdgcn_sched_barrier(0);  // every activation load goes out before the weight loads
    // lane (n, q): 8 weights of row n at K 32 s + 8 q, step s. Row-major: 64
    // bytes of each of 16 rows per wave load; tiled: the step's 1 KB entry.
    const uint4 *wrow =
        TILED ? reinterpret_cast<const uint4 *>(W) + int64_t(bx) * steps * 64 + lane
              : reinterpret_cast<const uint4 *>(W + int64_t(min(bx * 16 + n, N - 1)) * ldw + 8 * q);
    constexpr int STEP = TILED ? 64 : 4;  // uint4 entries from one step to the next
    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    uint4 w[WS];
    auto fetch = [&](int p) {  // steps p .. p + WS - 1 of the wave's range (clamped, no branches)
#pragma unroll
        for (int t = 0; t < WS; ++t) {
            const int s = min(s0 + min(p + t, max(ns - 1, 0)), steps - 1);
            const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wrow + s * STEP));
            w[t] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    };
    fetch(0);
    if constexpr (XPT > 0) {
        __builtin_amdgcn_sched_barrier(0);
        stage_regs_commit<XPT>(xv, M, K, xl);
        lds_barrier();
    } else {
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_below<WS>();  // this wave's activation loads (its oldest)
        __builtin_amdgcn_s_barrier();
    }
    const uint4 *xr[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xr[mb] = xl + min(mb * 16 + n, M - 1) * kc + q;
    for (int p = 0; p < ns; p += WS) {
        if (p > 0) fetch(p);
#pragma unroll
        for (int t = 0; t < WS; ++t)
            if (p + t < ns) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) acc[mb] = mfma16<XT>(xr[mb][(s0 + p + t) * 4], w[t], acc[mb]);
            }
    }
    ksplit_sum<MB, MR>(acc, red, KS, kp, kp, lane);
    if (kp == 0) store_rows<MB, MR>(acc, y, ys, y_bf16, accumulate, M, N, bx, lane, n_lo);
}


// SwiGLU x gate (see w16_gemv.hip)
__device__ __forceinline__ float sigmoid_gate(float gl) { return sigmoid_ref(gl); }
__device__ __forceinline__ uint16_t swiglu_h(float g, float u, float gate) {
    return __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(silu_ref(g) * u * gate));
}

struct SgPiece {
    float4 g0, g1, u0, u1;
    float gl;
};

__device__ __forceinline__ void sg_load(const float *v, int ldv, int n, int i, float rkn, SgPiece &p) {
    const int kn = n / 8, m = div_small(i, rkn), c = i - m * kn;
    // element loads: rows of 2n + 1 floats are not 16-byte aligned
    const float *g = v + int64_t(m) * ldv + c * 8, *u = g + n;
    p.g0 = make_float4(g[0], g[1], g[2], g[3]);
    p.g1 = make_float4(g[4], g[5], g[6], g[7]);
    p.u0 = make_float4(u[0], u[1], u[2], u[3]);
    p.u1 = make_float4(u[4], u[5], u[6], u[7]);
    p.gl = v[int64_t(m) * ldv + 2 * n];
}

__device__ __forceinline__ void sg_commit(const SgPiece &p, int n, int i, float rkn, uint4 *xl) {
    const int kn = n / 8, m = div_small(i, rkn), c = i - m * kn;
    const float gate = sigmoid_gate(p.gl);
    auto two = [&](float g0, float u0, float g1, float u1) {
        return uint32_t(swiglu_h(g0, u0, gate)) | (uint32_t(swiglu_h(g1, u1, gate)) << 16);
    };
    xl[m * x_row_stride(n) + c] = make_uint4(two(p.g0.x, p.u0.x, p.g0.y, p.u0.y), two(p.g0.z, p.u0.z, p.g0.w, p.u0.w),
                                             two(p.g1.x, p.u1.x, p.g1.y, p.u1.y), two(p.g1.z, p.u1.z, p.g1.w, p.u1.w));
}

template <int MB, int MR, int XPT, int WS>
__device__ __forceinline__ void w16_swiglu_block(const uint16_t *W, const float *v, int ldv, int M, int K, int N,
                                                 void *__restrict__ y, int ys, int y_bf16, int accumulate, int bx) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int KS = blockDim.x / WAVE;
    const int tid = threadIdx.x, kp = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE, q = lane / 16,
              n = lane % 16;
    const int steps = K / 32, spw = (steps + KS - 1) / KS, s0 = kp * spw, ns = min(spw, steps - s0);
    const int kc = x_row_stride(K), P = M * (K / 8), nt = blockDim.x;
    const float rkn = __builtin_amdgcn_rcpf(float(K / 8));
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    float *red = reinterpret_cast<float *>(xl + x_pieces(M, K));
    SgPiece p0, p1, p2, p3;  // named, not an array (see XRegs)
    if constexpr (XPT >= 1) sg_load(v, ldv, K, min(tid, P - 1), rkn, p0);
    if constexpr (XPT >= 2) sg_load(v, ldv, K, min(tid + nt, P - 1), rkn, p1);
    if constexpr (XPT >= 3) sg_load(v, ldv, K, min(tid + 2 * nt, P - 1), rkn, p2);
    if constexpr (XPT >= 4) sg_load(v, ldv, K, min(tid + 3 * nt, P - 1), rkn, p3);
    __builtin_amdgcn_sched_barrier(0);  // the activation loads go out before the weight loads
    const uint4 *wrow = reinterpret_cast<const uint4 *>(W) + int64_t(bx) * steps * 64 + lane;
    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    uint4 w[WS];
    auto fetch = [&](int p) {  // steps p .. p + WS - 1 of the wave's range (clamped, no branches)
#pragma unroll
        for (int t = 0; t < WS; ++t) {
            const int s = min(s0 + min(p + t, max(ns - 1, 0)), steps - 1);
            const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wrow + s * 64));
            w[t] = make_uint4(u[0], u[1], u[2], u[3]);
        }
    };
    fetch(0);
    __builtin_amdgcn_sched_barrier(0);
    // unconditional commits (a thread past the end rewrites the last piece
    // with the same value), as in stage_regs_commit
    if constexpr (XPT >= 1) sg_commit(p0, K, min(tid, P - 1), rkn, xl);
    if constexpr (XPT >= 2) sg_commit(p1, K, min(tid + nt, P - 1), rkn, xl);
    if constexpr (XPT >= 3) sg_commit(p2, K, min(tid + 2 * nt, P - 1), rkn, xl);
    if constexpr (XPT >= 4) sg_commit(p3, K, min(tid + 3 * nt, P - 1), rkn, xl);
    if constexpr (XPT == 0)
        for (int i = tid; i < P; i += nt) {
            SgPiece p;
            sg_load(v, ldv, K, i, rkn, p);
            sg_commit(p, K, i, rkn, xl);
        }
    lds_barrier();
    const uint4 *xr[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xr[mb] = xl + min(mb * 16 + n, M - 1) * kc + q;
    for (int p = 0; p < ns; p += WS) {
        if (p > 0) fetch(p);
#pragma unroll
        for (int t = 0; t < WS; ++t)
            if (p + t < ns) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) acc[mb] = mfma16<F16>(xr[mb][(s0 + p + t) * 4], w[t], acc[mb]);
            }
    }
    ksplit_sum<MB, MR>(acc, red, KS, kp, kp, lane);
    if (kp == 0) store_rows<MB, MR>(acc, y, ys, y_bf16, accumulate, M, N, bx, lane);
}

}  // namespace qwq4
