// Dense GEMV on 16-bit weights, and the shared expert's SwiGLU with its
// sigmoid gate.
//
// Reference roles: gpu::gemv_rows with fp16 weights (src/kernels/gemv.hip:7-42;
// the engine runs the shared expert's gate/up and down projections through
// it, src/engine/decode.hip:99-101) and ref::Model::linear on bf16 weights
// (src/ref/ref_model.cpp:86-97); gpu::swiglu_T (src/kernels/moe_route.hip:187-197).
//
// The weights are row-major [N][ldw] as the checkpoint holds them, or in the
// tiled layout qw_w16_tile writes once at load (below), fp16 with
// fp16 activations or bf16 with bf16 ones: the 16x16x32 MFMA takes both as
// they are, so a product needs no conversion and every product is exact
// (fp32 sums). The kernel shape is the q4 GEMV's (q4_gemv_impl.cuh): a block
// holds one 16-row tile, its KS waves split K, each wave requests its whole
// range of weight rows (16 B per lane per 32-element MFMA step, up to
// 8 or 16 steps at once, WS below) before anything waits, the activations are staged
// in LDS, and the KS partial sums are added through LDS in k-part order.
#include <type_traits>

#include "q4_gemv_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

constexpr int W16_MAX_KS = 8;  // waves per block

// WS: 32-element MFMA steps a wave keeps in flight (8 or 16: 32 or 64 VGPRs),
// the smallest that holds its range where one does (the shared expert's down
// projection, 6 steps per wave: 16 held 81-97 VGPRs, 4-5 waves per SIMD;
// 8 make it 10% faster per layer)
template <typename XT, int MB, int MR, int XPT, int WS, bool TILED>
__global__ __launch_bounds__(W16_MAX_KS *WAVE) void w16_gemv_kernel(const uint16_t *W, int ldw, const uint16_t *x,
                                                                    int xs, int M, int K, int N, void *__restrict__ y,
                                                                    int ys, int y_bf16, int accumulate, int n_lo) {
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
        TILED ? reinterpret_cast<const uint4 *>(W) + int64_t(blockIdx.x) * steps * 64 + lane
              : reinterpret_cast<const uint4 *>(W + int64_t(min(int(blockIdx.x) * 16 + n, N - 1)) * ldw + 8 * q);
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
    if (kp == 0) store_rows<MB, MR>(acc, y, ys, y_bf16, accumulate, M, N, blockIdx.x, lane, n_lo);
}

template <typename XT, int MB, int MR, bool TILED>
static void launch_w16_t(const W16Args &a, int KS, hipStream_t s) {
    const int threads = KS * WAVE;
    const size_t lds = dense_lds_bytes(a.M, a.K, MB, KS, KS);
    const int xpt = (a.M * (a.K / 8) + threads - 1) / threads;
    const unsigned blocks = unsigned((a.N + 15) / 16);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), threads, lds);
        kern<<<blocks, threads, lds, s>>>(a.W, a.ldw, a.x, a.xs, a.M, a.K, a.N, a.y, a.ys, a.y_bf16, a.accumulate,
                                          a.n_lo);
    };
    const int spw = (a.K / 32 + KS - 1) / KS;
    auto pick = [&](auto ws) {
        constexpr int W = decltype(ws)::value;
        if (xpt <= 1) go(w16_gemv_kernel<XT, MB, MR, 1, W, TILED>);
        else if (xpt <= 2) go(w16_gemv_kernel<XT, MB, MR, 2, W, TILED>);
        else if (xpt <= 4) go(w16_gemv_kernel<XT, MB, MR, 4, W, TILED>);
        else go(w16_gemv_kernel<XT, MB, MR, 0, W, TILED>);
    };
    if (spw <= 8) pick(std::integral_constant<int, 8>());
    else pick(std::integral_constant<int, 16>());
}

template <typename XT, bool TILED>
static void launch_w16_x(const W16Args &a, int KS, hipStream_t s) {
    if (a.M > 16) launch_w16_t<XT, 2, 4, TILED>(a, KS, s);
    else if (a.M == 1) launch_w16_t<XT, 1, 1, TILED>(a, KS, s);
    else if (a.M == 2) launch_w16_t<XT, 1, 2, TILED>(a, KS, s);
    else launch_w16_t<XT, 1, 4, TILED>(a, KS, s);
}

// K split: as many waves (up to 8) as the 32-element steps allow; fewer
// steps per wave mean more loads in flight per weight byte. (16 waves of 8
// steps for shapes with fewer row blocks than CUs measured slower.)
static int w16_ks(int K, int) { return K / 32 < W16_MAX_KS ? K / 32 : W16_MAX_KS; }

bool w16_fits(int M, int K, int N) {
    const int KS = w16_ks(K, N), MB = M > 16 ? 2 : 1;
    return dense_lds_bytes(M, K, MB, KS, KS) <= 160 * 1024;
}

static void launch_w16_fit(const W16Args &a, hipStream_t s) {
    const int KS = w16_ks(a.K, a.N);
    if (a.tiled) {
        if (a.f16) launch_w16_x<F16, true>(a, KS, s);
        else launch_w16_x<BF16, true>(a, KS, s);
    } else {
        if (a.f16) launch_w16_x<F16, false>(a, KS, s);
        else launch_w16_x<BF16, false>(a, KS, s);
    }
}

static void launch_w16_rows(const W16Args &a, hipStream_t s);

// Rows grouped over activation slices (rpg > 0; row n reads x + (n / rpg) * K,
// as gpu::gemv_rows does, src/kernels/gemv.hip:17): one launch per slice.
// Row-major weights start the launch at the slice's first row; tiled ones at
// its first 16-row tile, storing only the slice's rows (a tile that straddles
// two slices is computed in both launches).
void launch_w16_gemv(const W16Args &a, hipStream_t s) {
    if (a.rpg <= 0) {
        launch_w16_rows(a, s);
        return;
    }
    const size_t ysz = a.y_bf16 ? 2 : 4;
    for (int r0 = 0, sl = 0; r0 < a.N; r0 += a.rpg, ++sl) {
        const int r1 = r0 + a.rpg < a.N ? r0 + a.rpg : a.N, b0 = a.tiled ? r0 / 16 * 16 : r0;
        W16Args b = a;
        b.rpg = 0;
        b.W = a.tiled ? a.W + int64_t(b0) * a.K : a.W + int64_t(b0) * a.ldw;
        b.x = a.x + int64_t(sl) * a.K;
        b.y = static_cast<char *>(a.y) + int64_t(b0) * ysz;
        b.N = r1 - b0;
        b.n_lo = r0 - b0;
        launch_w16_rows(b, s);
    }
}

// Batches whose activations exceed LDS run as several launches of fewer rows.
static void launch_w16_rows(const W16Args &a, hipStream_t s) {
    if (w16_fits(a.M, a.K, a.N)) {
        launch_w16_fit(a, s);
        return;
    }
    int mc = 16;
    while (mc > 1 && !w16_fits(mc, a.K, a.N)) --mc;
    const size_t ysz = a.y_bf16 ? 2 : 4;
    for (int m0 = 0; m0 < a.M; m0 += mc) {
        W16Args b = a;
        b.M = a.M - m0 < mc ? a.M - m0 : mc;
        b.x = a.x + int64_t(m0) * a.xs;
        b.y = static_cast<char *>(a.y) + int64_t(m0) * a.ys * ysz;
        launch_w16_fit(b, s);
    }
}

// ------------------------------------------------------------ tiled layout
// Wt uint4 [ceil(N/16)][K/32][64]: entry (sub, s, 16 q + n) holds the 8
// elements of row 16 sub + n at K 32 s + 8 q .. +8 (zero past row N - 1),
// which is what lane 16 q + n feeds the 16x16x32 MFMA at step s; one step of
// a subtile is one contiguous 1 KB wave load. One thread per entry.
__global__ __launch_bounds__(256) void w16_tile_kernel(const uint16_t *__restrict__ W, int64_t ldw, int N, int K,
                                                       uint4 *__restrict__ Wt) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x, steps = K / 32;
    if (i >= (int64_t(N) + 15) / 16 * steps * 64) return;
    const int l = int(i % 64), q = l / 16, n = l % 16;
    const int64_t s = i / 64 % steps, sub = i / 64 / steps, row = sub * 16 + n;
    Wt[i] = row < N ? *reinterpret_cast<const uint4 *>(W + row * ldw + s * 32 + q * 8) : make_uint4(0, 0, 0, 0);
}

void launch_w16_tile(const uint16_t *W, int64_t ldw, int N, int K, void *Wt, hipStream_t s) {
    const int64_t n = (int64_t(N) + 15) / 16 * (K / 32) * 64;
    w16_tile_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(W, ldw, N, K, static_cast<uint4 *>(Wt));
}

// ---------------------------------------------------------- SwiGLU x gate
// h[t][j] = fp16(silu(v[t][j]) * v[t][n + j] * sigmoid(v[t][2n])): the shared
// expert's activation, v the output of its fused gate/up/gate-logit GEMV.
// Finite values beyond the fp16 range saturate (f32_to_f16_satfinite). The
// standalone kernel and the fused down projection below share these helpers,
// so both produce the same bits. silu and sigmoid are the reference's forms
// (silu_ref, sigmoid_ref), in the reference's order of the products
// (src/kernels/moe_route.hip:187-193).
__device__ __forceinline__ float sigmoid_gate(float gl) { return sigmoid_ref(gl); }
__device__ __forceinline__ uint16_t swiglu_h(float g, float u, float gate) {
    return __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(silu_ref(g) * u * gate));
}

__global__ __launch_bounds__(256) void swiglu_gate_kernel(const float *__restrict__ v, int ldv, int n, int T,
                                                          uint16_t *__restrict__ h) {
    const int t = blockIdx.y, j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const float *r = v + int64_t(t) * ldv;
    h[int64_t(t) * n + j] = swiglu_h(r[j], r[n + j], sigmoid_gate(r[2 * n]));
}

// --------------------------------- SwiGLU x gate folded into the down GEMV
// y = W h with h formed from v while the activations are staged (K = n):
// the w16 GEMV on tiled fp16 weights whose staging reads, per 8-element piece
// of h, 8 gate and 8 up values and the row's gate logit, and writes the 8
// fp16 values swiglu_gate_kernel would. One launch instead of two. Up to four
// pieces per thread go through registers, requested before the weight loads
// (XPT 1, 2, 4; 17 VGPRs a piece); more rows are staged by a loop after them
// (XPT 0), which waits for the weight loads too.
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
__global__ __launch_bounds__(W16_MAX_KS *WAVE) void w16_swiglu_kernel(const uint16_t *W, const float *v, int ldv, int M,
                                                                      int K, int N, void *__restrict__ y, int ys,
                                                                      int y_bf16, int accumulate) {
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
    const uint4 *wrow = reinterpret_cast<const uint4 *>(W) + int64_t(blockIdx.x) * steps * 64 + lane;
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
    if (kp == 0) store_rows<MB, MR>(acc, y, ys, y_bf16, accumulate, M, N, blockIdx.x, lane);
}

template <int MB, int MR>
static void launch_w16_swiglu_t(const W16SwigluArgs &a, hipStream_t s) {
    const int KS = w16_ks(a.n, a.N), threads = KS * WAVE;
    const size_t lds = dense_lds_bytes(a.M, a.n, MB, KS, KS);
    const int xpt = (a.M * (a.n / 8) + threads - 1) / threads;
    const unsigned blocks = unsigned((a.N + 15) / 16);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), threads, lds);
        kern<<<blocks, threads, lds, s>>>(a.Wt, a.v, a.ldv, a.M, a.n, a.N, a.y, a.ys, a.y_bf16, a.accumulate);
    };
    const int spw = (a.n / 32 + KS - 1) / KS;
    auto pick = [&](auto ws) {
        constexpr int W = decltype(ws)::value;
        if (xpt <= 1) go(w16_swiglu_kernel<MB, MR, 1, W>);
        else if (xpt <= 2) go(w16_swiglu_kernel<MB, MR, 2, W>);
        else if (xpt <= 4) go(w16_swiglu_kernel<MB, MR, 4, W>);
        else go(w16_swiglu_kernel<MB, MR, 0, W>);
    };
    if (spw <= 8) pick(std::integral_constant<int, 8>());
    else pick(std::integral_constant<int, 16>());
}

bool w16_swiglu_fits(int M, int n, int N) { return w16_fits(M, n, N); }

void launch_w16_swiglu(const W16SwigluArgs &a, hipStream_t s) {
    if (a.M > 16) launch_w16_swiglu_t<2, 4>(a, s);
    else if (a.M == 1) launch_w16_swiglu_t<1, 1>(a, s);
    else if (a.M == 2) launch_w16_swiglu_t<1, 2>(a, s);
    else launch_w16_swiglu_t<1, 4>(a, s);
}

void launch_swiglu_gate(const float *v, int ldv, int n, int T, uint16_t *h, hipStream_t s) {
    swiglu_gate_kernel<<<dim3(unsigned((n + 255) / 256), unsigned(T)), 256, 0, s>>>(v, ldv, n, T, h);
}

}  // namespace qwq4
