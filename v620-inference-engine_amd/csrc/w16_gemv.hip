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

#include "q4_kernels.hpp"
#include "w16_core.cuh"

namespace qwq4 {

template <typename XT, int MB, int MR, int XPT, int WS, bool TILED>
__global__ __launch_bounds__(W16_MAX_KS *WAVE) void w16_gemv_kernel(const uint16_t *W, int ldw, const uint16_t *x,
                                                                    int xs, int M, int K, int N, void *__restrict__ y,
                                                                    int ys, int y_bf16, int accumulate, int n_lo) {
    w16_gemv_block<XT, MB, MR, XPT, WS, TILED>(W, ldw, x, xs, M, K, N, y, ys, y_bf16, accumulate, n_lo, blockIdx.x);
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
template <int MB, int MR, int XPT, int WS>
__global__ __launch_bounds__(W16_MAX_KS *WAVE) void w16_swiglu_kernel(const uint16_t *W, const float *v, int ldv, int M,
                                                                      int K, int N, void *__restrict__ y, int ys,
                                                                      int y_bf16, int accumulate) {
    w16_swiglu_block<MB, MR, XPT, WS>(W, v, ldv, M, K, N, y, ys, y_bf16, accumulate, blockIdx.x);
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
