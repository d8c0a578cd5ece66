// Dense q4 GEMV for decode rows (M <= 32 per launch), on the gfx950
// 16x16x32 MFMA.
//
// Reference role: gpu::gemv_rows (src/kernels/gemv.hip:7-42, decode
// projections and LM head, fp16 weights there). The arithmetic is
// ref::Model::expert_linear (src/ref/ref_model.cpp:100-119) with a per-group
// zero point. The wave-level work (one 16-row subtile x a K range, lane map)
// is in q4_gemv_core.cuh.
#include "q4_gemv_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

// ------------------------------------------------------------ dense GEMV
// Two schedules over the same wave work (one 16-row subtile x a K range):
//   block   small and medium N: KS waves share a subtile (K split), each
//           block is one item of 8/KS subtiles, and every wave requests its
//           whole K range (<= 16 groups, <= 16 KB) before anything else;
//   stream  large N (LM head): persistent waves, one subtile at a time over
//           all of K in chunks of 8 groups, the next chunk (weights, scales,
//           zeros) in flight while the current one is computed; the stream
//           runs on across subtiles.
// Both stage the M activation rows (bf16) in LDS once per block. The MFMA
// accumulator starts at -144 * sum(x) of the group (an MFMA against a splat
// of -144), see q4_common.cuh. KS waves of a block sharing a subtile reduce
// their partial sums through LDS in a fixed order (deterministic).

__host__ __device__ inline size_t dense_lds_bytes(int M, int K, int MB) {
    return size_t(x_pieces(M, K)) * 16 + size_t(8) * MB * WAVE * 16;
}

__device__ __forceinline__ void stage_x_issue(const uint16_t *__restrict__ x, int xs, int M, int K, uint4 *xl) {
    stage_rows_issue([&](int m) { return x + int64_t(m) * xs; }, M, K, xl);
}

template <int MB>
__device__ __forceinline__ void store_rows(const f32x4 (&acc)[MB], void *y, int ys, int y_bf16, int accumulate,
                                           int M, int sub, int lane) {
    const int q = lane / 16, n = lane % 16;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m < M) store_y(y, int64_t(m) * ys + sub * 16 + n, acc[mb][r], y_bf16, accumulate);
        }
}

// ---- block schedule
template <int KS, int MB, bool HAS_Z, int GW>
__global__ __launch_bounds__(512) void q4_gemv_block_kernel(const uint32_t *Wt,
                                                            const uint16_t *St,
                                                            const uint16_t *Zt,
                                                            const uint16_t *__restrict__ x, int xs,
                                                            void *__restrict__ y, int ys, int y_bf16, int N, int K,
                                                            int M, int accumulate) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int SUB = 8 / KS;
    const int G = K / QGROUP, kc = K / 8, nsub = N / 16, gpk = G / KS;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, q = lane / 16, n = lane % 16;
    const int sl = wave / KS, kp = wave % KS, g0 = kp * gpk;
    const int sub = blockIdx.x * SUB + sl;
    // activations (L2) and then the wave's whole K range of weights (HBM) are
    // requested before anything waits
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    f32x4 *red = reinterpret_cast<f32x4 *>(xl + x_pieces(M, K));
    stage_x_issue(x, xs, M, K, xl);
    const Q4Tile t(Wt, St, Zt, min(sub, nsub - 1), G);
    WaveRange<GW, HAS_Z> wr;
    wr.fetch(t, g0, gpk, lane);
    __syncthreads();
    const uint4 *xr[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xr[mb] = xl + min(mb * 16 + n, M - 1) * kc + q * 4;
    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    wr.template compute<BF16, MB>(xr, acc);
    if constexpr (KS > 1) {
        if (kp != 0) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) red[(wave * MB + mb) * WAVE + lane] = acc[mb];
        }
        lds_barrier();
        if (kp == 0) {
#pragma unroll
            for (int j = 1; j < KS; ++j)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) acc[mb] += red[((wave + j) * MB + mb) * WAVE + lane];
        }
    }
    if (kp == 0 && sub < nsub) store_rows<MB>(acc, y, ys, y_bf16, accumulate, M, sub, lane);
}

// ---- stream schedule
constexpr int STREAM_CH = 4;

__host__ __device__ inline size_t stream_lds_bytes(int M, int K, int MB) {
    return size_t(x_pieces(M, K)) * 16 + size_t(K / QGROUP) * 16 * MB * 4;
}

template <int MB, bool HAS_Z>
__global__ __launch_bounds__(512) void q4_gemv_stream_kernel(const uint32_t *Wt, const uint16_t *St,
                                                             const uint16_t *Zt, const uint16_t *__restrict__ x,
                                                             int xs, void *__restrict__ y, int ys, int y_bf16, int N,
                                                             int K, int M, int accumulate) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int CH = STREAM_CH, MR = 16 * MB;
    const int G = K / QGROUP, kc = K / 8, nsub = N / 16, nch = (G + CH - 1) / CH;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, q = lane / 16, n = lane % 16;
    const int stride = gridDim.x * 8;
    int sub = blockIdx.x * 8 + wave, ch = 0;
    // one chunk: 4 groups of weights, their 4 scales (one 8-byte load) and zero word
    uint4 wc[CH], wn[CH];
    uint2 sc, sn;
    uint32_t zc = 0, zn = 0;
    auto fetch = [&](int sb, int chk, uint4 (&w)[CH], uint2 &sv, uint32_t &zv) {
        const Q4Tile t(Wt, St, Zt, min(sb, nsub - 1), G);
#pragma unroll
        for (int c = 0; c < CH; ++c) w[c] = t.word4(min(chk * CH + c, G - 1), lane);
        sv = *reinterpret_cast<const uint2 *>(t.s + chk * 64 + n * 4);
        if constexpr (HAS_Z) zv = t.z[chk * 16 + n];
    };
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    float *corr = reinterpret_cast<float *>(xl + x_pieces(M, K));
    stage_x_issue(x, xs, M, K, xl);
    fetch(sub, ch, wc, sc, zc);
    __syncthreads();
    // corr[g][m] = -144 * sum of group g of row min(m, M-1)
    for (int i = tid; i < G * MR; i += blockDim.x) {
        const int g = i / MR, m = min(i - g * MR, M - 1);
        const uint4 *src = xl + m * kc + g * 16;
        float sum = 0.f;
        for (int c = 0; c < 16; ++c) {
            const uint4 v = src[c];
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                sum += bf16_bits_to_f32(uint16_t(w4[j])) + bf16_bits_to_f32(uint16_t(w4[j] >> 16));
        }
        corr[i] = -144.f * sum;
    }
    lds_barrier();
    const uint4 *xr[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xr[mb] = xl + min(mb * 16 + n, M - 1) * kc + q * 4;
    f32x4 acc[MB];
    while (sub < nsub) {
        int nsb = sub, nchk = ch + 1;
        if (nchk == nch) {
            nchk = 0;
            nsb += stride;
        }
        fetch(nsb, nchk, wn, sn, zn);
        if (ch == 0) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int g = ch * CH + c;
            if (g >= G) break;
            const uint32_t zb = zero_bytes(HAS_Z ? (zc >> (4 * c)) & 0xfu : 8u);
            const uint32_t s2 = c < 2 ? sc.x : sc.y;
            const float s = f16_bits_to_f32(uint16_t(c % 2 ? s2 >> 16 : s2));
            uint4 b[4];
            b[0] = unpack8<BF16>(wc[c].x, zb);
            b[1] = unpack8<BF16>(wc[c].y, zb);
            b[2] = unpack8<BF16>(wc[c].z, zb);
            b[3] = unpack8<BF16>(wc[c].w, zb);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                f32x4 p = *reinterpret_cast<const f32x4 *>(corr + g * MR + mb * 16 + 4 * q);
#pragma unroll
                for (int t = 0; t < 4; ++t) p = mfma16<BF16>(xr[mb][g * 16 + t], b[t], p);
                acc[mb] += s * p;
            }
        }
        if (ch == nch - 1) store_rows<MB>(acc, y, ys, y_bf16, accumulate, M, sub, lane);
#pragma unroll
        for (int c = 0; c < CH; ++c) wc[c] = wn[c];
        sc = sn;
        zc = zn;
        sub = nsb;
        ch = nchk;
    }
}

template <int MB, bool HAS_Z>
static void launch_stream(const GemvArgs &a, size_t, hipStream_t s) {
    auto kern = q4_gemv_stream_kernel<MB, HAS_Z>;
    const size_t lds = stream_lds_bytes(a.M, a.K, MB);
    const int nsub = a.N / 16;
    const LaunchShape ls = persistent_shape(reinterpret_cast<const void *>(kern), 512, lds);
    const int want = (nsub + 7) / 8;
    const int blocks = want < ls.max_blocks ? want : ls.max_blocks;
    kern<<<blocks, 512, lds, s>>>(a.W, a.S, a.Z, a.x, a.xs, a.y, a.ys, a.y_bf16, a.N, a.K, a.M, a.accumulate);
}

template <int KS, int MB, bool HAS_Z, int GW>
static void launch_block(const GemvArgs &a, size_t lds, hipStream_t s) {
    auto kern = q4_gemv_block_kernel<KS, MB, HAS_Z, GW>;
    const int nsub = a.N / 16, blocks = (nsub + (8 / KS) - 1) / (8 / KS);
    if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), 512, lds);
    kern<<<blocks, 512, lds, s>>>(a.W, a.S, a.Z, a.x, a.xs, a.y, a.ys, a.y_bf16, a.N, a.K, a.M, a.accumulate);
}

template <int KS, int MB, bool HAS_Z>
static void launch_block_gw(const GemvArgs &a, size_t lds, hipStream_t s) {
    const int gpk = a.K / QGROUP / KS;
    if (gpk <= 4) launch_block<KS, MB, HAS_Z, 4>(a, lds, s);
    else if (gpk <= 8) launch_block<KS, MB, HAS_Z, 8>(a, lds, s);
    else launch_block<KS, MB, HAS_Z, 16>(a, lds, s);
}

template <int MB, bool HAS_Z>
static void launch_dense(const GemvArgs &a, hipStream_t s) {
    const int G = a.K / QGROUP, nsub = a.N / 16;
    const size_t lds = dense_lds_bytes(a.M, a.K, MB);
    int cus = 0, dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int64_t want = int64_t(12) * (cus > 0 ? cus : 256);  // waves: 12 per CU
    if (nsub >= want) {
        launch_stream<MB, HAS_Z>(a, lds, s);
        return;
    }
    // K split: the largest power of two <= 8 dividing G (measured: more,
    // shorter waves finish sooner than fewer, longer ones)
    int ks = 1;
    while (ks < 8 && G % (ks * 2) == 0) ks *= 2;
    if (G / ks > 16) {
        launch_stream<MB, HAS_Z>(a, lds, s);
        return;
    }
    switch (ks) {
        case 1: launch_block_gw<1, MB, HAS_Z>(a, lds, s); break;
        case 2: launch_block_gw<2, MB, HAS_Z>(a, lds, s); break;
        case 4: launch_block_gw<4, MB, HAS_Z>(a, lds, s); break;
        default: launch_block_gw<8, MB, HAS_Z>(a, lds, s); break;
    }
}

bool gemv_fits(int M, int K) {
    const int MB = M <= 16 ? 1 : 2;
    const size_t l1 = dense_lds_bytes(M, K, MB), l2 = stream_lds_bytes(M, K, MB);
    return (l1 > l2 ? l1 : l2) <= 160 * 1024;
}

static void launch_gemv_fit(const GemvArgs &a, hipStream_t s) {
    if (a.M <= 16) {
        if (a.Z) launch_dense<1, true>(a, s);
        else launch_dense<1, false>(a, s);
    } else {
        if (a.Z) launch_dense<2, true>(a, s);
        else launch_dense<2, false>(a, s);
    }
}

// Batches whose activations exceed LDS run as several launches of fewer rows.
void launch_gemv(const GemvArgs &a, hipStream_t s) {
    if (gemv_fits(a.M, a.K)) {
        launch_gemv_fit(a, s);
        return;
    }
    int mc = 16;
    while (mc > 1 && !gemv_fits(mc, a.K)) --mc;
    const size_t ysz = a.y_bf16 ? 2 : 4;
    for (int m0 = 0; m0 < a.M; m0 += mc) {
        GemvArgs b = a;
        b.M = a.M - m0 < mc ? a.M - m0 : mc;
        b.x = a.x + int64_t(m0) * a.xs;
        b.y = static_cast<char *>(a.y) + int64_t(m0) * a.ys * ysz;
        launch_gemv_fit(b, s);
    }
}

}  // namespace qwq4
