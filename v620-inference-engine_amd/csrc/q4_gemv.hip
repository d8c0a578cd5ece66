// q4 GEMV for decode rows (M <= 32) and the gathered per-expert GEMV of routed
// MoE tokens, on the gfx950 16x16x32 MFMA.
//
// Reference roles: gpu::gemv_rows (src/kernels/gemv.hip:7-42, decode
// projections and LM head, fp16 weights there) and gpu::moe_experts_P
// (src/kernels/moe_experts.hip:189-245). The arithmetic is
// ref::Model::expert_linear (src/ref/ref_model.cpp:100-119) with a per-group
// zero point.
//
// Work split. A wave owns a 16-row subtile of the tiled weights and a
// contiguous range of the 128-wide K groups; KS waves of a 512-thread block
// share one subtile (a K split, reduced through LDS in a fixed order), so
// small N still fills the chip. Lane l serves weight row n = l % 16 and
// K-quarter q = l / 16 of every group: one 16-byte load per lane per group,
// 1 KB of contiguous HBM per wave-instruction, the nibbles unpacked in
// registers (q4_common.cuh). The MFMA's other operand is the activations:
// lane l feeds token row m = l % 16, so the 16x16 result holds every
// (token, row) pair; each lane ends with one weight row n and four token rows
// 4(l/16) + r, so the group scale and zero are one value per lane.
#include "q4_wave.cuh"
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
// of -144), see q4_common.cuh.

__host__ __device__ inline int x_pieces(int M, int K);
__host__ __device__ inline size_t dense_lds_bytes(int M, int K, int MB) {
    return size_t(x_pieces(M, K)) * 16 + size_t(8) * MB * WAVE * 16;
}

// LDS-only barrier: orders this block's LDS traffic without draining the
// global-memory loads in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// x rows 0..M-1 of K bf16 -> LDS with direct global->LDS loads (no
// registers; 1 KB per wave instruction). They are issued before the weight
// loads, and the barrier that follows those waits for both, so activations
// (L2) and weights (HBM) are all requested before anything waits.
__host__ __device__ inline int x_pieces(int M, int K) {  // 16-byte pieces, rounded to whole waves
    return (M * (K / 8) + WAVE - 1) / WAVE * WAVE;
}

__device__ __forceinline__ void stage_x_issue(const uint16_t *__restrict__ x, int xs, int M, int K, uint4 *xl) {
    const int kc = K / 8, total = M * kc, wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int nw = blockDim.x / WAVE;
    for (int base = wave * WAVE; base < total; base += nw * WAVE) {
        const int i = min(base + lane, total - 1), m = i / kc, c = i - m * kc;
        __builtin_amdgcn_global_load_lds(x + int64_t(m) * xs + c * 8, xl + base, 16, 0, 0);
    }
}

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

// One group of one subtile: acc[mb] += s * (x . (q - z)) for the lane's rows.
template <int MB>
__device__ __forceinline__ void dense_group(const uint4 &w, uint32_t zb, float s, const uint4 *const (&xr)[MB], int g,
                                            f32x4 (&acc)[MB]) {
    const uint4 negb = make_uint4(BF16::NEG_BIAS, BF16::NEG_BIAS, BF16::NEG_BIAS, BF16::NEG_BIAS);
    uint4 b[4];
    b[0] = unpack8<BF16>(w.x, zb);
    b[1] = unpack8<BF16>(w.y, zb);
    b[2] = unpack8<BF16>(w.z, zb);
    b[3] = unpack8<BF16>(w.w, zb);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        uint4 a[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t] = xr[mb][g * 16 + t];
        f32x4 p = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) p = mfma16<BF16>(a[t], negb, p);
#pragma unroll
        for (int t = 0; t < 4; ++t) p = mfma16<BF16>(a[t], b[t], p);
        acc[mb] += s * p;
    }
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
    uint4 w[GW];
    uint32_t sv[GW], zv[GW];
#pragma unroll
    for (int c = 0; c < GW; ++c) {
        const int g = g0 + min(c, gpk - 1);
        w[c] = t.word4(g, lane);
        sv[c] = t.scale(g, n);
        if constexpr (HAS_Z) zv[c] = t.zero_word(g, n);
    }
    __syncthreads();
    const uint4 *xr[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xr[mb] = xl + min(mb * 16 + n, M - 1) * kc + q * 4;
    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < GW; ++c) {
        if (c >= gpk) break;
        const int g = g0 + c;
        const uint32_t zb = zero_bytes(HAS_Z ? Q4Tile::zero_of(zv[c], g) : 8u);
        dense_group<MB>(w[c], zb, f16_bits_to_f32(uint16_t(sv[c])), xr, g, acc);
    }
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

// ------------------------------------------------ routed-expert GEMVs
// grid (row blocks of one expert, max active experts). Block y serves the
// y-th expert with tokens (active[] ascending); its M tokens are the slots
// offsets[e] .. offsets[e+1]-1. Expert e's weights are rows e*F .. of the
// stacked [E*F][H] (gate, up) and [E*H][F] (down) tiled matrices.

// gate/up fused with SiLU * up: h[slot][F] (fp16).
template <int KS, int MB, bool HAS_Z>
__global__ __launch_bounds__(512) void moe_gate_up_gemv_kernel(
    const uint32_t *__restrict__ gw, const uint16_t *__restrict__ gs, const uint16_t *__restrict__ gz,
    const uint32_t *__restrict__ uw, const uint16_t *__restrict__ us, const uint16_t *__restrict__ uz,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ active, const int32_t *__restrict__ n_active,
    const int32_t *__restrict__ pair_tok, const uint16_t *__restrict__ x, int H, int F, uint16_t *__restrict__ h) {
    if (int(blockIdx.y) >= *n_active) return;
    constexpr int SUB = 8 / KS;
    const int e = active[blockIdx.y];
    const int base = offsets[e], M = offsets[e + 1] - base;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16, n = lane % 16;
    const int lsub = blockIdx.x * SUB + wave / KS, kp = wave % KS;
    const int G = H / QGROUP, gpk = G / KS, fsub = F / 16;
    const int64_t sub = int64_t(e) * fsub + min(lsub, fsub - 1);
    const Q4Tile tile[2] = {Q4Tile(gw, gs, gz, sub, G), Q4Tile(uw, us, uz, sub, G)};
    const uint16_t *arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) arow[mb] = x + int64_t(pair_tok[base + min(mb * 16 + n, M - 1)]) * H;
    f32x4 acc[MB][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb][0] = acc[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    q4_groups<BF16, MB, 2, HAS_Z, MB == 1 ? 4 : 2>(tile, arow, kp * gpk, kp * gpk + gpk, lane, acc);
    ksplit_reduce<MB, 2, KS>(acc, wave, kp, lane);
    if (kp != 0 || lsub >= fsub) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m < M) h[int64_t(base + m) * F + lsub * 16 + n] = silu_mul_f16(acc[mb][0][r], acc[mb][1][r]);
        }
}

// down: yp[slot][H] (fp32) = D_e h[slot].
template <int KS, int MB, bool HAS_Z>
__global__ __launch_bounds__(512) void moe_down_gemv_kernel(const uint32_t *__restrict__ dw,
                                                            const uint16_t *__restrict__ ds,
                                                            const uint16_t *__restrict__ dz,
                                                            const int32_t *__restrict__ offsets,
                                                            const int32_t *__restrict__ active,
                                                            const int32_t *__restrict__ n_active,
                                                            const uint16_t *__restrict__ h, int H, int F,
                                                            float *__restrict__ yp) {
    if (int(blockIdx.y) >= *n_active) return;
    constexpr int SUB = 8 / KS;
    const int e = active[blockIdx.y];
    const int base = offsets[e], M = offsets[e + 1] - base;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, q = lane / 16, n = lane % 16;
    const int lsub = blockIdx.x * SUB + wave / KS, kp = wave % KS;
    const int G = F / QGROUP, gpk = G / KS, hsub = H / 16;
    const int64_t sub = int64_t(e) * hsub + min(lsub, hsub - 1);
    const Q4Tile tile[1] = {Q4Tile(dw, ds, dz, sub, G)};
    const uint16_t *arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) arow[mb] = h + int64_t(base + min(mb * 16 + n, M - 1)) * F;
    f32x4 acc[MB][1];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    q4_groups<F16, MB, 1, HAS_Z, 4>(tile, arow, kp * gpk, kp * gpk + gpk, lane, acc);
    ksplit_reduce<MB, 1, KS>(acc, wave, kp, lane);
    if (kp != 0 || lsub >= hsub) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m < M) yp[int64_t(base + m) * H + lsub * 16 + n] = acc[mb][0][r];
        }
}

template <int KS, int MB, bool HAS_Z>
static void launch_moe_gemv_t(const MoeGemvArgs &a, int max_active, bool down, hipStream_t s) {
    const int rows = down ? a.H : a.F;
    const int subtiles = rows / 16;
    const dim3 grid(unsigned((subtiles + (8 / KS) - 1) / (8 / KS)), unsigned(max_active)), block(512);
    if (!down)
        moe_gate_up_gemv_kernel<KS, MB, HAS_Z><<<grid, block, 0, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets,
                                                                      a.active, a.n_active, a.pair_tok, a.x, a.H, a.F,
                                                                      a.h);
    else
        moe_down_gemv_kernel<KS, MB, HAS_Z><<<grid, block, 0, s>>>(a.dw, a.ds, a.dz, a.offsets, a.active, a.n_active,
                                                                   a.h, a.H, a.F, a.yp);
}

template <int KS>
static void launch_moe_gemv_ks(const MoeGemvArgs &a, int max_active, bool down, hipStream_t s) {
    const bool z = down ? a.dz != nullptr : a.gz != nullptr;
    if (a.T > 16) {
        if (z) launch_moe_gemv_t<KS, 2, true>(a, max_active, down, s);
        else launch_moe_gemv_t<KS, 2, false>(a, max_active, down, s);
    } else {
        if (z) launch_moe_gemv_t<KS, 1, true>(a, max_active, down, s);
        else launch_moe_gemv_t<KS, 1, false>(a, max_active, down, s);
    }
}

static void launch_moe_one(const MoeGemvArgs &a, bool down, hipStream_t s) {
    const int max_active = a.T * a.topk < a.E ? a.T * a.topk : a.E;
    const int rows = down ? a.H : a.F, G = (down ? a.F : a.H) / QGROUP;
    // the K split is sized for the expected number of distinct experts
    // E (1 - (1 - k/E)^T) of T tokens routed uniformly
    double miss = 1.0;
    for (int t = 0; t < a.T; ++t) miss *= 1.0 - double(a.topk) / a.E;
    int64_t expect = int64_t(a.E * (1.0 - miss));
    if (expect < a.topk) expect = a.topk;
    int ks = 1;
    while (ks < 8 && int64_t(rows / 16) * expect * ks < 2048 && G % (ks * 2) == 0) ks *= 2;
    switch (ks) {
        case 1: launch_moe_gemv_ks<1>(a, max_active, down, s); break;
        case 2: launch_moe_gemv_ks<2>(a, max_active, down, s); break;
        case 4: launch_moe_gemv_ks<4>(a, max_active, down, s); break;
        default: launch_moe_gemv_ks<8>(a, max_active, down, s); break;
    }
}

void launch_moe_gemv(const MoeGemvArgs &a, hipStream_t s) {
    launch_moe_one(a, false, s);
    launch_moe_one(a, true, s);
}

}  // namespace qwq4
