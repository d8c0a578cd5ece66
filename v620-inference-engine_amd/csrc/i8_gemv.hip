// Dense GEMV on int8 weights with an fp32 scale per group of 16 or 32 along K.
//
// Reference role: gpu::gemv_rows_i8 (src/kernels/gemv.hip:75-136, declared
// src/kernels/gemv.hpp:15-23), the engine's int8 copy of its fp16 dense
// weights (QW_INT8_DENSE, src/engine/decode.hip:52-70,119-125), quantised by
// quantize_rows_i8 (src/engine/weight_convert.cpp:92-108):
//   y[m*ys + n] (+)= sum_g scale[n][g] * sum_{k in g} W8[n][k] * x[m*xs + off(n) + k]
// with off(n) = (n / rpg) * K when rows are grouped over activation slices.
//
// The weights are tiled once at load (qw_i8_tile, below; the role the q4
// path's qw_q4_tile plays for pack_int4_words) from the quantiser's row-major
// [N][K] int8 and [N][K/group] fp32 scales. Kernel shape as the 16-bit GEMV
// (w16_gemv.hip): a block holds one 16-row tile, its KS waves split K in
// 64-element steps, the activations (fp16) and the tile's scales are staged
// in LDS, the KS partial sums are added through LDS in k-part order. A wave
// instruction reads 1 KB of contiguous weights (row-major rows read 64 bytes
// per row per instruction measured 20% slower), 16 bytes per lane: lane
// (n, q) gets row n's weights arranged so that every MFMA operand covers
// exactly one scale group, and the MFMA's fp32 result is scaled once, as the
// reference scales each group's fp32 dot product (16x16x32 MFMAs for groups
// of 32, 16x16x16 for groups of 16).
// int8 -> fp16 is exact: the byte b ^ 0x80 = b + 128 becomes the low byte of
// fp16 1024 + (b + 128), minus 1152. Products with fp16 activations are exact
// in fp32, so a group's sum differs from the reference's only by summation
// order.
#include <algorithm>
#include <type_traits>

#include "q4_gemv_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

constexpr int I8_MAX_KS = 16;  // waves per block

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// four int8 weights (byte i = element i) -> four fp16 (two dwords), exactly
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const f16x2 off{(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // e0, e1
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // e2, e3
    return make_uint2(__builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, lo) - off),
                      __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, hi) - off));
}

__device__ __forceinline__ uint4 i8x8_to_f16x8(uint32_t a, uint32_t b) {
    const uint2 l = i8x4_to_f16x4(a), h = i8x4_to_f16x4(b);
    return make_uint4(l.x, l.y, h.x, h.y);
}

__device__ __forceinline__ f32x4 mfma16x16(const uint2 &a, const uint2 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
}

// Direct global->LDS copy of `pieces` 16-byte pieces (whole waves of them are
// written: the LDS region is rounded up to 64 pieces).
__device__ __forceinline__ void stage_block_issue(const uint4 *src, int pieces, uint4 *dst) {
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, nw = blockDim.x / WAVE;
    for (int b = wave * WAVE; b < pieces; b += nw * WAVE)
        __builtin_amdgcn_global_load_lds(src + min(b + lane, pieces - 1), dst + b, 16, 0, 0);
}

// LDS pieces of a block's scales: 16 rows x K / GRP floats, whole waves
__host__ __device__ inline int i8_scale_pieces(int K, int group) { return (16 * (K / group) / 4 + WAVE - 1) / WAVE * WAVE; }

// GRP: scale group (16 or 32). MB row blocks of 16 tokens, MR rows of the
// last one formed. XPT: activation pieces per thread through registers (0:
// direct global->LDS). WS: 64-element steps a wave keeps in flight. NSL: row
// slices a 16-row tile can read (2 when rpg is not a multiple of 16).
template <int GRP, int MB, int MR, int XPT, int WS, int NSL>
__global__ __launch_bounds__(I8_MAX_KS *WAVE) void i8_gemv_kernel(const uint4 *Wt, const float *St, const uint16_t *x,
                                                                  int xs, int M, int K, int N, int rpg,
                                                                  void *__restrict__ y, int ys, int y_bf16,
                                                                  int accumulate) {
    static_assert(GRP == 16 || GRP == 32, "scale groups of 16 or 32");
    static_assert(NSL == 1 || XPT == 0, "two row slices are staged directly");
    extern __shared__ __align__(16) unsigned char smem[];
    const int KS = blockDim.x / WAVE;
    const int tid = threadIdx.x, kp = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE, q = lane / 16,
              n = lane % 16;
    const int steps = K / 64, spw = (steps + KS - 1) / KS, s0 = kp * spw, ns = min(spw, steps - s0);
    const int G = K / GRP, kc = x_row_stride(K);
    const int n0 = int(blockIdx.x) * 16;
    // activation slices of this tile: sl0 for its first row, sl1 for its last
    const int sl0 = rpg > 0 ? n0 / rpg : 0, sl1 = rpg > 0 ? min(n0 + 15, N - 1) / rpg : 0;
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    uint4 *sl = xl + x_pieces(NSL * M, K);
    float *red = reinterpret_cast<float *>(sl + i8_scale_pieces(K, GRP));
    const uint16_t *xb = x + int64_t(sl0) * K;
    XRegs xv;
    if constexpr (XPT > 0) stage_regs_issue<XPT>(xb, xs, M, K, xv);
    else if constexpr (NSL == 1) stage_x_issue(xb, xs, M, K, xl);
    else
        stage_rows_issue([&](int i) { return x + int64_t(i % M) * xs + int64_t(i < M ? sl0 : sl1) * K; }, NSL * M, K,
                         xl);
    // the tile's scales, [K / 64][16 rows][64 / GRP] floats, contiguous
    stage_block_issue(reinterpret_cast<const uint4 *>(St + int64_t(blockIdx.x) * 16 * G), 4 * G, sl);
    __builtin_amdgcn_sched_barrier(0);  // activations and scales go out before the weight loads
    // lane l of step s: 16 bytes of row n (see the tiled format above)
    const uint4 *wt = Wt + int64_t(blockIdx.x) * steps * WAVE + lane;
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    uint4 w[WS];
    auto fetch = [&](int p) {  // steps p .. p + WS - 1 of the wave's range (clamped, no branches)
#pragma unroll
        for (int t = 0; t < WS; ++t) {
            const int s = min(s0 + min(p + t, max(ns - 1, 0)), steps - 1);
            const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wt + s * WAVE));
            w[t] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    };
    f32x4 acc[NSL][MB];
#pragma unroll
    for (int j = 0; j < NSL; ++j)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[j][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    fetch(0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XPT > 0) stage_regs_commit<XPT>(xv, M, K, xl);
    wait_vm_below<WS>();  // this wave's activation and scale loads (its oldest)
    lds_barrier();
    // the second slice is computed only by tiles that straddle two
    const bool two = NSL == 2 && sl1 != sl0;
    const uint4 *xr[NSL][MB];
#pragma unroll
    for (int j = 0; j < NSL; ++j)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) xr[j][mb] = xl + (j * M + min(mb * 16 + n, M - 1)) * kc;
    constexpr int SPS = 64 / GRP;  // scales per step
    typedef float sv_t __attribute__((ext_vector_type(SPS)));
    const sv_t *scl = reinterpret_cast<const sv_t *>(sl) + n;
    const f32x4 zero = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < ns; p += WS) {
        if (p > 0) fetch(p);
#pragma unroll
        for (int t = 0; t < WS; ++t)
            if (p + t < ns) {
                const int s = s0 + p + t;
                const sv_t sc = scl[s * 16];
                if constexpr (GRP == 32) {
                    // K of the lane's 8 weights: 8 q (first group), 32 + 8 q (second)
                    const uint4 wa = i8x8_to_f16x8(w[t].x, w[t].y), wb = i8x8_to_f16x8(w[t].z, w[t].w);
#pragma unroll
                    for (int j = 0; j < NSL; ++j)
                        if (j == 0 || two) {
#pragma unroll
                            for (int mb = 0; mb < MB; ++mb) {
                                const f32x4 ra = mfma16<F16>(xr[j][mb][s * 8 + q], wa, zero);
                                const f32x4 rb = mfma16<F16>(xr[j][mb][s * 8 + 4 + q], wb, zero);
                                const int rows = mb == MB - 1 ? MR : 4;
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (r < rows) acc[j][mb][r] += sc[0] * ra[r] + sc[1] * rb[r];
                            }
                        }
                } else {
                    // dword g: K 16 g + 4 q .. + 3 of the step, group 4 s + g
                    const uint2 wg[4] = {i8x4_to_f16x4(w[t].x), i8x4_to_f16x4(w[t].y), i8x4_to_f16x4(w[t].z),
                                         i8x4_to_f16x4(w[t].w)};
#pragma unroll
                    for (int j = 0; j < NSL; ++j)
                        if (j == 0 || two) {
#pragma unroll
                            for (int mb = 0; mb < MB; ++mb) {
                                const uint2 *xh = reinterpret_cast<const uint2 *>(xr[j][mb]);
                                const int rows = mb == MB - 1 ? MR : 4;
#pragma unroll
                                for (int g = 0; g < 4; ++g) {
                                    const f32x4 rg = mfma16x16(xh[s * 16 + 4 * g + q], wg[g], zero);
#pragma unroll
                                    for (int r = 0; r < 4; ++r)
                                        if (r < rows) acc[j][mb][r] += sc[g] * rg[r];
                                }
                            }
                        }
                }
            }
    }
    // each lane keeps the slice of its own row
    if constexpr (NSL == 2) {
        if (min(n0 + n, N - 1) / rpg != sl0) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[0][mb] = acc[1][mb];
        }
    }
    ksplit_sum<MB, MR>(acc[0], red, KS, kp, kp, lane);
    if (kp == 0) store_rows<MB, MR>(acc[0], y, ys, y_bf16, accumulate, M, N, blockIdx.x, lane);
}

// ------------------------------------------------------------ tiled format
// Wt uint4 [ceil(N/16)][K/64][64]: entry (tile, s, lane l) holds 16 int8
// weights of row 16 tile + l % 16, q = l / 16, of the 64-element step s:
//   group 32: bytes 0-7 = K 64 s + 8 q .. + 7, bytes 8-15 = K 64 s + 32 + 8 q .. + 7
//   group 16: dword g = K 64 s + 16 g + 4 q .. + 3 (g = 0..3)
// so each 16x16x32 (16x16x16) MFMA operand covers one scale group. Rows past
// N are zero. St fp32 [ceil(N/16)][K/64][16][64/group]: the scales of the
// step's groups, per row.
__global__ void i8_tile_kernel(const int8_t *__restrict__ W8, const float *__restrict__ S, int N, int K, int group,
                               uint4 *__restrict__ Wt, float *__restrict__ St) {
    const int64_t steps = K / 64, total = int64_t((N + 15) / 16) * steps * WAVE;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
        const int l = int(i % WAVE), q = l / 16, nn = l % 16;
        const int64_t s = (i / WAVE) % steps, tile = i / (WAVE * steps), row = tile * 16 + nn;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (row < N) {
            const int8_t *r = W8 + row * K + s * 64;
            if (group == 32) {
                const uint2 a = *reinterpret_cast<const uint2 *>(r + 8 * q);
                const uint2 b = *reinterpret_cast<const uint2 *>(r + 32 + 8 * q);
                v = make_uint4(a.x, a.y, b.x, b.y);
            } else {
                const uint32_t *d = reinterpret_cast<const uint32_t *>(r + 4 * q);
                v = make_uint4(d[0], d[4], d[8], d[12]);
            }
        }
        Wt[i] = v;
        // scales: lane l < 16 writes row nn's scales of this step
        if (q == 0) {
            const int sps = 64 / group, G = K / group;
            for (int j = 0; j < sps; ++j)
                St[((tile * steps + s) * 16 + nn) * sps + j] = row < N ? S[row * G + s * sps + j] : 0.f;
        }
    }
}

void launch_i8_tile(const int8_t *W8, const float *S, int N, int K, int group, uint4 *Wt, float *St, hipStream_t s) {
    const int64_t total = int64_t((N + 15) / 16) * (K / 64) * WAVE;
    const unsigned blocks = unsigned(std::min<int64_t>((total + 255) / 256, 65536));
    i8_tile_kernel<<<blocks, 256, 0, s>>>(W8, S, N, K, group, Wt, St);
}

// K split: up to 8 waves; 16 when the row tiles would not give every CU two
// blocks (fewer blocks leave the weight stream short of loads in flight)
static int i8_ks(int K, int N) {
    const int ks = (N + 15) / 16 < 512 ? 16 : 8;
    return K / 64 < ks ? K / 64 : ks;
}

static int i8_nsl(int rpg) { return rpg > 0 && rpg % 16 != 0 ? 2 : 1; }

size_t i8_lds_bytes(int M, int K, int N, int group, int rpg) {
    const int KS = i8_ks(K, N), MB = M > 16 ? 2 : 1;
    return size_t(x_pieces(i8_nsl(rpg) * M, K) + i8_scale_pieces(K, group)) * 16 +
           size_t(red_slots(KS, KS)) * MB * WAVE * 16;  // one set of k-split slots (no persistent blocks)
}

template <int GRP, int MB, int MR, int NSL>
static void launch_i8_t(const I8Args &a, hipStream_t s) {
    const int KS = i8_ks(a.K, a.N), threads = KS * WAVE;
    const size_t lds = i8_lds_bytes(a.M, a.K, a.N, a.group, a.rpg);
    const int xpt = NSL == 1 ? (a.M * (a.K / 8) + threads - 1) / threads : 0;
    const unsigned blocks = unsigned((a.N + 15) / 16);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), threads, lds);
        kern<<<blocks, threads, lds, s>>>(a.W, a.S, a.x, a.xs, a.M, a.K, a.N, a.rpg, a.y, a.ys, a.y_bf16,
                                          a.accumulate);
    };
    const int spw = (a.K / 64 + KS - 1) / KS;
    auto pick = [&](auto ws) {
        constexpr int W = decltype(ws)::value;
        if constexpr (NSL == 2) go(i8_gemv_kernel<GRP, MB, MR, 0, W, 2>);
        else {
            if (xpt <= 1) go(i8_gemv_kernel<GRP, MB, MR, 1, W, 1>);
            else if (xpt <= 2) go(i8_gemv_kernel<GRP, MB, MR, 2, W, 1>);
            else if (xpt <= 4) go(i8_gemv_kernel<GRP, MB, MR, 4, W, 1>);
            else go(i8_gemv_kernel<GRP, MB, MR, 0, W, 1>);
        }
    };
    if (spw <= 4) pick(std::integral_constant<int, 4>());
    else pick(std::integral_constant<int, 8>());
}

template <int GRP, int NSL>
static void launch_i8_m(const I8Args &a, hipStream_t s) {
    if (a.M > 16) launch_i8_t<GRP, 2, 4, NSL>(a, s);
    else if (a.M == 1) launch_i8_t<GRP, 1, 1, NSL>(a, s);
    else if (a.M == 2) launch_i8_t<GRP, 1, 2, NSL>(a, s);
    else launch_i8_t<GRP, 1, 4, NSL>(a, s);
}

static void launch_i8_fit(const I8Args &a, hipStream_t s) {
    const bool two = i8_nsl(a.rpg) == 2;
    if (a.group == 32) two ? launch_i8_m<32, 2>(a, s) : launch_i8_m<32, 1>(a, s);
    else two ? launch_i8_m<16, 2>(a, s) : launch_i8_m<16, 1>(a, s);
}

bool i8_fits(int M, int K, int N, int group, int rpg) { return i8_lds_bytes(M, K, N, group, rpg) <= 160 * 1024; }

// Batches whose activations exceed LDS run as several launches of fewer rows
// (the caller has checked that one row fits).
void launch_i8_gemv(const I8Args &a, hipStream_t s) {
    if (i8_fits(a.M, a.K, a.N, a.group, a.rpg)) {
        launch_i8_fit(a, s);
        return;
    }
    int mc = 16;
    while (mc > 1 && !i8_fits(mc, a.K, a.N, a.group, a.rpg)) --mc;
    const size_t ysz = a.y_bf16 ? 2 : 4;
    for (int m0 = 0; m0 < a.M; m0 += mc) {
        I8Args b = a;
        b.M = a.M - m0 < mc ? a.M - m0 : mc;
        b.x = a.x + int64_t(m0) * a.xs;
        b.y = static_cast<char *>(a.y) + int64_t(m0) * a.ys * ysz;
        launch_i8_fit(b, s);
    }
}

}  // namespace qwq4
