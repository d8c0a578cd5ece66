// q4-dequant prefill GEMM: Y[t][n] = sum_k X[t][k] * W[n][k] for a chunk of
// T tokens (reference role: gpu::gemm, src/kernels/gemm.hip:10-18, which
// calls rocBLAS on fp16 weights; here the weights stay q4 in HBM and are
// dequantised on the fly into LDS).
//
// Numerics. Each weight is dequantised once, w = fp16((q - z) * s) (the
// subtraction exact, one rounding for the product), the way the reference's
// grouped expert GEMM does (src/kernels/moe_experts.hip:31-42). X is
// converted to fp16 by a pre-pass (exact for |x| in the fp16 normal range;
// finite values beyond it saturate at +-65504, infinities and NaN pass). Products and sums run on the fp16 MFMA with fp32
// accumulation. Rounding the dequantised weights to bf16 instead would cost
// ~1.4e-3 of max|y| (close to the 2e-3 bar); fp16 costs ~2e-4.
//
// Schedule: q4_gemm_core.cuh (block tile 256 or 128 tokens x 256 weight
// rows, 8 waves, LDS double-buffered K stages of 64). Blocks take their tiles
// in an XCD-aware order; the epilogue goes through LDS so that stores are
// 16 bytes per lane.
#include "q4_gemm_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

size_t gemm_workspace_bytes(int T, int K) {
    const size_t xh = size_t(T) * K * 2;
    return (xh + 255) & ~size_t(255);
}

// bf16 -> fp16 (finite values saturate, inf and NaN pass), 8 elements per thread.
__global__ __launch_bounds__(256) void x_to_f16_kernel(const uint16_t *__restrict__ X, int ldx, int T, int K,
                                                       uint16_t *__restrict__ Xh) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int kc = K / 8;
    if (i >= int64_t(T) * kc) return;
    const int64_t t = i / kc;
    const int c = int(i % kc);
    const uint4 v = *reinterpret_cast<const uint4 *>(X + t * ldx + c * 8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = bf16_bits_to_f32(uint16_t(w[j])), b = bf16_bits_to_f32(uint16_t(w[j] >> 16));
        o[j] = uint32_t(__builtin_bit_cast(uint16_t, f32_to_f16_satfinite(a))) |
               (uint32_t(__builtin_bit_cast(uint16_t, f32_to_f16_satfinite(b))) << 16);
    }
    *reinterpret_cast<uint4 *>(Xh + t * K + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
}

void launch_x_to_f16(const uint16_t *X, int ldx, int T, int K, uint16_t *Xh, hipStream_t s) {
    const int64_t n8 = int64_t(T) * (K / 8);
    x_to_f16_kernel<<<unsigned((n8 + 255) / 256), 256, 0, s>>>(X, ldx, T, K, Xh);
}

// One GB_M x BN output tile at tokens t0.., weight rows n0..
template <bool HAS_Z, int YT, int GB_M, int BN>
__device__ __forceinline__ void gemm_tile_at(const uint32_t *Wt, const uint16_t *St, const uint16_t *Zt,
                                             const uint16_t *__restrict__ Xh, int lda, int T, void *__restrict__ Y,
                                             int ldy, int N, int K, int t0, int n0) {
    using Sh = GemmShape<GB_M, BN>;
    const int tid = threadIdx.x, wave = tid / WAVE;
    const BRow b(Wt, St, Zt, min(n0 + b_tile_row<BN>(), N - 1), K / QGROUP);
    f32x16 acc[2][Sh::NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < Sh::NJ; ++j) acc[i][j] = f32x16{};
    const uint16_t *ap[GB_M / 32];
#pragma unroll
    for (int j = 0; j < GB_M / 32; ++j) ap[j] = Xh + int64_t(min(t0 + a_load_row(j), T - 1)) * lda;
    gemm_tile<GB_M, HAS_Z, BN>(ap, b, K, acc);

    const int wm = wave / Sh::NWN, wn2 = wave % Sh::NWN;
    constexpr int YB = YT == 0 ? 4 : 2;
    emit_tile<Sh::NJ, YB>(
        epi_slot(wave), acc,
        [](float v, int, int) {
            if constexpr (YT == 1) return f32_to_bf16_rne(v);
            else return __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(v));
        },
        [&](int tr, int col, uint4 v) {
            const int t = t0 + wm * 64 + tr, n = n0 + wn2 * Sh::WNR + col;
            if (t < T && n < N)
                *reinterpret_cast<uint4 *>(static_cast<unsigned char *>(Y) + (int64_t(t) * ldy + n) * YB) = v;
        });
}

// XCD-aware order: workgroups are dealt round-robin to the 8 XCDs; give each
// XCD a contiguous range of the nb items so that the blocks sharing an X tile
// run together and hit the same L2
__device__ __forceinline__ int xcd_item(int w, int nb) { return nb % 8 == 0 ? (w % 8) * (nb / 8) + w / 8 : w; }

template <bool HAS_Z, int YT, int GB_M, int BN = GB_N>
__global__ __launch_bounds__(G_THREADS) void q4_gemm_kernel(const uint32_t *Wt,
                                                            const uint16_t *St,
                                                            const uint16_t *Zt,
                                                            const uint16_t *__restrict__ Xh, int lda, int T,
                                                            void *__restrict__ Y, int ldy, int N, int K) {
    // token-major tile order (consecutive items share their X rows)
    const int lin = xcd_item(int(blockIdx.y * gridDim.x + blockIdx.x), int(gridDim.x * gridDim.y));
    const int by = lin / gridDim.x, bx = lin % gridDim.x;
    gemm_tile_at<HAS_Z, YT, GB_M, BN>(Wt, St, Zt, Xh, lda, T, Y, ldy, N, K, by * GB_M, bx * BN);
}

// 256 x 256 tiles that do not fill whole rounds of the chip: the first nbig
// (whole rounds) run as they are; each remaining tile runs as two 256 x 128
// halves, so the last round has twice the blocks at half the work each
// instead of a partly idle round of whole tiles. Tiles are numbered
// token-major over the 256 x 256 grid of nbx tiles per row.
template <bool HAS_Z, int YT>
__global__ __launch_bounds__(G_THREADS) void q4_gemm_mixed_kernel(const uint32_t *Wt, const uint16_t *St,
                                                                  const uint16_t *Zt,
                                                                  const uint16_t *__restrict__ Xh, int lda, int T,
                                                                  void *__restrict__ Y, int ldy, int N, int K,
                                                                  int nbx, int nbig, int nhalf) {
    const int w = blockIdx.x;
    if (w < nbig) {
        const int lin = xcd_item(w, nbig);
        gemm_tile_at<HAS_Z, YT, 256, 256>(Wt, St, Zt, Xh, lda, T, Y, ldy, N, K, lin / nbx * 256, lin % nbx * 256);
    } else {
        const int hw = xcd_item(w - nbig, nhalf), lin = nbig + hw / 2;
        gemm_tile_at<HAS_Z, YT, 256, 128>(Wt, St, Zt, Xh, lda, T, Y, ldy, N, K, lin / nbx * 256,
                                              lin % nbx * 256 + (hw % 2) * 128);
    }
}

template <bool HAS_Z, int YT, int GB_M, int BN = GB_N>
static void launch_gemm_t(const GemmArgs &a, const uint16_t *Xh, int lda, hipStream_t s) {
    auto kern = q4_gemm_kernel<HAS_Z, YT, GB_M, BN>;
    const dim3 grid(unsigned((a.N + BN - 1) / BN), unsigned((a.T + GB_M - 1) / GB_M));
    kern<<<grid, G_THREADS, 0, s>>>(a.W, a.S, a.Z, Xh, lda, a.T, a.Y, a.ldy, a.N, a.K);
}

// 256 x 256 tiles when they fill whole rounds of the chip (or many rounds);
// past one round with at most half a round left over, whole rounds of them
// plus the rest as 256 x 128 halves in the same launch (2048-token
// micro-batches of 4096->12288); else 256 tokens x 128 weight rows when those
// fill whole rounds (the same dequant work per MFMA); else 128 x 256.
template <bool HAS_Z, int YT>
static void launch_gemm_mixed(const GemmArgs &a, const uint16_t *Xh, int lda, int nbig, int nhalf, hipStream_t s) {
    const int nbx = (a.N + 255) / 256;
    q4_gemm_mixed_kernel<HAS_Z, YT><<<unsigned(nbig + nhalf), G_THREADS, 0, s>>>(
        a.W, a.S, a.Z, Xh, lda, a.T, a.Y, a.ldy, a.N, a.K, nbx, nbig, nhalf);
}

template <bool HAS_Z, int YT>
static void launch_gemm_m(const GemmArgs &a, const uint16_t *Xh, int lda, hipStream_t s) {
    int cus = 0, dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cus < 1) cus = 256;
    auto whole = [&](int64_t nb) {
        const double rounds = double(nb) / cus;
        return rounds >= 4.0 || (rounds >= 1.0 && rounds - double(int64_t(rounds)) < 0.01);
    };
    const int64_t t256 = (a.T + 255) / 256, nb = int64_t((a.N + 255) / 256) * t256;
    if (whole(nb)) launch_gemm_t<HAS_Z, YT, 256>(a, Xh, lda, s);
    else if (nb > cus && 2 * (nb % cus) <= cus)  // e.g. 2048 tokens x 12288 rows: 256 whole tiles + 256 halves
        launch_gemm_mixed<HAS_Z, YT>(a, Xh, lda, int(nb / cus * cus), int(2 * (nb % cus)), s);
    else if (whole(int64_t((a.N + 127) / 128) * t256)) launch_gemm_t<HAS_Z, YT, 256, 128>(a, Xh, lda, s);
    else launch_gemm_t<HAS_Z, YT, 128>(a, Xh, lda, s);
}

// bf16 rows go through the fp16 pre-pass into the workspace; fp16 rows
// (x_f16) are the MFMA operand as they are.
void launch_gemm(const GemmArgs &a, hipStream_t s) {
    const uint16_t *Xh = a.X;
    int lda = a.ldx;
    if (!a.x_f16) {
        uint16_t *w = static_cast<uint16_t *>(a.ws);
        launch_x_to_f16(a.X, a.ldx, a.T, a.K, w, s);
        Xh = w;
        lda = a.K;
    }
    if (a.Z) {
        if (a.y_type == 1) launch_gemm_m<true, 1>(a, Xh, lda, s);
        else if (a.y_type == 2) launch_gemm_m<true, 2>(a, Xh, lda, s);
        else launch_gemm_m<true, 0>(a, Xh, lda, s);
    } else {
        if (a.y_type == 1) launch_gemm_m<false, 1>(a, Xh, lda, s);
        else if (a.y_type == 2) launch_gemm_m<false, 2>(a, Xh, lda, s);
        else launch_gemm_m<false, 0>(a, Xh, lda, s);
    }
}

}  // namespace qwq4
