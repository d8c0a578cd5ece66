// q4-dequant prefill GEMM: Y[t][n] = sum_k X[t][k] * W[n][k] for a chunk of
// T tokens (reference role: gpu::gemm, src/kernels/gemm.hip:10-18, which
// calls rocBLAS on fp16 weights; here the weights stay q4 in HBM and are
// dequantised on the fly into LDS).
//
// Numerics. Each weight is dequantised once, w = fp16((q - z) * s) (the
// subtraction exact, one rounding for the product), the way the reference's
// grouped expert GEMM does (src/kernels/moe_experts.hip:31-42). X is
// converted to fp16 by a pre-pass (exact for |x| in the fp16 normal range,
// saturated at +-65504). Products and sums run on the fp16 MFMA with fp32
// accumulation. Rounding the dequantised weights to bf16 instead would cost
// ~1.4e-3 of max|y| (close to the 2e-3 bar); fp16 costs ~2e-4.
//
// Schedule. Block tile 256 tokens x 256 weight rows, 8 waves (4 x 2, two
// per SIMD) of 64 x 128 each on v_mfma_f32_32x32x16_f16; K in stages of 64,
// LDS double buffered (2 x (32 + 32) KB). For the next stage, the X tile goes
// global -> LDS by direct loads and the weight tile (8 KB of q4, tiled
// format; two threads per weight row) into registers, dequantised and
// written to LDS in two halves interleaved with the current stage's MFMAs;
// fragment reads run one 16-K step ahead. LDS rows are 128 B; 16-byte
// chunks are XOR-swizzled by row so fragment reads are bank-conflict free.
#include "q4_common.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

constexpr int GB_N = 256, GB_K = 64, G_THREADS = 512, G_WAVES = 8;
constexpr int TILE_BYTES = 256 * GB_K * 2;  // 32 KB: one operand of one stage (at most 256 rows)

size_t gemm_workspace_bytes(int T, int K) {
    const size_t xh = size_t(T) * K * 2;
    return (xh + 255) & ~size_t(255);
}

// bf16 -> fp16 (saturating), 8 elements per thread.
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
        float a = bf16_bits_to_f32(uint16_t(w[j])), b = bf16_bits_to_f32(uint16_t(w[j] >> 16));
        a = fminf(fmaxf(a, -65504.f), 65504.f);
        b = fminf(fmaxf(b, -65504.f), 65504.f);
        o[j] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(a))) |
               (uint32_t(__builtin_bit_cast(uint16_t, _Float16(b))) << 16);
    }
    *reinterpret_cast<uint4 *>(Xh + t * K + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
}

// byte offset of 16-byte chunk c (0..7) of row r in a [rows][64 fp16] tile.
// gfx950 LDS serves 256 B (64 banks) per cycle: the 16 rows one pass of a
// b128 access touches occupy two 128-byte halves (row parity), and within a
// half the chunk is XORed with r/2, so those 16 accesses hit 16 distinct
// 16-byte bank groups.
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// 8 packed nibbles (tiled word) -> 8 fp16 weights (q - z) * s
__device__ __forceinline__ uint4 dequant8(uint32_t w, uint32_t zb, h2 s2) {
    const uint4 u = unpack8<F16>(w, zb);  // 1040 + (q - z), exact
    const h2 bias = {(_Float16)1040.f, (_Float16)1040.f};
    uint4 r;
    r.x = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, u.x) - bias) * s2);
    r.y = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, u.y) - bias) * s2);
    r.z = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, u.z) - bias) * s2);
    r.w = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, u.w) - bias) * s2);
    return r;
}

// GB_M = 256: waves 4 (tokens) x 2 (rows) of 64 x 128; GB_M = 128: 2 x 4 of 64 x 64
template <bool HAS_Z, bool Y_BF16, int GB_M>
__global__ __launch_bounds__(G_THREADS) void q4_gemm_kernel(const uint32_t *__restrict__ Wt,
                                                            const uint16_t *__restrict__ St,
                                                            const uint16_t *__restrict__ Zt,
                                                            const uint16_t *__restrict__ Xh, int T, void *__restrict__ Y,
                                                            int ldy, int N, int K) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int G = K / QGROUP, nsub = N / 16, nk = K / GB_K;
    // XCD-aware tile order: workgroups are dealt round-robin to the 8 XCDs;
    // give each XCD a contiguous, token-major range of tiles so the blocks
    // sharing an X tile run together and hit the same L2
    int bx = blockIdx.x, by = blockIdx.y;
    {
        const int nb = gridDim.x * gridDim.y, w = blockIdx.y * gridDim.x + blockIdx.x;
        if (nb % 8 == 0) {
            const int lin = (w % 8) * (nb / 8) + w / 8;
            by = lin / gridDim.x;
            bx = lin % gridDim.x;
        }
    }
    const int t0 = by * GB_M, n0 = bx * GB_N;
    // stage buffers: A(i) at 2i * TILE_BYTES, B(i) right after it
    auto bufA = [&](int i) { return smem + 2 * i * TILE_BYTES; };
    auto bufB = [&](int i) { return smem + (2 * i + 1) * TILE_BYTES; };

    // ---- X tile: direct global->LDS loads, 1 KB (8 rows x 8 chunks) per
    // wave instruction; lane i -> row i/8, LDS slot i%8 holding the chunk
    // that swz() places there
    auto issue_a = [&](int ks, unsigned char *dst) {
        const int k0 = ks * GB_K;
#pragma unroll
        for (int j = 0; j < GB_M / 8 / G_WAVES; ++j) {  // GB_M / 64 instructions per wave
            const int rb = (j * G_WAVES + wave) * 8;
            const int r = rb + lane / 8, c = (lane % 8) ^ ((r >> 1) & 7);
            const int t = min(t0 + r, T - 1);
            __builtin_amdgcn_global_load_lds(Xh + int64_t(t) * K + k0 + c * 8, dst + rb * 128, 16, 0, 0);
        }
    };
    // ---- weight tile: thread pair (2r, 2r+1) owns weight row n0 + r, one
    // 32-element quarter each per stage
    const int brow = tid / 2, bq = tid % 2;
    const int wrow = n0 + brow, wsub = min(wrow / 16, nsub - 1), wn = wrow % 16;
    const uint4 *wbase = reinterpret_cast<const uint4 *>(Wt) + int64_t(wsub) * G * 64 + wn;
    const uint16_t *sbase = St + int64_t(wsub) * ((G + 3) / 4) * 64 + wn * 4;
    const uint16_t *zbase = HAS_Z ? Zt + int64_t(wsub) * ((G + 3) / 4) * 16 + wn : nullptr;
    uint4 wr;
    uint32_t sr = 0, zr = 0;
    auto issue_b = [&](int ks) {  // quarter 2(ks%2) + bq of group ks/2
        const int g = ks / 2;
        wr = wbase[g * 64 + ((ks % 2) * 2 + bq) * 16];
        sr = sbase[(g >> 2) * 64 + (g & 3)];
        if constexpr (HAS_Z) zr = zbase[(g >> 2) * 16];
    };
    // half h of the dequant (2 of the 4 words), written swizzled
    auto commit_b = [&](int ks, unsigned char *dst, int h) {
        const int g = ks / 2;
        const uint32_t zb = zero_bytes(HAS_Z ? (zr >> (4 * (g & 3))) & 0xfu : 8u);
        const _Float16 sc = __builtin_bit_cast(_Float16, uint16_t(sr));
        const h2 s2 = {sc, sc};
        const uint32_t words[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
        for (int c = 2 * h; c < 2 * h + 2; ++c)
            *reinterpret_cast<uint4 *>(dst + swz(brow, bq * 4 + c)) = dequant8(words[c], zb, s2);
    };

    // ---- MFMA tiles: wave (wm, wn2) owns tokens 64 wm.. x weight rows WNR wn2..
    constexpr int NWN = G_WAVES / (GB_M / 64), WNR = GB_N / NWN, NJ = WNR / 32;
    const int wm = wave / NWN, wn2 = wave % NWN, l32 = lane % 32, lh = lane / 32;
    f32x16 acc[2][NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16{};
    auto read_frags = [&](const unsigned char *a, const unsigned char *b, int kk, uint4 (&af)[2], uint4 (&bf)[NJ]) {
        const int c = kk * 2 + lh;
#pragma unroll
        for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const uint4 *>(a + swz(wm * 64 + i * 32 + l32, c));
#pragma unroll
        for (int j = 0; j < NJ; ++j) bf[j] = *reinterpret_cast<const uint4 *>(b + swz(wn2 * WNR + j * 32 + l32, c));
    };
    // MFMAs of one stage; fragments of step kk+1 are read during step kk,
    // and the next stage's weights are dequantised into LDS in two halves
    // between them (ksn < 0: nothing to dequantise)
    auto compute = [&](const unsigned char *a, const unsigned char *b, int ksn, unsigned char *dstb) {
        uint4 af[2], bf[NJ], an[2], bn[NJ];
        read_frags(a, b, 0, af, bf);
#pragma unroll
        for (int kk = 0; kk < GB_K / 16; ++kk) {
            if (kk + 1 < GB_K / 16) read_frags(a, b, kk + 1, an, bn);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32<F16>(af[i], bf[j], acc[i][j]);
            if (ksn >= 0 && (kk == 1 || kk == 3)) commit_b(ksn, dstb, kk / 2);
            // interleave: one MFMA, then up to four VALU instructions
#pragma unroll
            for (int q = 0; q < 2 * NJ; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) af[i] = an[i];
#pragma unroll
            for (int j = 0; j < NJ; ++j) bf[j] = bn[j];
        }
    };

    issue_a(0, bufA(0));
    issue_b(0);
    commit_b(0, bufB(0), 0);
    commit_b(0, bufB(0), 1);
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
        const int cur = ks & 1, nxt = cur ^ 1;
        const bool more = ks + 1 < nk;
        if (more) {
            issue_a(ks + 1, bufA(nxt));
            issue_b(ks + 1);
        }
        compute(bufA(cur), bufB(cur), more ? ks + 1 : -1, bufB(nxt));
        __syncthreads();
    }

    // ---- epilogue: lane holds weight row n = 32 j + l32 and tokens
    // 8(r/4) + 4 lh + r%4 of each 32 x 32 tile. Each 64 x 32 column slice of
    // the wave's tile is transposed through the wave's own LDS area (free
    // after the K loop) so that the stores are 16 bytes per lane along n.
    constexpr int YB = Y_BF16 ? 2 : 4, ROWB = 32 * YB, PER_ROW = ROWB / 16;
    unsigned char *ep = smem + wave * 64 * ROWB;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tr = i * 32 + (r / 4) * 8 + lh * 4 + (r % 4);
                if constexpr (Y_BF16)
                    *reinterpret_cast<uint16_t *>(ep + tr * ROWB + l32 * 2) = f32_to_bf16_rne(acc[i][j][r]);
                else
                    *reinterpret_cast<float *>(ep + tr * ROWB + l32 * 4) = acc[i][j][r];
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
        for (int p = lane; p < 64 * PER_ROW; p += WAVE) {
            const int tr = p / PER_ROW, pc = p % PER_ROW;
            const int t = t0 + wm * 64 + tr, n = n0 + wn2 * WNR + j * 32 + pc * (16 / YB);
            if (t < T && n < N)
                *reinterpret_cast<uint4 *>(static_cast<unsigned char *>(Y) + (int64_t(t) * ldy + n) * YB) =
                    *reinterpret_cast<const uint4 *>(ep + tr * ROWB + pc * 16);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
}

template <bool HAS_Z, bool Y_BF16, int GB_M>
static void launch_gemm_t(const GemmArgs &a, const uint16_t *Xh, hipStream_t s) {
    auto kern = q4_gemm_kernel<HAS_Z, Y_BF16, GB_M>;
    const size_t lds = 4 * size_t(TILE_BYTES);
    (void)persistent_shape(reinterpret_cast<const void *>(kern), G_THREADS, lds);  // sets the LDS limit
    const dim3 grid(unsigned((a.N + GB_N - 1) / GB_N), unsigned((a.T + GB_M - 1) / GB_M));
    kern<<<grid, G_THREADS, lds, s>>>(a.W, a.S, a.Z, Xh, a.T, a.Y, a.ldy, a.N, a.K);
}

// 256-token tiles when they fill whole rounds of the chip, else 128
template <bool HAS_Z, bool Y_BF16>
static void launch_gemm_m(const GemmArgs &a, const uint16_t *Xh, hipStream_t s) {
    int cus = 0, dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cus < 1) cus = 256;
    const int64_t nb = int64_t((a.N + GB_N - 1) / GB_N) * ((a.T + 255) / 256);
    const double rounds = double(nb) / cus;
    const bool big = rounds >= 4.0 || (rounds >= 1.0 && rounds - double(int64_t(rounds)) < 0.01);
    if (big) launch_gemm_t<HAS_Z, Y_BF16, 256>(a, Xh, s);
    else launch_gemm_t<HAS_Z, Y_BF16, 128>(a, Xh, s);
}

void launch_gemm(const GemmArgs &a, hipStream_t s) {
    uint16_t *Xh = static_cast<uint16_t *>(a.ws);
    const int64_t n8 = int64_t(a.T) * (a.K / 8);
    x_to_f16_kernel<<<unsigned((n8 + 255) / 256), 256, 0, s>>>(a.X, a.ldx, a.T, a.K, Xh);
    if (a.Z) {
        if (a.y_bf16) launch_gemm_m<true, true>(a, Xh, s);
        else launch_gemm_m<true, false>(a, Xh, s);
    } else {
        if (a.y_bf16) launch_gemm_m<false, true>(a, Xh, s);
        else launch_gemm_m<false, false>(a, Xh, s);
    }
}

}  // namespace qwq4
