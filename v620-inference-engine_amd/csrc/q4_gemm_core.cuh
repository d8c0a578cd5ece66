// Shared main loop of the q4-dequant MFMA GEMMs (dense prefill GEMM and the
// grouped expert GEMMs): one block computes a GB_M x 256 tile of
// A (fp16 rows, K long) times W^T (256 q4 weight rows of the tiled format).
//
// Schedule. 8 waves (two per SIMD); GB_M = 256: waves 4 (rows of A) x 2
// (weight rows) of 64 x 128 each, GB_M = 128: 2 x 4 of 64 x 64; MFMA
// v_mfma_f32_32x32x16_f16. K runs in stages of 64 through a double-buffered
// LDS (2 x (32 + 32) KB). For the next stage, the A tile goes global -> LDS
// by direct loads (1 KB = 8 rows per wave instruction, any row addresses)
// and the weight tile (8 KB of q4; two threads per weight row) into
// registers two stages ahead, dequantised and written to LDS in two halves
// interleaved with the MFMAs of the stage before its own; fragment reads run
// one 16-K step ahead.
//
// Numerics: each weight becomes fp16((q - z) * s) (exact subtraction, one
// rounding); products and sums run on the fp16 MFMA with fp32 accumulation.
#pragma once

#include "q4_common.cuh"

namespace qwq4 {

constexpr int GB_N = 256, GB_K = 64, G_THREADS = 512, G_WAVES = 8;
constexpr int TILE_BYTES = 256 * GB_K * 2;     // 32 KB: one operand of one stage (<= 256 rows)
constexpr size_t GEMM_LDS = 4 * size_t(TILE_BYTES);  // the stage buffers (static LDS)

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

template <int GB_M>
struct GemmShape {
    static constexpr int NWN = G_WAVES / (GB_M / 64);  // waves along the weight rows
    static constexpr int WNR = GB_N / NWN;             // weight rows per wave
    static constexpr int NJ = WNR / 32;                // 32-row MFMA tiles per wave
};

// The thread's weight row (thread pair 2r, 2r+1 owns tile row r): its tiled
// 16-byte entries, scales and zero words.
struct BRow {
    const uint4 *w;
    const uint16_t *s;
    const uint32_t *z;  // the 32-bit word holding this row's 16-bit zero word (zs: its shift)
    int zs;
    __device__ __forceinline__ BRow(const uint32_t *Wt, const uint16_t *St, const uint16_t *Zt, int64_t row, int G) {
        const int64_t sub = row / 16;
        const int n = int(row % 16), GC = (G + 3) / 4;
        w = reinterpret_cast<const uint4 *>(Wt) + sub * G * 64 + n;
        s = St + sub * GC * 64 + n * 4;
        z = Zt ? reinterpret_cast<const uint32_t *>(Zt + sub * GC * 16 + (n & ~1)) : nullptr;
        zs = (n & 1) * 16;
    }
};

// The A-tile row whose 16-byte pieces this thread loads in part j of a stage
// (j < GB_M / 64): the caller resolves it to a row pointer once per block.
__device__ __forceinline__ int a_load_row(int j) { return (j * G_WAVES + int(threadIdx.x) / WAVE) * 8 + int(threadIdx.x) % WAVE / 8; }

// acc += A_tile (GB_M x K; ap[j] = start of row a_load_row(j)) * W_tile^T
// (256 rows; this thread's row is b). Ends with a barrier; the LDS is free
// afterwards.
// The four stage buffers are distinct LDS objects: the compiler can then tell
// the direct-to-LDS loads into one A buffer from the fragment reads of the
// other, and does not drain every load in flight before those reads (with
// one LDS array it must assume they may alias). Returns the first buffer,
// free for the epilogue.
template <int GB_M, bool HAS_Z, class Acc>
__device__ __forceinline__ unsigned char *gemm_tile(const uint16_t *const *ap, const BRow &b, int K, Acc &acc) {
    using S = GemmShape<GB_M>;
    constexpr int NJ = S::NJ;
    __shared__ __align__(16) unsigned char lds_a0[TILE_BYTES], lds_a1[TILE_BYTES], lds_b0[TILE_BYTES],
        lds_b1[TILE_BYTES];
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int nk = K / GB_K;
    auto bufA = [&](int i) { return i ? lds_a1 : lds_a0; };
    auto bufB = [&](int i) { return i ? lds_b1 : lds_b0; };

    // A tile: lane i of an instruction -> row rb + i/8 (= a_load_row(j)), LDS
    // slot i%8 holding the chunk swz() places there
    auto issue_a = [&](int ks, unsigned char *dst) {
        const int k0 = ks * GB_K;
#pragma unroll
        for (int j = 0; j < GB_M / 8 / G_WAVES; ++j) {
            const int rb = (j * G_WAVES + wave) * 8;
            const int r = rb + lane / 8, c = (lane % 8) ^ ((r >> 1) & 7);
            __builtin_amdgcn_global_load_lds(ap[j] + k0 + c * 8, dst + rb * 128, 16, 0, 0);
        }
    };
    const int brow = tid / 2, bq = tid % 2;
    // raw weights of one stage: this thread's quarter 2(ks%2) + bq of group
    // ks/2, its scale and zero word
    struct BRaw {
        uint4 w;
        uint32_t s, z;
    };
    auto issue_b = [&](int ks, BRaw &r) {
        ks = min(ks, nk - 1);  // past the end: a valid (unused) load keeps the code branch-free
        const int g = ks / 2;
        r.w = b.w[g * 64 + ((ks % 2) * 2 + bq) * 16];
        r.s = b.s[(g >> 2) * 64 + (g & 3)];
        if constexpr (HAS_Z) r.z = b.z[(g >> 2) * 8] >> b.zs;  // (a 32-bit load: see BRow)
    };
    // half h of the dequant (2 of the 4 words), written swizzled
    auto commit_b = [&](int ks, const BRaw &r, unsigned char *dst, int h) {
        const int g = ks / 2;
        const uint32_t zb = zero_bytes(HAS_Z ? (r.z >> (4 * (g & 3))) & 0xfu : 8u);
        const _Float16 sc = __builtin_bit_cast(_Float16, uint16_t(r.s));
        const h2 s2 = {sc, sc};
        const uint32_t words[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
#pragma unroll
        for (int c = 2 * h; c < 2 * h + 2; ++c)
            *reinterpret_cast<uint4 *>(dst + swz(brow, bq * 4 + c)) = dequant8(words[c], zb, s2);
    };

    const int wm = wave / S::NWN, wn2 = wave % S::NWN, l32 = lane % 32, lh = lane / 32;
    auto read_frags = [&](const unsigned char *a, const unsigned char *bb, int kk, uint4 (&af)[2], uint4 (&bf)[NJ]) {
        const int c = kk * 2 + lh;
#pragma unroll
        for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const uint4 *>(a + swz(wm * 64 + i * 32 + l32, c));
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            bf[j] = *reinterpret_cast<const uint4 *>(bb + swz(wn2 * S::WNR + j * 32 + l32, c));
    };
    // MFMAs of one stage; fragments of step kk+1 are read during step kk, and
    // the next stage's weights (raw, loaded a stage earlier) are dequantised
    // in two halves between them
    auto compute = [&](const unsigned char *a, const unsigned char *bb, int ksn, const BRaw &rn, unsigned char *dstb) {
        uint4 af[2], bf[NJ], an[2], bn[NJ];
        read_frags(a, bb, 0, af, bf);
#pragma unroll
        for (int kk = 0; kk < GB_K / 16; ++kk) {
            if (kk + 1 < GB_K / 16) read_frags(a, bb, kk + 1, an, bn);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32<F16>(af[i], bf[j], acc[i][j]);
            if (ksn >= 0 && (kk == 1 || kk == 3)) commit_b(ksn, rn, dstb, kk / 2);
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

    // Stage ks (parity p): the A tile of ks + 1 goes to LDS by direct loads
    // and the raw weights of ks + 2 into register set p, both requested
    // before the stage's MFMAs (the barrier that ends the stage waits for
    // them); the weights of ks + 1 (set 1 - p, loaded during the previous
    // stage) are dequantised into LDS between the MFMAs.
    BRaw rs[2];
    issue_a(0, bufA(0));
    issue_b(0, rs[0]);
    commit_b(0, rs[0], bufB(0), 0);
    commit_b(0, rs[0], bufB(0), 1);
    issue_b(1, rs[1]);
    __syncthreads();
    auto stage = [&](int ks, BRaw &mine, const BRaw &next, int p) {
        const bool more = ks + 1 < nk;
        issue_b(ks + 2, mine);
        // unconditional (the last stage reloads its own K range into the
        // idle buffer): with a branch around them the compiler could no
        // longer count which loads are in flight and would drain them all
        issue_a(min(ks + 1, nk - 1), bufA(p ^ 1));
        compute(bufA(p), bufB(p), more ? ks + 1 : -1, next, bufB(p ^ 1));
        lds_barrier();  // (also waits for this wave's A loads of ks + 1)
    };
    for (int ks = 0; ks < nk; ks += 2) {  // nk is even (K is a multiple of 128)
        stage(ks, rs[0], rs[1], 0);
        stage(ks + 1, rs[1], rs[0], 1);
    }
    return lds_a0;
}

// Wave-private LDS transpose for the epilogue: the wave's acc[i][j] (rows
// 64 wm + 32 i + 8(r/4) + 4 lh + r%4, weight row 32 j + l32 of its slice) is
// handed to emit(row, col, 16-byte piece) one 64 x 32 column slice at a
// time, as 16-byte pieces along the weight-row axis. YB: bytes per output
// element (2: values rounded to bf16 / converted to fp16 by cvt, 4: fp32).
template <int NJ, int YB, class CvtFn, class EmitFn>
__device__ __forceinline__ void emit_tile(unsigned char *ep, const f32x16 (&acc)[2][NJ], CvtFn cvt, EmitFn emit) {
    constexpr int ROWB = 32 * YB, PER_ROW = ROWB / 16;
    const int lane = threadIdx.x % WAVE, l32 = lane % 32, lh = lane / 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tr = i * 32 + (r / 4) * 8 + lh * 4 + (r % 4);
                if constexpr (YB == 2)
                    *reinterpret_cast<uint16_t *>(ep + tr * ROWB + l32 * 2) = cvt(acc[i][j][r], tr, j * 32 + l32);
                else
                    *reinterpret_cast<float *>(ep + tr * ROWB + l32 * 4) = acc[i][j][r];
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
        for (int p = lane; p < 64 * PER_ROW; p += WAVE) {
            const int tr = p / PER_ROW, pc = p % PER_ROW;
            emit(tr, j * 32 + pc * (16 / YB), *reinterpret_cast<const uint4 *>(ep + tr * ROWB + pc * 16));
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
}

}  // namespace qwq4
