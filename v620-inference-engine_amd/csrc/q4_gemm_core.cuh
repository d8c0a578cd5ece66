// Shared main loop of the q4-dequant MFMA GEMMs (dense prefill GEMM and the
// grouped expert GEMMs): one block computes a GB_M x 256 tile of
// A (fp16 rows, K long) times W^T (256 q4 weight rows of the tiled format).
//
// Schedule. 8 waves (two per SIMD); GB_M = 256: waves 4 (rows of A) x 2
// (weight rows) of 64 x 128 each, GB_M = 128: 2 x 4 of 64 x 64; MFMA
// v_mfma_f32_32x32x16_f16. K runs in stages of 64 through a double-buffered
// LDS (2 x (32 + 32) KB). Besides its MFMAs each wave has one loading role:
//   waves 0-3 (one per SIMD) move the next stage's A tile global -> LDS by
//     direct loads (1 KB = 8 rows per wave instruction, any row addresses);
//   waves 4-7 load the weight tile (8 KB of q4, one thread per weight row)
//     into registers two stages ahead and dequantise it into LDS in two
//     halves interleaved with the MFMAs of the stage before its own.
// The roles run as separate code paths: a wave with direct-to-LDS loads in
// flight waits for all of its loads at every barrier, so the weight loads
// must not be issued by those waves or they would get one stage, not two.
// Fragment reads run one 16-K step ahead.
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
// The chunk is XORed with (r & 7) ^ bit 3 of r. Two access shapes use it:
// the weight dequant writes one row per lane (64 consecutive rows, one
// chunk), and the fragment reads take 32 consecutive rows at chunk c (lanes
// 0-31) and c+1 (lanes 32-63). Measured with SQ_LDS_BANK_CONFLICT on gfx950
// both are conflict-free under this XOR; the XOR with r/2 used before left
// the reads clean but served the b128 writes at half rate (conflict cycles
// = 1/2 of the active LDS cycles), and XOR with r & 7 alone does the same
// to the reads.
__device__ __forceinline__ int swz_x(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ swz_x(r)) << 4); }

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// 8 packed nibbles (tiled word) -> 8 fp16 weights (q - z) * s: the nibbles
// become fp16 1024 + q (unpack8 with no byte offset), 1024 + z is subtracted
// (exact), then one rounding multiply by s
__device__ __forceinline__ uint4 dequant8(uint32_t w, h2 bias, h2 s2) {
    const uint4 u = unpack8<F16>(w, 0u);  // 1024 + q, exact
    uint4 r;
    r.x = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, u.x) - bias) * s2);
    r.y = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, u.y) - bias) * s2);
    r.z = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, u.z) - bias) * s2);
    r.w = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, u.w) - bias) * s2);
    return r;
}

// the packed fp16 1024 + z of a zero point z (0..15)
__device__ __forceinline__ h2 zero_bias(uint32_t z) {
    const _Float16 b = __builtin_bit_cast(_Float16, uint16_t(0x6400u | z));
    return h2{b, b};
}

// GB_M rows of A by BN weight rows (BN = 256, or 128 where a 256 x 256
// grid would leave a partial round)
template <int GB_M, int BN = GB_N>
struct GemmShape {
    static constexpr int NWN = G_WAVES / (GB_M / 64);  // waves along the weight rows
    static constexpr int WNR = BN / NWN;               // weight rows per wave
    static constexpr int NJ = WNR / 32;                // 32-row MFMA tiles per wave
};

// The weight row a thread of waves 4-7 loads and dequantises: tile row
// tid % BN (b_tile_row<BN>()); its tiled 16-byte entries, scales and zero
// words. With BN = 128 two threads share a row, one per 32-K half of a stage.
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

constexpr int G_ROLE = G_WAVES / 2;  // waves per loading role

// The four stage buffers (A and weights, two stages each), at file scope so
// that every tile shape instantiated in one kernel shares them. Distinct
// objects: the compiler can then tell the direct-to-LDS loads into one A
// buffer from the fragment reads of the other, and does not drain every load
// in flight before those reads (with one LDS array it must assume they may
// alias).
static __shared__ __align__(16) unsigned char lds_a0[TILE_BYTES], lds_a1[TILE_BYTES], lds_b0[TILE_BYTES],
    lds_b1[TILE_BYTES];

constexpr int EPI_BYTES = 64 * 32 * 4;  // one wave's epilogue slot: a 64 x 32 slice of fp32

// The wave's epilogue slot once gemm_tile has returned: waves 0-3 in lds_a0,
// 4-7 in lds_b0 (lds_a1 and lds_b1 stay free for the caller).
__device__ __forceinline__ unsigned char *epi_slot(int wave) {
    return (wave < 4 ? lds_a0 : lds_b0) + (wave % 4) * EPI_BYTES;
}

template <int BN = GB_N>
__device__ __forceinline__ int b_tile_row() { return int(threadIdx.x) % BN; }

// The A-tile row whose 16-byte pieces a thread of waves 0-3 loads in part j
// of a stage (j < GB_M / 32): the caller resolves it to a row pointer once
// per block (for all threads; only waves 0-3 use them).
__device__ __forceinline__ int a_load_row(int j) {
    return (j * G_ROLE + int(threadIdx.x) / WAVE % G_ROLE) * 8 + int(threadIdx.x) % WAVE / 8;
}

// acc += A_tile (GB_M x K; ap[j] = start of row a_load_row(j)) * W_tile^T
// (BN rows; a weight-loading thread's row is b). Ends with a barrier; the
// LDS is free afterwards (epilogues: epi_slot).
template <int GB_M, bool HAS_Z, int BN = GB_N, class Acc>
__device__ __forceinline__ void gemm_tile(const uint16_t *const *ap, const BRow &b, int K, Acc &acc) {
    using S = GemmShape<GB_M, BN>;
    static_assert(BN == 256 || BN == 128, "weight tile of 256 or 128 rows");
    constexpr int NH = BN == 256 ? 2 : 1;  // 16-byte weight entries (32 K) per thread and stage
    constexpr int NJ = S::NJ;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
    const int nk = K / GB_K;
    auto bufA = [&](int i) { return i ? lds_a1 : lds_a0; };
    auto bufB = [&](int i) { return i ? lds_b1 : lds_b0; };

    // A tile (waves 0-3): lane i of an instruction -> row rb + i/8 (=
    // a_load_row(j)), LDS slot i%8 holding the chunk swz() places there
    auto issue_a = [&](int ks, unsigned char *dst) {
        const int k0 = ks * GB_K, wa = wave % G_ROLE;
#pragma unroll
        for (int j = 0; j < GB_M / 8 / G_ROLE; ++j) {
            const int rb = (j * G_ROLE + wa) * 8;
            const int r = rb + lane / 8, c = (lane % 8) ^ swz_x(r);
            __builtin_amdgcn_global_load_lds(ap[j] + k0 + c * 8, dst + rb * 128, 16, 0, 0);
        }
    };
    const int brow = b_tile_row<BN>(), bh = BN == 256 ? 0 : (tid % 256) / 128;  // bh: this thread's half (BN 128)
    // raw weights of one stage (waves 4-7): quarters 2(ks%2), 2(ks%2)+1 of
    // group ks/2 of this thread's row (BN 128: quarter 2(ks%2) + bh only),
    // its scale and zero word
    struct BRaw {  // exactly as loaded: nothing is computed from them before their use
        uint4 w0, w1;  // (w1 unused with BN 128)
        uint16_t s;
        uint32_t z;
    };
    auto issue_b = [&](int ks, BRaw &r) {
        ks = min(ks, nk - 1);  // past the end: a valid (unused) load keeps the code branch-free
        const int g = ks / 2;
        if constexpr (NH == 2) {
            r.w0 = b.w[g * 64 + ((ks % 2) * 2) * 16];
            r.w1 = b.w[g * 64 + ((ks % 2) * 2 + 1) * 16];
        } else {
            r.w0 = b.w[g * 64 + ((ks % 2) * 2 + bh) * 16];
        }
        r.s = b.s[(g >> 2) * 64 + (g & 3)];
        if constexpr (HAS_Z) r.z = b.z[(g >> 2) * 8];  // the 32-bit word holding the row's zeros (see BRow)
    };
    // half h of the dequant (one of the two 16-byte entries: 4 chunks),
    // written swizzled (BN 128: the thread's own half bh)
    auto commit_b = [&](int ks, const BRaw &r, unsigned char *dst, int h) {
        if constexpr (NH == 1) h = bh;
        const int g = ks / 2;
        // the scale and zero word are taken here, not earlier: the compiler
        // would otherwise work them out right after their loads (waiting
        // for them a stage early, and with them for everything issued since)
        uint32_t zw = HAS_Z ? r.z : 0u, sw = r.s;
        asm volatile("" : "+v"(zw), "+v"(sw));
        const h2 zb = zero_bias(HAS_Z ? (zw >> (b.zs + 4 * (g & 3))) & 0xfu : 8u);
        const _Float16 sc = __builtin_bit_cast(_Float16, uint16_t(sw));
        const h2 s2 = {sc, sc};
        const uint4 w = (NH == 1 || !h) ? r.w0 : r.w1;
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) *reinterpret_cast<uint4 *>(dst + swz(brow, h * 4 + c)) = dequant8(words[c], zb, s2);
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
    // MFMAs of one stage; fragments of step kk+1 are read during step kk;
    // extra(kk) runs between the MFMAs of step kk (the weight dequant)
    auto compute = [&](const unsigned char *a, const unsigned char *bb, auto extra) {
        uint4 af[2], bf[NJ], an[2], bn[NJ];
        read_frags(a, bb, 0, af, bf);
#pragma unroll
        for (int kk = 0; kk < GB_K / 16; ++kk) {
            if (kk + 1 < GB_K / 16) read_frags(a, bb, kk + 1, an, bn);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32<F16>(af[i], bf[j], acc[i][j]);
            extra(kk);
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

    if (wave < G_ROLE) {
        // A role. Stage ks (parity p): the A tile of ks + 1 goes to LDS
        // before the stage's MFMAs; the stage-ending barrier waits for it.
        issue_a(0, bufA(0));
        __syncthreads();
        auto stage = [&](int ks, int p) {
            // unconditional (the last stage reloads its own K range into the
            // idle buffer): with a branch around them the compiler could no
            // longer count which loads are in flight and would drain them all
            issue_a(min(ks + 1, nk - 1), bufA(p ^ 1));
            compute(bufA(p), bufB(p), [](int) {});
            lds_barrier();
        };
        for (int ks = 0; ks < nk; ks += 2) {  // nk is even (K is a multiple of 128)
            stage(ks, 0);
            stage(ks + 1, 1);
        }
    } else {
        // Weight role. Stage ks (parity p): the raw weights of ks + 2 into
        // register set p, those of ks + 1 (set 1 - p) dequantised into LDS
        // between the MFMAs; no direct loads pending, so the barriers wait
        // for LDS traffic only and the weight loads keep two stages.
        // With 256 weight rows these waves issue ahead of the A-role waves
        // of their SIMD (wave priority): their dequant and loads then do not
        // queue behind the other wave's MFMAs, which fill the gaps (256 x 256:
        // +3%; with 128 rows, half the dequant per thread, it costs 2%).
        if constexpr (BN == 256) __builtin_amdgcn_s_setprio(2);
        BRaw rs[2];
        issue_b(0, rs[0]);
        commit_b(0, rs[0], bufB(0), 0);
        if constexpr (NH == 2) commit_b(0, rs[0], bufB(0), 1);
        issue_b(1, rs[1]);
        __syncthreads();
        auto stage = [&](int ks, BRaw &mine, const BRaw &next, int p) {
            const bool more = ks + 1 < nk;
            issue_b(ks + 2, mine);
            compute(bufA(p), bufB(p), [&](int kk) {
                if (more && (kk == 1 || (NH == 2 && kk == 3))) commit_b(ks + 1, next, bufB(p ^ 1), kk / 2);
            });
            lds_barrier();
        };
        for (int ks = 0; ks < nk; ks += 2) {
            stage(ks, rs[0], rs[1], 0);
            stage(ks + 1, rs[1], rs[0], 1);
        }
        if constexpr (BN == 256) __builtin_amdgcn_s_setprio(0);
    }
}

// A BM-row tile (BM a multiple of 32 up to 160) by 512 weight rows, weights dequantised
// in registers: wave w owns weight rows 64 w .. 64 w + 63 as two 32-row
// groups (b0: 64 w + lane % 32, b1: 64 w + 32 + lane % 32) and computes all
// BM rows of A against both (acc[i][j]: A rows 32 i .., group j). Every
// weight row feeds one wave, which dequantises it itself (one tiled entry
// per row, stage and lane, requested two stages ahead, one word per 16-K
// step), so each dequantised word serves 2 BM / 32 MFMAs, and each A
// fragment read from LDS serves two MFMAs (half the LDS reads per MFMA of a
// one-group-per-wave form, 32 weight rows per wave, which the grouped GEMMs
// used before: 1.96 against 1.82-1.86 ms per config-5 chunk). Only A goes
// through LDS: wave w moves rows 64 j + 8 w .. + 7 (arow[j]: this lane's
// row, 64 j + 8 w + lane / 8; rows past BM none). Four-wave blocks of 256
// weight rows (two blocks per CU) measured slower (down GEMM 835 against
// 661 us).
// (USE: a tag per call site; the host pass rejects one specialization
// called from two kernels' device code)
template <int BM, bool HAS_Z, int USE>
__device__ __forceinline__ void gemm_tile_rd2(const uint16_t *const (&arow)[(BM + 63) / 64], const BRow &b0,
                                              const BRow &b1, int K, f32x16 (&acc)[BM / 32][2]) {
    static_assert(BM % 32 == 0 && BM <= 160, "tiles of 32 to 160 rows");
    constexpr int NI = BM / 32, NA = (BM + 63) / 64;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
    const int l32 = lane % 32, lh = lane / 32, nk = K / GB_K;
    constexpr int NLD = HAS_Z ? 6 : 4;  // weight-side loads per stage and lane
    auto bufA = [&](int i) { return i ? lds_a1 : lds_a0; };
    auto issue_a = [&](int ks, unsigned char *dst) {
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int rb = 64 * j + wave * 8, r = rb + lane / 8, c = (lane % 8) ^ swz_x(r);
            if (rb < BM)  // (wave-uniform)
                __builtin_amdgcn_global_load_lds(arow[j] + ks * GB_K + c * 8, dst + rb * 128, 16, 0, 0);
        }
    };
    struct WR {
        uint4 w0, w1;
        uint16_t s0, s1;
        uint32_t z0, z1;
    };
    auto issue_w = [&](int ks, WR &r) {
        ks = min(ks, nk - 1);  // past the end: a valid (unused) load
        const int g = ks / 2, e = g * 64 + ((ks % 2) * 2 + lh) * 16, so = (g >> 2) * 64 + (g & 3);
        r.w0 = b0.w[e];
        r.w1 = b1.w[e];
        r.s0 = b0.s[so];
        r.s1 = b1.s[so];
        if constexpr (HAS_Z) {
            r.z0 = b0.z[(g >> 2) * 8];
            r.z1 = b1.z[(g >> 2) * 8];
        }
    };
    auto compute = [&](const unsigned char *a, const WR &r, int ks) {
        uint32_t s0 = r.s0, s1 = r.s1, z0 = HAS_Z ? r.z0 : 0u, z1 = HAS_Z ? r.z1 : 0u;
        asm volatile("" : "+v"(s0), "+v"(s1), "+v"(z0), "+v"(z1));  // taken here, not at their loads (see commit_b)
        const int g = ks / 2;
        const h2 zb0 = zero_bias(HAS_Z ? (z0 >> (b0.zs + 4 * (g & 3))) & 0xfu : 8u);
        const h2 zb1 = zero_bias(HAS_Z ? (z1 >> (b1.zs + 4 * (g & 3))) & 0xfu : 8u);
        const _Float16 c0 = __builtin_bit_cast(_Float16, uint16_t(s0)), c1 = __builtin_bit_cast(_Float16, uint16_t(s1));
        const h2 sa = {c0, c0}, sb = {c1, c1};
        const uint32_t wa[4] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w}, wb[4] = {r.w1.x, r.w1.y, r.w1.z, r.w1.w};
        uint4 af[NI], an[NI];
        auto rd = [&](int kk, uint4 (&f)[NI]) {
#pragma unroll
            for (int i = 0; i < NI; ++i) f[i] = *reinterpret_cast<const uint4 *>(a + swz(i * 32 + l32, kk + 4 * lh));
        };
        rd(0, af);
#pragma unroll
        for (int kk = 0; kk < GB_K / 16; ++kk) {
            if (kk + 1 < GB_K / 16) rd(kk + 1, an);
            const uint4 f0 = dequant8(wa[kk], zb0, sa), f1 = dequant8(wb[kk], zb1, sb);
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                acc[i][0] = mfma32<F16>(af[i], f0, acc[i][0]);
                acc[i][1] = mfma32<F16>(af[i], f1, acc[i][1]);
            }
#pragma unroll
            for (int i = 0; i < NI; ++i) af[i] = an[i];
        }
    };
    WR w0, w1;
    issue_a(0, bufA(0));
    issue_w(0, w0);
    issue_w(1, w1);
    wait_vm_below<NLD>();  // A(0) and W(0) here; W(1) stays in flight
    __builtin_amdgcn_s_barrier();
    auto stage = [&](int ks, int p, WR &cur) {
        issue_a(min(ks + 1, nk - 1), bufA(p ^ 1));
        compute(bufA(p), cur, ks);
        issue_w(ks + 2, cur);
        wait_vm_below<NLD>();  // everything but W(ks + 2): A(ks + 1) and W(ks + 1) arrived
        __builtin_amdgcn_s_barrier();
    };
    for (int ks = 0; ks < nk; ks += 2) {  // nk is even (K is a multiple of 128)
        stage(ks, 0, w0);
        stage(ks + 1, 1, w1);
    }
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
