// Wave-level pieces of the q4 GEMVs (dense decode rows and routed experts).
//
// A wave owns a 16-row subtile of the tiled weights and a range of the
// 128-wide K groups. Lane l serves weight row n = l % 16 and K quarter
// q = l / 16 of every group: one 16-byte load per lane per group, 1 KB of
// contiguous HBM per wave instruction, nibbles unpacked in registers
// (q4_common.cuh). The MFMA's other operand is the activations, staged in
// LDS: lane l feeds token row m = l % 16, so the 16x16 result holds every
// (token, row) pair; each lane ends with one weight row n and four token rows
// 4(l/16) + r, so the group scale and zero are one value per lane.
#pragma once

#include "q4_common.cuh"

namespace qwq4 {

// LDS row stride, in 16-byte pieces, of staged activation rows of K
// elements: K / 8, plus one piece when K / 8 is a multiple of 64. A b128 read
// pass serves 16 lanes that read 16 different rows at the same column; with a
// row stride that is a multiple of 256 bytes they would all hit the same
// banks (a 16-way conflict at 16 rows), the extra piece spreads them over 16
// bank groups. Padded rows are staged row by row (each wave instruction's
// 64 pieces stay inside one row).
__host__ __device__ inline int x_row_stride(int K) {
    const int kc = K / 8;
    return kc % 64 == 0 ? kc + 1 : kc;
}

// 16-byte pieces of M staged rows, rounded to whole waves.
__host__ __device__ inline int x_pieces(int M, int K) { return (M * x_row_stride(K) + WAVE - 1) / WAVE * WAVE; }

// Rows 0..M-1 (row m starts at row(m)) of K 16-bit elements -> LDS, row m at
// xl + m * x_row_stride(K), by direct global->LDS loads (no registers; 1 KB
// per wave instruction). Issued before the weight loads; the barrier that
// follows those waits for both, so activations (L2) and weights (HBM) are
// requested before anything waits. With padded rows the row address is
// wave-uniform (row(m) may then come from a scalar load, which does not wait
// behind vector loads in flight).
template <class RowFn>
__device__ __forceinline__ void stage_rows_issue(RowFn row, int M, int K, uint4 *xl) {
    const int kc = K / 8, wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, nw = blockDim.x / WAVE;
    if (kc % WAVE == 0) {
        const int st = kc + 1;
        for (int m = 0; m < M; ++m) {
            const uint16_t *r = row(m);
            for (int c = wave * WAVE; c < kc; c += nw * WAVE)
                __builtin_amdgcn_global_load_lds(r + (c + lane) * 8, xl + m * st + c, 16, 0, 0);
        }
    } else {
        const int total = M * kc;
        for (int base = wave * WAVE; base < total; base += nw * WAVE) {
            const int i = min(base + lane, total - 1), m = i / kc, c = i - m * kc;
            __builtin_amdgcn_global_load_lds(row(m) + c * 8, xl + base, 16, 0, 0);
        }
    }
}

// The lane index, as a value the compiler cannot see through: per-lane
// addresses derived from it inside a loop are recomputed per iteration
// instead of being hoisted out and held (2 registers each) across it.
__device__ __forceinline__ int opaque_lane() {
    int l = int(threadIdx.x) % WAVE;
    asm volatile("" : "+v"(l));
    return l;
}

// A wave's whole K range of one subtile (groups g0 .. g0 + n - 1, n <= GW),
// requested up front into registers. CH4: the range is whole 4-group chunks
// (g0 and n multiples of 4), so each chunk's scales are one 8-byte load and
// its zeros one 16-bit word; otherwise one scale and one zero load per group.
// (A compile-time choice: a runtime branch between the two puts waits between
// the loads.)
template <int GW, bool HAS_Z, bool CH4 = false>
struct WaveRange {
    // vector-memory instructions fetch() issues
    static constexpr int LOADS = CH4 ? GW / 4 * (HAS_Z ? 2 : 1) + GW : GW * (HAS_Z ? 3 : 2);
    uint4 w[GW];
    // scales and zero words as loaded: with whole chunks two fp16 scales per
    // word and one zero word per chunk (unpacked where used: holding them
    // one per group costs 1.5 registers a group)
    static constexpr int NSV = CH4 ? GW / 2 : GW, NZV = CH4 ? GW / 4 : GW;
    uint32_t sv[NSV], zv[NZV];
    __device__ __forceinline__ uint32_t scale_bits(int c) const {
        if constexpr (CH4) return (sv[c >> 1] >> ((c & 1) * 16)) & 0xffffu;
        else return sv[c];
    }
    __device__ __forceinline__ uint32_t zero_word(int c) const {
        if constexpr (CH4) return zv[c >> 2];
        else return zv[c];
    }
    int g0, n;
    __device__ __forceinline__ void fetch(const Q4Tile &t, int g0_, int n_, int lane) {
        g0 = g0_;
        n = n_;
        const int r = lane % 16;
        // scales and zeros first: group c's compute then waits only for the
        // words up to c (loads complete in order), not for the whole range
        if constexpr (CH4) {
            static_assert(GW % 4 == 0, "whole chunks");
#pragma unroll
            for (int j = 0; j < GW / 4; ++j) {
                const int gc = (g0 >> 2) + min(j, n / 4 - 1);
                const uint2 s4 = *reinterpret_cast<const uint2 *>(t.s + gc * 64 + r * 4);
                sv[2 * j] = s4.x;
                sv[2 * j + 1] = s4.y;
                if constexpr (HAS_Z) zv[j] = t.z[gc * 16 + r];
            }
        } else {
#pragma unroll
            for (int c = 0; c < GW; ++c) {
                const int g = g0 + min(c, n - 1);
                sv[c] = t.scale(g, r);
                if constexpr (HAS_Z) zv[c] = t.zero_word(g, r);
            }
        }
#pragma unroll
        for (int c = 0; c < GW; ++c) w[c] = t.word4_stream(g0 + min(c, n - 1), lane);
    }
};

// Activation pieces held in registers (up to 4 per thread). Named members
// rather than an array: an array that lives across the scheduling barriers
// below is kept in scratch memory by the compiler.
struct XRegs {
    uint4 v0, v1, v2, v3;
    __device__ __forceinline__ void set(int j, const uint4 &v) {
        if (j == 0) v0 = v;
        else if (j == 1) v1 = v;
        else if (j == 2) v2 = v;
        else v3 = v;
    }
    __device__ __forceinline__ uint4 get(int j) const { return j == 0 ? v0 : j == 1 ? v1 : j == 2 ? v2 : v3; }
};

// i / d for 0 <= i < 2^20 and 1 <= d < 2^16 without an integer division
// (a ~40-instruction sequence on the GPU): (i + 0.5) / d is at least 0.5 / d
// away from an integer, and rd = rcp(d) (within 1 ulp) leaves a relative
// error of a few 2^-24, far inside that margin.
__device__ __forceinline__ int div_small(int i, float rd) { return int((float(i) + 0.5f) * rd); }

// Activation rows through registers: thread t takes pieces t, t + nt, ...
// of the M x K/8 pieces (XPT >= M * K / 8 / blockDim.x, XPT <= 4). Issued
// before the weight loads; unlike direct-to-LDS loads (after which the
// compiler drains every load in flight before the first LDS read), the
// compiler then waits for exactly these, so each weight group is computed as
// soon as it arrives.
template <int XPT>
__device__ __forceinline__ void stage_regs_issue(const uint16_t *x, int xs, int M, int K, XRegs &xv) {
    static_assert(XPT >= 1 && XPT <= 4, "up to 4 pieces per thread");
    const int kn = K / 8, P = M * kn, nt = blockDim.x;
    const float rkn = __builtin_amdgcn_rcpf(float(kn));
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        const int i = min(int(threadIdx.x) + j * nt, P - 1), m = div_small(i, rkn), c = i - m * kn;
        xv.set(j, *reinterpret_cast<const uint4 *>(x + int64_t(m) * xs + c * 8));
    }
}

// ... then into LDS (row m at xl + m * x_row_stride(K)).
template <int XPT>
__device__ __forceinline__ void stage_regs_commit(const XRegs &xv, int M, int K, uint4 *xl) {
    const int kn = K / 8, kc = x_row_stride(K), P = M * kn, nt = blockDim.x;
    const float rkn = __builtin_amdgcn_rcpf(float(kn));
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        // unconditional store (a thread past the end rewrites the last piece
        // with the same value): a conditional one lets the compiler sink the
        // load down to it, behind the weight loads and their wait
        const int i = min(int(threadIdx.x) + j * nt, P - 1), m = div_small(i, rkn), c = i - m * kn;
        xl[m * kc + c] = xv.get(j);
    }
}

// Sum of the activations over each of a wave's groups g0 .. g0 + n - 1
// (n <= GW), per token row, for the zero-point start of the group's product
// (compute_zq): an MFMA chain of the group's four 32-element slices against
// a splat of 1 (exact products, fp32 sums), on the staged activations only,
// so it runs while the weights are in flight. sums[c][mb] is in the MFMA
// result layout (lane: rows 4 (l / 16) + r of row block mb).
// P4 (at most 4 token rows, MB == 1): four groups share one chain. Row
// 4c + m of such a tile holds token m of group gb + c (xp_of(gb): the lane's
// fragment of the tile starting at group gb), so each row goes through
// exactly the arithmetic it gets in a tile of its own, and 4 MFMAs serve what
// would take 16; the sums of rows r < MR are read out per (group, token) into
// element r of every lane (wave-uniform values).
template <typename T, int MB, int GW, bool P4, int MR, class XpFn>
__device__ __forceinline__ void group_sums(const uint4 *const (&xr)[MB], XpFn xp_of, int g0, int n,
                                           f32x4 (&sums)[GW][MB]) {
    const uint4 one = make_uint4(T::ONE, T::ONE, T::ONE, T::ONE);
    if constexpr (P4) {
        static_assert(MB == 1 && GW % 4 == 0, "packed sums: one row block, whole tiles of four groups");
#pragma unroll
        for (int tl = 0; tl < GW / 4; ++tl) {
            if (4 * tl < n) {
                const uint4 *xp = xp_of(g0 + 4 * tl);
                f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < 4; ++t) c = mfma16<T>(xp[t], one, c);
                const float cv[4] = {c[0], c[1], c[2], c[3]};
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        sums[4 * tl + g][0][r] =
                            r < MR ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv[r]), 16 * g))
                                   : 0.f;
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < GW; ++c) {
            if (c < n) {
                const int g = g0 + c;
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    sums[c][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int t = 0; t < 4; ++t) sums[c][mb] = mfma16<T>(xr[mb][g * 16 + t], one, sums[c][mb]);
                }
            }
        }
    }
}

// NS subtiles over the same groups (wr[j] fetched with equal g0 and n): per
// group, as its weights arrive, the product of the activations with the
// operands BASE + UNIT q (unpack8_q) onto a start of -(BASE + UNIT z) *
// sum(x), which leaves UNIT * sum x * (q - z) (every product exact in fp32),
// times the group scale / UNIT (a power of two) into acc. Only elements r < MR of the last row block are formed
// (rows past the batch are never read).
template <typename T, int MB, int NS, int GW, bool HAS_Z, bool CH4, int MR>
__device__ __forceinline__ void compute_zq(const WaveRange<GW, HAS_Z, CH4> (&wr)[NS], const uint4 *const (&xr)[MB],
                                           const f32x4 (&sums)[GW][MB], f32x4 (&acc)[NS][MB]) {
    const int g0 = wr[0].g0, n = wr[0].n;
#pragma unroll
    for (int c = 0; c < GW; ++c) {
        if (c < n) {
            const int g = g0 + c;
            uint4 a[MB][4];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int t = 0; t < 4; ++t) a[mb][t] = xr[mb][g * 16 + t];
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const float nz = -(T::BASE + T::UNIT * float(HAS_Z ? Q4Tile::zero_of(wr[j].zero_word(c), g) : 8u));
                const uint32_t sbits = wr[j].scale_bits(c);
                uint4 b[4];
                b[0] = unpack8_q<T>(wr[j].w[c].x);
                b[1] = unpack8_q<T>(wr[j].w[c].y);
                b[2] = unpack8_q<T>(wr[j].w[c].z);
                b[3] = unpack8_q<T>(wr[j].w[c].w);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    constexpr int R = 4;
                    const int rows = mb == MB - 1 ? MR : R;
                    f32x4 p;
#pragma unroll
                    for (int r = 0; r < R; ++r) p[r] = r < rows ? sums[c][mb][r] * nz : 0.f;
#pragma unroll
                    for (int t = 0; t < 4; ++t) p = mfma16<T>(a[mb][t], b[t], p);
                    const float sc = f16_bits_to_f32(uint16_t(sbits)) * (1.f / T::UNIT);
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        if (r < rows) acc[j][mb][r] += sc * p[r];
                }
            }
        }
    }
}

// compute_zq for one subtile and one row block with each group's sum of
// activations formed beside its product (no per-group sums held across the
// range: for kernels whose registers go to a longer weight range). Per
// 32-element slice the activation fragment feeds both MFMAs (the sum against
// a splat of 1, the product against BASE + UNIT q) and the weight word is
// unpacked just before its use, so one fragment and one unpacked word are
// live at a time; the zero-point term -(BASE + UNIT z) * sum(x) is added to
// the product at the end of the group.
template <typename T, int GW, bool HAS_Z, bool CH4>
__device__ __forceinline__ void compute_zq_inline(const WaveRange<GW, HAS_Z, CH4> &wr, const uint4 *xr, f32x4 &acc) {
    const uint4 one = make_uint4(T::ONE, T::ONE, T::ONE, T::ONE);
#pragma unroll
    for (int c = 0; c < GW; ++c) {
        if (c < wr.n) {
            const int g = wr.g0 + c;
            const uint32_t words[4] = {wr.w[c].x, wr.w[c].y, wr.w[c].z, wr.w[c].w};
            f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f}, p = sum;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint4 a = xr[g * 16 + t];
                sum = mfma16<T>(a, one, sum);
                p = mfma16<T>(a, unpack8_q<T>(words[t]), p);
            }
            const float nz = -(T::BASE + T::UNIT * float(HAS_Z ? Q4Tile::zero_of(wr.zero_word(c), g) : 8u));
            acc += (f16_bits_to_f32(uint16_t(wr.scale_bits(c))) * (1.f / T::UNIT)) * (p + sum * nz);
        }
    }
}

// The lane's fragment of a packed correction tile (token n % 4 of group
// gb + n / 4, groups past the last one clamped to it) in rows staged at xl
// with row stride kc (pieces), M rows, G groups.
__device__ __forceinline__ const uint4 *packed_fragment(const uint4 *xl, int kc, int M, int G, int gb, int lane) {
    const int n = lane % 16, q = lane / 16;
    return xl + min(n & 3, M - 1) * kc + min(gb + (n >> 2), G - 1) * 16 + q * 4;
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

// ---- the row-block tail shared by the dense GEMVs: k-split partial sums
// through LDS, then the output rows

// partial sums: one slot per wave that is not a k-part 0, double-buffered
__host__ __device__ inline int red_slots(int waves, int KS) { return waves - waves / KS; }

// LDS: staged rows, then the partial-sum slots
__host__ __device__ inline size_t dense_lds_bytes(int M, int K, int MB, int waves, int KS) {
    return size_t(x_pieces(M, K)) * 16 + size_t(2) * red_slots(waves, KS) * MB * WAVE * 16;
}

__device__ __forceinline__ void stage_x_issue(const uint16_t *__restrict__ x, int xs, int M, int K, uint4 *xl) {
    stage_rows_issue([&](int m) { return x + int64_t(m) * xs; }, M, K, xl);
}

// Accumulator elements a lane keeps: MR of the last row block, 4 of the others.
template <int MB, int MR>
constexpr int acc_elems() { return (MB - 1) * 4 + MR; }

// Rows n_lo <= row < N of the subtile are stored (n_lo > 0: a launch whose
// first rows belong to another activation slice, see launch_gemv).
template <int MB, int MR>
__device__ __forceinline__ void store_rows(const f32x4 (&acc)[MB], void *y, int ys, int y_bf16, int accumulate,
                                           int M, int N, int sub, int lane, int n_lo = 0) {
    const int q = lane / 16, n = lane % 16, row = sub * 16 + n;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < (mb == MB - 1 ? MR : 4); ++r) {
            const int m = mb * 16 + 4 * q + r;
            if (m < M && row < N && row >= n_lo) store_y(y, int64_t(m) * ys + row, acc[mb][r], y_bf16, accumulate);
        }
}

// Sums the KS partials of each subtile into the k-part 0 wave's acc, in
// k-part order. Buffer rb: one slot of acc_elems() x 64 floats (element-major,
// so a wave's write of one element is 64 consecutive floats) per wave with
// k-part != 0, red_slots of them.
template <int MB, int MR>
__device__ __forceinline__ void ksplit_sum(f32x4 (&acc)[MB], float *rb, int KS, int wave, int kp, int lane) {
    if (KS == 1) return;
    constexpr int PER = acc_elems<MB, MR>();
    const int slot0 = (wave / KS) * (KS - 1);  // the subtile's first partial slot
    if (kp != 0) {
        float *d = rb + (slot0 + kp - 1) * PER * WAVE + lane;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < (mb == MB - 1 ? MR : 4); ++r) d[(mb * 4 + r) * WAVE] = acc[mb][r];
    }
    lds_barrier();
    if (kp == 0) {
        // four partials in flight per step (KS is a runtime value), added in
        // k-part order
        for (int i0 = 1; i0 < KS; i0 += 4) {
            float part[4][PER];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float *p = rb + (slot0 + min(i0 + j, KS - 1) - 1) * PER * WAVE + lane;
#pragma unroll
                for (int e = 0; e < PER; ++e) part[j][e] = p[e * WAVE];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (i0 + j < KS) {
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                        for (int r = 0; r < (mb == MB - 1 ? MR : 4); ++r) acc[mb][r] += part[j][mb * 4 + r];
                }
        }
    }
}

}  // namespace qwq4
