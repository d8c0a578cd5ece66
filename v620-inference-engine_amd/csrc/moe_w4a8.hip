// W4A8 grouped expert GEMMs for prefill chunks: the reference's opt-in,
// lossy int8-activation path (gpu::moe_experts_w4a8,
// src/kernels/moe_w4a8.hip:13-215; selected by the engine with q8 scratch,
// src/engine/prefill.hip:333), on the gfx950 int8 MFMA.
//
// Arithmetic: activation rows are quantised per (row, 128-group) as the
// reference does, sc = max|x| / 127, q = rint(x * (1 / sc)); weights are
// widened exactly to int8 q - z; per 128-wide K group the int8 products are
// summed exactly in int32 (v_mfma_i32_32x32x32_i8), then
// acc = fma(float(I) * s_w, s_x, acc) in fp32, groups in order. The
// reference sums per 64-wide step and rescales each step with the same group
// scales; float(I) is exact either way (|I| < 2^24), so the two differ only
// in the fp32 roundings of the rescale (about 1e-7 of the result). Gate/up
// writes h = fp16(silu(g) * u); h rows are quantised the same way for the
// down projection, which writes yp in fp16.
//
// Schedule (the fp16 core's, q4_gemm_core.cuh, in int8): work is the routing
// tile list (mixed tiles of 32 to 160 slots, run as 128- and 64-slot blocks);
// a block of 8 waves takes one entry and 128 weight rows (gate/up: 64 gate
// and the same 64 up rows, interleaved by 32). K runs in stages of 128 (one
// scale group) through a double-buffered LDS; an int8 row of a stage is 128
// bytes, the fp16 core's row geometry, so its buffers, swizzle and direct
// loads serve unchanged:
//   waves 0-3 move the next stage's quantised A rows global -> LDS by direct
//     loads, and the rows' activation scales of that group;
//   waves 4-7 (two threads per weight row) load the q4 entries two stages
//     ahead and widen them into LDS between the MFMAs.
// Each wave holds MT 32x32 tiles (128-slot blocks: 2, 64: 1; a 256-slot
// list entry runs as two 128-slot blocks): per stage 4 int8 MFMAs per tile
// into int32, then the rescale (three VALU operations per accumulator).
#include <type_traits>

#include "q4_gemm_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int W8_TILE_M = -32;  // the routing's mixed tiles of 32 to 160 slots (the grouped path's list)

int moe_w4a8_tile_m() { return W8_TILE_M; }

// ------------------------------------------------------------ quantiser
// One wave per (row, group of 128): two elements per lane.
// One (row, 128-group) per 16-lane row of a wave (four per wave): lane i of
// the row holds elements 8 i .. 8 i + 7 (one 16-byte load), the group's
// amax is a maximum over the 16 lanes, and each element is quantised as
// rint(x * (1 / sc)) with sc = amax / 127 (1 for an all-zero group).
template <bool F16>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t *__restrict__ x, int64_t ldx, int rows,
                                                         int K, int8_t *__restrict__ q, float *__restrict__ scale) {
    const int G = K / QGROUP, li = threadIdx.x % 16;
    const int64_t item = int64_t(blockIdx.x) * (blockDim.x / 16) + threadIdx.x / 16;
    const bool live = item < int64_t(rows) * G;
    const int64_t it = live ? item : int64_t(rows) * G - 1;  // (every lane takes part in the shuffles)
    const int64_t r = it / G;
    const int g = int(it % G);
    const uint4 u = *reinterpret_cast<const uint4 *>(x + r * ldx + g * QGROUP + 8 * li);
    auto cvt = [](uint16_t b) { return F16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b); };
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[2 * j] = cvt(uint16_t(w[j]));
        v[2 * j + 1] = cvt(uint16_t(w[j] >> 16));
    }
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));  // within the 16-lane row
    const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
    uint32_t pk[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) pk[j / 4] |= uint32_t(int(__builtin_rintf(v[j] * inv)) & 0xff) << (8 * (j % 4));
    if (live) {
        *reinterpret_cast<uint2 *>(q + r * K + g * QGROUP + 8 * li) = make_uint2(pk[0], pk[1]);
        if (li == 0) scale[r * G + g] = sc;
    }
}

// The same quantisation, one (row, group) per wave and two elements per lane:
// for rows whose stride or base do not allow 16-byte loads.
template <bool F16>
__global__ __launch_bounds__(256) void quant_rows_pair_kernel(const uint16_t *__restrict__ x, int64_t ldx, int rows,
                                                              int K, int8_t *__restrict__ q, float *__restrict__ scale) {
    const int G = K / QGROUP, lane = threadIdx.x % WAVE;
    const int64_t item = int64_t(blockIdx.x) * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (item >= int64_t(rows) * G) return;
    const int64_t r = item / G;
    const int g = int(item % G);
    const uint32_t pair = *reinterpret_cast<const uint32_t *>(x + r * ldx + g * QGROUP + 2 * lane);
    auto cvt = [](uint16_t b) { return F16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b); };
    const float v0 = cvt(uint16_t(pair)), v1 = cvt(uint16_t(pair >> 16));
    float mx = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const float sc = mx > 0.f ? mx / 127.f : 1.f, inv = 1.f / sc;
    const int q0 = int(__builtin_rintf(v0 * inv)), q1 = int(__builtin_rintf(v1 * inv));
    *reinterpret_cast<uint16_t *>(q + r * K + g * QGROUP + 2 * lane) = uint16_t((q0 & 0xff) | ((q1 & 0xff) << 8));
    if (lane == 0) scale[r * G + g] = sc;
}

void launch_quant_rows(const uint16_t *x, int x_f16, int64_t ldx, int rows, int K, int8_t *q, float *scale,
                       hipStream_t s) {
    const int64_t items = int64_t(rows) * (K / QGROUP);
    if (ldx % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0) {
        const unsigned blocks = unsigned((items + 15) / 16);
        if (x_f16) quant_rows_kernel<true><<<blocks, 256, 0, s>>>(x, ldx, rows, K, q, scale);
        else quant_rows_kernel<false><<<blocks, 256, 0, s>>>(x, ldx, rows, K, q, scale);
    } else {
        const unsigned blocks = unsigned((items + 3) / 4);
        if (x_f16) quant_rows_pair_kernel<true><<<blocks, 256, 0, s>>>(x, ldx, rows, K, q, scale);
        else quant_rows_pair_kernel<false><<<blocks, 256, 0, s>>>(x, ldx, rows, K, q, scale);
    }
}

// ------------------------------------------------------------ GEMM pieces
// A word of a tiled q4 entry (elements j < 4 in the low nibbles of bytes j,
// j + 4 in the high nibbles) -> eight int8 q - z in K order. Bytes carry 128
// while subtracting (128 + q - z >= 113: no borrow), then lose it.
__device__ __forceinline__ uint2 widen8(uint32_t w, uint32_t zz) {
    const uint32_t lo = (((w & 0x0f0f0f0fu) | 0x80808080u) - zz) ^ 0x80808080u;
    const uint32_t hi = ((((w >> 4) & 0x0f0f0f0fu) | 0x80808080u) - zz) ^ 0x80808080u;
    return make_uint2(lo, hi);
}

__device__ __forceinline__ i32x16 mfma_i8(const uint4 &a, const uint4 &b, const i32x16 &c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                                 0);
}

static __device__ __forceinline__ uint16_t f16_sat(float v) {
    return __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(v));
}


constexpr int W8_BN = 128;  // weight rows per block
constexpr int W8_K = 128;   // K per stage (one scale group)

// activation scales of a stage's tile rows (waves 0-3 fill them), two stages
static __shared__ __align__(16) float w8_lsx[2][256];

// Block shapes: BM = 128 or 64 slot rows (list entries of 96 and 32 slots
// run at the next height, 160 as 128 + 64); waves 2 (slots) x 4 (weight rows), each MT
// 32-row slot tiles by one 32-row weight tile.
template <int BM>
struct W8Shape {
    static_assert(BM == 128 || BM == 64, "128 or 64 slot rows");
    static constexpr int MT = BM / 64;  // 32-row tiles per wave along the slots
    static constexpr int NT = 1;        // 32-row tiles per wave along the weight rows
    static constexpr int WN = 4;        // waves along the weight rows
};

// acc[mi][nj] += A (BM slot rows, quantised; ap[j]: row a_load_row(j); sxr:
// the scale row of tile row tid, for tid < BM) x W^T (128 weight rows; this
// B-role thread's row b, its K half bh; scale rows sw_row[nj] of the lane's
// columns), K columns (a multiple of 128).
// (USE tags the caller, 0 gate/up, 1 down: each call site instantiates its own
// specialization; the host compilation pass rejects a second call site of a
// shared one)
template <int BM, bool HAS_Z, int USE, class ApT, class SwT, class AccT>
__device__ __forceinline__ void w8_tile(const ApT &ap, const float *sxr, const BRow &b, const SwT &sw_row, int K,
                                        AccT &acc) {
    using S = W8Shape<BM>;
    constexpr int MT = S::MT, NT = S::NT;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
    const int nk = K / W8_K, G = K / QGROUP;
    auto bufA = [&](int i) { return i ? lds_a1 : lds_a0; };
    auto bufB = [&](int i) { return i ? lds_b1 : lds_b0; };
    const int mi0 = (wave / S::WN) * MT, nj0 = (wave % S::WN) * NT, l32 = lane % 32, lh = lane / 32;
    i32x16 ip[MT][NT];

    // MFMAs of one stage (4 slabs of 32 K) and the group's rescale; extra(q)
    // runs after slab q (the B role's widening)
    auto compute = [&](const unsigned char *a, const unsigned char *bb, const float *lsx, int g, auto extra) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j) ip[i][j] = i32x16{};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 af[MT], bf[NT];
#pragma unroll
            for (int i = 0; i < MT; ++i) af[i] = *reinterpret_cast<const uint4 *>(a + swz((mi0 + i) * 32 + l32, 2 * q + lh));
#pragma unroll
            for (int j = 0; j < NT; ++j) bf[j] = *reinterpret_cast<const uint4 *>(bb + swz((nj0 + j) * 32 + l32, 2 * q + lh));
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j) ip[i][j] = mfma_i8(af[i], bf[j], ip[i][j]);
            extra(q);
        }
        float sw[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) sw[j] = f16_bits_to_f32(sw_row[j][(g >> 2) * 64 + (g & 3)]);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            float sx[16];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float4 v = *reinterpret_cast<const float4 *>(&lsx[(mi0 + i) * 32 + 8 * u + 4 * lh]);
                sx[4 * u] = v.x;
                sx[4 * u + 1] = v.y;
                sx[4 * u + 2] = v.z;
                sx[4 * u + 3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(float(ip[i][j][r]) * sw[j], sx[r], acc[i][j][r]);
        }
    };

    if (wave < G_ROLE) {
        // A role: the quantised rows of stage ks + 1 by direct loads, and the
        // group's activation scales of the tile rows
        auto issue_a = [&](int ks, unsigned char *dst) {
            const int k0 = ks * W8_K, wa = wave % G_ROLE;
#pragma unroll
            for (int j = 0; j < BM / 32; ++j) {
                const int rb = (j * G_ROLE + wa) * 8;
                const int r = rb + lane / 8, c = (lane % 8) ^ swz_x(r);
                __builtin_amdgcn_global_load_lds(ap[j] + k0 + c * 16, dst + rb * 128, 16, 0, 0);
            }
        };
        issue_a(0, bufA(0));
        if (tid < BM) w8_lsx[0][tid] = sxr[0];
        __syncthreads();
        auto stage = [&](int ks, int p) {
            const int kn = min(ks + 1, nk - 1);
            issue_a(kn, bufA(p ^ 1));
            const float sv = sxr[kn];
            compute(bufA(p), bufB(p), w8_lsx[p], ks, [](int) {});
            if (tid < BM) w8_lsx[p ^ 1][tid] = sv;
            lds_barrier();
        };
        int ks = 0;
        for (; ks + 1 < nk; ks += 2) {
            stage(ks, 0);
            stage(ks + 1, 1);
        }
        if (ks < nk) stage(ks, 0);
    } else {
        // weight role: row (tid - 256) / 2, K half bh of each stage
        const int br = (tid - G_THREADS / 2) / 2, bh = tid % 2;
        (void)G;
        struct BRaw {
            uint4 w0, w1;
            uint32_t z;
        };
        auto issue_b = [&](int ks, BRaw &r) {
            ks = min(ks, nk - 1);  // past the end: a valid, unused load keeps the code branch-free
            r.w0 = b.w[ks * 64 + (2 * bh) * 16];
            r.w1 = b.w[ks * 64 + (2 * bh + 1) * 16];
            if constexpr (HAS_Z) r.z = b.z[(ks >> 2) * 8];
        };
        // entry e (32 K) of the raw weights -> int8 chunks 4 bh + 2 e, + 1
        auto commit_b = [&](int ks, const BRaw &r, unsigned char *dst, int e) {
            uint32_t zw = HAS_Z ? r.z : 0u;
            asm volatile("" : "+v"(zw));
            const uint32_t zz = HAS_Z ? ((zw >> (b.zs + 4 * (ks & 3))) & 0xfu) * 0x01010101u : 0x08080808u;
            const uint4 w = e ? r.w1 : r.w0;
            const uint2 x0 = widen8(w.x, zz), x1 = widen8(w.y, zz), x2 = widen8(w.z, zz), x3 = widen8(w.w, zz);
            *reinterpret_cast<uint4 *>(dst + swz(br, 4 * bh + 2 * e)) = make_uint4(x0.x, x0.y, x1.x, x1.y);
            *reinterpret_cast<uint4 *>(dst + swz(br, 4 * bh + 2 * e + 1)) = make_uint4(x2.x, x2.y, x3.x, x3.y);
        };
        BRaw rs[2];
        issue_b(0, rs[0]);
        commit_b(0, rs[0], bufB(0), 0);
        commit_b(0, rs[0], bufB(0), 1);
        issue_b(1, rs[1]);
        __syncthreads();
        auto stage = [&](int ks, BRaw &mine, const BRaw &next, int p) {
            const bool more = ks + 1 < nk;
            issue_b(ks + 2, mine);
            compute(bufA(p), bufB(p), w8_lsx[p], ks, [&](int q) {
                if (more && (q == 1 || q == 3)) commit_b(ks + 1, next, bufB(p ^ 1), q / 2);
            });
            lds_barrier();
        };
        int ks = 0;
        for (; ks + 1 < nk; ks += 2) {
            stage(ks, rs[0], rs[1], 0);
            stage(ks + 1, rs[1], rs[0], 1);
        }
        if (ks < nk) stage(ks, rs[0], rs[1], 0);
    }
}

// The block's slots: list entry blockIdx.y (expert, first slot); real slots
// M of a block of `rows` (128 for entries of 96 to 160 slots, 64 for 32 and
// 64; a 160-slot entry's last 32 in a second 64-slot pass of the same block),
// all in list order.
struct W8Entry {
    int e, base, M, rows;
    int rest;  // slots past the first 128 of a 160-slot entry, run as a second 64-slot pass
};
static __device__ __forceinline__ bool w8_entry(const W8Args &a, W8Entry &t) {
    const int tile = blockIdx.y;
    if (tile >= *a.n_tiles) return false;
    t.e = a.tile_e[tile];
    const int m0 = a.tile_m0[tile], rem = a.offsets[t.e + 1] - a.offsets[t.e] - m0;
    const int rows = tile_rows(rem, W8_TILE_M);
    const int real = min(rows, rem);
    t.rows = rows > 64 ? 128 : 64;
    t.base = a.offsets[t.e] + m0;
    t.M = min(t.rows, real);
    t.rest = real - t.M;
    return true;
}

// gate/up tile: block rows r of the 128: 32-row group r / 32 is gate when
// even, up when odd, for h columns j0 + 32 (r / 64) + r % 32.
template <int BM, bool HAS_Z>
__device__ __forceinline__ void gate_up_w8(const W8Args &a, const W8Entry &t) {
    using S = W8Shape<BM>;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, l32 = lane % 32, lh = lane / 32;
    const int j0 = blockIdx.x * 64, G = a.H / QGROUP;
    const int64_t eF = int64_t(t.e) * a.F;
    auto brow = [&](int r) {
        const int64_t row = eF + min(j0 + (r / 64) * 32 + r % 32, a.F - 1);
        return ((r / 32) & 1) ? BRow(a.uw, a.us, a.uz, row, G) : BRow(a.gw, a.gs, a.gz, row, G);
    };
    const int32_t *pt = a.pair_tok + t.base;
    const int8_t *ap[BM / 32];
#pragma unroll
    for (int j = 0; j < BM / 32; ++j) ap[j] = a.qx + int64_t(pt[min(a_load_row(j), t.M - 1)]) * a.H;
    const BRow b = brow(max(0, min((tid - G_THREADS / 2) / 2, W8_BN - 1)));
    const int mi0 = (wave / S::WN) * S::MT, nj0 = (wave % S::WN) * S::NT;
    const uint16_t *swr[S::NT];
#pragma unroll
    for (int j = 0; j < S::NT; ++j) swr[j] = brow((nj0 + j) * 32 + l32).s;
    // the scale row a thread t < BM stages: its slot's token
    const float *sxp = a.sx + int64_t(pt[min(tid, t.M - 1)]) * G;
    f32x16 acc[S::MT][S::NT];
#pragma unroll
    for (int i = 0; i < S::MT; ++i)
#pragma unroll
        for (int j = 0; j < S::NT; ++j) acc[i][j] = f32x16{};
    w8_tile<BM, HAS_Z, 0>(ap, sxp, b, swr, a.H, acc);
    // h = fp16(silu(g) * u): tile nj holds gate (nj even) or up (odd) of
    // columns j0 + 32 (nj / 2) + l32
    auto put = [&](int i, int col, const f32x16 &g, const f32x16 &u) {
        const int j = j0 + col + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = (mi0 + i) * 32 + 8 * (r / 4) + 4 * lh + r % 4;
            if (m < t.M && j < a.F) a.h[int64_t(t.base + m) * a.F + j] = f16_sat(silu_ref(g[r]) * u[r]);
        }
    };
    {
        // gate and up of a column group sit in waves wn and wn + 1: the up
        // wave hands its accumulators over through LDS (free after the loop)
        float *xb = reinterpret_cast<float *>(lds_a0) + (wave / 2) * (S::MT * 16 * WAVE);
        if (nj0 & 1) {
#pragma unroll
            for (int i = 0; i < S::MT; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) xb[(i * 16 + r) * WAVE + lane] = acc[i][0][r];
        }
        __syncthreads();
        if (!(nj0 & 1)) {
#pragma unroll
            for (int i = 0; i < S::MT; ++i) {
                f32x16 u;
#pragma unroll
                for (int r = 0; r < 16; ++r) u[r] = xb[(i * 16 + r) * WAVE + lane];
                put(i, (nj0 / 2) * 32, acc[i][0], u);
            }
        }
    }
}

template <bool HAS_Z>
__global__ __launch_bounds__(G_THREADS) void moe_gate_up_w4a8_kernel(W8Args a) {
    W8Entry t;
    if (!w8_entry(a, t)) return;
    if (t.rows == 128) gate_up_w8<128, HAS_Z>(a, t);
    else gate_up_w8<64, HAS_Z>(a, t);
    if (t.rest > 0) {
        __syncthreads();  // the first pass's LDS is consumed
        gate_up_w8<64, HAS_Z>(a, W8Entry{t.e, t.base + 128, t.rest, 64, 0});
    }
}

// down tile: block rows are down rows n0 .. n0 + 127 of expert e
template <int BM, bool HAS_Z>
__device__ __forceinline__ void down_w8(const W8Args &a, const W8Entry &t) {
    using S = W8Shape<BM>;
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, l32 = lane % 32, lh = lane / 32;
    const int n0 = blockIdx.x * W8_BN, G = a.F / QGROUP;
    const int64_t eH = int64_t(t.e) * a.H;
    auto brow = [&](int r) { return BRow(a.dw, a.ds, a.dz, eH + min(n0 + r, a.H - 1), G); };
    const int8_t *ap[BM / 32];
#pragma unroll
    for (int j = 0; j < BM / 32; ++j) ap[j] = a.qh + int64_t(t.base + min(a_load_row(j), t.M - 1)) * a.F;
    const BRow b = brow(max(0, min((tid - G_THREADS / 2) / 2, W8_BN - 1)));
    const int mi0 = (wave / S::WN) * S::MT, nj0 = (wave % S::WN) * S::NT;
    const uint16_t *swr[S::NT];
#pragma unroll
    for (int j = 0; j < S::NT; ++j) swr[j] = brow((nj0 + j) * 32 + l32).s;
    const float *sxp = a.sh + int64_t(t.base + min(tid, t.M - 1)) * G;  // the slot of tile row tid
    f32x16 acc[S::MT][S::NT];
#pragma unroll
    for (int i = 0; i < S::MT; ++i)
#pragma unroll
        for (int j = 0; j < S::NT; ++j) acc[i][j] = f32x16{};
    w8_tile<BM, HAS_Z, 1>(ap, sxp, b, swr, a.F, acc);
#pragma unroll
    for (int i = 0; i < S::MT; ++i)
#pragma unroll
        for (int j = 0; j < S::NT; ++j) {
            const int n = n0 + (nj0 + j) * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = (mi0 + i) * 32 + 8 * (r / 4) + 4 * lh + r % 4;
                if (m < t.M && n < a.H) a.yp[int64_t(t.base + m) * a.H + n] = f16_sat(acc[i][j][r]);
            }
        }
}

template <bool HAS_Z>
__global__ __launch_bounds__(G_THREADS) void moe_down_w4a8_kernel(W8Args a) {
    W8Entry t;
    if (!w8_entry(a, t)) return;
    if (t.rows == 128) down_w8<128, HAS_Z>(a, t);
    else down_w8<64, HAS_Z>(a, t);
    if (t.rest > 0) {
        __syncthreads();  // the first pass's LDS is consumed
        down_w8<64, HAS_Z>(a, W8Entry{t.e, t.base + 128, t.rest, 64, 0});
    }
}

size_t moe_w4a8_workspace_bytes(int T, int topk, int H, int F) {
    auto up = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t P = size_t(T) * topk;
    return up(size_t(T) * H) + up(size_t(T) * (H / QGROUP) * 4) + up(P * F) + up(P * (F / QGROUP) * 4);
}

// x quantised, gate/up, h quantised, down: four launches on one stream.
void launch_moe_w4a8(W8Args a, const uint16_t *x, int x_f16, int T, int topk, hipStream_t s) {
    auto up = [](size_t b) { return (b + 255) & ~size_t(255); };
    unsigned char *w = static_cast<unsigned char *>(a.ws);
    const size_t P = size_t(T) * topk;
    a.qx = reinterpret_cast<int8_t *>(w);
    w += up(size_t(T) * a.H);
    a.sx = reinterpret_cast<float *>(w);
    w += up(size_t(T) * (a.H / QGROUP) * 4);
    a.qh = reinterpret_cast<int8_t *>(w);
    w += up(P * a.F);
    a.sh = reinterpret_cast<float *>(w);
    launch_quant_rows(x, x_f16, a.H, T, a.H, const_cast<int8_t *>(a.qx), const_cast<float *>(a.sx), s);
    const int max_tiles = int(P / -W8_TILE_M) + a.E;
    if (a.gz) moe_gate_up_w4a8_kernel<true><<<dim3(unsigned(a.F / 64), unsigned(max_tiles)), G_THREADS, 0, s>>>(a);
    else moe_gate_up_w4a8_kernel<false><<<dim3(unsigned(a.F / 64), unsigned(max_tiles)), G_THREADS, 0, s>>>(a);
    launch_quant_rows(a.h, 1, a.F, int(P), a.F, const_cast<int8_t *>(a.qh), const_cast<float *>(a.sh), s);
    if (a.dz) moe_down_w4a8_kernel<true><<<dim3(unsigned(a.H / W8_BN), unsigned(max_tiles)), G_THREADS, 0, s>>>(a);
    else moe_down_w4a8_kernel<false><<<dim3(unsigned(a.H / W8_BN), unsigned(max_tiles)), G_THREADS, 0, s>>>(a);
}

}  // namespace qwq4
