// W4A8 grouped expert GEMMs for prefill chunks: the reference's opt-in,
// lossy int8-activation path (gpu::moe_experts_w4a8,
// src/kernels/moe_w4a8.hip:13-215; selected by the engine with q8 scratch,
// src/engine/prefill.hip:333), on the gfx950 int8 MFMA.
//
// Arithmetic (as the reference's): activation rows are quantised per (row,
// 128-group), sc = max|x| / 127, q = rint(x * (1 / sc)); weights are widened
// exactly to int8 q - z; per 64-wide K step the int8 products are summed
// exactly in int32, then acc = fma(float(I) * s_w, s_x, acc) in fp32, steps
// in order. Gate/up writes h = fp16(silu(g) * u); h rows are quantised the
// same way for the down projection, which writes yp in fp16.
//
// Schedule. Work is the routing tile list with tiles of 64 slots
// (qw_moe_route with tile_m = 64). A block (4 waves) takes one list entry and
// 64 h columns (gate/up: 64 gate and the same 64 up rows) or 128 down rows.
// K runs in 64-wide steps through a double-buffered LDS: the next step's
// activation pieces and q4 weight entries are loaded into registers before
// the current step's MFMAs and written to LDS after them (weights widened to
// int8 on the way). Each wave holds two 32x32 tiles: one v_mfma_i32_32x32x32_i8
// pair per tile and step, then the step's rescale (three VALU operations per
// accumulator: the VALU, not the matrix core, bounds this kernel).
#include "q4_gemm_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int W8_TILE = 64;  // slots per tile (the routing's tile_m)
constexpr int W8_STEP = 64;  // K per step

int moe_w4a8_tile_m() { return W8_TILE; }

// ------------------------------------------------------------ quantiser
// One wave per (row, group of 128): two elements per lane.
template <bool F16>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t *__restrict__ x, int64_t ldx, int rows,
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
    const unsigned blocks = unsigned((items + 3) / 4);
    if (x_f16) quant_rows_kernel<true><<<blocks, 256, 0, s>>>(x, ldx, rows, K, q, scale);
    else quant_rows_kernel<false><<<blocks, 256, 0, s>>>(x, ldx, rows, K, q, scale);
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

// LDS tile rows of 64 int8 (4 chunks of 16 bytes); chunk c of row r sits at
// c ^ ((r >> 1) & 3): the 8 lanes of a b128 read pass (8 consecutive rows,
// one chunk) then cover all 8 16-byte bank groups of a 128-byte line.
__device__ __forceinline__ int w8_off(int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 3)) << 4); }

__device__ __forceinline__ i32x16 mfma_i8(const uint4 &a, const uint4 &b, const i32x16 &c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                                 0);
}

// Weight rows of a block: 128 rows of the tiled format, one thread pair per
// row (thread t loads row t / 2: the entry of quarter 2 (s % 2) + t % 2 of
// step s, 32 K).
struct W8B {
    BRow row;
    int half;
    __device__ __forceinline__ uint4 load(int s) const {
        const int g = s / 2;
        return row.w[g * 64 + ((s % 2) * 2 + half) * 16];
    }
    __device__ __forceinline__ uint32_t zz(int s) const {  // the step's zero in every byte
        if (!row.z) return 0x08080808u;
        const int g = s / 2;
        return ((row.z[(g >> 2) * 8] >> (row.zs + 4 * (g & 3))) & 0xfu) * 0x01010101u;
    }
};

// The main loop of one 64-slot tile by 128 weight rows. Slot i of the tile
// reads quantised row arow(i) (i < M); tile row r is weight row brow(r) (a
// BRow). Wave (wm, wn) forms two 32x32 tiles t = 0, 1: slots 32 wm .. and
// tile rows tb[t] .. (lane column tb[t] + lane % 32), rescaled per step with
// the scale of its column and those of its 16 slots (staged in LDS per
// group). acc[t] ends in the 32x32 MFMA result layout.
template <class ARowFn, class BRowFn>
__device__ __forceinline__ void w4a8_tile(const int8_t *q8, const float *sx, int K, int M, ARowFn arow, BRowFn brow,
                                          const int (&tb)[2], f32x16 (&acc)[2]) {
    __shared__ __align__(16) int8_t la[2][W8_TILE * W8_STEP], lb[2][128 * W8_STEP];
    __shared__ __align__(16) float lsx[W8_TILE];
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, l32 = lane % 32, lh = lane / 32;
    const int wm = wave / 2, G = K / QGROUP, steps = K / W8_STEP;
    // this thread's activation piece (slot row tid / 4, chunk tid % 4), the
    // slot whose scales it stages (tid < 64), and its weight row
    const int ar = tid / 4, ac = tid % 4, br = tid / 2, bh = tid % 2;
    const int8_t *asrc = q8 + int64_t(arow(min(ar, M - 1))) * K + ac * 16;
    const float *sxr = sx + int64_t(arow(min(tid % W8_TILE, M - 1))) * G;
    const W8B wb{brow(br), bh};
    const BRow sc0 = brow(tb[0] + l32), sc1 = brow(tb[1] + l32);
    uint4 an, bn;
    uint32_t zn;
    auto load = [&](int s) {
        an = *reinterpret_cast<const uint4 *>(asrc + s * W8_STEP);
        bn = wb.load(s);
        zn = wb.zz(s);
    };
    auto commit = [&](int p) {
        *reinterpret_cast<uint4 *>(&la[p][w8_off(ar, ac)]) = an;
        const uint2 x0 = widen8(bn.x, zn), x1 = widen8(bn.y, zn), x2 = widen8(bn.z, zn), x3 = widen8(bn.w, zn);
        *reinterpret_cast<uint4 *>(&lb[p][w8_off(br, 2 * bh)]) = make_uint4(x0.x, x0.y, x1.x, x1.y);
        *reinterpret_cast<uint4 *>(&lb[p][w8_off(br, 2 * bh + 1)]) = make_uint4(x2.x, x2.y, x3.x, x3.y);
    };
    acc[0] = f32x16{};
    acc[1] = f32x16{};
    load(0);
    commit(0);
    float sxv[16];
    for (int s = 0; s < steps; ++s) {
        const int p = s & 1, g = s / 2;
        if (s % 2 == 0 && tid < W8_TILE) lsx[tid] = sxr[g];
        if (s + 1 < steps) load(s + 1);
        __syncthreads();  // step s's tiles and the group's scales are in LDS
        if (s % 2 == 0) {
            // the lane's 16 slots 32 wm + 8 (r / 4) + 4 lh + r % 4
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = *reinterpret_cast<const float4 *>(&lsx[32 * wm + 8 * j + 4 * lh]);
                sxv[4 * j] = v.x;
                sxv[4 * j + 1] = v.y;
                sxv[4 * j + 2] = v.z;
                sxv[4 * j + 3] = v.w;
            }
        }
        const float sw[2] = {f16_bits_to_f32(sc0.s[(g >> 2) * 64 + (g & 3)]),
                             f16_bits_to_f32(sc1.s[(g >> 2) * 64 + (g & 3)])};
        uint4 af[2], bf[2][2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {  // two 32-K halves of the step; lane half lh takes 16 K of each
            af[k] = *reinterpret_cast<const uint4 *>(&la[p][w8_off(32 * wm + l32, 2 * k + lh)]);
#pragma unroll
            for (int t = 0; t < 2; ++t)
                bf[t][k] = *reinterpret_cast<const uint4 *>(&lb[p][w8_off(tb[t] + l32, 2 * k + lh)]);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            i32x16 ip = i32x16{};
            ip = mfma_i8(af[0], bf[t][0], ip);
            ip = mfma_i8(af[1], bf[t][1], ip);
            // acc += float(I) * s_w * s_x, the last multiply-add fused as the
            // reference's compiler contracts it (moe_w4a8.hip:110-116)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(float(ip[r]) * sw[t], sxv[r], acc[t][r]);
        }
        __syncthreads();  // every read of buffer p is done before it is refilled
        if (s + 1 < steps) commit(p ^ 1);
    }
}

static __device__ __forceinline__ uint16_t f16_sat(float v) {
    return __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(v));
}

// the reference's silu: x * (1 / (1 + exp(-x))) (src/kernels/common.cuh:94-99)
static __device__ __forceinline__ float silu_ref(float g) { return g * (1.f / (1.f + __expf(-g))); }

// The 64-slot tile of list entry blockIdx.y: expert, first slot, real slots.
struct W8Entry {
    int e, base, M;
};
static __device__ __forceinline__ bool w8_entry(const int32_t *offsets, const int32_t *tile_e,
                                                const int32_t *tile_m0, const int32_t *n_tiles, W8Entry &t) {
    const int tile = blockIdx.y;
    if (tile >= *n_tiles) return false;
    t.e = tile_e[tile];
    const int m0 = tile_m0[tile];
    t.base = offsets[t.e] + m0;
    t.M = min(W8_TILE, offsets[t.e + 1] - offsets[t.e] - m0);
    return true;
}

// gate/up: tile rows 0-63 are gate rows j0 .., rows 64-127 the same up rows;
// wave (wm, wn) holds gate (t = 0) and up (t = 1) of columns j0 + 32 wn ..;
// h = fp16(silu(g) * u) (finite values beyond the fp16 range saturate).
__global__ __launch_bounds__(256) void moe_gate_up_w4a8_kernel(W8Args a) {
    W8Entry t;
    if (!w8_entry(a.offsets, a.tile_e, a.tile_m0, a.n_tiles, t)) return;
    const int j0 = blockIdx.x * 64, wave = threadIdx.x / WAVE, wm = wave / 2, wn = wave % 2;
    const int lane = threadIdx.x % WAVE, l32 = lane % 32, lh = lane / 32, G = a.H / QGROUP;
    const int32_t *pt = a.pair_tok + t.base;
    const int64_t eF = int64_t(t.e) * a.F;
    const int tb[2] = {32 * wn, 64 + 32 * wn};
    f32x16 acc[2];
    w4a8_tile(
        a.qx, a.sx, a.H, t.M, [&](int i) { return pt[i]; },
        [&](int r) {
            const int64_t row = eF + min(j0 + r % 64, a.F - 1);
            return r < 64 ? BRow(a.gw, a.gs, a.gz, row, G) : BRow(a.uw, a.us, a.uz, row, G);
        },
        tb, acc);
    const int j = j0 + 32 * wn + l32;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int m = 32 * wm + 8 * (q / 4) + 4 * lh + q % 4;
        if (m < t.M && j < a.F) a.h[int64_t(t.base + m) * a.F + j] = f16_sat(silu_ref(acc[0][q]) * acc[1][q]);
    }
}

// down: tile rows are down rows n0 .. n0 + 127 of expert e; wave (wm, wn)
// holds rows n0 + 64 wn + 32 t ..; yp = fp16 (saturating).
__global__ __launch_bounds__(256) void moe_down_w4a8_kernel(W8Args a) {
    W8Entry t;
    if (!w8_entry(a.offsets, a.tile_e, a.tile_m0, a.n_tiles, t)) return;
    const int n0 = blockIdx.x * 128, wave = threadIdx.x / WAVE, wm = wave / 2, wn = wave % 2;
    const int lane = threadIdx.x % WAVE, l32 = lane % 32, lh = lane / 32, G = a.F / QGROUP;
    const int64_t eH = int64_t(t.e) * a.H;
    const int tb[2] = {64 * wn, 64 * wn + 32};
    f32x16 acc[2];
    const int base = t.base;
    w4a8_tile(
        a.qh, a.sh, a.F, t.M, [&](int i) { return base + i; },
        [&](int r) { return BRow(a.dw, a.ds, a.dz, eH + min(n0 + r, a.H - 1), G); }, tb, acc);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int n = n0 + tb[tt] + l32;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int m = 32 * wm + 8 * (q / 4) + 4 * lh + q % 4;
            if (m < t.M && n < a.H) a.yp[int64_t(base + m) * a.H + n] = f16_sat(acc[tt][q]);
        }
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
    const int max_tiles = int(P / W8_TILE) + a.E;
    moe_gate_up_w4a8_kernel<<<dim3(unsigned(a.F / 64), unsigned(max_tiles)), 256, 0, s>>>(a);
    launch_quant_rows(a.h, 1, a.F, int(P), a.F, const_cast<int8_t *>(a.qh), const_cast<float *>(a.sh), s);
    moe_down_w4a8_kernel<<<dim3(unsigned(a.H / 128), unsigned(max_tiles)), 256, 0, s>>>(a);
}

}  // namespace qwq4
