// MoE routing, gather indices and the weighted combine.
//
// Reference: the math of ref::Model::moe (src/ref/ref_model.cpp:412-431) and
// the deterministic slot order of gpu::moe_route_B
// (src/kernels/moe_route.hip:65-165), for any batch: decode rows and 4096-token
// prefill chunks use the same code (the reference's prefill scatter,
// moe_route.hip:28-58, fills slots with atomics and is nondeterministic; this
// one is not).
//
//   p_e      = expf(l_e - max l)                            per token
//   top k    by (p descending, expert index ascending)
//   w_i      = float(double(p_i) / sum_{j<k} double(p_j))    sum in selection order
//   slots    experts ascending; within an expert, tokens ascending
//
// expf is the C library's: the reference calls std::exp on a float
// (ref_model.cpp:418), i.e. glibc's expf, which is not correctly rounded (it
// returns the other neighbour of the exact value for ~74,000 of the floats in
// [-4, 0)). Where two logits' exponentials are equal under one rounding and
// not under the other, the (p, index) order picks different experts, so the
// device evaluates glibc's algorithm itself (expf_glibc below) and matches the
// CPU path bit for bit: selection, order and weights.

#include <type_traits>

#include "q4_common.cuh"
#include "route_core.cuh"
#include "w16_core.cuh"

#include "q4_kernels.hpp"

namespace qwq4 {

template <int PER>
__global__ __launch_bounds__(256) void route_topk_kernel(const float *__restrict__ logits, int T, int E, int k,
                                                         int32_t *__restrict__ top_e, float *__restrict__ top_w) {
    const int t = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (t >= T) return;
    ExpfGlibc ex;
    ex.load(lane);
    const float *l = logits + int64_t(t) * E;
    topk_wave<PER>(ex, [&](int i) { return l[i]; }, E, k, lane, top_e + int64_t(t) * k, top_w + int64_t(t) * k);
}

// ---- slots of a larger batch: one block per 64-token chunk
// Every block counts the selections of all tokens (totals) and of the tokens
// before its chunk (prefix) from top_e with LDS atomics, scans the totals over
// the experts (offsets), and gives each of its chunk's pairs the slot
// offsets[e] + prefix[e] + (its token's rank among the chunk's tokens of e,
// a popcount below its bit in the expert's 64-bit chunk mask). Block 0 also
// writes counts, offsets, the active list and the tile list. No block reads
// what another writes, so one launch needs no hand-off between blocks.
constexpr int SLOT_CHUNK = 64;

// exclusive scan over the first E threads' values (1024-thread block); the
// total is returned in every thread
__device__ __forceinline__ int block_scan_excl(int v, int E, int *s_w, int &total) {
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const uint32_t inc = wave_scan_incl(uint32_t(tid < E ? v : 0));
    if (lane == WAVE - 1) s_w[wave] = int(inc);
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < int(blockDim.x) / WAVE; ++w) {
        before += w < wave ? s_w[w] : 0;
        all += s_w[w];
    }
    __syncthreads();
    total = all;
    return before + int(inc) - (tid < E ? v : 0);
}

__global__ __launch_bounds__(1024) void route_slots_kernel(RouteArgs a) {
    __shared__ int s_all[1024], s_pre[1024], s_base[1024], s_w[16];
    __shared__ unsigned long long s_mask[1024];
    const int tid = threadIdx.x, T = a.T, E = a.E, k = a.topk, P = T * k;
    const int t0 = int(blockIdx.x) * SLOT_CHUNK, nt = min(SLOT_CHUNK, T - t0), pk = t0 * k;
    if (tid < E) {
        s_all[tid] = 0;
        s_pre[tid] = 0;
        s_mask[tid] = 0ull;
    }
    __syncthreads();
    // eight selections requested per thread before their counts (one memory
    // round trip per eight instead of per selection)
    for (int i0 = tid; i0 < P; i0 += 8 * int(blockDim.x)) {
        int ev[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) ev[u] = a.top_e[min(i0 + u * int(blockDim.x), P - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = i0 + u * int(blockDim.x);
            if (i < P) {
                atomicAdd(&s_all[ev[u]], 1);
                if (i < pk) atomicAdd(&s_pre[ev[u]], 1);
            }
        }
    }
    __syncthreads();
    const int c = tid < E ? s_all[tid] : 0;
    int total;
    const int off = block_scan_excl(c, E, s_w, total);
    if (tid < E) s_base[tid] = off + s_pre[tid];
    if (blockIdx.x == 0) {
        int n_act, n_tiles = 0;
        const int act = block_scan_excl(c > 0, E, s_w, n_act);
        const int ntl = a.tile_m != 0 && tid < E ? tile_count(c, a.tile_m) : 0;
        const int tile0 = a.tile_m != 0 ? block_scan_excl(ntl, E, s_w, n_tiles) : 0;
        if (tid < E) {
            a.offsets[tid] = off;
            a.counts[tid] = c;
            if (c > 0) a.active[act] = tid;
            for (int j = 0, m0 = 0; j < ntl; ++j, m0 += tile_rows(c - m0, a.tile_m)) {
                a.tile_e[tile0 + j] = tid;
                a.tile_m0[tile0 + j] = m0;
            }
        }
        if (tid == 0) {
            a.offsets[E] = total;
            *a.n_active = n_act;
            if (a.tile_m != 0) *a.n_tiles = n_tiles;
        }
    }
    // the chunk's pairs: token bits per expert, then ranks
    for (int i = tid; i < nt * k; i += blockDim.x) atomicOr(&s_mask[a.top_e[pk + i]], 1ull << (i / k));
    __syncthreads();
    for (int i = tid; i < nt * k; i += blockDim.x) {
        const int e = a.top_e[pk + i], tl = i / k;
        const int slot = s_base[e] + __popcll(s_mask[e] & ((1ull << tl) - 1ull));
        a.tok_slot[pk + i] = slot;
        a.pair_tok[slot] = t0 + tl;
    }
}

// Decode batches (T <= 64): selections and slots in one launch. A token
// picks an expert at most once, so the tokens of expert e are the set bits of
// one 64-bit mask; a pair's rank among them is a popcount below its bit.
// The whole routing of a decode batch by one block of 1024 threads; logit(t)
// gives token t's row loader (expert index -> logit).
// Static LDS of the routing body (in every kernel that routes): its top-k,
// mask, offset and scan arrays. Launchers count it against the CU's 160 KiB.
constexpr size_t ROUTE_STATIC_LDS = 64 * 64 * 4 + 1024 * 8 + 1024 * 4 + 16 * 2 * 4;

template <int PER, class RowFn>
__device__ __forceinline__ void route_small_body(const RouteArgs &a, const ExpfGlibc &ex, RowFn logit_row) {
    __shared__ int32_t s_te[64 * 64];
    __shared__ unsigned long long s_mask[1024];
    __shared__ int32_t s_off[1024];
    __shared__ uint32_t s_sum[16][2];
    static_assert(sizeof(s_te) + sizeof(s_mask) + sizeof(s_off) + sizeof(s_sum) == ROUTE_STATIC_LDS, "static LDS");
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int T = a.T, E = a.E, k = a.topk, P = T * k;
    if (tid < E) s_mask[tid] = 0ull;
    for (int t = wave; t < T; t += 16)
        topk_wave<PER>(ex, logit_row(t), E, k, lane, s_te + t * k, a.top_w + int64_t(t) * k);
    __syncthreads();
    for (int i = tid; i < P; i += blockDim.x) {
        a.top_e[i] = s_te[i];
        atomicOr(&s_mask[s_te[i]], 1ull << (i / k));
    }
    __syncthreads();
    // exclusive scans over the experts (one per thread): pairs and non-empty
    // experts packed in one word (both < 2^16), tiles in another
    const int c = tid < E ? __popcll(s_mask[tid]) : 0;
    const int nt = a.tile_m != 0 ? tile_count(c, a.tile_m) : 0;
    const uint32_t v0 = uint32_t(c) | (uint32_t(c > 0) << 16), v1 = uint32_t(nt);
    const uint32_t i0 = wave_scan_incl(v0), i1 = a.tile_m != 0 ? wave_scan_incl(v1) : 0u;
    if (lane == WAVE - 1) {
        s_sum[wave][0] = i0;
        s_sum[wave][1] = i1;
    }
    __syncthreads();
    uint32_t e0 = i0 - v0, e1 = i1 - v1;
    for (int w = 0; w < wave; ++w) {
        e0 += s_sum[w][0];
        e1 += s_sum[w][1];
    }
    const int off = int(e0 & 0xffffu), act = int(e0 >> 16), tile0 = int(e1);
    if (tid < E) {
        s_off[tid] = off;
        a.offsets[tid] = off;
        a.counts[tid] = c;
        if (c > 0) a.active[act] = tid;
        for (int j = 0, m0 = 0; j < nt; ++j, m0 += tile_rows(c - m0, a.tile_m)) {
            a.tile_e[tile0 + j] = tid;
            a.tile_m0[tile0 + j] = m0;
        }
        if (tid == E - 1) {
            a.offsets[E] = off + c;
            *a.n_active = act + (c > 0);
            if (a.tile_m != 0) *a.n_tiles = tile0 + nt;
        }
    }
    __syncthreads();
    for (int i = tid; i < P; i += blockDim.x) {
        const int e = s_te[i], t = i / k;
        const int slot = s_off[e] + __popcll(s_mask[e] & ((1ull << t) - 1ull));
        a.tok_slot[i] = slot;
        a.pair_tok[slot] = t;
    }
}

template <int PER>
__global__ __launch_bounds__(1024) void route_small_kernel(RouteArgs a) {
    ExpfGlibc ex;
    ex.load(threadIdx.x % WAVE);
    route_small_body<PER>(a, ex, [&](int t) {
        const float *l = a.logits + int64_t(t) * a.E;
        return [l](int i) { return l[i]; };
    });
}

// ---- router GEMV and routing of a decode batch in one launch
// Block (g, ks) computes the fp32 logits of experts 16g .. 16g + 15 (one per
// wave) over K slice ks for every token and writes them as partial sums. The
// last block of group g to finish adds its slices into the logits; the last
// group to finish routes. With at most two logits per thread of a block
// (T * E <= 2048) the last block of the whole grid does both instead.
// Counters (device scope) are cleared for the next call by the blocks that
// count last.
__device__ __forceinline__ float wave_sum_f32(float v) {
#define QW_FSUM_STEP(ctrl) v += __builtin_bit_cast(float, QW_DPP(__builtin_bit_cast(uint32_t, v), ctrl, 0xf, 0xf, false));
    QW_FSUM_STEP(DPP_XOR1)
    QW_FSUM_STEP(DPP_XOR2)
    QW_FSUM_STEP(DPP_HALF_MIRROR)
    QW_FSUM_STEP(DPP_MIRROR)
#undef QW_FSUM_STEP
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// The routing block's copy of every logit into LDS (agent-scope loads, eight
// in flight per thread before their writes), then a barrier.
__device__ __forceinline__ void load_logits_lds(const float *logits, int n, float *sl) {
    const int bd = blockDim.x;
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * bd) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = ld_agent(logits + min(i0 + j * bd, n - 1));
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (i0 + j * bd < n) sl[i0 + j * bd] = v[j];
    }
    __syncthreads();
}

// Whether the K-sliced router's last block routes from LDS: the T x E logits
// fit beside the routing's static arrays.
__host__ __device__ inline bool router_lds_route(int T, int E) { return size_t(T) * E * 4 <= 96 * 1024; }

// A run of 8 router weights as loaded -> fp32: fp32 bits in raw0 / raw1, or
// 8 fp16 in raw0 (w_f16, exact widening).
__device__ __forceinline__ void widen_run(const uint4 &raw0, const uint4 &raw1, int w_f16, float4 &w0, float4 &w1) {
    if (w_f16) {
        w0 = float4{f16_bits_to_f32(uint16_t(raw0.x)), f16_bits_to_f32(uint16_t(raw0.x >> 16)),
                    f16_bits_to_f32(uint16_t(raw0.y)), f16_bits_to_f32(uint16_t(raw0.y >> 16))};
        w1 = float4{f16_bits_to_f32(uint16_t(raw0.z)), f16_bits_to_f32(uint16_t(raw0.z >> 16)),
                    f16_bits_to_f32(uint16_t(raw0.w)), f16_bits_to_f32(uint16_t(raw0.w >> 16))};
    } else {
        w0 = __builtin_bit_cast(float4, raw0);
        w1 = __builtin_bit_cast(float4, raw1);
    }
}

template <int PER>
__global__ __launch_bounds__(1024) void router_route_kernel(RouteArgs a, RouterArgs r) {
    extern __shared__ __align__(16) unsigned char smem[];  // x slice, [T][kl]
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    ExpfGlibc ex;
    ex.load(lane);
    const int T = a.T, E = a.E, H = r.H, kc = r.kl / 8, k0 = blockIdx.y * r.kl;
    const int e = blockIdx.x * 16 + wave;
    // kl <= 512: each lane owns at most one run of 8 weights of its expert's
    // slice; they are requested before the activations are staged. Lanes
    // past the slice (and waves past E) read a valid run and zero it: the
    // token loop below then has no branch around the weights, so the wait
    // for them is not repeated per token. On this GPU stores count on the
    // same counter as loads, so each repeated wait also waited for the
    // previous token's logit store (one memory round trip per token).
    const bool mine = e < E && lane < kc;
    const int64_t wo = int64_t(min(e, E - 1)) * H + k0 + min(lane, kc - 1) * 8;
    // as loaded (fp32 bits, or 8 fp16 in raw0), widened after the activations
    // are staged (fp16 -> fp32 is exact: the same products as fp32 weights
    // holding the same values)
    uint4 raw0, raw1 = make_uint4(0u, 0u, 0u, 0u);
    if (r.w_f16) {
        raw0 = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(r.w) + wo);
    } else {
        const float *wp = static_cast<const float *>(r.w) + wo;
        raw0 = *reinterpret_cast<const uint4 *>(wp);
        raw1 = *reinterpret_cast<const uint4 *>(wp + 4);
    }
    uint4 *xs = reinterpret_cast<uint4 *>(smem);
    // activation pieces: four loads in flight per thread before their writes
    for (int i0 = tid; i0 < T * kc; i0 += 4 * int(blockDim.x)) {
        uint4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = min(i0 + j * int(blockDim.x), T * kc - 1), t = i / kc, c = i - t * kc;
            v[j] = *reinterpret_cast<const uint4 *>(r.x + int64_t(t) * H + k0 + c * 8);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (i0 + j * int(blockDim.x) < T * kc) xs[i0 + j * blockDim.x] = v[j];
    }
    __syncthreads();
    // the weights' one wait, here: every token below then finds them ready
    // (each token's block is guarded by t < T, and the compiler would
    // otherwise wait again in each)
    float4 w0, w1;
    widen_run(raw0, raw1, r.w_f16, w0, w1);
    if (!mine) w0 = w1 = float4{0.f, 0.f, 0.f, 0.f};
    asm volatile("" ::"v"(w0.x), "v"(w0.y), "v"(w0.z), "v"(w0.w), "v"(w1.x), "v"(w1.y), "v"(w1.z), "v"(w1.w));
    // x rows bf16 or fp16 (a block-uniform choice; both conversions are exact)
    auto dots = [&](auto cvt) {
        if (e >= E) return;
#pragma unroll
        for (int t = 0; t < 64; ++t) {
            if (t < T) {
                float s = 0.f;
                {
                    const uint4 v = xs[t * kc + min(lane, kc - 1)];
                    s = fmaf(w0.x, cvt(uint16_t(v.x)), s);
                    s = fmaf(w0.y, cvt(uint16_t(v.x >> 16)), s);
                    s = fmaf(w0.z, cvt(uint16_t(v.y)), s);
                    s = fmaf(w0.w, cvt(uint16_t(v.y >> 16)), s);
                    s = fmaf(w1.x, cvt(uint16_t(v.z)), s);
                    s = fmaf(w1.y, cvt(uint16_t(v.z >> 16)), s);
                    s = fmaf(w1.z, cvt(uint16_t(v.w)), s);
                    s = fmaf(w1.w, cvt(uint16_t(v.w >> 16)), s);
                }
                const float v = wave_sum_f32(s);
                if (lane == 0) st_agent(r.part + (int64_t(blockIdx.y) * T + t) * E + e, v);
            }
        }
    };
    if (r.x_f16) dots([](uint16_t b) { return f16_bits_to_f32(b); });
    else dots([](uint16_t b) { return bf16_bits_to_f32(b); });
    const int ksplit = gridDim.y, TE = T * E;
    // the sum of a logit's slices, in slice order (up to 8 loads in flight)
    auto slice_sum = [&](int o) {
        float v = 0.f;
        for (int j0 = 0; j0 < ksplit; j0 += 8) {
            float pv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) pv[j] = j0 + j < ksplit ? ld_agent(r.part + int64_t(j0 + j) * TE + o) : 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) v += pv[j];
        }
        return v;
    };
    // The routing block reads the logits from LDS (the activation slice's
    // area, free by then) when they fit: one memory round trip for all of
    // them instead of one per token and wave.
    const bool lds_route = router_lds_route(T, E);
    float *sl = reinterpret_cast<float *>(smem);
    auto route = [&]() {
        if (lds_route) {
            route_small_body<PER>(a, ex, [&](int t) {
                const float *l = sl + t * E;
                return [l](int i) { return l[i]; };
            });
        } else {
            route_small_body<PER>(a, ex, [&](int t) {
                const float *l = r.logits + int64_t(t) * E;
                return [l](int i) { return ld_agent(l + i); };
            });
        }
    };
    if (T * E <= 2 * int(blockDim.x)) {
        // few logits (decode batches): the last block of the whole grid sums
        // every logit's slices (the same additions in the same order as the
        // per-group sums below) and routes, one hand-off instead of two
        if (!count_last_block(r.counter, int(gridDim.x * gridDim.y))) return;
        for (int o = tid; o < TE; o += blockDim.x) {
            const float v = slice_sum(o);
            st_agent(r.logits + o, v);
            sl[o] = v;  // (T * E fits: at most 2048 logits)
        }
        __syncthreads();
        route_small_body<PER>(a, ex, [&](int t) {
            const float *l = sl + t * E;
            return [l](int i) { return l[i]; };
        });
        return;
    }
    // the last slice block of each group of 16 experts adds the group's
    // slices in slice order
    if (!count_last_block(r.counter + 1 + blockIdx.x, int(gridDim.y))) return;
    const int e0 = blockIdx.x * 16, ng = min(16, E - e0);
    for (int i = tid; i < T * ng; i += blockDim.x) {
        const int t = i / ng, o = t * E + e0 + (i - t * ng);
        st_agent(r.logits + o, slice_sum(o));
    }
    // and the last group to finish routes
    if (!count_last_block(r.counter, int(gridDim.x))) return;
    if (lds_route) load_logits_lds(r.logits, TE, sl);
    route();
}

// ---- decode batches (T <= 8): full-K router blocks, one hand-off
// Block b computes the complete fp32 logits of experts EPB b .. EPB b + EPB - 1
// for every token: WPE waves per expert split K into WPE contiguous parts,
// each lane sums runs of 8 weights (all of its weight loads requested before
// the activations are staged), the wave reduces, and the WPE part sums are
// added in part order. With no K split across blocks there is no partial-sum
// pass, and only E / EPB blocks count into the hand-off counter (device-scope
// atomics on one counter serialise at about 18 ns each). The last block reads
// every logit once into LDS and routes from there.
// ROUTE false: the logits only, by plain stores (the kernel boundary makes
// them visible to the next launch), no count and no routing.
// bx: the block's expert group (an argument, so that a kernel running other
// work in the same grid can call it for a part of its blocks)
template <int PER, int EPB, int WPE, int NCH, bool ROUTE>
__device__ __forceinline__ void router_full_block(const RouteArgs &a, const RouterArgs &r, int bx) {
    extern __shared__ __align__(16) unsigned char smem[];  // x [T][H] | part sums [T][EPB][WPE] | logits [T][E]
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int T = a.T, E = a.E, H = r.H, kw = H / WPE, nch = kw / 8;
    const int el = wave / WPE, wp = wave % WPE, e = min(bx * EPB + el, E - 1);
    ExpfGlibc ex;
    ex.load(lane);
    // the lane's runs of 8 weights: chunks lane, lane + 64, .. of its part
    // (as loaded; widened to fp32 once the activations are staged)
    uint4 wraw[NCH][2];
    const int64_t wo = int64_t(e) * H + wp * kw;
    if (r.w_f16) {
        const uint16_t *wr = static_cast<const uint16_t *>(r.w) + wo;
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            wraw[j][0] = *reinterpret_cast<const uint4 *>(wr + min(lane + j * WAVE, nch - 1) * 8);
            wraw[j][1] = make_uint4(0u, 0u, 0u, 0u);
        }
    } else {
        const float *wr = static_cast<const float *>(r.w) + wo;
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            const int c = min(lane + j * WAVE, nch - 1);
            wraw[j][0] = *reinterpret_cast<const uint4 *>(wr + c * 8);
            wraw[j][1] = *reinterpret_cast<const uint4 *>(wr + c * 8 + 4);
        }
    }
    uint4 *xs = reinterpret_cast<uint4 *>(smem);
    const int xc = H / 8;
    for (int i = tid; i < T * xc; i += blockDim.x) {
        const int t = i / xc, c = i - t * xc;
        xs[i] = *reinterpret_cast<const uint4 *>(r.x + int64_t(t) * H + c * 8);
    }
    float *part = reinterpret_cast<float *>(xs + T * xc);  // [T][EPB][WPE]
    float *sl = part + T * EPB * WPE;                     // [T][E] (last block)
    __syncthreads();
    float4 w[NCH][2];
#pragma unroll
    for (int j = 0; j < NCH; ++j) widen_run(wraw[j][0], wraw[j][1], r.w_f16, w[j][0], w[j][1]);
    auto dots = [&](auto cvt) {
        for (int t = 0; t < T; ++t) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                if (lane + j * WAVE < nch) {
                    const uint4 v = xs[t * xc + wp * (kw / 8) + lane + j * WAVE];
                    s = fmaf(w[j][0].x, cvt(uint16_t(v.x)), s);
                    s = fmaf(w[j][0].y, cvt(uint16_t(v.x >> 16)), s);
                    s = fmaf(w[j][0].z, cvt(uint16_t(v.y)), s);
                    s = fmaf(w[j][0].w, cvt(uint16_t(v.y >> 16)), s);
                    s = fmaf(w[j][1].x, cvt(uint16_t(v.z)), s);
                    s = fmaf(w[j][1].y, cvt(uint16_t(v.z >> 16)), s);
                    s = fmaf(w[j][1].z, cvt(uint16_t(v.w)), s);
                    s = fmaf(w[j][1].w, cvt(uint16_t(v.w >> 16)), s);
                }
            }
            const float v = wave_sum_f32(s);
            if (lane == 0) part[(t * EPB + el) * WPE + wp] = v;
        }
    };
    if (r.x_f16) dots([](uint16_t b) { return f16_bits_to_f32(b); });
    else dots([](uint16_t b) { return bf16_bits_to_f32(b); });
    __syncthreads();
    for (int i = tid; i < T * EPB; i += blockDim.x) {
        const int t = i / EPB, j = i - t * EPB, ee = bx * EPB + j;
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < WPE; ++q) v += part[i * WPE + q];
        if (ee < E) {
            if constexpr (ROUTE) st_agent(r.logits + int64_t(t) * E + ee, v);
            else r.logits[int64_t(t) * E + ee] = v;
        }
    }
    if constexpr (ROUTE) {
        if (!count_last_block(r.counter, int(gridDim.x))) return;
        load_logits_lds(r.logits, T * E, sl);
        route_small_body<PER>(a, ex, [&](int t) {
            const float *l = sl + t * E;
            return [l](int i) { return l[i]; };
        });
    }
}

template <int PER, int EPB, int WPE, int NCH, bool ROUTE = true>
__global__ __launch_bounds__(EPB *WPE *WAVE) void router_full_kernel(RouteArgs a, RouterArgs r) {
    router_full_block<PER, EPB, WPE, NCH, ROUTE>(a, r, int(blockIdx.x));
}

// The full-K router serves T <= 8 (activations staged whole) and H up to
// 8192 (runs of 8 weights: at most 8 per lane with 2 waves per expert)
// (E <= 512: the routing's per-lane logits then fit the 1024-thread block's
// registers)
// (and its activations, part sums and logits in LDS beside the routing's
// static arrays fit the CU's 160 KiB: at H = 8192 and T = 8 only E <= 64 fits,
// at H = 4096 every E up to 512 does)
static size_t router_full_lds(int T, int E, int H) {
    constexpr int EPB = 8, WPE = 2;
    return size_t(T) * H * 2 + size_t(T) * EPB * WPE * 4 + size_t(T) * E * 4;
}
bool router_full_ok(int T, int E, int H) {
    return T <= 8 && H % 1024 == 0 && H <= 8192 && E <= 512 && E % 8 == 0 &&
           router_full_lds(T, E, H) + ROUTE_STATIC_LDS <= 160 * 1024;
}

static void launch_router_full(const RouteArgs &a, const RouterArgs &r, hipStream_t s) {
    constexpr int EPB = 8, WPE = 2;
    const int per = (a.E + WAVE - 1) / WAVE;
    const size_t lds = router_full_lds(a.T, a.E, r.H);
    const unsigned grid = unsigned((a.E + EPB - 1) / EPB);
    const int nch = r.H / WPE / 8;  // runs of 8 per wave
    auto go = [&](auto kern) {
        if (lds > 48 * 1024) raise_lds_limit(reinterpret_cast<const void *>(kern));
        kern<<<grid, EPB * WPE * WAVE, lds, s>>>(a, r);
    };
    auto pick = [&](auto nc) {
        constexpr int NC = decltype(nc)::value;
        if (per <= 1) go(router_full_kernel<1, EPB, WPE, NC>);
        else if (per <= 2) go(router_full_kernel<2, EPB, WPE, NC>);
        else if (per <= 4) go(router_full_kernel<4, EPB, WPE, NC>);
        else go(router_full_kernel<8, EPB, WPE, NC>);
    };
    if (nch <= 2 * WAVE) pick(std::integral_constant<int, 2>());
    else if (nch <= 4 * WAVE) pick(std::integral_constant<int, 4>());
    else pick(std::integral_constant<int, 8>());
}

bool router_logits_ok(int T, int E, int H) { return router_full_ok(T, E, H); }

bool router_split_ok(int T, int E, int H) { return T >= 2 && T <= 8 && router_logits_ok(T, E, H); }

template <int EPB, int WPE>
static void launch_router_logits_t(const RouterArgs &r, int T, int E, hipStream_t s) {
    RouteArgs a{};
    a.T = T;
    a.E = E;
    const size_t lds = size_t(T) * r.H * 2 + size_t(T) * EPB * WPE * 4 + size_t(T) * E * 4;
    const unsigned grid = unsigned((E + EPB - 1) / EPB);
    const int nch = r.H / WPE / 8;
    auto go = [&](auto kern) {
        if (lds > 48 * 1024) raise_lds_limit(reinterpret_cast<const void *>(kern));
        kern<<<grid, EPB * WPE * WAVE, lds, s>>>(a, r);
    };
    if (nch <= WAVE) go(router_full_kernel<1, EPB, WPE, 1, false>);
    else if (nch <= 2 * WAVE) go(router_full_kernel<1, EPB, WPE, 2, false>);
    else if (nch <= 4 * WAVE) go(router_full_kernel<1, EPB, WPE, 4, false>);
    else go(router_full_kernel<1, EPB, WPE, 8, false>);
}

// One expert per block, its K split over 8 waves (256 blocks at E = 256):
// with no routing tail, the launch is the weight stream and its latency, and
// more blocks in flight shorten it (batch 1, same box: 29.9 us per MoE block
// against 30.3 with 4 experts per block and 30.4-31.2 with 8).
void launch_router_logits(const RouterArgs &r, int T, int E, hipStream_t s) {
    launch_router_logits_t<1, 8>(r, T, E, s);
}

// ---- up to 8 tokens with the shared expert: blocks 0 .. E - 1 compute the
// router logits (as launch_router_logits), blocks E .. compute 16 rows each
// of the shared expert's gate/up/gate-logit GEMV (as qw_w16_gemv_tiled): two
// independent GEMVs over the same activation rows in one launch, which also
// gives the CUs the router leaves idle (E blocks) work.
template <int NCH, typename SXT, int SMR, int SXPT, int SWS>
__global__ __launch_bounds__(8 * WAVE) void router_logits_shgu_kernel(RouteArgs a, RouterArgs r, ShExpertArgs sh) {
    const int b = blockIdx.x, N = 2 * sh.Fs + 1;
    if (b < a.E) router_full_block<1, 1, 8, NCH, false>(a, r, b);
    else w16_gemv_block<SXT, 1, SMR, SXPT, SWS, true>(sh.gu, 0, r.x, r.H, a.T, r.H, N, sh.v, N, 0, 0, 0, b - a.E);
}

bool shared_logits_ok(int T, int H, int Fs) {
    return T >= 1 && T <= 8 && H % 256 == 0 && H <= 8192 && Fs % 256 == 0 && Fs <= 4096;
}

void launch_router_logits_shgu(const RouterArgs &r, int T, int E, const ShExpertArgs &sh, hipStream_t s) {
    RouteArgs a{};
    a.T = T;
    a.E = E;
    const int H = r.H, N = 2 * sh.Fs + 1;
    // the router's LDS as launch_router_logits sizes it, the GEMV's as qw_w16_gemv's
    const size_t lr = size_t(T) * H * 2 + size_t(T) * 8 * 4 + size_t(T) * E * 4,
                 lw = dense_lds_bytes(T, H, 1, W16_MAX_KS, W16_MAX_KS);
    const size_t lds = lr > lw ? lr : lw;
    const unsigned grid = unsigned(E + (N + 15) / 16);
    const int xpt = (T * (H / 8) + 8 * WAVE - 1) / (8 * WAVE);
    auto go = [&](auto kern) {
        if (lds > 48 * 1024) raise_lds_limit(reinterpret_cast<const void *>(kern));
        kern<<<grid, 8 * WAVE, lds, s>>>(a, r, sh);
    };
    auto by_nch = [&](auto sxt, auto smr, auto sxpt, auto sws) {
        using SXT = decltype(sxt);
        constexpr int SMR = decltype(smr)::value, SXPT = decltype(sxpt)::value, SWS = decltype(sws)::value;
        if (H / 64 <= WAVE) go(router_logits_shgu_kernel<1, SXT, SMR, SXPT, SWS>);
        else go(router_logits_shgu_kernel<2, SXT, SMR, SXPT, SWS>);
    };
    auto by_ws = [&](auto sxt, auto smr, auto sxpt) {
        if (H / 32 / W16_MAX_KS <= 8) by_nch(sxt, smr, sxpt, std::integral_constant<int, 8>());
        else by_nch(sxt, smr, sxpt, std::integral_constant<int, 16>());
    };
    // loads per thread of the activation staging as launch_w16_t picks them
    auto by_xpt = [&](auto sxt, auto smr) {
        if (xpt <= 1) by_ws(sxt, smr, std::integral_constant<int, 1>());
        else if (xpt <= 2) by_ws(sxt, smr, std::integral_constant<int, 2>());
        else if (xpt <= 4) by_ws(sxt, smr, std::integral_constant<int, 4>());
        else by_ws(sxt, smr, std::integral_constant<int, 0>());
    };
    // rows per MFMA pass as launch_w16_x picks them
    auto by_mr = [&](auto sxt) {
        if (T == 1) by_xpt(sxt, std::integral_constant<int, 1>());
        else if (T == 2) by_xpt(sxt, std::integral_constant<int, 2>());
        else by_xpt(sxt, std::integral_constant<int, 4>());
    };
    if (r.x_f16) by_mr(F16{});
    else by_mr(BF16{});
}

// ---- router logits on the fp32 MFMA (9 to 32 tokens): block (g, s) forms
// the partial logits of experts 16 g .. 16 g + 15 over K slice s (512 wide)
// for every token, part[s][t][e]; the routing launch after it adds the
// slices in slice order. No per-token wave reductions (the dot products'
// cost in router_route_kernel) and no cross-block hand-off. Wave w takes
// 64 K of the slice: per 16-K step lane (q, n) loads 4 consecutive weights
// of expert 16 g + n and 4 activations of token 16 tt + n at K 4 q, and
// v_mfma_f32_16x16x4f32 j adds the products of their j-th elements (tokens
// as rows, experts as columns: the lane ends with expert 16 g + n, tokens
// 16 tt + 4 q + r). Fp16 weights and 16-bit activations widen exactly. The
// 8 waves' tiles are added in wave order through LDS.
template <int TT>
__global__ __launch_bounds__(8 * WAVE) void router_mfma_kernel(RouterArgs r, int T, int E) {
    __shared__ f32x4 red[8][TT][WAVE];
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE, q = lane / 16, n = lane % 16;
    const int e0 = int(blockIdx.x) * 16, sl = int(blockIdx.y), H = r.H;
    const int k0 = sl * 512 + wave * 64 + 4 * q;
    const int e = min(e0 + n, E - 1);
    constexpr int STEPS = 4;  // 64 K per wave in 16-K steps
    uint4 wraw[STEPS];
    uint2 xraw[TT][STEPS];
#pragma unroll
    for (int c = 0; c < STEPS; ++c) {
        const int k = k0 + 16 * c;
        if (r.w_f16) {
            const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(r.w) + int64_t(e) * H + k);
            wraw[c] = make_uint4(v.x, v.y, 0u, 0u);
        } else {
            wraw[c] = *reinterpret_cast<const uint4 *>(static_cast<const float *>(r.w) + int64_t(e) * H + k);
        }
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
            xraw[tt][c] = *reinterpret_cast<const uint2 *>(r.x + int64_t(min(16 * tt + n, T - 1)) * H + k);
    }
    const bool ev = e0 + n < E;
    f32x4 acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < STEPS; ++c) {
        float w[4];
        if (r.w_f16) {
            w[0] = f16_bits_to_f32(uint16_t(wraw[c].x));
            w[1] = f16_bits_to_f32(uint16_t(wraw[c].x >> 16));
            w[2] = f16_bits_to_f32(uint16_t(wraw[c].y));
            w[3] = f16_bits_to_f32(uint16_t(wraw[c].y >> 16));
        } else {
            w[0] = __builtin_bit_cast(float, wraw[c].x);
            w[1] = __builtin_bit_cast(float, wraw[c].y);
            w[2] = __builtin_bit_cast(float, wraw[c].z);
            w[3] = __builtin_bit_cast(float, wraw[c].w);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = ev ? w[j] : 0.f;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            const bool tv = 16 * tt + n < T;
            const uint32_t lo = xraw[tt][c].x, hi = xraw[tt][c].y;
            const uint16_t xs[4] = {uint16_t(lo), uint16_t(lo >> 16), uint16_t(hi), uint16_t(hi >> 16)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float xv = r.x_f16 ? f16_bits_to_f32(xs[j]) : bf16_bits_to_f32(xs[j]);
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(tv ? xv : 0.f, w[j], acc[tt], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) red[wave][tt][lane] = acc[tt];
    __syncthreads();
    if (tid < TT * WAVE) {
        const int tt = tid / WAVE, l = tid % WAVE, qq = l / 16, nn = l % 16;
        f32x4 v = red[0][tt][l];
#pragma unroll
        for (int w = 1; w < 8; ++w) v += red[w][tt][l];
        const int ee = e0 + nn;
        if (ee < E) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int t = 16 * tt + 4 * qq + rr;
                if (t < T) r.part[(int64_t(sl) * T + t) * E + ee] = v[rr];
            }
        }
    }
}

bool router_mfma_ok(int T, int E, int H, int kl) {
    // H / 512 slices: 1, 2, 4, 8 or 16 (launch_route_part's counts)
    const int S = H / 512;
    return T >= 9 && T <= 32 && E >= 1 && E <= 1024 && kl == 512 && H % 512 == 0 && (S & (S - 1)) == 0 && S <= 16;
}

void launch_router_mfma(const RouterArgs &r, int T, int E, hipStream_t s) {
    const dim3 grid(unsigned((E + 15) / 16), unsigned(r.H / 512));
    if (T <= 16) router_mfma_kernel<1><<<grid, 8 * WAVE, 0, s>>>(r, T, E);
    else router_mfma_kernel<2><<<grid, 8 * WAVE, 0, s>>>(r, T, E);
}

// The routing launches over partial logits (part[s][t][e], S slices added
// in slice order; the sums also go to logits, the rows a.logits names), as
// launch_route. S is a compile-time count, so a lane's slice loads all go
// out before the first add.
template <int S>
__device__ __forceinline__ float sum_slices(const float *p, int64_t plane, int i) {
    float pv[S];
#pragma unroll
    for (int sl = 0; sl < S; ++sl) pv[sl] = p[sl * plane + i];
    float v = pv[0];
#pragma unroll
    for (int sl = 1; sl < S; ++sl) v += pv[sl];
    return v;
}

template <int PER, int S>
__global__ __launch_bounds__(1024) void route_small_part_kernel(RouteArgs a, const float *part, float *logits) {
    ExpfGlibc ex;
    ex.load(threadIdx.x % WAVE);
    const int64_t plane = int64_t(a.T) * a.E;
    route_small_body<PER>(a, ex, [&](int t) {
        const float *p = part + int64_t(t) * a.E;
        float *lo = logits + int64_t(t) * a.E;
        return [p, lo, plane](int i) {
            const float v = sum_slices<S>(p, plane, i);
            lo[i] = v;
            return v;
        };
    });
}

template <int PER, int S>
__global__ __launch_bounds__(256) void route_topk_part_kernel(const float *__restrict__ part, int T, int E, int k,
                                                              float *__restrict__ logits, int32_t *__restrict__ top_e,
                                                              float *__restrict__ top_w) {
    const int t = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (t >= T) return;
    ExpfGlibc ex;
    ex.load(lane);
    const int64_t plane = int64_t(T) * E;
    const float *p = part + int64_t(t) * E;
    float *lo = logits + int64_t(t) * E;
    topk_wave<PER>(
        ex,
        [&](int i) {
            const float v = sum_slices<S>(p, plane, i);
            lo[i] = v;
            return v;
        },
        E, k, lane, top_e + int64_t(t) * k, top_w + int64_t(t) * k);
}

template <int S>
static void launch_route_part_s(const RouteArgs &a, const float *part, float *logits, hipStream_t s) {
    const int per = (a.E + WAVE - 1) / WAVE;
    if (a.T <= 16) {
        if (per <= 1) route_small_part_kernel<1, S><<<1, 1024, 0, s>>>(a, part, logits);
        else if (per <= 2) route_small_part_kernel<2, S><<<1, 1024, 0, s>>>(a, part, logits);
        else if (per <= 4) route_small_part_kernel<4, S><<<1, 1024, 0, s>>>(a, part, logits);
        else if (per <= 8) route_small_part_kernel<8, S><<<1, 1024, 0, s>>>(a, part, logits);
        else route_small_part_kernel<16, S><<<1, 1024, 0, s>>>(a, part, logits);
    } else {
        const unsigned g = unsigned((a.T + 3) / 4);
        if (per <= 4) route_topk_part_kernel<4, S><<<g, 256, 0, s>>>(part, a.T, a.E, a.topk, logits, a.top_e, a.top_w);
        else if (per <= 8) route_topk_part_kernel<8, S><<<g, 256, 0, s>>>(part, a.T, a.E, a.topk, logits, a.top_e, a.top_w);
        else route_topk_part_kernel<16, S><<<g, 256, 0, s>>>(part, a.T, a.E, a.topk, logits, a.top_e, a.top_w);
        route_slots_kernel<<<unsigned((a.T + SLOT_CHUNK - 1) / SLOT_CHUNK), 1024, 0, s>>>(a);
    }
}

void launch_route_part(const RouteArgs &a, const float *part, int S, float *logits, hipStream_t s) {
    switch (S) {
        case 1: launch_route_part_s<1>(a, part, logits, s); break;
        case 2: launch_route_part_s<2>(a, part, logits, s); break;
        case 4: launch_route_part_s<4>(a, part, logits, s); break;
        case 8: launch_route_part_s<8>(a, part, logits, s); break;
        default: launch_route_part_s<16>(a, part, logits, s); break;
    }
}

size_t router_lds_bytes(int T, int kl, int E) {
    const size_t x = size_t(T) * kl * 2, l = router_lds_route(T, E) ? size_t(T) * E * 4 : 0;
    return x > l ? x : l;
}

void launch_router_route(const RouteArgs &a, const RouterArgs &r, hipStream_t s) {
    if (router_full_ok(a.T, a.E, r.H)) {
        launch_router_full(a, r, s);
        return;
    }
    // callers guarantee kl in {128, 512}, H % kl == 0 and T <= 64
    const int per = (a.E + WAVE - 1) / WAVE;
    const dim3 grid(unsigned((a.E + 15) / 16), unsigned(r.H / r.kl));
    const size_t lds = router_lds_bytes(a.T, r.kl, a.E);
    auto go = [&](auto kern) {
        if (lds > 48 * 1024) raise_lds_limit(reinterpret_cast<const void *>(kern));
        kern<<<grid, 1024, lds, s>>>(a, r);
    };
    if (per <= 1) go(router_route_kernel<1>);
    else if (per <= 2) go(router_route_kernel<2>);
    else if (per <= 4) go(router_route_kernel<4>);
    else if (per <= 8) go(router_route_kernel<8>);
    else go(router_route_kernel<16>);
}

void launch_route(const RouteArgs &a, hipStream_t s) {
    // one block while each of its 16 waves routes at most one token; beyond,
    // top-k in parallel blocks and the slots in a second launch (32 tokens:
    // 9.8 against 12.1 us)
    if (a.T <= 16) {
        const int per = (a.E + WAVE - 1) / WAVE;
        if (per <= 1) route_small_kernel<1><<<1, 1024, 0, s>>>(a);
        else if (per <= 2) route_small_kernel<2><<<1, 1024, 0, s>>>(a);
        else if (per <= 4) route_small_kernel<4><<<1, 1024, 0, s>>>(a);
        else if (per <= 8) route_small_kernel<8><<<1, 1024, 0, s>>>(a);
        else route_small_kernel<16><<<1, 1024, 0, s>>>(a);
    } else {
        const int per = (a.E + WAVE - 1) / WAVE;
        const unsigned g = unsigned((a.T + 3) / 4);
        if (per <= 4) route_topk_kernel<4><<<g, 256, 0, s>>>(a.logits, a.T, a.E, a.topk, a.top_e, a.top_w);
        else if (per <= 8) route_topk_kernel<8><<<g, 256, 0, s>>>(a.logits, a.T, a.E, a.topk, a.top_e, a.top_w);
        else route_topk_kernel<16><<<g, 256, 0, s>>>(a.logits, a.T, a.E, a.topk, a.top_e, a.top_w);
        route_slots_kernel<<<unsigned((a.T + SLOT_CHUNK - 1) / SLOT_CHUNK), 1024, 0, s>>>(a);
    }
}

// ---- 2 to 4 tokens with the shared expert: block 0 routes the batch (as
// route_small_kernel; 8 waves cover T <= 8 tokens and, one thread per expert,
// E <= 512), blocks 1 .. run the shared expert's SwiGLU-gate + down GEMV (as
// qw_w16_swiglu_gemv_tiled, 16 output rows each). Both read only what the
// router-logits launch before them wrote.
template <int PER, int SMR, int SXPT, int SWS>
__global__ __launch_bounds__(8 * WAVE) void route_shdown_kernel(RouteArgs a, ShExpertArgs sh, int H) {
    if (blockIdx.x == 0) {
        ExpfGlibc ex;
        ex.load(threadIdx.x % WAVE);
        route_small_body<PER>(a, ex, [&](int t) {
            const float *l = a.logits + int64_t(t) * a.E;
            return [l](int i) { return l[i]; };
        });
    } else {
        w16_swiglu_block<1, SMR, SXPT, SWS>(sh.down, sh.v, 2 * sh.Fs + 1, a.T, sh.Fs, H, sh.out, H, 0, 0,
                                            int(blockIdx.x) - 1);
    }
}

bool launch_route_shdown(const RouteArgs &a, const ShExpertArgs &sh, int H, hipStream_t s) {
    const int T = a.T, Fs = sh.Fs;
    if (T < 2 || T > 4 || a.E > 8 * WAVE || a.tile_m != 0 || Fs % 256 != 0 || !w16_swiglu_fits(T, Fs, H)) return false;
    const size_t lds = dense_lds_bytes(T, Fs, 1, W16_MAX_KS, W16_MAX_KS);
    if (lds + ROUTE_STATIC_LDS > 160 * 1024) return false;
    const unsigned grid = unsigned(1 + (H + 15) / 16);
    const int xpt = (T * (Fs / 8) + 8 * WAVE - 1) / (8 * WAVE), per = (a.E + WAVE - 1) / WAVE;
    auto go = [&](auto kern) {
        if (lds > 48 * 1024) raise_lds_limit(reinterpret_cast<const void *>(kern));
        kern<<<grid, 8 * WAVE, lds, s>>>(a, sh, H);
    };
    auto by_per = [&](auto smr, auto sxpt, auto sws) {
        constexpr int SMR = decltype(smr)::value, SXPT = decltype(sxpt)::value, SWS = decltype(sws)::value;
        if (per <= 1) go(route_shdown_kernel<1, SMR, SXPT, SWS>);
        else if (per <= 2) go(route_shdown_kernel<2, SMR, SXPT, SWS>);
        else if (per <= 4) go(route_shdown_kernel<4, SMR, SXPT, SWS>);
        else go(route_shdown_kernel<8, SMR, SXPT, SWS>);
    };
    // staging width and weight steps per wave as launch_w16_swiglu picks them
    auto by_ws = [&](auto smr, auto sxpt) {
        if ((Fs / 32 + W16_MAX_KS - 1) / W16_MAX_KS <= 8) by_per(smr, sxpt, std::integral_constant<int, 8>());
        else by_per(smr, sxpt, std::integral_constant<int, 16>());
    };
    auto by_xpt = [&](auto smr) {
        if (xpt <= 1) by_ws(smr, std::integral_constant<int, 1>());
        else if (xpt <= 2) by_ws(smr, std::integral_constant<int, 2>());
        else by_ws(smr, std::integral_constant<int, 4>());
    };
    if (T == 2) by_xpt(std::integral_constant<int, 2>());
    else by_xpt(std::integral_constant<int, 4>());
    return true;
}

// ---- 5 to 8 tokens with the shared expert: block 0 routes the batch (as in
// route_shdown_kernel), blocks 1 .. form the shared expert's SwiGLU-gate rows
// h [T][Fs] (as swiglu_gate_kernel, 512 elements per block) for the down GEMV
// launch that follows.
template <int PER>
__global__ __launch_bounds__(8 * WAVE) void route_shgate_kernel(RouteArgs a, const float *v, int n, uint16_t *h) {
    if (blockIdx.x == 0) {
        ExpfGlibc ex;
        ex.load(threadIdx.x % WAVE);
        route_small_body<PER>(a, ex, [&](int t) {
            const float *l = a.logits + int64_t(t) * a.E;
            return [l](int i) { return l[i]; };
        });
    } else {
        const int i = (int(blockIdx.x) - 1) * int(blockDim.x) + int(threadIdx.x);
        if (i >= a.T * n) return;
        const int t = i / n, j = i - t * n;
        const float *r = v + int64_t(t) * (2 * n + 1);
        h[i] = swiglu_h(r[j], r[n + j], sigmoid_gate(r[2 * n]));
    }
}

bool launch_route_shgate(const RouteArgs &a, const ShExpertArgs &sh, uint16_t *h, hipStream_t s) {
    if (a.T < 1 || a.T > 8 || a.E > 8 * WAVE || a.tile_m != 0) return false;
    const int n = sh.Fs, per = (a.E + WAVE - 1) / WAVE;
    const unsigned grid = unsigned(1 + (a.T * n + 8 * WAVE - 1) / (8 * WAVE));
    if (per <= 1) route_shgate_kernel<1><<<grid, 8 * WAVE, 0, s>>>(a, sh.v, n, h);
    else if (per <= 2) route_shgate_kernel<2><<<grid, 8 * WAVE, 0, s>>>(a, sh.v, n, h);
    else if (per <= 4) route_shgate_kernel<4><<<grid, 8 * WAVE, 0, s>>>(a, sh.v, n, h);
    else route_shgate_kernel<8><<<grid, 8 * WAVE, 0, s>>>(a, sh.v, n, h);
    return true;
}

// out[t][j] = shared[t][j] + sum_i w[t][i] * yp[slot[t][i]][j], i in selection
// order (src/kernels/moe_route.hip:168-185, 201-224). 4 columns per thread.
// C consecutive groups of 4 elements of a yp row (fp32, or fp16 with YP16):
// one 16-byte load per 4 fp32 values or per 8 fp16 values.
template <bool YP16, int C>
__device__ __forceinline__ void yp_row(const void *yp, int64_t row, int H, int j, float4 (&v)[C]) {
    if constexpr (YP16) {
        const uint16_t *p = static_cast<const uint16_t *>(yp) + row * H + j;
        uint32_t u[2 * C];
        if constexpr (C == 2) {
            const uint4 q = *reinterpret_cast<const uint4 *>(p);
            u[0] = q.x, u[1] = q.y, u[2] = q.z, u[3] = q.w;
        } else {
            const uint2 q = *reinterpret_cast<const uint2 *>(p);
            u[0] = q.x, u[1] = q.y;
        }
#pragma unroll
        for (int c = 0; c < C; ++c)
            v[c] = make_float4(f16_bits_to_f32(uint16_t(u[2 * c])), f16_bits_to_f32(uint16_t(u[2 * c] >> 16)),
                               f16_bits_to_f32(uint16_t(u[2 * c + 1])), f16_bits_to_f32(uint16_t(u[2 * c + 1] >> 16)));
    } else {
#pragma unroll
        for (int c = 0; c < C; ++c) v[c] = *reinterpret_cast<const float4 *>(static_cast<const float *>(yp) + row * H + j + 4 * c);
    }
}

// 4 C consecutive elements of a shared row (fp32, or fp16 with SH16).
template <bool SH16, int C>
__device__ __forceinline__ void shared_row(const void *shared, int64_t off, float4 (&v)[C]) {
    if constexpr (SH16) {
        const uint16_t *p = static_cast<const uint16_t *>(shared) + off;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const uint2 q = *reinterpret_cast<const uint2 *>(p + 4 * c);
            v[c] = make_float4(f16_bits_to_f32(uint16_t(q.x)), f16_bits_to_f32(uint16_t(q.x >> 16)),
                               f16_bits_to_f32(uint16_t(q.y)), f16_bits_to_f32(uint16_t(q.y >> 16)));
        }
    } else {
#pragma unroll
        for (int c = 0; c < C; ++c) v[c] = *reinterpret_cast<const float4 *>(static_cast<const float *>(shared) + off + 4 * c);
    }
}

// Four fp32 values -> 4 elements of type OT (QW_T_* numbering: 0 fp32,
// 1 bf16 round to nearest even, 2 fp16 round to nearest even with finite
// values beyond +-65504 saturated) at o.
template <int OT>
__device__ __forceinline__ void store4(void *out, int64_t o, float4 v) {
    if constexpr (OT == 0) {
        *reinterpret_cast<float4 *>(static_cast<float *>(out) + o) = v;
    } else {
        auto cv = [](float f) -> uint32_t {
            if constexpr (OT == 1) return f32_to_bf16_rne(f);
            else return __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(f));
        };
        uint2 pk;
        pk.x = cv(v.x) | (cv(v.y) << 16);
        pk.y = cv(v.z) | (cv(v.w) << 16);
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(out) + o) = pk;
    }
}

// out[t][j] = shared[t][j] + sum_i w_i yp[slot_i][j], selections in order;
// a thread takes 4 C consecutive elements (C = 2 where H allows: 16-byte
// loads of fp16 rows). A negative slot (a selection held by another rank in
// the reference's expert-parallel layout) adds nothing.
template <bool YP16, int C, bool SH16, int OT>
__global__ __launch_bounds__(256) void combine_kernel(const void *__restrict__ yp, const int32_t *__restrict__ tok_slot,
                                                      const float *__restrict__ tok_w, const void *__restrict__ shared,
                                                      int k, int H, void *__restrict__ out) {
    const int t = blockIdx.x, j = (blockIdx.y * 256 + threadIdx.x) * 4 * C;
    if (j >= H) return;
    float4 acc[C];
    if (shared) shared_row<SH16, C>(shared, int64_t(t) * H + j, acc);
    else
#pragma unroll
        for (int c = 0; c < C; ++c) acc[c] = make_float4(0, 0, 0, 0);
    // up to 8 selections' rows requested together, then added in selection
    // order (the same sums as one at a time)
    for (int i0 = 0; i0 < k; i0 += 8) {
        float4 v[8][C];
        float w[8];
        int sl[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = min(i0 + u, k - 1);
            w[u] = tok_w[t * k + i];
            sl[u] = tok_slot[t * k + i];
            yp_row<YP16, C>(yp, int64_t(max(sl[u], 0)), H, j, v[u]);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (i0 + u < k && sl[u] >= 0) {
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    acc[c].x += w[u] * v[u][c].x;
                    acc[c].y += w[u] * v[u][c].y;
                    acc[c].z += w[u] * v[u][c].z;
                    acc[c].w += w[u] * v[u][c].w;
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) store4<OT>(out, int64_t(t) * H + j + 4 * c, acc[c]);
}

template <bool YP16, int C, bool SH16>
static void launch_combine_o(const void *yp, const int32_t *tok_slot, const float *tok_w, const void *shared, int T,
                             int topk, int H, void *out, int out_type, hipStream_t s) {
    const dim3 grid(unsigned(T), unsigned((H / (4 * C) + 255) / 256));
    if (out_type == 1) combine_kernel<YP16, C, SH16, 1><<<grid, 256, 0, s>>>(yp, tok_slot, tok_w, shared, topk, H, out);
    else if (out_type == 2) combine_kernel<YP16, C, SH16, 2><<<grid, 256, 0, s>>>(yp, tok_slot, tok_w, shared, topk, H, out);
    else combine_kernel<YP16, C, SH16, 0><<<grid, 256, 0, s>>>(yp, tok_slot, tok_w, shared, topk, H, out);
}

template <bool YP16, int C>
static void launch_combine_s(const void *yp, const int32_t *tok_slot, const float *tok_w, const void *shared,
                             int shared_f16, int T, int topk, int H, void *out, int out_type, hipStream_t s) {
    if (shared_f16) launch_combine_o<YP16, C, true>(yp, tok_slot, tok_w, shared, T, topk, H, out, out_type, s);
    else launch_combine_o<YP16, C, false>(yp, tok_slot, tok_w, shared, T, topk, H, out, out_type, s);
}

void launch_combine(const void *yp, int yp_f16, const int32_t *tok_slot, const float *tok_w, const void *shared,
                    int shared_f16, int T, int topk, int H, void *out, int out_type, hipStream_t s) {
    if (H % 8 == 0) {
        if (yp_f16) launch_combine_s<true, 2>(yp, tok_slot, tok_w, shared, shared_f16, T, topk, H, out, out_type, s);
        else launch_combine_s<false, 2>(yp, tok_slot, tok_w, shared, shared_f16, T, topk, H, out, out_type, s);
    } else {
        if (yp_f16) launch_combine_s<true, 1>(yp, tok_slot, tok_w, shared, shared_f16, T, topk, H, out, out_type, s);
        else launch_combine_s<false, 1>(yp, tok_slot, tok_w, shared, shared_f16, T, topk, H, out, out_type, s);
    }
}

}  // namespace qwq4
