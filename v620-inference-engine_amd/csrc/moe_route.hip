// MoE routing, gather indices and the weighted combine.
//
// Reference: the math of ref::Model::moe (src/ref/ref_model.cpp:412-431) and
// the deterministic slot order of gpu::moe_route_B
// (src/kernels/moe_route.hip:65-165), for any batch: decode rows and 4096-token
// prefill chunks use the same code (the reference's prefill scatter,
// moe_route.hip:28-58, fills slots with atomics and is nondeterministic; this
// one is not).
//
//   p_e      = float(exp(l_e - max l))                      per token
//   top k    by (p descending, expert index ascending)
//   w_i      = float(double(p_i) / sum_{j<k} double(p_j))    sum in selection order
//   slots    experts ascending; within an expert, tokens ascending
//
// exp is evaluated in double and rounded once to float, i.e. the correctly
// rounded expf the CPU path uses, so selection and weights match it bit for
// bit.
#include <climits>

#include "q4_common.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

constexpr int MAX_PER = 16;  // logits per lane: E <= 1024

// One wave routes one token. Lane j < k ends with the j-th selection.
__device__ __forceinline__ void topk_wave(const float *l, int E, int k, int lane, int32_t *te, float *tw) {
    float p[MAX_PER];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < MAX_PER; ++i) {
        const int idx = lane + WAVE * i;
        p[i] = idx < E ? l[idx] : -INFINITY;
        mx = fmaxf(mx, p[i]);
    }
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, WAVE));
#pragma unroll
    for (int i = 0; i < MAX_PER; ++i) {
        const int idx = lane + WAVE * i;
        p[i] = idx < E ? float(exp(double(p[i] - mx))) : -2.f;
    }
    double top = 0.0;
    int my_e = 0;
    float my_p = 0.f;
    for (int j = 0; j < k; ++j) {
        float bv = -3.f;
        int bi = INT_MAX;
#pragma unroll
        for (int i = 0; i < MAX_PER; ++i)
            if (p[i] > bv) {  // ascending index within the lane: the first maximum wins
                bv = p[i];
                bi = lane + WAVE * i;
            }
#pragma unroll
        for (int o = WAVE / 2; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, WAVE);
            const int oi = __shfl_xor(bi, o, WAVE);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if ((bi % WAVE) == lane) {
#pragma unroll
            for (int i = 0; i < MAX_PER; ++i)
                if (i == bi / WAVE) p[i] = -1.f;
        }
        top += double(bv);
        if (lane == j) {
            my_e = bi;
            my_p = bv;
        }
    }
    if (lane < k) {
        te[lane] = my_e;
        tw[lane] = float(double(my_p) / top);
    }
}

__global__ __launch_bounds__(256) void route_topk_kernel(const float *__restrict__ logits, int T, int E, int k,
                                                         int32_t *__restrict__ top_e, float *__restrict__ top_w) {
    const int t = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (t >= T) return;
    topk_wave(logits + int64_t(t) * E, E, k, lane, top_e + int64_t(t) * k, top_w + int64_t(t) * k);
}

struct SlotLds {
    int32_t *cnt, *off;
    unsigned long long *mask;  // [16 waves][E]
    uint16_t *cc;              // [chunks][E]
};

__host__ __device__ inline size_t slot_lds_layout(int T, int E, SlotLds *p, unsigned char *base) {
    const size_t n_chunks = size_t(T + WAVE - 1) / WAVE;
    size_t o = 0;
    const size_t cnt = o;
    o += size_t(E) * 4;
    const size_t off = o;
    o += size_t(E + 1) * 4;
    o = (o + 7) & ~size_t(7);
    const size_t mask = o;
    o += size_t(16) * E * 8;
    const size_t cc = o;
    o += n_chunks * E * 2;
    if (p) {
        p->cnt = reinterpret_cast<int32_t *>(base + cnt);
        p->off = reinterpret_cast<int32_t *>(base + off);
        p->mask = reinterpret_cast<unsigned long long *>(base + mask);
        p->cc = reinterpret_cast<uint16_t *>(base + cc);
    }
    return o;
}

size_t route_lds_bytes(int T, int E) { return slot_lds_layout(T, E, nullptr, nullptr); }

// counts, offsets, active list, tile list and slots from the selections te
// (LDS or global). Whole block (1024 threads) participates.
__device__ void route_slots(const int32_t *te, const RouteArgs &a, SlotLds L) {
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int T = a.T, E = a.E, k = a.topk, P = T * k;
    for (int e = tid; e < E; e += blockDim.x) L.cnt[e] = 0;
    for (int i = tid; i < 16 * E; i += blockDim.x) L.mask[i] = 0ull;
    __syncthreads();
    for (int i = tid; i < P; i += blockDim.x) atomicAdd(&L.cnt[te[i]], 1);
    __syncthreads();
    if (wave == 0) {  // three exclusive scans over the experts: pairs, non-empty experts, tiles
        const int per = (E + WAVE - 1) / WAVE, e0 = lane * per;
        int c_pairs = 0, c_act = 0, c_tiles = 0;
        for (int i = 0; i < per; ++i) {
            const int e = e0 + i;
            if (e < E) {
                const int c = L.cnt[e];
                c_pairs += c;
                c_act += c > 0;
                c_tiles += a.tile_m > 0 ? (c + a.tile_m - 1) / a.tile_m : 0;
            }
        }
        int ip = c_pairs, ia = c_act, it = c_tiles;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            const int np = __shfl_up(ip, o, WAVE), na = __shfl_up(ia, o, WAVE), nt = __shfl_up(it, o, WAVE);
            if (lane >= o) {
                ip += np;
                ia += na;
                it += nt;
            }
        }
        int rp = ip - c_pairs, ra = ia - c_act, rt = it - c_tiles;
        for (int i = 0; i < per; ++i) {
            const int e = e0 + i;
            if (e >= E) break;
            const int c = L.cnt[e];
            L.off[e] = rp;
            a.offsets[e] = rp;
            a.counts[e] = c;
            if (c > 0) a.active[ra++] = e;
            if (a.tile_m > 0)
                for (int m0 = 0; m0 < c; m0 += a.tile_m) {
                    a.tile_e[rt] = e;
                    a.tile_m0[rt] = m0;
                    ++rt;
                }
            rp += c;
        }
        if (lane == WAVE - 1) {
            L.off[E] = rp;
            a.offsets[E] = rp;
            *a.n_active = ra;
            if (a.tile_m > 0) *a.n_tiles = rt;
        }
    }
    __syncthreads();
    // per-chunk (64 tokens) counts of every expert, then their exclusive
    // prefix over chunks, then each pair's rank inside its chunk from a bitmask
    const int n_chunks = (T + WAVE - 1) / WAVE, rounds = (n_chunks + 15) / 16;
    unsigned long long *M = L.mask + size_t(wave) * E;
    for (int pass = 0; pass < 2; ++pass) {
        for (int r = 0; r < rounds; ++r) {
            const int c = r * 16 + wave, t = c * WAVE + lane;
            if (c < n_chunks && t < T)
                for (int j = 0; j < k; ++j) atomicOr(&M[te[t * k + j]], 1ull << lane);
            __syncthreads();
            if (c < n_chunks) {
                if (pass == 0) {
                    for (int e = lane; e < E; e += WAVE) L.cc[size_t(c) * E + e] = uint16_t(__popcll(M[e]));
                } else if (t < T) {
                    const unsigned long long below = (1ull << lane) - 1ull;
                    for (int j = 0; j < k; ++j) {
                        const int e = te[t * k + j];
                        const int slot = L.off[e] + L.cc[size_t(c) * E + e] + __popcll(M[e] & below);
                        a.tok_slot[t * k + j] = slot;
                        a.pair_tok[slot] = t;
                    }
                }
            }
            __syncthreads();
            for (int e = lane; e < E; e += WAVE) M[e] = 0ull;
            __syncthreads();
        }
        if (pass == 0) {
            for (int e = tid; e < E; e += blockDim.x) {
                int run = 0;
                for (int c = 0; c < n_chunks; ++c) {
                    const int v = L.cc[size_t(c) * E + e];
                    L.cc[size_t(c) * E + e] = uint16_t(run);
                    run += v;
                }
            }
            __syncthreads();
        }
    }
}

// Decode batches (T <= 64): selections and slots in one launch. A token
// picks an expert at most once, so the tokens of expert e are the set bits of
// one 64-bit mask; a pair's rank among them is a popcount below its bit.
__global__ __launch_bounds__(1024) void route_small_kernel(RouteArgs a) {
    __shared__ int32_t s_te[64 * 64];
    __shared__ unsigned long long s_mask[1024];
    __shared__ int32_t s_off[1024];
    __shared__ int32_t s_sum[16][3];
    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int T = a.T, E = a.E, k = a.topk, P = T * k;
    if (tid < E) s_mask[tid] = 0ull;
    for (int t = wave; t < T; t += 16)
        topk_wave(a.logits + int64_t(t) * E, E, k, lane, s_te + t * k, a.top_w + int64_t(t) * k);
    __syncthreads();
    for (int i = tid; i < P; i += blockDim.x) {
        a.top_e[i] = s_te[i];
        atomicOr(&s_mask[s_te[i]], 1ull << (i / k));
    }
    __syncthreads();
    // exclusive scans over the experts (one per thread): pairs, non-empty
    // experts, tiles
    const int c = tid < E ? __popcll(s_mask[tid]) : 0;
    const int v[3] = {c, c > 0, a.tile_m > 0 ? (c + a.tile_m - 1) / a.tile_m : 0};
    int inc[3] = {v[0], v[1], v[2]};
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int u = __shfl_up(inc[j], o, WAVE);
            if (lane >= o) inc[j] += u;
        }
    }
    if (lane == WAVE - 1) {
#pragma unroll
        for (int j = 0; j < 3; ++j) s_sum[wave][j] = inc[j];
    }
    __syncthreads();
    int ex[3] = {inc[0] - v[0], inc[1] - v[1], inc[2] - v[2]};
    for (int w = 0; w < wave; ++w) {
#pragma unroll
        for (int j = 0; j < 3; ++j) ex[j] += s_sum[w][j];
    }
    if (tid < E) {
        s_off[tid] = ex[0];
        a.offsets[tid] = ex[0];
        a.counts[tid] = c;
        if (c > 0) a.active[ex[1]] = tid;
        for (int j = 0; j < v[2]; ++j) {
            a.tile_e[ex[2] + j] = tid;
            a.tile_m0[ex[2] + j] = j * a.tile_m;
        }
        if (tid == E - 1) {
            a.offsets[E] = ex[0] + c;
            *a.n_active = ex[1] + v[1];
            if (a.tile_m > 0) *a.n_tiles = ex[2] + v[2];
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

__global__ __launch_bounds__(1024) void route_slots_kernel(RouteArgs a) {
    extern __shared__ unsigned char smem[];
    SlotLds L;
    slot_lds_layout(a.T, a.E, &L, smem);
    route_slots(a.top_e, a, L);
}

void launch_route(const RouteArgs &a, hipStream_t s) {
    const size_t lds = route_lds_bytes(a.T, a.E);
    if (a.T <= 64) {
        route_small_kernel<<<1, 1024, 0, s>>>(a);
    } else {
        if (lds > 48 * 1024)
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(route_slots_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        route_topk_kernel<<<(a.T + 3) / 4, 256, 0, s>>>(a.logits, a.T, a.E, a.topk, a.top_e, a.top_w);
        route_slots_kernel<<<1, 1024, lds, s>>>(a);
    }
}

// out[t][j] = shared[t][j] + sum_i w[t][i] * yp[slot[t][i]][j], i in selection
// order (src/kernels/moe_route.hip:168-185, 201-224). 4 columns per thread.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ yp, const int32_t *__restrict__ tok_slot,
                                                      const float *__restrict__ tok_w, const float *__restrict__ shared,
                                                      int k, int H, void *__restrict__ out, int out_bf16) {
    const int t = blockIdx.x, j = (blockIdx.y * 256 + threadIdx.x) * 4;
    if (j >= H) return;
    float4 acc = shared ? *reinterpret_cast<const float4 *>(shared + int64_t(t) * H + j) : make_float4(0, 0, 0, 0);
    for (int i = 0; i < k; ++i) {
        const int slot = tok_slot[t * k + i];
        const float w = tok_w[t * k + i];
        const float4 v = *reinterpret_cast<const float4 *>(yp + int64_t(slot) * H + j);
        acc.x += w * v.x;
        acc.y += w * v.y;
        acc.z += w * v.z;
        acc.w += w * v.w;
    }
    if (out_bf16) {
        uint16_t *o = static_cast<uint16_t *>(out) + int64_t(t) * H + j;
        uint2 pk;
        pk.x = uint32_t(f32_to_bf16_rne(acc.x)) | (uint32_t(f32_to_bf16_rne(acc.y)) << 16);
        pk.y = uint32_t(f32_to_bf16_rne(acc.z)) | (uint32_t(f32_to_bf16_rne(acc.w)) << 16);
        *reinterpret_cast<uint2 *>(o) = pk;
    } else {
        *reinterpret_cast<float4 *>(static_cast<float *>(out) + int64_t(t) * H + j) = acc;
    }
}

void launch_combine(const float *yp, const int32_t *tok_slot, const float *tok_w, const float *shared, int T, int topk,
                    int H, void *out, int out_bf16, hipStream_t s) {
    const dim3 grid(unsigned(T), unsigned((H / 4 + 255) / 256));
    combine_kernel<<<grid, 256, 0, s>>>(yp, tok_slot, tok_w, shared, topk, H, out, out_bf16);
}

}  // namespace qwq4
