// Gathered per-expert q4 GEMVs for routed decode tokens (reference role:
// gpu::moe_experts_P, src/kernels/moe_experts.hip:177-245; arithmetic of
// ref::Model::moe, src/ref/ref_model.cpp:434-463).
//
// grid (row blocks of one expert, max active experts). Block y serves the
// y-th expert with tokens (active[] ascending); its M tokens are the slots
// offsets[e] .. offsets[e+1]-1, slot p carrying token pair_tok[p]. Expert e's
// weights are rows e*F .. of the stacked [E*F][H] gate and up matrices and
// rows e*H .. of the [E*H][F] down matrix (tiled format).
//
// The block runs over the expert's tokens in chunks of R rows (as many as fit
// the LDS budget; with decode batches nearly every expert has one chunk, so
// its weights come from HBM once per call however many tokens chose it). Per
// chunk each wave requests its whole K range of one subtile up front, the
// chunk's rows (x gathered through pair_tok, or h) go to LDS by direct loads,
// every wave multiplies, and the KS partial sums of each subtile are reduced
// through LDS in a fixed order.
//   gate/up  waves = subtiles x {gate, up} x KS; the reducing wave also
//            forms h = silu(g) * u (fp16, saturated, the reference's fp16
//            intermediate) from the two sums it holds.
//   down     waves = subtiles x KS; yp fp32, or fp16 (YP16: rounded to
//            nearest even, finite values beyond +-65504 saturated; the
//            reference's moe_experts_P output).
#include <type_traits>

#include "q4_gemv_core.cuh"
#include "q4_kernels.hpp"
#include "route_core.cuh"
#include "w16_core.cuh"

namespace qwq4 {

__host__ __device__ inline size_t moe_lds_bytes(int R, int K) {
    return size_t(x_pieces(R, K)) * 16 + size_t(8) * WAVE * 16;
}

__device__ __forceinline__ uint16_t silu_mul_f16(float g, float u) {
    return __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(silu_ref(g) * u));
}

// yp element as stored: the fp32 sum, or its fp16 rounding (YP16) as a
// float, so a fused combine adds exactly what the unfused one reads back.
template <bool YP16>
__device__ __forceinline__ float yp_value(float v) {
    if constexpr (YP16) return float(f32_to_f16_satfinite(v));
    else return v;
}

template <bool YP16>
__device__ __forceinline__ void store_yp(void *yp, int64_t i, float v) {
    if constexpr (YP16) static_cast<uint16_t *>(yp)[i] = __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(v));
    else static_cast<float *>(yp)[i] = v;
}

// The fused combine's output element (type c.out_type: 0 fp32, 1 bf16,
// 2 fp16 saturated).
__device__ __forceinline__ void store_out(const CombineArgs &c, int64_t i, float v) {
    if (c.out_type == 1) static_cast<uint16_t *>(c.out)[i] = f32_to_bf16_rne(v);
    else if (c.out_type == 2) static_cast<uint16_t *>(c.out)[i] = __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(v));
    else static_cast<float *>(c.out)[i] = v;
}

// A wave-uniform read of routing data through the scalar cache (the
// constant address space): counted apart from the vector loads, so waiting
// for it does not wait for the weight requests issued before it (vector
// loads complete in order: a vector load of a token index issued after the
// weights would hold the activation rows back until every weight word had
// arrived).
__device__ __forceinline__ int ld_uniform(const int32_t *p, int i) {
    typedef const __attribute__((address_space(4))) int32_t cint;
    return ((cint *)(p))[__builtin_amdgcn_readfirstlane(i)];
}

__device__ __forceinline__ float ld_uniform_f32(const float *p, int i) {
    typedef const __attribute__((address_space(4))) float cfloat;
    return ((cfloat *)(p))[__builtin_amdgcn_readfirstlane(i)];
}

// Reads the block's expert: n_active and active[y] are requested together
// (one latency), and the weight loads need only e.
// (by: the block's active-expert rank)
__device__ __forceinline__ int block_expert_at(const int32_t *n_active, const int32_t *active, int E, int by) {
    const int na = ld_uniform(n_active, 0), e = ld_uniform(active, by);
    return by < na ? min(max(e, 0), E - 1) : -1;
}

__device__ __forceinline__ int block_expert(const int32_t *n_active, const int32_t *active, int E) {
    return block_expert_at(n_active, active, E, int(blockIdx.y));
}

// (bx, by): the block's column block and active-expert rank (arguments, so
// that a kernel running other work in the same grid can call it)
template <typename XT, int KS, int GW, bool HAS_Z, bool CH4, bool MULTI>
__device__ __forceinline__ void moe_gate_up_gemv_block(
    const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us,
    const uint16_t *uz, const int32_t *__restrict__ offsets, const int32_t *__restrict__ active,
    const int32_t *__restrict__ n_active, const int32_t *__restrict__ pair_tok, const uint16_t *__restrict__ x, int E,
    int H, int F, int R, uint16_t *__restrict__ h, int bx, int by) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int e = block_expert_at(n_active, active, E, by);
    if (e < 0) return;
    constexpr int SUB = 8 / (2 * KS);
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE, q = lane / 16,
              n = lane % 16;
    const int sl = wave / (2 * KS), mat = (wave / KS) % 2, kp = wave % KS;
    const int G = H / QGROUP, gpk = G / KS, fsub = F / 16, kc = x_row_stride(H);
    const int lsub = bx * SUB + sl;
    const int64_t sub = int64_t(e) * fsub + min(lsub, fsub - 1);
    const Q4Tile t = mat ? Q4Tile(uw, us, uz, sub, G) : Q4Tile(gw, gs, gz, sub, G);
    // the first chunk's weights go out before the slot range is known (an
    // active expert has at least one token)
    WaveRange<GW, HAS_Z, CH4> wr;
    wr.fetch(t, kp * gpk, gpk, opaque_lane());
    const int base = ld_uniform(offsets, e), M = ld_uniform(offsets, e + 1) - base;
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    f32x4 *red = reinterpret_cast<f32x4 *>(xl + x_pieces(R, H));
    // one chunk of mc rows from slot base + m0 (weights in wr)
    auto chunk = [&](int m0) {
        const int mc = min(R, M - m0);
        // (stage_rows_issue asks for one row at a time, wave-uniform, when a
        // row is whole waves of 16-byte pieces; else per lane)
        const bool rows_uniform = (H / 8) % WAVE == 0;
        stage_rows_issue(
            [&](int m) {
                const int i = base + m0 + m;
                return x + int64_t(rows_uniform ? ld_uniform(pair_tok, i) : pair_tok[i]) * H;
            },
            mc, H, xl);
        __syncthreads();
        const uint4 *xr[1] = {xl + min(n, mc - 1) * kc + q * 4};
        f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
        compute_zq_inline<XT>(wr, xr[0], acc[0]);
        red[wave * WAVE + lane] = acc[0];
        lds_barrier();
        if (mat == 0 && kp == 0 && lsub < fsub) {
            f32x4 g = red[wave * WAVE + lane], u = red[(wave + KS) * WAVE + lane];
#pragma unroll
            for (int j = 1; j < KS; ++j) {
                g += red[(wave + j) * WAVE + lane];
                u += red[(wave + KS + j) * WAVE + lane];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * q + r;
                if (m < mc) h[int64_t(base + m0 + m) * F + lsub * 16 + n] = silu_mul_f16(g[r], u[r]);
            }
        }
    };
    // the first chunk (its weights are already requested; M >= 1), then,
    // when an expert can have more than R tokens (MULTI), further ones, each
    // refetching its weights (from L2). Without that loop the kernel needs 72
    // VGPRs instead of 88, so a batch-1 grid (768 blocks) is resident in one
    // round.
    chunk(0);
    if constexpr (MULTI) {
        for (int m0 = R; m0 < M; m0 += R) {
            wr.fetch(t, kp * gpk, gpk, opaque_lane());
            lds_barrier();  // the previous chunk's rows and partials are consumed
            chunk(m0);
        }
    }
}

template <typename XT, int KS, int GW, bool HAS_Z, bool CH4, bool MULTI>
__global__ __launch_bounds__(512) void moe_gate_up_gemv_kernel(
    const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us,
    const uint16_t *uz, const int32_t *__restrict__ offsets, const int32_t *__restrict__ active,
    const int32_t *__restrict__ n_active, const int32_t *__restrict__ pair_tok, const uint16_t *__restrict__ x, int E,
    int H, int F, int R, uint16_t *__restrict__ h) {
    moe_gate_up_gemv_block<XT, KS, GW, HAS_Z, CH4, MULTI>(gw, gs, gz, uw, us, uz, offsets, active, n_active, pair_tok,
                                                          x, E, H, F, R, h, int(blockIdx.x), int(blockIdx.y));
}

// Batches of up to 4 tokens: every token row goes to LDS first (row t at
// t * kc, direct loads, issued before anything waits), then the expert's
// weights; the compute then waits only for the weights, group by group as
// they arrive, instead of for all of them behind the rows of the expert's
// tokens. The MFMA's token row n reads row pair_tok[base + n].
template <typename XT, int KS, int GW, bool HAS_Z, bool CH4>
__global__ __launch_bounds__(512) void moe_gate_up_small_kernel(
    const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us,
    const uint16_t *uz, const int32_t *__restrict__ offsets, const int32_t *__restrict__ active,
    const int32_t *__restrict__ n_active, const int32_t *__restrict__ pair_tok, const uint16_t *__restrict__ x, int E,
    int H, int F, int T, uint16_t *__restrict__ h) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    stage_rows_issue([&](int m) { return x + int64_t(m) * H; }, T, H, xl);
    __builtin_amdgcn_sched_barrier(0);
    const int e = block_expert(n_active, active, E);
    if (e < 0) {
        wait_vm_below<0>();  // the rows' direct loads land before the block's LDS is released
        return;
    }
    constexpr int SUB = 8 / (2 * KS);
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE, q = lane / 16,
              n = lane % 16;
    const int sl = wave / (2 * KS), mat = (wave / KS) % 2, kp = wave % KS;
    const int G = H / QGROUP, gpk = G / KS, fsub = F / 16, kc = x_row_stride(H);
    const int lsub = blockIdx.x * SUB + sl;
    const int64_t sub = int64_t(e) * fsub + min(lsub, fsub - 1);
    const Q4Tile tl = mat ? Q4Tile(uw, us, uz, sub, G) : Q4Tile(gw, gs, gz, sub, G);
    WaveRange<GW, HAS_Z, CH4> wr;
    wr.fetch(tl, kp * gpk, gpk, opaque_lane());
    const int base = ld_uniform(offsets, e), M = ld_uniform(offsets, e + 1) - base;
    int tok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) tok[i] = ld_uniform(pair_tok, base + min(i, M - 1));
    f32x4 *red = reinterpret_cast<f32x4 *>(xl + x_pieces(T, H));
    const int mr = min(n, M - 1);
    const int trow = mr == 0 ? tok[0] : mr == 1 ? tok[1] : mr == 2 ? tok[2] : tok[3];
    const uint4 *xr = xl + trow * kc + q * 4;
    // the rows (this wave's oldest loads) of every wave, not the weights
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_below<WaveRange<GW, HAS_Z, CH4>::LOADS>();
    __builtin_amdgcn_s_barrier();
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    compute_zq_inline<XT>(wr, xr, acc);
    red[wave * WAVE + lane] = acc;
    lds_barrier();
    if (mat == 0 && kp == 0 && lsub < fsub) {
        f32x4 g = red[wave * WAVE + lane], u = red[(wave + KS) * WAVE + lane];
#pragma unroll
        for (int j = 1; j < KS; ++j) {
            g += red[(wave + j) * WAVE + lane];
            u += red[(wave + KS + j) * WAVE + lane];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * q + r;
            if (m < M) h[int64_t(base + m) * F + lsub * 16 + n] = silu_mul_f16(g[r], u[r]);
        }
    }
}

// ---- decode batches that route themselves (the kernel takes T <= 4, k <= 8:
// at most 32 selections; moe_local_route_ok picks where it pays). The router
// launch then only writes the logits, with no
// cross-block hand-off (its counted last block, reload and routing took
// about 4 us of the batch-1 block), and every gate/up block routes the batch
// from the logits before its weight requests: wave t < T picks token t's
// top k (topk_wave, the routing kernels' code: the C library's expf, order
// (p desc, index asc), weights renormalised in double), then every wave
// derives the slots from the selections in LDS. A selection (t, j) of
// expert e gets the slot off(e) + #(earlier tokens of e), off(e) = the
// selections of smaller experts: experts ascending, tokens ascending, the
// order of the routing kernels. Block y serves the y-th active expert
// (ascending); block (0, 0) writes the routing outputs for the down
// projection, the combine and the caller.
struct LocalRoute {
    const float *logits;  // [T][E]
    int32_t *top_e, *tok_slot, *pair_tok, *offsets, *active, *n_active;
    float *top_w;
};

// One wave's view of the batch's routing: lane i < P holds selection i
// (token i / k): its expert, slot, and whether it is its expert's first
// selection (then act is the expert's rank among the active ones and cnt
// its number of tokens).
struct LaneRoute {
    int e, slot, act, cnt;
    bool first;
};

__device__ __forceinline__ LaneRoute lane_route(const int32_t *s_te, int P, int k, int lane) {
    LaneRoute r;
    const bool live = lane < P;
    r.e = live ? s_te[lane] : 0x7fffffff;
    const int t = lane / k;  // (one division; the loop reads the other lanes' tokens)
    int off = 0, rank = 0, cnt = 0;
    for (int l = 0; l < P; ++l) {
        const int el = __builtin_amdgcn_readlane(r.e, l), tl = __builtin_amdgcn_readlane(t, l);
        off += el < r.e;
        rank += el == r.e && tl < t;
        cnt += el == r.e;
    }
    r.first = live && rank == 0;
    const uint64_t fm = __ballot(r.first);
    int act = 0;
    for (int l = 0; l < P; ++l) {
        const int el = __builtin_amdgcn_readlane(r.e, l);
        act += ((fm >> l) & 1ull) && el < r.e;
    }
    r.slot = off + rank;
    r.act = act;
    r.cnt = cnt;
    return r;
}

// (bx, by): the block's column block and active-expert rank (arguments, so
// that a kernel running other work in the same grid can call it)
template <typename XT, int KS, int GW, bool HAS_Z, bool CH4, int PER>
__device__ __forceinline__ void moe_gate_up_routed_block(const uint32_t *gw, const uint16_t *gs, const uint16_t *gz,
                                                         const uint32_t *uw, const uint16_t *us, const uint16_t *uz,
                                                         const LocalRoute &lr, const uint16_t *__restrict__ x, int E,
                                                         int H, int F, int T, int k, uint16_t *__restrict__ h, int bx,
                                                         int by) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int32_t s_te[64];
    __shared__ float s_tw[64];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE, q = lane / 16,
              n = lane % 16;
    const int P = T * k;
    // every token row goes to LDS first (direct loads, row t at t * kc), in
    // flight while the batch is routed: the weights then are the only loads
    // the compute waits for, group by group as they arrive
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    stage_rows_issue([&](int m) { return x + int64_t(m) * H; }, T, H, xl);
    if (wave < T) {
        ExpfGlibc ex;
        ex.load(lane);
        const float *l = lr.logits + int64_t(wave) * E;
        topk_wave<PER>(ex, [&](int i) { return l[i]; }, E, k, lane, s_te + wave * k, s_tw + wave * k);
    }
    __syncthreads();
    const LaneRoute rt = lane_route(s_te, P, k, lane);
    const uint64_t mine = __ballot(rt.first && rt.act == by);
    const int n_act = __popcll(__ballot(rt.first));  // (every lane takes part in the ballot)
    if (bx == 0 && by == 0 && wave == 0) {
        if (lane < P) {
            lr.top_e[lane] = rt.e;
            lr.top_w[lane] = s_tw[lane];
            lr.tok_slot[lane] = rt.slot;
            lr.pair_tok[rt.slot] = lane / k;
            if (rt.first) {
                lr.active[rt.act] = rt.e;
                lr.offsets[rt.e] = rt.slot;
                lr.offsets[rt.e + 1] = rt.slot + rt.cnt;
            }
        }
        if (lane == 0) *lr.n_active = n_act;
    }
    if (mine == 0ull) return;  // fewer active experts than blocks
    const int src = __builtin_ctzll(mine);
    const int e = __builtin_amdgcn_readlane(rt.e, src), M = __builtin_amdgcn_readlane(rt.cnt, src);
    constexpr int SUB = 8 / (2 * KS);
    const int sl = wave / (2 * KS), mat = (wave / KS) % 2, kp = wave % KS;
    const int G = H / QGROUP, gpk = G / KS, fsub = F / 16, kc = x_row_stride(H);
    const int lsub = bx * SUB + sl;
    const int64_t sub = int64_t(e) * fsub + min(lsub, fsub - 1);
    const Q4Tile tl = mat ? Q4Tile(uw, us, uz, sub, G) : Q4Tile(gw, gs, gz, sub, G);
    WaveRange<GW, HAS_Z, CH4> wr;
    wr.fetch(tl, kp * gpk, gpk, opaque_lane());
    const int base = __builtin_amdgcn_readlane(rt.slot, src);
    // the expert's tokens in slot order: its selections' lanes ascending
    // (lane = t k + j, so ascending lanes are ascending tokens)
    const uint64_t em = __ballot(lane < P && rt.e == e);
    int tok[4];
    {
        uint64_t m = em;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tok[i] = m ? __builtin_ctzll(m) / k : 0;
            m &= m - 1;
        }
    }
    f32x4 *red = reinterpret_cast<f32x4 *>(xl + x_pieces(T, H));
    // the lane's token row: the expert's (min(n, M - 1))-th token
    const int mr = min(n, M - 1);
    const int trow = mr == 0 ? tok[0] : mr == 1 ? tok[1] : mr == 2 ? tok[2] : tok[3];
    const uint4 *xr = xl + trow * kc + q * 4;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    compute_zq_inline<XT>(wr, xr, acc);
    red[wave * WAVE + lane] = acc;
    lds_barrier();
    if (mat == 0 && kp == 0 && lsub < fsub) {
        f32x4 g = red[wave * WAVE + lane], u = red[(wave + KS) * WAVE + lane];
#pragma unroll
        for (int j = 1; j < KS; ++j) {
            g += red[(wave + j) * WAVE + lane];
            u += red[(wave + KS + j) * WAVE + lane];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * q + r;
            if (m < M) h[int64_t(base + m) * F + lsub * 16 + n] = silu_mul_f16(g[r], u[r]);
        }
    }
}

template <typename XT, int KS, int GW, bool HAS_Z, bool CH4, int PER>
__global__ __launch_bounds__(512) void moe_gate_up_routed_kernel(
    const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us,
    const uint16_t *uz, LocalRoute lr, const uint16_t *__restrict__ x, int E, int H, int F, int T, int k,
    uint16_t *__restrict__ h) {
    moe_gate_up_routed_block<XT, KS, GW, HAS_Z, CH4, PER>(gw, gs, gz, uw, us, uz, lr, x, E, H, F, T, k, h,
                                                           int(blockIdx.x), int(blockIdx.y));
}

// CMB: the last block of each row block (over the active experts, counted
// on a device-scope counter) also forms the combined output of those rows
// for every token, in the fixed selection order, then clears the counter.
template <int KS, int GW, bool HAS_Z, bool CH4, bool CMB, bool MULTI, bool YP16>
__global__ __launch_bounds__(512) void moe_down_gemv_kernel(const uint32_t *dw, const uint16_t *ds, const uint16_t *dz,
                                                            const int32_t *__restrict__ offsets,
                                                            const int32_t *__restrict__ active,
                                                            const int32_t *__restrict__ n_active,
                                                            const uint16_t *__restrict__ h, int E, int H, int F, int R,
                                                            void *__restrict__ yp, CombineArgs c, int T, int topk) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int e = block_expert(n_active, active, E);
    if (e < 0) return;
    constexpr int SUB = 8 / KS;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE, q = lane / 16,
              n = lane % 16;
    const int sl = wave / KS, kp = wave % KS;
    const int G = F / QGROUP, gpk = G / KS, hsub = H / 16, kc = x_row_stride(F);
    const int lsub = blockIdx.x * SUB + sl;
    const Q4Tile t(dw, ds, dz, int64_t(e) * hsub + min(lsub, hsub - 1), G);
    WaveRange<GW, HAS_Z, CH4> wr;
    wr.fetch(t, kp * gpk, gpk, opaque_lane());
    const int base = ld_uniform(offsets, e), M = ld_uniform(offsets, e + 1) - base;
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    f32x4 *red = reinterpret_cast<f32x4 *>(xl + x_pieces(R, F));
    auto chunk = [&](int m0) {
        const int mc = min(R, M - m0);
        stage_rows_issue([&](int m) { return h + int64_t(base + m0 + m) * F; }, mc, F, xl);
        __syncthreads();
        const uint4 *xr[1] = {xl + min(n, mc - 1) * kc + q * 4};
        f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
        compute_zq_inline<F16>(wr, xr[0], acc[0]);
        if constexpr (KS > 1) {
            red[wave * WAVE + lane] = acc[0];
            lds_barrier();
            if (kp == 0) {
#pragma unroll
                for (int j = 1; j < KS; ++j) acc[0] += red[(wave + j) * WAVE + lane];
            }
        }
        if (kp == 0 && lsub < hsub) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * q + r;
                const int64_t i = int64_t(base + m0 + m) * H + lsub * 16 + n;
                if constexpr (CMB && YP16) {
                    // fp16 pairs of adjacent rows (lanes n, n ^ 1) as one
                    // agent-coherent 32-bit store by the even lane
                    const uint32_t hv = __builtin_bit_cast(uint16_t, f32_to_f16_satfinite(acc[0][r]));
                    const uint32_t pv = uint32_t(__shfl_xor(int(hv), 1));
                    if (m < mc && (n & 1) == 0)
                        st_agent_u32(reinterpret_cast<uint32_t *>(static_cast<uint16_t *>(yp) + i), hv | (pv << 16));
                } else if (m < mc) {
                    if constexpr (CMB) st_agent(static_cast<float *>(yp) + i, acc[0][r]);
                    else store_yp<YP16>(yp, i, acc[0][r]);
                }
            }
        }
    };
    // the first chunk, then (MULTI) further ones refetching their weights, as
    // in the gate/up kernel
    chunk(0);
    if constexpr (MULTI) {
        for (int m0 = R; m0 < M; m0 += R) {
            wr.fetch(t, kp * gpk, gpk, opaque_lane());
            lds_barrier();
            chunk(m0);
        }
    }
    if constexpr (CMB) {
        if (!count_last_block(&c.counters[blockIdx.x], *n_active)) return;
        // The combine of rows r0 .. r0 + nr - 1 for every token, in the
        // order of the unfused combine (shared row, then the selections in
        // order). Per pass over qc selections: every (token, selection,
        // row) value of yp is requested at once (one latency) into LDS (the
        // staging area, free now), then each output element adds its own in
        // order.
        const int r0 = blockIdx.x * SUB * 16, nr = min(SUB * 16, H - r0), nt = blockDim.x;
        float *ybuf = reinterpret_cast<float *>(smem);
        for (int e0 = 0; e0 < T * nr; e0 += nt) {
            const int ne = min(nt, T * nr - e0), e = e0 + tid;
            const int tk = e / nr, j = r0 + (e - tk * nr);
            float v = 0.f;
            if (tid < ne && c.shared) v = c.shared[int64_t(tk) * H + j];
            for (int q0 = 0; q0 < topk; q0 += c.qc) {
                const int qn = min(c.qc, topk - q0);
                for (int p = tid; p < ne * qn; p += nt) {
                    const int qq = p / ne, ee = e0 + (p - qq * ne), tk2 = ee / nr, j2 = r0 + (ee - tk2 * nr);
                    const int64_t yi = int64_t(c.tok_slot[tk2 * topk + q0 + qq]) * H + j2;
                    if constexpr (YP16) {
                        const uint32_t w = ld_agent_u32(
                            reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(yp) + (yi & ~int64_t(1))));
                        ybuf[p] = f16_bits_to_f32(uint16_t(w >> ((yi & 1) * 16)));
                    } else {
                        ybuf[p] = ld_agent(static_cast<const float *>(yp) + yi);
                    }
                }
                __syncthreads();
                if (tid < ne)
                    for (int qq = 0; qq < qn; ++qq) v += c.tok_w[tk * topk + q0 + qq] * ybuf[qq * ne + tid];
                __syncthreads();
            }
            if (tid < ne) store_out(c, int64_t(tk) * H + j, v);
        }
    }
}

// Batch 1 with the combine (T = 1, k <= 8, the down K split in 2): block b
// holds output rows 16 b .. 16 b + 15 of all k selected experts; wave
// (y, kp) computes the y-th active expert (ascending; at T = 1 that is slot
// y) over K half kp, exactly as the general kernel's subtile does. The k
// results meet in LDS and the block forms its 16 outputs itself, in the
// combine's order (shared row, then the selections in order): no yp round
// trip through memory and no cross-block count before the combine. yp is
// still written (an output of the decode block).
template <int GW, bool HAS_Z, bool CH4, bool YP16>
__global__ __launch_bounds__(1024) void moe_down_t1_kernel(const uint32_t *dw, const uint16_t *ds, const uint16_t *dz,
                                                           const int32_t *__restrict__ active,
                                                           const int32_t *__restrict__ n_active,
                                                           const uint16_t *__restrict__ h, int E, int H, int F,
                                                           void *__restrict__ yp, CombineArgs c, int topk) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE, q = lane / 16,
              n = lane % 16;
    const int y = wave / 2, kp = wave % 2;
    // the h rows of the k slots (at T = 1 every slot is one active expert's)
    // and the shared row go out first, beside the routing reads: by the time
    // the weights are requested they are in flight, and the compute then
    // waits for the weights group by group as they arrive
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    stage_rows_issue([&](int m) { return h + int64_t(m) * F; }, topk, F, xl);
    const float shv = c.shared && tid < 16 ? c.shared[blockIdx.x * 16 + tid] : 0.f;
    __builtin_amdgcn_sched_barrier(0);
    // n_active and active[y] requested together (one latency); the weight
    // loads need only e (active holds E entries: the read stays inside them,
    // the value is used only for y < n_active <= E)
    const int na = ld_uniform(n_active, 0), ea = ld_uniform(active, min(y, E - 1));
    const int rows = min(na, topk);
    const bool live = y < rows;  // wave-uniform
    const int e = live ? min(max(ea, 0), E - 1) : 0;
    const int G = F / QGROUP, gpk = G / 2, hsub = H / 16, kc = x_row_stride(F);
    const Q4Tile t(dw, ds, dz, int64_t(e) * hsub + blockIdx.x, G);
    WaveRange<GW, HAS_Z, CH4> wr;
    wr.fetch(t, kp * gpk, gpk, opaque_lane());
    // the combine's inputs, requested now so that their latency is hidden:
    // the selections' slots and weights (block-uniform, scalar loads) and
    // the shared row's values (wave 0)
    int slot_q[8];
    float w_q[8];
#pragma unroll
    for (int qq = 0; qq < 8; ++qq) {
        slot_q[qq] = qq < topk ? ld_uniform(c.tok_slot, qq) : 0;
        w_q[qq] = qq < topk ? ld_uniform_f32(c.tok_w, qq) : 0.f;
    }
    f32x4 *red = reinterpret_cast<f32x4 *>(xl + x_pieces(8, F));
    float *yb = reinterpret_cast<float *>(red + 8 * WAVE);  // [8][16]
    // the h rows (this wave's oldest loads) of every wave, not the weights
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_below<WaveRange<GW, HAS_Z, CH4>::LOADS>();
    __builtin_amdgcn_s_barrier();
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    if (live) compute_zq_inline<F16>(wr, xl + y * kc + q * 4, acc);
    if (kp == 1) red[y * WAVE + lane] = acc;
    lds_barrier();
    if (kp == 0 && live) {
        acc += red[y * WAVE + lane];
        if (q == 0) {
            yb[y * 16 + n] = yp_value<YP16>(acc[0]);
            store_yp<YP16>(yp, int64_t(y) * H + blockIdx.x * 16 + n, acc[0]);
        }
    }
    __syncthreads();
    if (tid < 16) {
        const int j = blockIdx.x * 16 + tid;
        float v = 0.f;
        if (c.shared) v = shv;
#pragma unroll
        for (int qq = 0; qq < 8; ++qq)
            if (qq < topk) v += w_q[qq] * yb[slot_q[qq] * 16 + tid];
        store_out(c, j, v);
    }
}

// K split: the largest power of two <= kmax dividing G with at most 16 groups
// per wave; GW: the register budget for a wave's groups.
static int pick_ks(int G, int kmax) {
    int ks = 1;
    while (ks < kmax && G % (ks * 2) == 0) ks *= 2;
    return ks;
}

// Down projection: a split of 2 where a wave's range stays within 16
// groups (fewer, larger blocks: each has more weight bytes in flight for its
// fixed costs), else up to 8.
static int down_ks(int G) {
    int ks = pick_ks(G, 2);
    while (G / ks > 16 && ks < 8 && G % (ks * 2) == 0) ks *= 2;
    return ks;
}

template <int KS, int GW, bool HAS_Z, bool CH4>
static void launch_gate_up_routed(const MoeGemvArgs &a, int max_active, hipStream_t s) {
    const LocalRoute lr{a.route_logits, a.top_e, a.tok_slot, const_cast<int32_t *>(a.pair_tok),
                        const_cast<int32_t *>(a.offsets), const_cast<int32_t *>(a.active),
                        const_cast<int32_t *>(a.n_active), a.top_w};
    const int per = (a.E + WAVE - 1) / WAVE;
    const size_t lds = moe_lds_bytes(a.T, a.H);
    constexpr int SUB = 8 / (2 * KS);
    const dim3 grid(unsigned((a.F / 16 + SUB - 1) / SUB), unsigned(max_active));
    auto go = [&](auto kern) {
        if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), 512, lds);
        kern<<<grid, 512, lds, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, lr, a.x, a.E, a.H, a.F, a.T, a.topk, a.h);
    };
    auto pick = [&](auto xt) {
        using XT = decltype(xt);
        if (per <= 1) go(moe_gate_up_routed_kernel<XT, KS, GW, HAS_Z, CH4, 1>);
        else if (per <= 2) go(moe_gate_up_routed_kernel<XT, KS, GW, HAS_Z, CH4, 2>);
        else if (per <= 4) go(moe_gate_up_routed_kernel<XT, KS, GW, HAS_Z, CH4, 4>);
        else go(moe_gate_up_routed_kernel<XT, KS, GW, HAS_Z, CH4, 8>);
    };
    if (a.x_f16) pick(F16{});
    else pick(BF16{});
}

// ---- batch 1 with the shared expert: blocks 0 .. gx gy - 1 are the routed
// gate/up blocks (column block b % gx, active expert b / gx, their launch
// order), the blocks after them compute 16 rows each of the shared expert's
// SwiGLU-down GEMV (as qw_w16_swiglu_gemv_tiled) from the gate/up/gate-logit
// rows the block's first launch wrote.
template <typename XT, int GW, bool HAS_Z, int PER, int SWS>
__global__ __launch_bounds__(512) void gate_up_routed_shdown_kernel(
    const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us,
    const uint16_t *uz, LocalRoute lr, const uint16_t *__restrict__ x, int E, int H, int F, int k,
    uint16_t *__restrict__ h, ShExpertArgs sh, int gx, int gy) {
    const int b = blockIdx.x;
    if (b < gx * gy)
        moe_gate_up_routed_block<XT, 4, GW, HAS_Z, true, PER>(gw, gs, gz, uw, us, uz, lr, x, E, H, F, 1, k, h, b % gx,
                                                             b / gx);
    else
        w16_swiglu_block<1, 1, 1, SWS>(sh.down, sh.v, 2 * sh.Fs + 1, 1, sh.Fs, H, sh.out, H, 0, 0, b - gx * gy);
}

bool launch_gate_up_routed_shdown(const MoeGemvArgs &a, const ShExpertArgs &sh, hipStream_t s) {
    const int G = a.H / QGROUP;
    // the routed launch's shape: K split in 4 over whole 4-group chunks
    if (!a.route_logits || a.T != 1 || G % 16 != 0 || G / 4 > 8 || (a.gz != nullptr) != (a.uz != nullptr)) return false;
    const int gx = a.F / 16, gy = a.topk < a.E ? a.topk : a.E, per = (a.E + WAVE - 1) / WAVE;
    const LocalRoute lr{a.route_logits, a.top_e, a.tok_slot, const_cast<int32_t *>(a.pair_tok),
                        const_cast<int32_t *>(a.offsets), const_cast<int32_t *>(a.active),
                        const_cast<int32_t *>(a.n_active), a.top_w};
    const size_t l1 = moe_lds_bytes(1, a.H), l2 = dense_lds_bytes(1, sh.Fs, 1, W16_MAX_KS, W16_MAX_KS);
    const size_t lds = l1 > l2 ? l1 : l2;
    const unsigned grid = unsigned(gx * gy + a.H / 16);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024) raise_lds_limit(reinterpret_cast<const void *>(kern));
        kern<<<grid, 512, lds, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, lr, a.x, a.E, a.H, a.F, a.topk, a.h, sh, gx,
                                    gy);
    };
    auto by_ws = [&](auto xt, auto gw, auto hz, auto pr) {
        using XT = decltype(xt);
        constexpr int GW = decltype(gw)::value, PER = decltype(pr)::value;
        constexpr bool HZ = decltype(hz)::value;
        if (sh.Fs / 32 / W16_MAX_KS <= 8) go(gate_up_routed_shdown_kernel<XT, GW, HZ, PER, 8>);
        else go(gate_up_routed_shdown_kernel<XT, GW, HZ, PER, 16>);
    };
    auto by_per = [&](auto xt, auto gw, auto hz) {
        if (per <= 1) by_ws(xt, gw, hz, std::integral_constant<int, 1>());
        else if (per <= 2) by_ws(xt, gw, hz, std::integral_constant<int, 2>());
        else if (per <= 4) by_ws(xt, gw, hz, std::integral_constant<int, 4>());
        else by_ws(xt, gw, hz, std::integral_constant<int, 8>());
    };
    auto by_z = [&](auto xt, auto gw) {
        if (a.gz) by_per(xt, gw, std::true_type());
        else by_per(xt, gw, std::false_type());
    };
    auto by_gw = [&](auto xt) {
        if (G / 4 == 8) by_z(xt, std::integral_constant<int, 8>());
        else by_z(xt, std::integral_constant<int, 4>());
    };
    if (a.x_f16) by_gw(F16{});
    else by_gw(BF16{});
    return true;
}

// ---- 5 to 32 tokens with the shared expert: grid rows y < max_active run the
// gate/up GEMV of the y-th active expert (as moe_gate_up_gemv_kernel with
// the K split in 4 over whole 4-group chunks, GW = 4 or 8 groups per wave), the rows
// after them the shared expert's down GEMV over its SwiGLU rows sh_h (as
// qw_w16_gemv_tiled, 16 output rows per block). The two read different
// inputs of earlier launches (the routing, sh_h) and write different outputs.
template <typename XT, int GW, bool HAS_Z, bool MULTI, int SMB, int SXPT, int SWS>
__global__ __launch_bounds__(512) void gate_up_shdown_gemv_kernel(
    const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us,
    const uint16_t *uz, const int32_t *__restrict__ offsets, const int32_t *__restrict__ active,
    const int32_t *__restrict__ n_active, const int32_t *__restrict__ pair_tok, const uint16_t *__restrict__ x, int E,
    int H, int F, int R, uint16_t *__restrict__ h, int max_active, ShExpertArgs sh, const uint16_t *sh_h, int T) {
    const int by = int(blockIdx.y);
    if (by < max_active) {
        moe_gate_up_gemv_block<XT, 4, GW, HAS_Z, true, MULTI>(gw, gs, gz, uw, us, uz, offsets, active, n_active,
                                                              pair_tok, x, E, H, F, R, h, int(blockIdx.x), by);
    } else {
        const int i = (by - max_active) * int(gridDim.x) + int(blockIdx.x);
        if (i < (H + 15) / 16)
            w16_gemv_block<F16, SMB, 4, SXPT, SWS, true>(sh.down, 0, sh_h, sh.Fs, T, sh.Fs, H, sh.out, H, 0, 0, 0, i);
    }
}

bool launch_gate_up_shdown(const MoeGemvArgs &a, const ShExpertArgs &sh, const uint16_t *sh_h, hipStream_t s) {
    const int G = a.H / QGROUP;
    // the gate/up shapes of launch_gw with the K split in 4: 4 or 8 groups per
    // wave, whole 4-group chunks (H 2048 and 4096)
    if (a.route_logits || a.T < 5 || a.T > 32 || pick_ks(G, 4) != 4 || (G / 4 != 4 && G / 4 != 8) ||
        sh.Fs % 256 != 0 || (a.gz != nullptr) != (a.uz != nullptr) || !w16_fits(a.T, sh.Fs, a.H))
        return false;
    // the gate/up launch's shape (launch_one, launch_gate_up): rows per chunk
    // as many as keep the staged activations within 32 KB
    int R = a.T < 16 ? a.T : 16;
    while (R > 1 && size_t(R) * a.H * 2 > 32 * 1024) --R;
    const int max_active = a.T * a.topk < a.E ? a.T * a.topk : a.E, gx = a.F / 16;
    const int shb = (a.H + 15) / 16, rows = (shb + gx - 1) / gx;
    const int smb = a.T > 16 ? 2 : 1;
    const size_t l1 = moe_lds_bytes(R, a.H), l2 = dense_lds_bytes(a.T, sh.Fs, smb, W16_MAX_KS, W16_MAX_KS);
    // every block of the grid gets the larger LDS size: merge only where that
    // leaves as many gate/up blocks per CU as the gate/up launch alone has
    // (16 or more rows of the down GEMV stage more than the gate/up's chunk:
    // 202 against 189-193 us per block at 16 tokens, 420 against 296 at 32)
    if ((160 * 1024) / l2 < (160 * 1024) / l1) return false;
    const size_t lds = l1 > l2 ? l1 : l2;
    const dim3 grid(unsigned(gx), unsigned(max_active + rows));
    // the down GEMV's template shape as qw_w16_gemv_tiled picks it for T rows
    // of K = Fs (8 waves: Fs / 32 >= 8; 4 rows per MFMA pass, two row tiles
    // above 16 rows)
    const int xpt = (a.T * (sh.Fs / 8) + 8 * WAVE - 1) / (8 * WAVE);
    const bool ws16 = (sh.Fs / 32 + W16_MAX_KS - 1) / W16_MAX_KS > 8;
    auto go = [&](auto kern) {
        if (lds > 64 * 1024) raise_lds_limit(reinterpret_cast<const void *>(kern));
        kern<<<grid, 512, lds, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets, a.active, a.n_active, a.pair_tok,
                                    a.x, a.E, a.H, a.F, R, a.h, max_active, sh, sh_h, a.T);
    };
    auto by_ws = [&](auto xt, auto hz, auto mu, auto sxpt) {
        using XT = decltype(xt);
        constexpr bool HZ = decltype(hz)::value, MU = decltype(mu)::value;
        constexpr int SXPT = decltype(sxpt)::value;
        auto by_mb = [&](auto mb) {
            constexpr int MB = decltype(mb)::value;
            if (G / 4 == 4) {
                if (ws16) go(gate_up_shdown_gemv_kernel<XT, 4, HZ, MU, MB, SXPT, 16>);
                else go(gate_up_shdown_gemv_kernel<XT, 4, HZ, MU, MB, SXPT, 8>);
            } else {
                if (ws16) go(gate_up_shdown_gemv_kernel<XT, 8, HZ, MU, MB, SXPT, 16>);
                else go(gate_up_shdown_gemv_kernel<XT, 8, HZ, MU, MB, SXPT, 8>);
            }
        };
        if (smb == 2) by_mb(std::integral_constant<int, 2>());
        else by_mb(std::integral_constant<int, 1>());
    };
    auto by_xpt = [&](auto xt, auto hz, auto mu) {
        if (xpt <= 1) by_ws(xt, hz, mu, std::integral_constant<int, 1>());
        else if (xpt <= 2) by_ws(xt, hz, mu, std::integral_constant<int, 2>());
        else if (xpt <= 4) by_ws(xt, hz, mu, std::integral_constant<int, 4>());
        else by_ws(xt, hz, mu, std::integral_constant<int, 0>());
    };
    auto by_multi = [&](auto xt, auto hz) {
        if (a.T <= R) by_xpt(xt, hz, std::false_type());
        else by_xpt(xt, hz, std::true_type());
    };
    auto by_z = [&](auto xt) {
        if (a.gz) by_multi(xt, std::true_type());
        else by_multi(xt, std::false_type());
    };
    if (a.x_f16) by_z(F16{});
    else by_z(BF16{});
    return true;
}

// Batch 1 only. Routing in every block costs each block the top-k's
// latency (about 1.3 us of its 8 serial wave-maximum rounds) before its
// weight requests; at batch 1 (768 blocks, one round) that is less than the
// router's hand-off it replaces (30.3 against 31.7 us per MoE block, same
// box), at batch 2 (1536 blocks, two rounds, each paying it) it is more
// (52.5 against 47.2 us), and at batch 4 more again.
bool moe_local_route_ok(int T, int E, int topk) { return T == 1 && topk <= 8 && E <= 512; }

template <int KS, int GW, bool HAS_Z, bool CH4>
static void launch_gate_up(const MoeGemvArgs &a, int max_active, int R, hipStream_t s) {
    if (a.route_logits) {
        launch_gate_up_routed<KS, GW, HAS_Z, CH4>(a, max_active, s);
        return;
    }
    constexpr int SUB = 8 / (2 * KS);
    const dim3 grid(unsigned((a.F / 16 + SUB - 1) / SUB), unsigned(max_active));
    if (a.T <= 4) {
        auto kern = a.x_f16 ? moe_gate_up_small_kernel<F16, KS, GW, HAS_Z, CH4>
                            : moe_gate_up_small_kernel<BF16, KS, GW, HAS_Z, CH4>;
        const size_t lds = moe_lds_bytes(a.T, a.H);
        if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), 512, lds);
        kern<<<grid, 512, lds, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets, a.active, a.n_active, a.pair_tok,
                                    a.x, a.E, a.H, a.F, a.T, a.h);
        return;
    }
    // an expert has at most T tokens: one chunk of R rows holds them when R >= T
    auto kern = a.T <= R ? (a.x_f16 ? moe_gate_up_gemv_kernel<F16, KS, GW, HAS_Z, CH4, false>
                                    : moe_gate_up_gemv_kernel<BF16, KS, GW, HAS_Z, CH4, false>)
                         : (a.x_f16 ? moe_gate_up_gemv_kernel<F16, KS, GW, HAS_Z, CH4, true>
                                    : moe_gate_up_gemv_kernel<BF16, KS, GW, HAS_Z, CH4, true>);
    const size_t lds = moe_lds_bytes(R, a.H);
    if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), 512, lds);
    kern<<<grid, 512, lds, s>>>(a.gw, a.gs, a.gz, a.uw, a.us, a.uz, a.offsets, a.active, a.n_active, a.pair_tok, a.x,
                                a.E, a.H, a.F, R, a.h);
}

template <int KS, int GW, bool HAS_Z, bool CH4, bool CMB, bool YP16>
static void launch_down_c(const MoeGemvArgs &a, int max_active, int R, hipStream_t s) {
    if constexpr (CMB && KS == 2 && GW <= 8) {  // GW 16 would spill at 1024 threads
        if (a.T == 1 && a.topk <= 8) {
            const size_t lds = size_t(x_pieces(8, a.F)) * 16 + size_t(8) * WAVE * 16 + 8 * 16 * 4;
            moe_down_t1_kernel<GW, HAS_Z, CH4, YP16><<<unsigned(a.H / 16), 1024, lds, s>>>(
                a.dw, a.ds, a.dz, a.active, a.n_active, a.h, a.E, a.H, a.F, a.yp, *a.cmb, a.topk);
            return;
        }
    }
    auto kern = a.T <= R ? moe_down_gemv_kernel<KS, GW, HAS_Z, CH4, CMB, false, YP16>
                         : moe_down_gemv_kernel<KS, GW, HAS_Z, CH4, CMB, true, YP16>;
    const size_t lds = moe_lds_bytes(R, a.F);
    if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), 512, lds);
    constexpr int SUB = 8 / KS;
    const dim3 grid(unsigned((a.H / 16 + SUB - 1) / SUB), unsigned(max_active));
    CombineArgs c = a.cmb ? *a.cmb : CombineArgs{};
    c.qc = int(lds / 4 / 512);  // yp values of up to 512 elements x qc selections fit the staging LDS
    if (c.qc > a.topk) c.qc = a.topk;
    if (c.qc < 1) c.qc = 1;
    kern<<<grid, 512, lds, s>>>(a.dw, a.ds, a.dz, a.offsets, a.active, a.n_active, a.h, a.E, a.H, a.F, R, a.yp, c,
                                a.T, a.topk);
}

template <int KS, int GW, bool HAS_Z, bool CH4>
static void launch_down(const MoeGemvArgs &a, int max_active, int R, hipStream_t s) {
    if (a.yp_f16) {
        if (a.cmb) launch_down_c<KS, GW, HAS_Z, CH4, true, true>(a, max_active, R, s);
        else launch_down_c<KS, GW, HAS_Z, CH4, false, true>(a, max_active, R, s);
    } else {
        if (a.cmb) launch_down_c<KS, GW, HAS_Z, CH4, true, false>(a, max_active, R, s);
        else launch_down_c<KS, GW, HAS_Z, CH4, false, false>(a, max_active, R, s);
    }
}

template <bool DOWN, int KS, int GW, bool HAS_Z, bool CH4>
static void launch_kind(const MoeGemvArgs &a, int max_active, int R, hipStream_t s) {
    if constexpr (DOWN) launch_down<KS, GW, HAS_Z, CH4>(a, max_active, R, s);
    else launch_gate_up<KS, GW, HAS_Z, CH4>(a, max_active, R, s);
}

template <bool DOWN, int KS, bool HAS_Z>
static void launch_gw(const MoeGemvArgs &a, int max_active, int R, int gpk, hipStream_t s) {
    if (gpk == 4) launch_kind<DOWN, KS, 4, HAS_Z, true>(a, max_active, R, s);
    else if (gpk < 4) launch_kind<DOWN, KS, 4, HAS_Z, false>(a, max_active, R, s);
    else if (gpk == 6) launch_kind<DOWN, KS, 6, HAS_Z, false>(a, max_active, R, s);  // down at F = 1536
    else if (gpk == 8) launch_kind<DOWN, KS, 8, HAS_Z, true>(a, max_active, R, s);
    else if (gpk < 8) launch_kind<DOWN, KS, 8, HAS_Z, false>(a, max_active, R, s);
    else if (gpk % 4 == 0) launch_kind<DOWN, KS, 16, HAS_Z, true>(a, max_active, R, s);
    else launch_kind<DOWN, KS, 16, HAS_Z, false>(a, max_active, R, s);
}

template <bool DOWN, bool HAS_Z>
static void launch_one(const MoeGemvArgs &a, int max_active, hipStream_t s) {
    const int K = DOWN ? a.F : a.H, G = K / QGROUP;
    const int ks = DOWN ? down_ks(G) : pick_ks(G, 4);
    const int gpk = G / ks;
    // rows per block: a decode batch's tokens of one expert, as many as keep
    // the staged activations within 32 KB (two blocks per CU)
    int R = a.T < 16 ? a.T : 16;
    while (R > 1 && size_t(R) * K * 2 > 32 * 1024) --R;
    switch (ks) {
        case 1: launch_gw<DOWN, 1, HAS_Z>(a, max_active, R, gpk, s); break;
        case 2: launch_gw<DOWN, 2, HAS_Z>(a, max_active, R, gpk, s); break;
        case 4: launch_gw<DOWN, 4, HAS_Z>(a, max_active, R, gpk, s); break;
        default:
            if constexpr (DOWN) launch_gw<DOWN, 8, HAS_Z>(a, max_active, R, gpk, s);
            break;
    }
}

int moe_down_row_blocks(int H, int F) {
    const int sub = 8 / down_ks(F / QGROUP);
    return (H / 16 + sub - 1) / sub;
}

bool moe_gemv_supported(int H, int F) {
    // each wave holds at most 16 groups of its K range
    return H / QGROUP / pick_ks(H / QGROUP, 4) <= 16 && F / QGROUP / down_ks(F / QGROUP) <= 16;
}

void launch_moe_down(const MoeGemvArgs &a, hipStream_t s) {
    const int max_active = a.T * a.topk < a.E ? a.T * a.topk : a.E;
    if (a.dz) launch_one<true, true>(a, max_active, s);
    else launch_one<true, false>(a, max_active, s);
}

void launch_moe_gemv(const MoeGemvArgs &a, hipStream_t s) {
    const int max_active = a.T * a.topk < a.E ? a.T * a.topk : a.E;
    if (a.gz) launch_one<false, true>(a, max_active, s);
    else launch_one<false, false>(a, max_active, s);
    if (a.dz) launch_one<true, true>(a, max_active, s);
    else launch_one<true, false>(a, max_active, s);
}

}  // namespace qwq4
