// Dense q4 GEMV for decode rows (M <= 32 per launch), on the gfx950
// 16x16x32 MFMA: the kernel and its launch-shape choice, instantiated per
// activation type by q4_gemv.hip (bf16) and q4_gemv_f16.hip (fp16).
//
// Reference role: gpu::gemv_rows (src/kernels/gemv.hip:7-42, decode
// projections and LM head, fp16 weights there). The arithmetic is
// ref::Model::expert_linear (src/ref/ref_model.cpp:100-119) with a per-group
// zero point. The wave-level work (one 16-row subtile x a K range, lane map)
// is in q4_gemv_core.cuh.
#pragma once

#include "q4_gemv_core.cuh"
#include "q4_kernels.hpp"

namespace qwq4 {

// ------------------------------------------------------------ dense GEMV
// Work item = SUB consecutive 16-row subtiles; each subtile's K groups are
// split over KS waves (a block has KS * SUB <= 16 waves), a wave's range being
// gpk = G / KS groups, ideally 4 (one 4-group chunk: its scales are one 8-byte
// load, its zeros one 16-bit word). Every wave requests its whole range of
// weights (after the block's activation rows, bf16, staged in LDS by direct
// loads) before anything waits. The MFMA accumulator starts at -144 * sum(x)
// of the group (an MFMA against a splat of -144), see q4_common.cuh. The KS
// partial sums of a subtile are reduced through LDS in a fixed order
// (deterministic).
//
// Blocks are as many as stay resident in one round: block b takes items b,
// b + gridDim.x, ... with the activations staged once. With more than one
// item per block (PF) the next item's weights are requested before the
// current one is computed. A wave range of more than GW groups runs in
// passes of GW.

constexpr int DENSE_GW = 4;

template <typename XT, int NW, int MB, bool HAS_Z, bool CH4, bool PF, bool KSNW, int XPT, bool P4, int MR>
// Argument order: what the weight and activation requests need first (the
// first 14 dwords are preloaded into SGPRs at wave launch), the output last.
__global__ __launch_bounds__(NW * WAVE) void q4_gemv_block_kernel(const uint32_t *Wt, const uint16_t *St, const uint16_t *Zt,
                                                             const uint16_t *x, int xs, int M, int K, int N, int KS_,
                                                             int SUB_, void *__restrict__ y, int ys, int y_bf16,
                                                             int accumulate, int n_lo) {
    // KSNW: one subtile per item, split over all NW waves, each wave exactly
    // GW groups (all compile-time)
    const int KS = KSNW ? NW : KS_, SUB = KSNW ? 1 : SUB_;
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int GW = DENSE_GW;
    const int G = KSNW ? NW * GW : K / QGROUP, kc = x_row_stride(K), nsub = (N + 15) / 16, gpk = KSNW ? GW : G / KS,
              items = (nsub + SUB - 1) / SUB;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE,
              q = lane / 16, n = lane % 16, waves = KSNW ? NW : int(blockDim.x) / WAVE;
    const int sl = wave / KS, kp = wave % KS, g0 = kp * gpk;
    auto tile_of = [&](int item) { return Q4Tile(Wt, St, Zt, min(item * SUB + sl, nsub - 1), G); };
    uint4 *xl = reinterpret_cast<uint4 *>(smem);
    float *red = reinterpret_cast<float *>(xl + x_pieces(M, K));
    // XPT > 0 (at most 4 pieces per thread): activations through registers, so that
    // each weight group is computed as it arrives; else direct into LDS
    // (the compiler then drains every load in flight before the first LDS
    // read)
    XRegs xv;
    if constexpr (XPT > 0) stage_regs_issue<XPT>(x, xs, M, K, xv);
    else stage_x_issue(x, xs, M, K, xl);
    __builtin_amdgcn_sched_barrier(0);  // every activation load goes out before the weight loads
    WaveRange<GW, HAS_Z, CH4> wr[1];
    wr[0].fetch(tile_of(blockIdx.x), g0, min(gpk, GW), lane);
    if constexpr (XPT > 0) {
        __builtin_amdgcn_sched_barrier(0);  // and the LDS writes of the activations (which wait for them) after both
        stage_regs_commit<XPT>(xv, M, K, xl);
        lds_barrier();
    } else {
        // the direct loads of the activations are this wave's oldest loads in
        // flight: wait for them alone, then for every wave's
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_below<WaveRange<GW, HAS_Z, CH4>::LOADS>();
        __builtin_amdgcn_s_barrier();
    }
    const uint4 *xr[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xr[mb] = xl + min(mb * 16 + n, M - 1) * kc + q * 4;
    // the lane's fragment of the packed correction tile (P4): token n % 4
    // of group gb + n / 4
    auto xp_of = [&](int gb) { return packed_fragment(xl, kc, M, G, gb, lane); };
    f32x4 sums[GW][MB];
    group_sums<XT, MB, GW, P4, MR>(xr, xp_of, g0, min(gpk, GW), sums);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!PF) {
        f32x4 acc[1][MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[0][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
        compute_zq<XT, MB, 1, GW, HAS_Z, CH4, MR>(wr, xr, sums, acc);
        // longer ranges: further passes of GW groups
        for (int p = GW; p < gpk; p += GW) {
            wr[0].fetch(tile_of(blockIdx.x), g0 + p, min(gpk - p, GW), opaque_lane());
            group_sums<XT, MB, GW, P4, MR>(xr, xp_of, g0 + p, min(gpk - p, GW), sums);
            compute_zq<XT, MB, 1, GW, HAS_Z, CH4, MR>(wr, xr, sums, acc);
        }
        ksplit_sum<MB, MR>(acc[0], red, KS, wave, kp, lane);
        const int sub = blockIdx.x * SUB + sl;
        if (kp == 0 && sub < nsub) store_rows<MB, MR>(acc[0], y, ys, y_bf16, accumulate, M, N, sub, lane, n_lo);
    } else {
        // gpk <= GW here
        WaveRange<GW, HAS_Z, CH4> wn[1];
        int par = 0;
        for (int item = blockIdx.x; item < items; item += gridDim.x) {
            wn[0].fetch(tile_of(min(item + int(gridDim.x), items - 1)), g0, gpk, opaque_lane());
            f32x4 acc[1][MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[0][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
            compute_zq<XT, MB, 1, GW, HAS_Z, CH4, MR>(wr, xr, sums, acc);  // the corrections of the block's groups serve every item
            // partials double-buffered by item parity: the barrier of item
            // i + 1 orders item i's reads before item i + 2's writes
            ksplit_sum<MB, MR>(acc[0], red + par * (red_slots(waves, KS) * acc_elems<MB, MR>() * WAVE), KS, wave, kp,
                               lane);
            par ^= 1;
            const int sub = item * SUB + sl;
            if (kp == 0 && sub < nsub) store_rows<MB, MR>(acc[0], y, ys, y_bf16, accumulate, M, N, sub, lane, n_lo);
            wr[0] = wn[0];
        }
    }
}

// K split: gpk = 4 where G allows (KS = G / 4 <= 16), else the largest
// divisor of G up to 16 (fewest groups per wave). SUB: subtiles per item,
// filling blocks of 8, 12 or 16 waves (the kernel's launch bound NW).
static void dense_split(int G, int &KS, int &SUB, int &NW) {
    KS = 1;
    if (G % 4 == 0 && G / 4 <= 16) KS = G / 4;
    else
        for (int k = 16; k >= 1; --k)
            if (G % k == 0) {
                KS = k;
                break;
            }
    NW = 16;
    for (int nw : {8, 12, 16})
        if (nw % KS == 0) {
            NW = nw;
            break;
        }
    SUB = NW / KS;
}

// Blocks of one item each (items beyond the resident blocks run in further
// rounds). XPT: pieces of activations per thread through registers, 0 for
// direct loads into LDS.
template <typename XT, int NW, int MB, bool HAS_Z, bool CH4, bool KSNW, bool P4, int XPT, int MR>
static void launch_dense_one(const GemvArgs &a, int KS, int SUB, int items, size_t lds, hipStream_t s) {
    auto kern = q4_gemv_block_kernel<XT, NW, MB, HAS_Z, CH4, false, KSNW, XPT, P4, MR>;
    const int threads = KS * SUB * WAVE;
    if (lds > 64 * 1024) (void)persistent_shape(reinterpret_cast<const void *>(kern), threads, lds);  // LDS limit
    kern<<<items, threads, lds, s>>>(a.W, a.S, a.Z, a.x, a.xs, a.M, a.K, a.N, KS, SUB, a.y, a.ys,
                                     a.y_bf16, a.accumulate, a.n_lo);
}

// Small batches (at most 4 activation pieces per thread) stage through
// registers and run one item per block. Larger ones stage directly into LDS;
// when their items exceed one round of resident blocks, the blocks stay
// resident and prefetch their next item (PF). P4: batches of at most 4 rows
// (packed group corrections).
template <typename XT, int NW, int MB, bool HAS_Z, bool CH4, bool KSNW, bool P4, int MR>
static void launch_dense_t(const GemvArgs &a, int KS, int SUB, hipStream_t s) {
    const int waves = KS * SUB, threads = waves * WAVE, gpk = a.K / QGROUP / KS;
    const int nsub = (a.N + 15) / 16, items = (nsub + SUB - 1) / SUB;
    const int xpt = (a.M * (a.K / 8) + threads - 1) / threads;
    if constexpr (MB == 1) {
        // batches of 4 rows over more items than one round of resident
        // blocks (the LM head) run faster as the persistent prefetching blocks
        // below (151936 rows at batch 4: 60 against 65 us; at batches 1-3
        // the register path stays ahead: 51 against 58 at batch 1, 57.5
        // against 59 at batch 3)
        bool regs = xpt <= 4;
        if (regs && a.M >= 4 && gpk <= DENSE_GW) {
            auto pf = q4_gemv_block_kernel<XT, NW, MB, HAS_Z, CH4, true, KSNW, 0, P4, MR>;
            const size_t lds = dense_lds_bytes(a.M, a.K, MB, waves, KS);
            regs = items <= persistent_shape(reinterpret_cast<const void *>(pf), threads, lds).max_blocks;
        }
        if (regs) {
            const size_t lds = dense_lds_bytes(a.M, a.K, MB, waves, KS);
            if (xpt <= 1) launch_dense_one<XT, NW, MB, HAS_Z, CH4, KSNW, P4, 1, MR>(a, KS, SUB, items, lds, s);
            else if (xpt <= 2) launch_dense_one<XT, NW, MB, HAS_Z, CH4, KSNW, P4, 2, MR>(a, KS, SUB, items, lds, s);
            else launch_dense_one<XT, NW, MB, HAS_Z, CH4, KSNW, P4, 4, MR>(a, KS, SUB, items, lds, s);
            return;
        }
    }
    const size_t lds = dense_lds_bytes(a.M, a.K, MB, waves, KS);
    auto one = q4_gemv_block_kernel<XT, NW, MB, HAS_Z, CH4, false, KSNW, 0, P4, MR>;
    const LaunchShape ls = persistent_shape(reinterpret_cast<const void *>(one), threads, lds);
    if (items <= ls.max_blocks || gpk > DENSE_GW) {
        launch_dense_one<XT, NW, MB, HAS_Z, CH4, KSNW, P4, 0, MR>(a, KS, SUB, items, lds, s);
        return;
    }
    auto pf = q4_gemv_block_kernel<XT, NW, MB, HAS_Z, CH4, true, KSNW, 0, P4, MR>;
    const LaunchShape lp = persistent_shape(reinterpret_cast<const void *>(pf), threads, lds);
    // every resident slot gets a block; blocks take items grid-stride, so a
    // CU's blocks together hold an even share of the items and every slot
    // keeps weight loads in flight
    const int blocks = items < lp.max_blocks ? items : lp.max_blocks;
    pf<<<blocks, threads, lds, s>>>(a.W, a.S, a.Z, a.x, a.xs, a.M, a.K, a.N, KS, SUB, a.y, a.ys,
                                    a.y_bf16, a.accumulate, a.n_lo);
}

template <typename XT, int MB, bool HAS_Z, bool CH4, bool P4, int MR>
static void launch_dense_nw(const GemvArgs &a, int KS, int SUB, int NW, hipStream_t s) {
    const bool fit = KS == NW && a.K / QGROUP == NW * DENSE_GW;
    if (NW == 8) {
        if (fit) launch_dense_t<XT, 8, MB, HAS_Z, CH4, true, P4, MR>(a, KS, SUB, s);
        else launch_dense_t<XT, 8, MB, HAS_Z, CH4, false, P4, MR>(a, KS, SUB, s);
    } else if (NW == 12) {
        if (fit) launch_dense_t<XT, 12, MB, HAS_Z, CH4, true, P4, MR>(a, KS, SUB, s);
        else launch_dense_t<XT, 12, MB, HAS_Z, CH4, false, P4, MR>(a, KS, SUB, s);
    } else {
        if (fit) launch_dense_t<XT, 16, MB, HAS_Z, CH4, true, P4, MR>(a, KS, SUB, s);
        else launch_dense_t<XT, 16, MB, HAS_Z, CH4, false, P4, MR>(a, KS, SUB, s);
    }
}

template <typename XT, int MB, bool HAS_Z>
static void launch_dense(const GemvArgs &a, hipStream_t s) {
    int KS, SUB, NW;
    dense_split(a.K / QGROUP, KS, SUB, NW);
    const bool ch4 = (a.K / QGROUP / KS) % 4 == 0, p4 = MB == 1 && a.M <= 4;
    // MR: accumulator rows a lane can hold tokens in (batches of 1 and 2
    // keep only those)
    if (ch4) {
        if (p4 && a.M == 1) launch_dense_nw<XT, MB, HAS_Z, true, MB == 1, 1>(a, KS, SUB, NW, s);
        else if (p4 && a.M == 2) launch_dense_nw<XT, MB, HAS_Z, true, MB == 1, 2>(a, KS, SUB, NW, s);
        else if (p4) launch_dense_nw<XT, MB, HAS_Z, true, MB == 1, 4>(a, KS, SUB, NW, s);
        else launch_dense_nw<XT, MB, HAS_Z, true, false, 4>(a, KS, SUB, NW, s);
    } else {
        if (p4 && a.M == 1) launch_dense_nw<XT, MB, HAS_Z, false, MB == 1, 1>(a, KS, SUB, NW, s);
        else if (p4 && a.M == 2) launch_dense_nw<XT, MB, HAS_Z, false, MB == 1, 2>(a, KS, SUB, NW, s);
        else if (p4) launch_dense_nw<XT, MB, HAS_Z, false, MB == 1, 4>(a, KS, SUB, NW, s);
        else launch_dense_nw<XT, MB, HAS_Z, false, false, 4>(a, KS, SUB, NW, s);
    }
}

template <typename XT>
void launch_gemv_fit_t(const GemvArgs &a, hipStream_t s) {
    if (a.M <= 16) {
        if (a.Z) launch_dense<XT, 1, true>(a, s);
        else launch_dense<XT, 1, false>(a, s);
    } else {
        if (a.Z) launch_dense<XT, 2, true>(a, s);
        else launch_dense<XT, 2, false>(a, s);
    }
}

}  // namespace qwq4
