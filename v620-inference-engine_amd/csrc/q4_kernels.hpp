// Internal launcher interface between the C-ABI layer (capi.cpp) and the HIP
// kernels. Shapes are validated by the caller (capi.cpp) before any launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace qwq4 {

// Grid size of a persistent kernel on the current device: CUs times the
// resident blocks per CU for this kernel, block size and dynamic LDS. Sets the
// kernel's dynamic-LDS limit when it exceeds the 64 KiB default. Cached.
struct LaunchShape {
    int max_blocks, cus;
};
LaunchShape persistent_shape(const void *kernel, int threads, size_t lds);
// Raises a kernel's dynamic-LDS limit (once per kernel and device) to what the
// CU's 160 KiB leave beside its static LDS.
void raise_lds_limit(const void *kernel);

struct GemvArgs {
    const uint32_t *W;
    const uint16_t *S;
    const uint16_t *Z;
    const uint16_t *x;
    int xs;
    void *y;
    int ys, y_bf16, N, K, M, accumulate;
    int x_f16 = 0;  // x rows are fp16 (else bf16)
    int rpg = 0;    // rows per activation slice (0: one slice), as in gpu::gemv_rows
    int n_lo = 0;   // rows below n_lo are computed but not stored (internal)
};
void launch_gemv(const GemvArgs &a, hipStream_t s);

// Weighted combine folded into the down projection (see launch_moe_gemv):
// out[t][j] = shared[t][j] + sum_i tok_w[t][i] * yp[tok_slot[t][i]][j].
struct CombineArgs {
    int32_t *counters;  // one per down row block, zero between calls
    const int32_t *tok_slot;
    const float *tok_w;
    const float *shared;  // fp32 [T][H] or null
    void *out;
    int out_type;  // 0 fp32, 1 bf16, 2 fp16
    int qc;  // selections staged per pass of the combine (set by the launcher)
};
// Down row blocks of the decode experts for H (the counters combine needs).
int moe_down_row_blocks(int H, int F);

// The shared expert of a fused decode block (tiled 16-bit weights of x's
// type, qw_w16_tile): v = gu x ([T][2 Fs + 1] fp32: gate, up, gate logit),
// out = down swiglu_gate(v) ([T][H] fp32), the rows the combine adds.
struct ShExpertArgs {
    const uint16_t *gu;    // [2 Fs + 1][H]
    const uint16_t *down;  // [H][Fs]
    int Fs;
    float *v;
    float *out;
};
struct MoeGemvArgs {
    const uint32_t *gw;
    const uint16_t *gs;
    const uint16_t *gz;
    const uint32_t *uw;
    const uint16_t *us;
    const uint16_t *uz;
    const uint32_t *dw;
    const uint16_t *ds;
    const uint16_t *dz;
    int E, H, F;
    const int32_t *offsets, *active, *n_active, *pair_tok;
    const uint16_t *x;
    int T, topk;
    uint16_t *h;
    void *yp;                // fp32, or fp16 with yp_f16
    const CombineArgs *cmb;  // null: yp only
    int x_f16 = 0;           // x rows are fp16 (else bf16)
    int yp_f16 = 0;
    // Non-null: the gate/up blocks route the batch themselves from these
    // logits [T][E] (moe_local_route_ok), and block (0, 0) writes the
    // routing outputs: top_e, top_w, tok_slot and the offsets, active,
    // n_active and pair_tok above (which are then outputs, not inputs).
    const float *route_logits = nullptr;
    int32_t *top_e = nullptr, *tok_slot = nullptr;
    float *top_w = nullptr;
};
// Whether the gate/up decode GEMV can route a batch of T tokens itself.
bool moe_local_route_ok(int T, int E, int topk);
void launch_moe_gemv(const MoeGemvArgs &a, hipStream_t s);
// The down projection (with the folded combine where it applies) alone, after
// a gate/up launch of the caller's.
void launch_moe_down(const MoeGemvArgs &a, hipStream_t s);
// Batch 1 gate/up routed in its blocks with the shared expert's SwiGLU-down
// GEMV in the same launch; false (nothing launched) where the shapes do not
// fit that launch.
bool launch_gate_up_routed_shdown(const MoeGemvArgs &a, const ShExpertArgs &sh, hipStream_t s);
// 5 to 8 tokens: the gate/up GEMV (as launch_moe_gemv's) and the shared
// expert's down GEMV over its SwiGLU rows sh_h [T][Fs] in one launch; false
// (nothing launched) where the shapes do not allow it.
bool launch_gate_up_shdown(const MoeGemvArgs &a, const ShExpertArgs &sh, const uint16_t *sh_h, hipStream_t s);
// Whether the expert GEMVs take these sizes (a wave holds <= 16 groups of its K range).
bool moe_gemv_supported(int H, int F);

struct MoeGroupedArgs {
    const uint32_t *gw;
    const uint16_t *gs;
    const uint16_t *gz;
    const uint32_t *uw;
    const uint16_t *us;
    const uint16_t *uz;
    const uint32_t *dw;
    const uint16_t *ds;
    const uint16_t *dz;
    int E, H, F;
    const int32_t *offsets, *pair_tok, *tile_e, *tile_m0, *n_tiles;
    const uint16_t *x;
    int T, topk;
    uint16_t *h;
    void *yp;       // fp32, or fp16 with yp_f16
    void *ws;
    int x_f16 = 0;  // x rows are fp16 (no pre-pass)
    int yp_f16 = 0;
};
// Tokens per tile the grouped kernels expect in the routing tile list.
int moe_grouped_tile_m();
size_t moe_grouped_workspace_bytes(int T, int topk, int E, int H, int F);
void launch_moe_grouped(const MoeGroupedArgs &a, hipStream_t s);

struct RouteArgs {
    const float *logits;
    int T, E, topk, tile_m;
    int32_t *top_e;
    float *top_w;
    int32_t *counts, *offsets, *tok_slot, *pair_tok, *active, *n_active;
    int32_t *tile_e, *tile_m0, *n_tiles;
};
// fp32 router GEMV fused with the decode routing (T <= 64).
struct RouterArgs {
    const void *w;      // [E][H] fp32, or fp16 (w_f16)
    const uint16_t *x;  // bf16 or fp16 [T][H]
    int H, kl;          // K slice per block (a multiple of 8 dividing H)
    float *part;        // [H / kl][T][E] partial logits
    float *logits;      // [T][E]
    int32_t *counter;   // [1 + ceil(E / 16)], zero between calls
    int x_f16 = 0;      // x rows are fp16 (else bf16)
    int w_f16 = 0;      // router weights are fp16 (the engine's w.router), else fp32
};
// Up to 8 tokens: the shared expert's gate/up GEMV in the router-logits launch
// (and at batch 1 its down GEMV beside the routed gate/up) where the shapes
// allow (T <= 8, H and Fs multiples of 256, H <= 8192, Fs <= 4096).
bool shared_logits_ok(int T, int H, int Fs);
void launch_router_logits_shgu(const RouterArgs &r, int T, int E, const ShExpertArgs &sh, hipStream_t s);
// 2 to 4 tokens: the routing (one block, as launch_route) and the shared
// expert's SwiGLU-gate + down GEMV in one launch; false (nothing launched)
// where the shapes do not allow it.
bool launch_route_shdown(const RouteArgs &a, const ShExpertArgs &sh, int H, hipStream_t s);
// Up to 8 tokens: the routing and the shared expert's SwiGLU-gate rows h
// [T][Fs] (sh.v's gate, up and gate-logit columns, as launch_swiglu_gate) in
// one launch; false (nothing launched) where the shapes do not allow it.
bool launch_route_shgate(const RouteArgs &a, const ShExpertArgs &sh, uint16_t *h, hipStream_t s);
// 9 to 32 tokens: partial router logits per 512-wide K slice on the fp32
// MFMA (r.part [H / 512][T][E]), then routing launches that add the slices
// in slice order (writing the sums to logits) and route as launch_route.
bool router_mfma_ok(int T, int E, int H, int kl);
void launch_router_mfma(const RouterArgs &r, int T, int E, hipStream_t s);
void launch_route_part(const RouteArgs &a, const float *part, int S, float *logits, hipStream_t s);
size_t router_lds_bytes(int T, int kl, int E);
void launch_router_route(const RouteArgs &a, const RouterArgs &r, hipStream_t s);
// The fp32 router GEMV alone (logits, no routing and no hand-off), for the
// batches whose expert GEMVs route themselves; false if the full-K router
// does not take the shape.
bool router_logits_ok(int T, int E, int H);
void launch_router_logits(const RouterArgs &r, int T, int E, hipStream_t s);
// Decode batches whose router runs as the logits launch (one block per
// expert) followed by the routing launch instead of one launch of E / 8
// blocks with the routing in its last block.
bool router_split_ok(int T, int E, int H);
// LDS bytes the slot pass needs for (T, E); the C-ABI rejects larger inputs.
void launch_route(const RouteArgs &a, hipStream_t s);

// out_type: 0 fp32, 1 bf16, 2 fp16; shared fp32, or fp16 with shared_f16.
void launch_combine(const void *yp, int yp_f16, const int32_t *tok_slot, const float *tok_w, const void *shared,
                    int shared_f16, int T, int topk, int H, void *out, int out_type, hipStream_t s);

// checkpoint order <-> tiled device format (q4_common.cuh)
void launch_tile(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, uint32_t *Wt,
                 uint16_t *St, uint16_t *Zt, hipStream_t s);
void launch_untile(const uint32_t *Wt, const uint16_t *St, const uint16_t *Zt, int64_t N, int64_t K, uint32_t *W,
                   uint16_t *S, uint32_t *Z, hipStream_t s);
bool gemv_fits(int M, int K);
void launch_unpack(const uint32_t *W, int64_t N, int64_t K, uint8_t *out, hipStream_t s);
void launch_dequant(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, float *out,
                    hipStream_t s);
void launch_bf16_to_f16(const uint16_t *in, uint16_t *out, int64_t n, hipStream_t s);
void launch_read_probe(const void *p, int64_t bytes, hipStream_t s);
void launch_from_engine_order(const uint32_t *in, uint32_t *out, int64_t n_words, hipStream_t s);

// Dense GEMV on 16-bit weights (row-major [N][ldw]; fp16 weights with fp16
// x, or bf16 with bf16).
struct W16Args {
    const uint16_t *W;
    int ldw;
    const uint16_t *x;
    int xs;
    void *y;
    int ys, y_bf16, N, K, M, accumulate, f16;
    int tiled;     // W in the layout of launch_w16_tile (ldw unused)
    int rpg = 0;   // rows per activation slice (0: one slice), as in gpu::gemv_rows
    int n_lo = 0;  // rows below n_lo are computed but not stored (internal)
};
bool w16_fits(int M, int K, int N);
void launch_w16_gemv(const W16Args &a, hipStream_t s);
void launch_w16_tile(const uint16_t *W, int64_t ldw, int N, int K, void *Wt, hipStream_t s);
// y = W h, h[m][j] = fp16(silu(v[m][j]) v[m][n + j] sigmoid(v[m][2n])) formed
// while staging (the shared expert's swiglu_T folded into its down GEMV); W
// fp16 [N][n] in the tiled layout of launch_w16_tile.
struct W16SwigluArgs {
    const uint16_t *Wt;
    const float *v;
    int ldv, n;
    void *y;
    int ys, y_bf16, N, M, accumulate;
};
bool w16_swiglu_fits(int M, int n, int N);
void launch_w16_swiglu(const W16SwigluArgs &a, hipStream_t s);
// Dense GEMV on int8 weights (tiled by launch_i8_tile from row-major [N][K])
// with an fp32 scale per group of `group` (16 or 32) along K; fp16
// activation rows, row slices of rpg rows (0: none) as in gpu::gemv_rows_i8.
struct I8Args {
    const uint4 *W;
    const float *S;
    int group;
    const uint16_t *x;
    int xs;
    void *y;
    int ys, y_bf16, N, K, M, rpg, accumulate;
};
size_t i8_lds_bytes(int M, int K, int N, int group, int rpg);
bool i8_fits(int M, int K, int N, int group, int rpg);
void launch_i8_tile(const int8_t *W8, const float *S, int N, int K, int group, uint4 *Wt, float *St, hipStream_t s);
void launch_i8_gemv(const I8Args &a, hipStream_t s);
void launch_swiglu_gate(const float *v, int ldv, int n, int T, uint16_t *h, hipStream_t s);

// W4A8 grouped expert GEMMs (moe_w4a8.hip): tiled q4 weights as for the
// grouped fp16 path, the routing tile list with 64-slot tiles, fp16 h and yp.
// qx / sx / qh / sh point into the workspace (set by launch_moe_w4a8).
struct W8Args {
    const uint32_t *gw, *uw, *dw;
    const uint16_t *gs, *gz, *us, *uz, *ds, *dz;
    int E, H, F;
    const int32_t *offsets, *pair_tok, *tile_e, *tile_m0, *n_tiles;
    uint16_t *h, *yp;
    void *ws;
    const int8_t *qx, *qh;
    const float *sx, *sh;
};
int moe_w4a8_tile_m();
size_t moe_w4a8_workspace_bytes(int T, int topk, int H, int F);
void launch_moe_w4a8(W8Args a, const uint16_t *x, int x_f16, int T, int topk, hipStream_t s);
void launch_quant_rows(const uint16_t *x, int x_f16, int64_t ldx, int rows, int K, int8_t *q, float *scale,
                       hipStream_t s);

struct GemmArgs {
    const uint32_t *W;
    const uint16_t *S;
    const uint16_t *Z;
    const uint16_t *X;
    int ldx, T;
    void *Y;
    int ldy, y_type, N, K;  // y_type: 0 fp32, 1 bf16, 2 fp16
    void *ws;  // workspace: fp16 copy of X (bf16 rows only)
    int x_f16 = 0;  // X rows are fp16 (else bf16)
};
size_t gemm_workspace_bytes(int T, int K);
// bf16 [T][ldx] -> fp16 [T][K] (saturating), the GEMMs' A operand.
void launch_x_to_f16(const uint16_t *X, int ldx, int T, int K, uint16_t *Xh, hipStream_t s);
void launch_gemm(const GemmArgs &a, hipStream_t s);

}  // namespace qwq4
