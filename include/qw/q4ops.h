/* q4ops.h -- C ABI of the MI355X (gfx950) q4 matmul path of qw.
 *
 * Drop-in operator layer for the reference engine's quantized matmul roles
 * (manuelbaez/v620-inference-engine, paths relative to that repository):
 *   qw_q4_gemv            gpu::gemv_rows            src/kernels/gemv.hpp:13-14
 *   qw_q4_gemm            gpu::gemm (rocBLAS)       src/kernels/gemm.hpp:14-15
 *   qw_moe_route          gpu::moe_route_B, and
 *                         gpu::moe_route_T + moe_scatter_T
 *                                                   src/kernels/moe.hpp:17-27
 *   qw_moe_experts_gemv   gpu::moe_experts_P        src/kernels/moe.hpp:35-37
 *   qw_moe_experts_grouped gpu::moe_experts_T       src/kernels/moe.hpp:29-32
 *   qw_moe_experts_w4a8   gpu::moe_experts_w4a8     src/kernels/moe_tiling.hpp:14-20
 *   qw_quant_rows_i8      quant_rows_kernel         src/kernels/moe_w4a8.hip:17-36
 *   qw_moe_combine        gpu::moe_combine_B/T      src/kernels/moe.hpp:42-46
 *   qw_w16_gemv           gpu::gemv_rows (fp16 W)   src/kernels/gemv.hpp:13-14
 *   qw_w16_gemv_tiled     gpu::gemv_rows (fp16 W)   src/kernels/gemv.hpp:13-14 (weights tiled at load)
 *   qw_w16_swiglu_gemv_tiled  gpu::swiglu_T + gemv_rows  src/kernels/moe_route.hip:187-197, gemv.hpp:13-14
 *                         ref::Model::linear        src/ref/ref_model.cpp:86-97
 *   qw_i8_gemv            gpu::gemv_rows_i8         src/kernels/gemv.hpp:15-23
 *   qw_swiglu_gate        gpu::swiglu_T             src/kernels/moe_route.hip:187-197
 *   qw_q4_unpack / qw_q4_dequant                    src/ref/ref_model.cpp:108-114
 *   qw_q4_from_engine_order (inverse of pack_int4_words)
 *                                                   src/engine/weight_convert.cpp:61-71
 *
 * Conventions
 *   - Every pointer is a device pointer owned by the caller; nothing here
 *     allocates, frees or synchronises, so all calls are safe under HIP graph
 *     capture. `stream` is a hipStream_t (NULL = the default stream).
 *   - Functions return 0 on success and a negative code on error:
 *       QW_Q4_EINVAL  a bad shape, stride, alignment or null pointer (nothing
 *                     was launched; qw_q4_last_error() says which);
 *       QW_Q4_ELAUNCH the HIP launch failed (hipGetLastError).
 *     Unlike the reference launchers (which return void and ignore launch
 *     errors, and silently skip an unsupported row count), no unsupported
 *     case is a silent no-op.
 *   - Calls on different streams are independent; the library holds no state
 *     beyond the per-thread error string.
 *
 * q4 weight formats
 *   Checkpoint order (compressed-tensors, docs/MODEL.md:34-37), the input of
 *   qw_q4_tile and the format of the bit-exact surface (unpack, dequant):
 *     W  uint32 [N][K/8]        element 8c+i of row n in bits 4i..4i+3 of word c
 *     S  fp16   [N][K/128]      scale per 128-element group along K
 *     Z  uint32 [N][ceil(G/8)]  4-bit zero of group g in bits 4(g%8) of word g/8
 *                               (G = K/128); NULL = zero 8 for every group, the
 *                               reference's symmetric format
 *   Tiled device order (what the matmul entry points read; written once at
 *   load time by qw_q4_tile, the way the reference repacks at load time with
 *   pack_int4_words, src/engine/weight_convert.cpp:61-71):
 *     Wt uint32, N*K/8 words     16-row x 128-column tiles, 1 KB each, in the
 *                               order one wave64 reads them (see q4_common.cuh)
 *     St fp16, Zt u16            scales and zeros regrouped per 16-row tile
 *   Sizes: qw_q4_tiled_size. weight = (q - z) * s, exactly, in fp32.
 *   K must be a multiple of 128 and N (rows) of 16. Activations are bf16
 *   (uint16 bit patterns); accumulation is fp32.
 */
#ifndef QW_Q4OPS_H
#define QW_Q4OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QW_Q4_OK 0
#define QW_Q4_EINVAL (-1)
#define QW_Q4_ELAUNCH (-2)

/* Element types of outputs and intermediates that take more than one
 * (arguments named *_type). */
#define QW_T_F32 0
#define QW_T_BF16 1
#define QW_T_F16 2

/* Version of this ABI (bumped on any signature change). */
int qw_q4_abi_version(void);

/* Message for the last error returned on this thread ("" if none). */
const char *qw_q4_last_error(void);

/* Load-time repack to the tiled device format (role of pack_int4_words,
 * src/engine/weight_convert.cpp:61-71), its inverse, and the buffer sizes.
 * Z may be NULL (then Zt is not written / not read). */
void qw_q4_tiled_size(int64_t N, int64_t K, size_t *wt_bytes, size_t *st_bytes, size_t *zt_bytes);
int qw_q4_tile(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, uint32_t *Wt,
               uint16_t *St, uint16_t *Zt, void *stream);
int qw_q4_untile(const uint32_t *Wt, const uint16_t *St, const uint16_t *Zt, int64_t N, int64_t K, uint32_t *W,
                 uint16_t *S, uint32_t *Z, void *stream);

/* Decode GEMV (replaces gpu::gemv_rows, src/kernels/gemv.hpp:13-14), tiled
 * weights (Wt, St, Zt or NULL):
 *   y[m*ys + n] (+)= sum_k W[n][k] * x[m*xs + off(n) + k],   m < M, n < N
 * off(n) = (n / rpg) * K when rpg > 0 (row n reads activation slice n / rpg:
 * the engine's hyper-connection down projection, src/engine/decode.hip:55-59),
 * else 0. rpg 0 or >= 16, at most 64 slices (each runs as one launch; rpg need
 * not be a multiple of 16).
 * x rows of stride xs (elements, a multiple of 8, x 16-byte aligned; with
 * M > 1 and rpg > 0, xs covers every slice): bf16 (x_f16 = 0) or fp16
 * (x_f16 = 1, the engine's decode rows, src/kernels/gemv.hpp:11-14); y fp32
 * (y_bf16 = 0) or bf16 (y_bf16 = 1, round to nearest even) rows of stride ys;
 * accumulate != 0 adds to y. 1 <= M <= 32. Every product is exact, sums in
 * fp32. */
int qw_q4_gemv(const uint32_t *W, const uint16_t *S, const uint16_t *Z, const uint16_t *x, int x_f16, int xs, void *y,
               int ys, int y_bf16, int N, int K, int M, int rpg, int accumulate, void *stream);

/* Dense GEMV on 16-bit weights (the role of gpu::gemv_rows with fp16
 * weights, src/kernels/gemv.hpp:13-14, which the engine runs the shared
 * expert's projections through, src/engine/decode.hip:99-101; and of
 * ref::Model::linear on bf16 weights, src/ref/ref_model.cpp:86-97):
 *   y[m*ys + n] (+)= sum_k W[n*ldw + k] * x[m*xs + off(n) + k],   m < M, n < N
 * f16 = 1: W and x fp16; f16 = 0: W and x bf16 (the MFMA takes matching
 * types; every product is exact, sums in fp32). W row-major, ldw >= K a
 * multiple of 8, 16-byte aligned; K a multiple of 32; any N >= 1; x rows of
 * stride xs and row slices (rpg, off(n)) as in qw_q4_gemv; y fp32 or bf16
 * (y_bf16). 1 <= M <= 32. */
int qw_w16_gemv(const uint16_t *W, int ldw, const uint16_t *x, int xs, int f16, void *y, int ys, int y_bf16, int N,
                int K, int M, int rpg, int accumulate, void *stream);

/* Bytes of the tiled layout of a 16-bit [N][K] matrix (N padded to a
 * multiple of 16 rows). */
size_t qw_w16_tiled_size(int N, int K);

/* Load-time conversion of a 16-bit row-major [N][ldw] matrix (fp16 or bf16,
 * the bits are moved unchanged) into the tiled layout qw_w16_gemv_tiled
 * reads: each 32-element step of a 16-row tile is one contiguous 1 KB piece,
 * so every wave load of the GEMV is contiguous (the row-major GEMV's loads
 * take 64 bytes from each of 16 rows). No counterpart in the reference, whose
 * gemv_rows reads the row-major matrix (src/kernels/gemv.hip:7-42); the
 * engine's loader would call it once per matrix, as it converts q4 weights
 * (src/engine/weight_convert.cpp:61-71). Device buffers, 16-byte aligned;
 * ldw >= K a multiple of 8, K a multiple of 32, N >= 1. */
int qw_w16_tile(const uint16_t *W, int ldw, int N, int K, void *Wt, void *stream);

/* qw_w16_gemv on weights in the tiled layout (qw_w16_tile); the same
 * arguments and results, bit for bit, without ldw. */
int qw_w16_gemv_tiled(const void *Wt, const uint16_t *x, int xs, int f16, void *y, int ys, int y_bf16, int N, int K,
                      int M, int rpg, int accumulate, void *stream);

/* The shared expert's SwiGLU x gate folded into its down projection: the
 * result of qw_swiglu_gate(v, ldv, n, M, h) followed by
 * qw_w16_gemv_tiled(Wt, h, n, 1, y, ys, y_bf16, N, n, M, accumulate), bit for
 * bit, in one launch and without h:
 *   h[m][j] = fp16(silu(v[m][j]) * v[m][n + j] * sigmoid(v[m][2n]))
 *   y[m*ys + i] (+)= sum_j Wt[i][j] * h[m][j],   i < N, m < M
 * Replaces swiglu_T + gemv_rows (src/kernels/moe_route.hip:187-197,
 * src/engine/decode.hip:99-101), which the reference runs as two launches.
 * Wt: fp16 [N][n] tiled by qw_w16_tile (16-byte aligned); v fp32 [M][ldv]
 * (ldv >= 2n + 1); n a multiple of 32; y fp32 or bf16; 1 <= M <= 32. Every
 * block forms all of h, so this is the faster form up to about 4 rows; with
 * more rows the two launches (h formed once) are faster. */
int qw_w16_swiglu_gemv_tiled(const void *Wt, const float *v, int ldv, int n, void *y, int ys, int y_bf16, int N, int M,
                             int accumulate, void *stream);

/* Dense GEMV on int8 weights (replaces gpu::gemv_rows_i8,
 * src/kernels/gemv.hpp:15-23, src/kernels/gemv.hip:75-136; the engine's int8
 * copy of its dense weights, src/engine/decode.hip:52-70,119-125):
 *   y[m*ys + n] (+)= sum_g scale[n][g] * sum_{k in group g} W8[n][k] * x[m*xs + off(n) + k]
 * off(n) = (n / rpg) * K when rpg > 0 (row n reads activation slice n / rpg),
 * else 0. Wt / St: the weights and scales in the kernel format written by
 * qw_i8_tile, both 16-byte aligned; group 16 or 32 (the reference's
 * I8_GROUP); K a multiple of 64; any N >= 1; rpg 0 or >= 16; x fp16 rows of
 * stride xs (a multiple of 8, covering every slice when M > 1), 16-byte
 * aligned; y fp32 or bf16 (y_bf16). 1 <= M <= 32. Each group's int8 x fp16
 * products are exact and summed in fp32, then scaled, as in the reference. */
int qw_i8_gemv(const void *Wt, const float *St, int group, const uint16_t *x, int xs, void *y, int ys, int y_bf16,
               int N, int K, int M, int rpg, int accumulate, void *stream);

/* Bytes of the kernel format of an int8 [N][K] matrix: weights (Wt) and
 * scales (St). N is padded to a multiple of 16 rows. */
void qw_i8_tiled_size(int N, int K, int group, size_t *w_bytes, size_t *s_bytes);

/* Load-time conversion (the role pack_int4_words plays for q4,
 * src/engine/weight_convert.cpp:61-71): W8 int8 row-major [N][K] and scale
 * fp32 [N][K / group], as quantize_rows_i8 writes them
 * (src/engine/weight_convert.cpp:92-108), into Wt / St (sizes from
 * qw_i8_tiled_size). Device buffers; W8 8-byte aligned, Wt 16-byte aligned. */
int qw_i8_tile(const int8_t *W8, const float *scale, int N, int K, int group, void *Wt, float *St, void *stream);

/* The shared expert's activation (replaces gpu::swiglu_T,
 * src/kernels/moe_route.hip:187-197; math of src/ref/ref_model.cpp:468-476):
 *   h[t][j] = fp16(silu(v[t][j]) * v[t][n + j] * sigmoid(v[t][2n]))
 * v fp32 [T][ldv] (ldv >= 2n + 1): the output of the fused gate / up /
 * gate-logit projection; h fp16 [T][n], finite values beyond +-65504
 * saturate. */
int qw_swiglu_gate(const float *v, int ldv, int n, int T, uint16_t *h, void *stream);

/* Prefill GEMM (replaces gpu::gemm, src/kernels/gemm.hpp:14-15, with tiled
 * q4 weights): Y[t][n] = sum_k X[t][k] * W[n][k], t < T. X rows of stride
 * ldx, bf16 (x_f16 = 0) or fp16 (x_f16 = 1, the reference's prefill rows);
 * Y rows of stride ldy, y_type QW_T_F32, QW_T_BF16 (round to nearest even)
 * or QW_T_F16 (the reference's f16_out, which the engine passes for most
 * prefill projections, src/engine/prefill.hip:218-334: round to nearest
 * even, finite values beyond +-65504 saturate). For bf16 rows, `workspace` (device
 * memory of at least qw_q4_gemm_workspace_size(T, K) bytes, 256-byte
 * aligned) is scratch for the fp16 pre-pass; it holds nothing between calls.
 * fp16 rows need none (workspace may be NULL).
 * Numerics: X runs through the MFMAs as fp16 (the reference's prefill rows
 * are fp16, src/engine/prefill.hip): exact for |x| in the fp16 normal range;
 * finite |x| > 65504 saturates to +-65504, infinities and NaN pass through
 * (a NaN in row t makes row t of Y NaN); weights are fp16((q - z) * s);
 * sums in fp32. */
size_t qw_q4_gemm_workspace_size(int T, int K);
int qw_q4_gemm(const uint32_t *W, const uint16_t *S, const uint16_t *Z, const uint16_t *X, int x_f16, int ldx, int T,
               void *Y, int ldy, int y_type, int N, int K, void *workspace, size_t workspace_bytes, void *stream);

/* Routing of T tokens over E experts (replaces gpu::moe_route_B for decode
 * rows and gpu::moe_route_T + moe_scatter_T for prefill, moe.hpp:17-27; math
 * of ref::Model::moe, src/ref/ref_model.cpp:412-431):
 *   p = expf(l - max l) (the C library's expf, evaluated bit for bit on the
 *   device); top k by (p desc, index asc);
 *   top_w = float(p / sum of the k selected p, in double)
 * Outputs (all device int32 unless noted):
 *   top_e [T][k], top_w [T][k] (fp32), counts [E], offsets [E+1],
 *   tok_slot [T][k] (slot of each selection), pair_tok [T*k] (token of each
 *   slot), active [E] (experts with pairs, ascending; first *n_active valid),
 *   n_active [1].
 * Slots are deterministic: experts ascending, tokens ascending within one.
 * tile_m != 0 also writes a tile list (for qw_moe_experts_grouped): per
 * expert ascending, tiles over its slots offsets[e] + m0 ..:
 *   tile_e, tile_m0 [T*k/|tile_m| + E], n_tiles [1]  (tile_m 0: may be NULL).
 *   tile_m > 0: tiles of tile_m slots. tile_m = -g (mixed): the tile starting
 *   rem slots before the end of the expert's range has 4g slots when rem > 5g,
 *   else rem rounded up to a multiple of g (whole 4g tiles, then one tile for
 *   the rest, a rest of at most g joining the last whole tile).
 * Limits: 1 <= k <= min(E, 64), E <= 1024, T * k < 2^30. Above 16 tokens the
 * slots are assigned by one block per 64 tokens. */
int qw_moe_route(const float *logits, int T, int E, int topk, int tile_m, int32_t *top_e, float *top_w,
                 int32_t *counts, int32_t *offsets, int32_t *tok_slot, int32_t *pair_tok, int32_t *active,
                 int32_t *n_active, int32_t *tile_e, int32_t *tile_m0, int32_t *n_tiles, void *stream);

/* Gathered per-expert GEMVs for decode batches (replaces gpu::moe_experts_P,
 * moe.hpp:35-37). For every slot p of expert e (from qw_moe_route):
 *   h[p]  = silu(G_e x[pair_tok[p]]) * (U_e x[pair_tok[p]])     fp16 [T*k][F]
 *   yp[p] = D_e h[p]                             fp32 or fp16 [T*k][H]
 * yp fp32 (yp_f16 = 0) or fp16 (yp_f16 = 1: the reference's moe_experts_P
 * output, src/kernels/moe.hpp:35-37, and the engine's b.yp buffer; round to
 * nearest even, finite values beyond +-65504 saturate), 4-byte aligned.
 * Weights are tiled (qw_q4_tile) over the stacked experts: gate and up as one
 * [E*F][H] matrix each, down as [E*H][F]; zeros may be NULL. x [T][H], bf16
 * (x_f16 = 0) or fp16 (x_f16 = 1).
 * F and H multiples of 128. 1 <= T <= 32. Each expert's weights are read
 * once per call however many of the batch's tokens chose it. */
int qw_moe_experts_gemv(const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                        const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                        const uint16_t *dz, int E, int H, int F, const int32_t *offsets, const int32_t *active,
                        const int32_t *n_active, const int32_t *pair_tok, const uint16_t *x, int x_f16, int T,
                        int topk, uint16_t *h, void *yp, int yp_f16, void *stream);

/* Grouped per-expert GEMMs for prefill chunks (replaces gpu::moe_experts_T,
 * moe.hpp:29-32): the same outputs as qw_moe_experts_gemv for any T, over
 * the (expert, tile) list qw_moe_route writes when called with
 * tile_m = qw_moe_grouped_tile_m() (mixed tiles, -32: 32 to 160 slots). x [T][H] bf16 (x_f16 = 0) or fp16 (x_f16 = 1). For bf16 x,
 * workspace: at least qw_moe_grouped_workspace_size(...) bytes (an fp16
 * copy of x), 256-byte aligned; fp16 x needs none. x and h pass through fp16 as in qw_q4_gemm (finite
 * values beyond +-65504 saturate, infinities and NaN pass through). yp
 * [T*k][H] (16-byte aligned) is fp32 (yp_f16 = 0) or fp16 (yp_f16 = 1, the
 * reference's choice, src/kernels/moe.hpp:20-25: half the bytes written by
 * the down GEMM and read by the combine; finite values beyond +-65504
 * saturate). H a multiple of 8. */
int qw_moe_grouped_tile_m(void);
size_t qw_moe_grouped_workspace_size(int T, int topk, int E, int H, int F);
int qw_moe_experts_grouped(const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                           const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                           const uint16_t *dz, int E, int H, int F, const int32_t *offsets, const int32_t *pair_tok,
                           const int32_t *tile_e, const int32_t *tile_m0, const int32_t *n_tiles, const uint16_t *x,
                           int x_f16, int T, int topk, uint16_t *h, void *yp, int yp_f16, void *workspace,
                           size_t workspace_bytes, void *stream);

/* W4A8 grouped expert GEMMs (replaces gpu::moe_experts_w4a8,
 * src/kernels/moe_tiling.hpp:14-20, src/kernels/moe_w4a8.hip:13-215: the
 * reference's opt-in int8-activation path, lossy by design). Activation rows
 * are quantised per (row, 128-group) as qw_quant_rows_i8 does; weights are
 * widened exactly to int8 q - z; per 64-wide K step the products are summed
 * in int32 and added as fp32 float(I) * s_w * s_x. Gate/up write
 *   h[p] = fp16(silu(g) * u)                     fp16 [T*k][F]
 * and the down projection, on h quantised the same way,
 *   yp[p] = fp16(D_e . h[p])                     fp16 [T*k][H]
 * (finite values beyond +-65504 saturate). Weights tiled as for
 * qw_moe_experts_grouped; tile list from qw_moe_route with
 * tile_m = qw_moe_w4a8_tile_m() (the grouped path's list: -32, mixed tiles
 * of 32 to 160 slots). The int32 sums run per 128-wide group (the reference:
 * per 64-wide step; the fp32 rescale roundings differ by about 1e-7 of the
 * result). x [T][H] fp16 (x_f16 = 1,
 * the reference's rows) or bf16. H and F multiples of 128. workspace: at
 * least qw_moe_w4a8_workspace_size(T, topk, H, F) bytes, 256-byte aligned
 * (the quantised rows and their scales, the reference's q8 / q8s). */
int qw_moe_w4a8_tile_m(void);
size_t qw_moe_w4a8_workspace_size(int T, int topk, int H, int F);
int qw_moe_experts_w4a8(const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                        const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                        const uint16_t *dz, int E, int H, int F, const int32_t *offsets, const int32_t *pair_tok,
                        const int32_t *tile_e, const int32_t *tile_m0, const int32_t *n_tiles, const uint16_t *x,
                        int x_f16, int T, int topk, uint16_t *h, uint16_t *yp, void *workspace, size_t workspace_bytes,
                        void *stream);

/* The W4A8 activation quantiser (quant_rows_kernel,
 * src/kernels/moe_w4a8.hip:17-36): per row and group of 128 along K,
 *   scale[r][g] = max|x| / 127 (1 for an all-zero group),
 *   q[r][k] = rint(x[r][k] * (1 / scale[r][g]))   (round half to even)
 * x rows of stride ldx (elements), fp16 (x_f16 = 1) or bf16; q int8 [rows][K],
 * scale fp32 [rows][K / 128]. K a multiple of 128. */
int qw_quant_rows_i8(const uint16_t *x, int x_f16, int rows, int K, int ldx, int8_t *q, float *scale, void *stream);

/* Weighted combine (replaces gpu::moe_combine_B/T, moe.hpp:42-46):
 *   out[t][j] = shared[t][j] + sum_{i<k, slot >= 0} tok_w[t][i] * yp[tok_slot[t][i]][j]
 * yp fp32 (yp_f16 = 0) or fp16 (yp_f16 = 1); shared [T][H] fp32
 * (shared_f16 = 0, moe_combine_B) or fp16 (shared_f16 = 1, moe_combine_T),
 * or NULL; out of out_type QW_T_F32 (moe_combine_B), QW_T_F16 (moe_combine_T;
 * round to nearest even, finite values beyond +-65504 saturate) or QW_T_BF16.
 * A negative slot (a selection another rank holds, in the reference's
 * expert-parallel layout) adds nothing, as in the reference. H % 4 == 0.
 * Sums in fp32: the shared value, then the selections in order. */
int qw_moe_combine(const void *yp, int yp_f16, const int32_t *tok_slot, const float *tok_w, const void *shared,
                   int shared_f16, int T, int topk, int H, void *out, int out_type, void *stream);

/* Format surface (bit-exact): nibbles as bytes [N][K]; dequantised fp32
 * weights [N][K]; reference-engine word order -> checkpoint word order. */
int qw_q4_unpack(const uint32_t *W, int64_t N, int64_t K, uint8_t *out, void *stream);
int qw_q4_dequant(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, float *out,
                  void *stream);
int qw_q4_from_engine_order(const uint32_t *in, uint32_t *out, int64_t n_words, void *stream);

/* A routed-MoE decode block in three to six launches (the engine's decode step calls
 * router GEMV -> route -> experts -> combine back to back, src/engine/decode.hip:99-111;
 * math of ref::Model::moe, src/ref/ref_model.cpp:406-463):
 *   logits = x . router_w^T, router_w [E][H] fp32 (router_f16 = 0, the reference
 *   model's fp32 router) or fp16 (router_f16 = 1, the engine's w.router, which
 *   decode.hip:101 runs through gemv_rows); fp16 weights are widened exactly, so
 *   fp16 weights and fp32 weights holding the same values give the same bits;
 *   sums in fp32;
 *   routing as qw_moe_route; experts as qw_moe_experts_gemv;
 *   out[t] = shared[t] + sum_i top_w[t][i] * yp[tok_slot[t][i]]   (out_type)
 * Launches: at T = 1 the router writes the logits and the gate/up blocks
 * route; at T = 2..8 the logits launch is followed by the routing launch;
 * at 9..32 partial logits per 512-wide K slice come from the fp32 MFMA and
 * the routing launch adds them (slice order); elsewhere the router GEMV and
 * routing share a launch. Up to T = 2 the
 * combine runs inside the down projection, above that in a launch of its own. Outputs: out
 * (QW_T_F32, the engine's moe_combine_B rows, QW_T_BF16 or QW_T_F16), logits
 * [T][E], top_e, top_w, tok_slot [T][k], h, yp (fp32 or fp16 with yp_f16, as
 * qw_moe_experts_gemv; the combine adds the values yp holds). shared fp32 [T][H] or NULL (e.g. the shared
 * expert's output). x [T][H] bf16 (x_f16 = 0) or fp16 (x_f16 = 1). 1 <= T <= 32.
 * workspace: qw_moe_decode_workspace_size(...) bytes, 256-byte aligned, filled
 * with zeros once before its first use (it holds completion counters that
 * every call leaves at zero); calls that share a workspace must not overlap. */
size_t qw_moe_decode_workspace_size(int T, int E, int topk, int H, int F);
int qw_moe_decode(const void *router_w, int router_f16, const uint16_t *x, int x_f16, int T, int E, int topk,
                  const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us,
                  const uint16_t *uz,
                  const uint32_t *dw, const uint16_t *ds, const uint16_t *dz, int H, int F, const float *shared,
                  void *out, int out_type, float *logits, int32_t *top_e, float *top_w, int32_t *tok_slot,
                  uint16_t *h, void *yp, int yp_f16, void *workspace, size_t workspace_bytes, void *stream);

/* qw_moe_decode with the shared expert (the engine's decode.hip:98-101 before
 * the routed block): sh_v = sh_gu x ([T][2 Fs + 1] fp32: gate, up and gate
 * logit rows, the engine's b.shp), sh_out = sh_down swiglu_gate(sh_v) ([T][H]
 * fp32, the engine's b.sh_out), and out = sh_out + the routed experts'
 * combine. sh_gu [2 Fs + 1][H] is tiled 16-bit (qw_w16_tile) of x's type
 * (fp16 with x_f16 = 1, bf16 else); sh_down [H][Fs] is tiled fp16; the
 * arithmetic is that of qw_w16_gemv_tiled and qw_w16_swiglu_gemv_tiled (up
 * to T = 4; qw_swiglu_gate + qw_w16_gemv_tiled above, the same values)
 * followed by qw_moe_decode with shared = sh_out, bit for bit. Up
 * to T = 8 the shared expert's gate/up GEMV runs in the router-logits launch
 * and its down GEMV in the routed gate/up launch (T = 1) or the routing
 * launch (T = 2 to 4; from 5 the routing launch forms the SwiGLU rows and
 * the down GEMV rides in the experts' gate/up launch, as it does above 8
 * tokens where the LDS allows), instead of launches of their own. Fs a multiple of 32. workspace:
 * qw_moe_decode_with_shared_workspace_size(...) bytes (that of qw_moe_decode
 * plus T * Fs * 2), zeroed once as for qw_moe_decode. */
size_t qw_moe_decode_with_shared_workspace_size(int T, int E, int topk, int H, int F, int Fs);
int qw_moe_decode_with_shared(const void *router_w, int router_f16, const uint16_t *x, int x_f16, int T, int E,
                              int topk, const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                              const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                              const uint16_t *dz, int H, int F, const void *sh_gu, const void *sh_down, int Fs,
                              float *sh_v, float *sh_out, void *out, int out_type, float *logits, int32_t *top_e,
                              float *top_w, int32_t *tok_slot, uint16_t *h, void *yp, int yp_f16, void *workspace,
                              size_t workspace_bytes, void *stream);

/* qw_moe_decode without a workspace argument: it allocates nothing and
 * needs no caller scratch. No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops). The scratch (completion counters, partial router
 * logits, routing arrays) is one library-held device array per GPU of
 * qw_moe_decode_static_max_bytes() = 4 MiB, kept until the process ends.
 * Every shape qw_moe_decode accepts fits (T <= 32, E <= 1024, k <= 64 and
 * the supported H, F: at most about 3.97 MB). The completion counters start
 * at zero (the array is zero when the library loads) and every completed call
 * leaves them at zero. A call that returns QW_Q4_ELAUNCH after some of its
 * kernels were enqueued enqueues a clearing kernel behind them; after any
 * other failure of the device work (a kernel fault, a capture that was
 * abandoned mid-call), call qw_moe_decode_static_reset before the next call.
 * All calls on one GPU share the array: calls that overlap on one GPU (on
 * different streams, or from different threads) race and must not be
 * issued. */
size_t qw_moe_decode_static_max_bytes(void);
int qw_moe_decode_static(const void *router_w, int router_f16, const uint16_t *x, int x_f16, int T, int E, int topk,
                         const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                         const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                         const uint16_t *dz, int H, int F, const float *shared, void *out, int out_type,
                         float *logits, int32_t *top_e, float *top_w, int32_t *tok_slot, uint16_t *h, void *yp,
                         int yp_f16, void *stream);
/* Clears the completion counters of the current GPU's static scratch (one
 * small kernel on `stream`; no allocation, no memset node). */
int qw_moe_decode_static_reset(void *stream);

/* Scale conversion as the reference does it at load (weight_convert.cpp:19-26):
 * bf16 -> fp16 bits, magnitudes above 65504 saturated, round to nearest even. */
int qw_bf16_to_f16(const uint16_t *in, uint16_t *out, int64_t n, void *stream);

/* Measurement aid, no counterpart in the reference: reads `bytes` (a multiple
 * of 32768) at p with the dense GEMV's load shape and computes nothing; with
 * bytes == 0 it launches one empty block. Benchmarks time it beside the GEMV
 * to show the per-launch floor and the read-only ceiling of one launch. */
int qw_read_probe(const void *p, int64_t bytes, void *stream);

/* ---- Checkpoint loading (role of the reference's loader, src/core/safetensors.cpp
 * and src/engine/weights.hip:352-402).
 * A safetensors file, mapped read-only and indexed by tensor name. */
typedef struct qw_st_file qw_st_file;
int qw_st_open(const char *path, qw_st_file **out);
void qw_st_close(qw_st_file *f);
/* Number of tensors and the i-th name (sorted), for listing. */
int qw_st_count(const qw_st_file *f);
const char *qw_st_name(const qw_st_file *f, int i);
/* One tensor's header entry: dtype ("I32", "BF16", ...; dtype holds >= 16
 * bytes), shape (up to 8 dims), and its bytes in the mapping (host memory). */
int qw_st_tensor(const qw_st_file *f, const char *name, char *dtype, int64_t *shape, int *ndim, const void **data,
                 size_t *nbytes);

/* One compressed-tensors q4 projection, "<prefix>.weight_packed" (I32
 * [N][K/8], checkpoint order) and "<prefix>.weight_scale" (BF16 or F16
 * [N][K/128]), straight into the tiled device format (symmetric: zero 8, Zt
 * not written). Wt/St may point inside a larger tiled matrix (stacked
 * experts): see qw_q4_tiled_offset. `staging` is device memory of at least
 * qw_q4_load_staging_size(N, K) bytes, 256-byte aligned, in use until the
 * stream's work is done. The copy from the mapping is synchronous. */
size_t qw_q4_load_staging_size(int64_t N, int64_t K);
int qw_q4_load(const qw_st_file *f, const char *prefix, int64_t N, int64_t K, uint32_t *Wt, uint16_t *St, void *staging,
               size_t staging_bytes, void *stream);
/* Byte offsets of row row0 (a multiple of 16) inside tiled Wt, St, Zt of K
 * columns: expert e of a stacked [E*F][K] matrix starts at row e*F. */
void qw_q4_tiled_offset(int64_t row0, int64_t K, size_t *wt_off, size_t *st_off, size_t *zt_off);

/* ---- Converted-weights cache (role of the reference's WeightCache,
 * src/engine/weights.hip:26-164): the buffers a load fills, in order, kept in
 * one file; the next load with the same key uploads them instead of reading
 * and converting the checkpoint. `key` identifies the checkpoint (the caller
 * hashes its files, sizes and conversion options); the library adds its own
 * tiled-layout version. qw_wcache_open never fails on a missing, stale or
 * damaged file: *mode = 2 (replaying) when `path` is a complete cache with this
 * key, else 1 (recording into "<path>.tmp", renamed by qw_wcache_finish), or
 * 0 (off; qw_q4_last_error says why). put/get copy synchronously on `stream`
 * (load time only, not capture-safe); src/dst are device memory when
 * on_device, else host memory. put is a no-op unless recording; get fails
 * (EINVAL) unless replaying a piece of exactly `bytes` bytes. */
typedef struct qw_wcache qw_wcache;
int qw_wcache_open(const char *path, uint64_t key, qw_wcache **out, int *mode);
int qw_wcache_put(qw_wcache *c, const void *src, size_t bytes, int on_device, void *stream);
int qw_wcache_get(qw_wcache *c, void *dst, size_t bytes, int on_device, void *stream);
/* Recording: completes and renames the file. Replaying: fails unless every
 * piece was read. */
int qw_wcache_finish(qw_wcache *c);
void qw_wcache_close(qw_wcache *c);

#ifdef __cplusplus
}
#endif

#endif /* QW_Q4OPS_H */
