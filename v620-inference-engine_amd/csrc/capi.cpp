// C-ABI layer (include/qw/q4ops.h): argument checks, then one launch per
// kernel on the caller's stream. Nothing here allocates or synchronises.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "q4_kernels.hpp"
#include "qw/q4ops.h"
#include "st_loader.hpp"
#include "wcache.hpp"

struct qw_wcache {
    qwq4::WCache c;
    std::vector<unsigned char> host;  // staging of device pieces being recorded
};

struct qw_st_file {
    qwq4::StFile f;
    std::vector<const qwq4::StTensor *> order;
};

namespace {

thread_local std::string g_err;

int fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return QW_Q4_EINVAL;
}

int launched(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_err = std::string(what) + ": " + hipGetErrorString(e);
        return QW_Q4_ELAUNCH;
    }
    g_err.clear();
    return QW_Q4_OK;
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

hipStream_t st(void *s) { return static_cast<hipStream_t>(s); }

#define REQUIRE(cond, ...)                             \
    do {                                               \
        if (!(cond)) return fail(__VA_ARGS__);         \
    } while (0)

int check_q4(const char *fn, const uint32_t *W, const uint16_t *S, int64_t N, int64_t K) {
    REQUIRE(W && S, "%s: null weight or scale pointer", fn);
    REQUIRE(N >= 16 && N % 16 == 0, "%s: N = %lld must be a positive multiple of 16", fn, (long long)N);
    REQUIRE(K >= 128 && K % 128 == 0, "%s: K = %lld must be a positive multiple of 128", fn, (long long)K);
    REQUIRE(aligned(W, 16), "%s: W must be 16-byte aligned", fn);
    REQUIRE(aligned(S, 8), "%s: S must be 8-byte aligned", fn);
    return 0;
}

// checkpoint-order arguments of the format functions (N any, K % 8 or 128)
int check_ckpt(const char *fn, const uint32_t *W, const uint16_t *S, int64_t N, int64_t K) {
    REQUIRE(W && S, "%s: null weight or scale pointer", fn);
    REQUIRE(N >= 1, "%s: N = %lld must be >= 1", fn, (long long)N);
    REQUIRE(K >= 128 && K % 128 == 0, "%s: K = %lld must be a positive multiple of 128", fn, (long long)K);
    REQUIRE(aligned(W, 16) && aligned(S, 2), "%s: W must be 16-byte aligned", fn);
    return 0;
}

// Activation rows and row grouping of the dense GEMVs: rpg = 0 (every row
// reads x[m * xs ...]) or rpg >= 16 rows per slice (row n reads slice n / rpg
// at x + m * xs + (n / rpg) * K, gpu::gemv_rows, src/kernels/gemv.hpp:11-14);
// at most 64 slices (one launch each). With more than one row, the stride
// covers every slice.
int check_rpg(const char *fn, int rpg, int N, int K, int M, const void *x, int xs) {
    REQUIRE(rpg == 0 || rpg >= 16, "%s: rpg = %d (need 0 or >= 16)", fn, rpg);
    const int64_t slices = rpg > 0 ? (int64_t(N) + rpg - 1) / rpg : 1;
    REQUIRE(slices <= 64, "%s: rpg = %d gives %lld slices of N = %d (at most 64)", fn, rpg, (long long)slices, N);
    REQUIRE(xs >= K && xs % 8 == 0 && aligned(x, 16) && (M == 1 || int64_t(xs) >= slices * K),
            "%s: x stride %d must be >= K, a multiple of 8 and cover %lld slices of K = %d, x 16-byte aligned", fn, xs,
            (long long)slices, K);
    return 0;
}

}  // namespace

extern "C" {

int qw_q4_abi_version(void) { return 5; }

const char *qw_q4_last_error(void) { return g_err.c_str(); }

int qw_q4_gemv(const uint32_t *W, const uint16_t *S, const uint16_t *Z, const uint16_t *x, int x_f16, int xs, void *y,
               int ys, int y_bf16, int N, int K, int M, int rpg, int accumulate, void *stream) {
    if (int r = check_q4("qw_q4_gemv", W, S, N, K)) return r;
    REQUIRE(x && y, "qw_q4_gemv: null x or y");
    REQUIRE(M >= 1 && M <= 32, "qw_q4_gemv: M = %d outside 1..32", M);
    if (int r = check_rpg("qw_q4_gemv", rpg, N, K, M, x, xs)) return r;
    REQUIRE(ys >= N || M == 1, "qw_q4_gemv: y stride %d < N", ys);
    REQUIRE(aligned(y, y_bf16 ? 2 : 4), "qw_q4_gemv: y misaligned");
    qwq4::GemvArgs a{W, S, Z, x, xs, y, ys, y_bf16 != 0, N, K, M, accumulate != 0};
    a.x_f16 = x_f16 != 0;
    a.rpg = rpg;
    qwq4::launch_gemv(a, st(stream));
    return launched("qw_q4_gemv");
}

int qw_w16_gemv(const uint16_t *W, int ldw, const uint16_t *x, int xs, int f16, void *y, int ys, int y_bf16, int N,
                int K, int M, int rpg, int accumulate, void *stream) {
    REQUIRE(W && x && y, "qw_w16_gemv: null W, x or y");
    REQUIRE(N >= 1 && K >= 32 && K % 32 == 0, "qw_w16_gemv: N = %d, K = %d (need N >= 1, K a positive multiple of 32)",
            N, K);
    REQUIRE(ldw >= K && ldw % 8 == 0 && aligned(W, 16), "qw_w16_gemv: ldw %d must be >= K, a multiple of 8, W 16-byte aligned", ldw);
    REQUIRE(M >= 1 && M <= 32, "qw_w16_gemv: M = %d outside 1..32", M);
    if (int r = check_rpg("qw_w16_gemv", rpg, N, K, M, x, xs)) return r;
    REQUIRE(ys >= N || M == 1, "qw_w16_gemv: y stride %d < N", ys);
    REQUIRE(aligned(y, y_bf16 ? 2 : 4), "qw_w16_gemv: y misaligned");
    qwq4::W16Args a{W, ldw, x, xs, y, ys, y_bf16 != 0, N, K, M, accumulate != 0, f16 != 0, 0};
    a.rpg = rpg;
    qwq4::launch_w16_gemv(a, st(stream));
    return launched("qw_w16_gemv");
}

size_t qw_w16_tiled_size(int N, int K) {
    return N > 0 && K > 0 ? size_t((N + 15) / 16) * 16 * size_t(K) * 2 : 0;
}

int qw_w16_tile(const uint16_t *W, int ldw, int N, int K, void *Wt, void *stream) {
    REQUIRE(W && Wt, "qw_w16_tile: null W or Wt");
    REQUIRE(N >= 1 && K >= 32 && K % 32 == 0, "qw_w16_tile: N = %d, K = %d (need N >= 1, K a positive multiple of 32)",
            N, K);
    REQUIRE(ldw >= K && ldw % 8 == 0 && aligned(W, 16) && aligned(Wt, 16),
            "qw_w16_tile: ldw %d must be >= K, a multiple of 8; W and Wt 16-byte aligned", ldw);
    qwq4::launch_w16_tile(W, ldw, N, K, Wt, st(stream));
    return launched("qw_w16_tile");
}

int qw_w16_gemv_tiled(const void *Wt, const uint16_t *x, int xs, int f16, void *y, int ys, int y_bf16, int N, int K,
                      int M, int rpg, int accumulate, void *stream) {
    REQUIRE(Wt && x && y, "qw_w16_gemv_tiled: null Wt, x or y");
    REQUIRE(N >= 1 && K >= 32 && K % 32 == 0,
            "qw_w16_gemv_tiled: N = %d, K = %d (need N >= 1, K a positive multiple of 32)", N, K);
    REQUIRE(aligned(Wt, 16), "qw_w16_gemv_tiled: Wt must be 16-byte aligned");
    REQUIRE(M >= 1 && M <= 32, "qw_w16_gemv_tiled: M = %d outside 1..32", M);
    if (int r = check_rpg("qw_w16_gemv_tiled", rpg, N, K, M, x, xs)) return r;
    REQUIRE(ys >= N || M == 1, "qw_w16_gemv_tiled: y stride %d < N", ys);
    REQUIRE(aligned(y, y_bf16 ? 2 : 4), "qw_w16_gemv_tiled: y misaligned");
    qwq4::W16Args a{static_cast<const uint16_t *>(Wt), K, x, xs, y, ys, y_bf16 != 0, N, K, M, accumulate != 0,
                    f16 != 0, 1};
    a.rpg = rpg;
    qwq4::launch_w16_gemv(a, st(stream));
    return launched("qw_w16_gemv_tiled");
}

int qw_w16_swiglu_gemv_tiled(const void *Wt, const float *v, int ldv, int n, void *y, int ys, int y_bf16, int N, int M,
                             int accumulate, void *stream) {
    REQUIRE(Wt && v && y, "qw_w16_swiglu_gemv_tiled: null Wt, v or y");
    REQUIRE(N >= 1 && n >= 32 && n % 32 == 0,
            "qw_w16_swiglu_gemv_tiled: N = %d, n = %d (need N >= 1, n a positive multiple of 32)", N, n);
    REQUIRE(M >= 1 && M <= 32, "qw_w16_swiglu_gemv_tiled: M = %d outside 1..32", M);
    REQUIRE(aligned(Wt, 16) && aligned(v, 4) && (M == 1 || ldv >= 2 * n + 1),
            "qw_w16_swiglu_gemv_tiled: ldv %d must be >= 2n + 1; Wt 16-byte, v 4-byte aligned", ldv);
    REQUIRE(ys >= N || M == 1, "qw_w16_swiglu_gemv_tiled: y stride %d < N", ys);
    REQUIRE(aligned(y, y_bf16 ? 2 : 4), "qw_w16_swiglu_gemv_tiled: y misaligned");
    REQUIRE(qwq4::w16_swiglu_fits(M, n, N), "qw_w16_swiglu_gemv_tiled: %d rows of n = %d exceed the staging LDS", M, n);
    qwq4::W16SwigluArgs a{static_cast<const uint16_t *>(Wt), v, ldv, n, y, ys, y_bf16 != 0, N, M, accumulate != 0};
    qwq4::launch_w16_swiglu(a, st(stream));
    return launched("qw_w16_swiglu_gemv_tiled");
}

void qw_i8_tiled_size(int N, int K, int group, size_t *w_bytes, size_t *s_bytes) {
    const size_t tiles = N > 0 ? size_t((N + 15) / 16) : 0, k = K > 0 ? size_t(K) : 0;
    if (w_bytes) *w_bytes = tiles * 16 * k;
    if (s_bytes) *s_bytes = group > 0 ? tiles * 16 * (k / size_t(group)) * 4 : 0;
}

static int i8_shape(const char *fn, int N, int K, int group) {
    REQUIRE(group == 16 || group == 32, "%s: group %d (need 16 or 32)", fn, group);
    REQUIRE(N >= 1 && K >= 64 && K % 64 == 0, "%s: N = %d, K = %d (need N >= 1, K a positive multiple of 64)", fn, N,
            K);
    return 0;
}

int qw_i8_tile(const int8_t *W8, const float *scale, int N, int K, int group, void *Wt, float *St, void *stream) {
    REQUIRE(W8 && scale && Wt && St, "qw_i8_tile: null pointer");
    if (int rc = i8_shape("qw_i8_tile", N, K, group)) return rc;
    REQUIRE(aligned(W8, 8) && aligned(Wt, 16) && aligned(St, 4) && aligned(scale, 4), "qw_i8_tile: misaligned buffer");
    qwq4::launch_i8_tile(W8, scale, N, K, group, static_cast<uint4 *>(Wt), St, st(stream));
    return launched("qw_i8_tile");
}

int qw_i8_gemv(const void *Wt, const float *St, int group, const uint16_t *x, int xs, void *y, int ys, int y_bf16, int N,
               int K, int M, int rpg, int accumulate, void *stream) {
    REQUIRE(Wt && St && x && y, "qw_i8_gemv: null Wt, St, x or y");
    if (int rc = i8_shape("qw_i8_gemv", N, K, group)) return rc;
    REQUIRE(aligned(Wt, 16) && aligned(St, 16), "qw_i8_gemv: Wt and St must be 16-byte aligned");
    REQUIRE(M >= 1 && M <= 32, "qw_i8_gemv: M = %d outside 1..32", M);
    REQUIRE(rpg == 0 || rpg >= 16, "qw_i8_gemv: rpg = %d (need 0 or >= 16)", rpg);
    const int64_t slices = rpg > 0 ? (int64_t(N) + rpg - 1) / rpg : 1;
    REQUIRE(xs % 8 == 0 && aligned(x, 16) && (M == 1 || int64_t(xs) >= slices * K),
            "qw_i8_gemv: x stride %d must be a multiple of 8 and cover %lld slices of K = %d, x 16-byte aligned", xs,
            (long long)slices, K);
    REQUIRE(ys >= N || M == 1, "qw_i8_gemv: y stride %d < N", ys);
    REQUIRE(aligned(y, y_bf16 ? 2 : 4), "qw_i8_gemv: y misaligned");
    REQUIRE(qwq4::i8_fits(1, K, N, group, rpg), "qw_i8_gemv: K = %d too large for one staged row", K);
    qwq4::I8Args a{static_cast<const uint4 *>(Wt), St, group, x, xs, y, ys, y_bf16 != 0, N, K, M, rpg, accumulate != 0};
    qwq4::launch_i8_gemv(a, st(stream));
    return launched("qw_i8_gemv");
}

int qw_swiglu_gate(const float *v, int ldv, int n, int T, uint16_t *h, void *stream) {
    REQUIRE(v && h, "qw_swiglu_gate: null v or h");
    REQUIRE(n >= 1 && T >= 1 && ldv >= 2 * n + 1, "qw_swiglu_gate: n = %d, T = %d, ldv = %d (need ldv >= 2n + 1)", n, T,
            ldv);
    REQUIRE(T <= 65535, "qw_swiglu_gate: T = %d > 65535", T);
    qwq4::launch_swiglu_gate(v, ldv, n, T, h, st(stream));
    return launched("qw_swiglu_gate");
}

size_t qw_q4_gemm_workspace_size(int T, int K) {
    if (T < 1 || K < 128) return 0;
    return qwq4::gemm_workspace_bytes(T, K);
}

int qw_q4_gemm(const uint32_t *W, const uint16_t *S, const uint16_t *Z, const uint16_t *X, int x_f16, int ldx, int T,
               void *Y, int ldy, int y_type, int N, int K, void *workspace, size_t workspace_bytes, void *stream) {
    if (int r = check_q4("qw_q4_gemm", W, S, N, K)) return r;
    REQUIRE(X && Y, "qw_q4_gemm: null X or Y");
    REQUIRE(T >= 1, "qw_q4_gemm: T = %d must be >= 1", T);
    REQUIRE(ldx >= K && ldx % 8 == 0 && aligned(X, 16), "qw_q4_gemm: ldx %d must be >= K, a multiple of 8, X 16-byte aligned", ldx);
    REQUIRE(ldy >= N, "qw_q4_gemm: ldy %d < N", ldy);
    REQUIRE(y_type == QW_T_F32 || y_type == QW_T_BF16 || y_type == QW_T_F16, "qw_q4_gemm: y_type = %d (0 fp32, 1 bf16, 2 fp16)",
            y_type);
    REQUIRE(aligned(Y, 16) && ldy % (y_type == QW_T_F32 ? 4 : 8) == 0,
            "qw_q4_gemm: Y must be 16-byte aligned with rows of a multiple of 16 bytes (ldy %d)", ldy);
    const size_t need = x_f16 ? 0 : qwq4::gemm_workspace_bytes(T, K);
    REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 256)),
            "qw_q4_gemm: workspace needs %zu bytes, 256-byte aligned (got %zu)", need, workspace_bytes);
    qwq4::GemmArgs a{W, S, Z, X, ldx, T, Y, ldy, y_type, N, K, workspace};
    a.x_f16 = x_f16 != 0;
    qwq4::launch_gemm(a, st(stream));
    return launched("qw_q4_gemm");
}

int qw_moe_route(const float *logits, int T, int E, int topk, int tile_m, int32_t *top_e, float *top_w,
                 int32_t *counts, int32_t *offsets, int32_t *tok_slot, int32_t *pair_tok, int32_t *active,
                 int32_t *n_active, int32_t *tile_e, int32_t *tile_m0, int32_t *n_tiles, void *stream) {
    REQUIRE(logits && top_e && top_w && counts && offsets && tok_slot && pair_tok && active && n_active,
            "qw_moe_route: null pointer");
    REQUIRE(T >= 1 && E >= 1 && E <= 1024, "qw_moe_route: T = %d, E = %d (need T >= 1, 1 <= E <= 1024)", T, E);
    REQUIRE(topk >= 1 && topk <= E && topk <= 64, "qw_moe_route: topk = %d outside 1..min(E, 64)", topk);
    REQUIRE(tile_m > -4096 && tile_m < 4096, "qw_moe_route: |tile_m| >= 4096");
    REQUIRE(tile_m == 0 || (tile_e && tile_m0 && n_tiles), "qw_moe_route: tile_m != 0 needs the tile outputs");
    REQUIRE(int64_t(T) * topk < (1 << 30), "qw_moe_route: too many pairs");
    qwq4::RouteArgs a{logits, T, E, topk, tile_m, top_e, top_w, counts, offsets, tok_slot, pair_tok, active,
                      n_active, tile_e, tile_m0, n_tiles};
    qwq4::launch_route(a, st(stream));
    return launched("qw_moe_route");
}

int qw_moe_experts_gemv(const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                        const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                        const uint16_t *dz, int E, int H, int F, const int32_t *offsets, const int32_t *active,
                        const int32_t *n_active, const int32_t *pair_tok, const uint16_t *x, int x_f16, int T,
                        int topk, uint16_t *h, void *yp, int yp_f16, void *stream) {
    if (int r = check_q4("qw_moe_experts_gemv(gate)", gw, gs, int64_t(E) * F, H)) return r;
    if (int r = check_q4("qw_moe_experts_gemv(up)", uw, us, int64_t(E) * F, H)) return r;
    if (int r = check_q4("qw_moe_experts_gemv(down)", dw, ds, int64_t(E) * H, F)) return r;
    REQUIRE(offsets && active && n_active && pair_tok && x && h && yp, "qw_moe_experts_gemv: null pointer");
    REQUIRE(T >= 1 && T <= 32, "qw_moe_experts_gemv: T = %d outside 1..32", T);
    REQUIRE(qwq4::moe_gemv_supported(H, F), "qw_moe_experts_gemv: H = %d, F = %d too large", H, F);
    REQUIRE(topk >= 1 && topk <= E, "qw_moe_experts_gemv: topk = %d outside 1..E", topk);
    REQUIRE(aligned(x, 16) && aligned(h, 16) && aligned(yp, 4), "qw_moe_experts_gemv: x/h must be 16-byte aligned, yp 4");
    qwq4::MoeGemvArgs a{gw, gs, gz, uw, us, uz, dw, ds, dz, E, H, F, offsets, active, n_active, pair_tok,
                        x, T, topk, h, yp};
    a.x_f16 = x_f16 != 0;
    a.yp_f16 = yp_f16 != 0;
    qwq4::launch_moe_gemv(a, st(stream));
    return launched("qw_moe_experts_gemv");
}

size_t qw_moe_grouped_workspace_size(int T, int topk, int E, int H, int F) {
    if (T < 1 || topk < 1 || E < 1) return 0;
    return qwq4::moe_grouped_workspace_bytes(T, topk, E, H, F);
}

int qw_moe_grouped_tile_m(void) { return qwq4::moe_grouped_tile_m(); }

int qw_moe_experts_grouped(const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                           const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                           const uint16_t *dz, int E, int H, int F, const int32_t *offsets, const int32_t *pair_tok,
                           const int32_t *tile_e, const int32_t *tile_m0, const int32_t *n_tiles, const uint16_t *x,
                           int x_f16, int T, int topk, uint16_t *h, void *yp, int yp_f16, void *workspace,
                           size_t workspace_bytes, void *stream) {
    if (int r = check_q4("qw_moe_experts_grouped(gate)", gw, gs, int64_t(E) * F, H)) return r;
    if (int r = check_q4("qw_moe_experts_grouped(up)", uw, us, int64_t(E) * F, H)) return r;
    if (int r = check_q4("qw_moe_experts_grouped(down)", dw, ds, int64_t(E) * H, F)) return r;
    REQUIRE(offsets && pair_tok && tile_e && tile_m0 && n_tiles && x && h && yp,
            "qw_moe_experts_grouped: null pointer");
    REQUIRE(T >= 1 && topk >= 1 && topk <= E, "qw_moe_experts_grouped: T = %d, topk = %d", T, topk);
    REQUIRE(aligned(x, 16) && aligned(h, 16) && aligned(yp, 16), "qw_moe_experts_grouped: x/h/yp must be 16-byte aligned");
    REQUIRE(H % 8 == 0, "qw_moe_experts_grouped: H = %d must be a multiple of 8", H);
    const size_t need = x_f16 ? 0 : qwq4::moe_grouped_workspace_bytes(T, topk, E, H, F);
    REQUIRE(need == 0 || (workspace && workspace_bytes >= need && aligned(workspace, 256)),
            "qw_moe_experts_grouped: workspace needs %zu bytes, 256-byte aligned", need);
    qwq4::MoeGroupedArgs a{gw, gs, gz, uw, us, uz, dw, ds, dz, E, H, F, offsets, pair_tok, tile_e, tile_m0, n_tiles,
                           x, T, topk, h, yp, workspace};
    a.x_f16 = x_f16 != 0;
    a.yp_f16 = yp_f16 != 0;
    qwq4::launch_moe_grouped(a, st(stream));
    return launched("qw_moe_experts_grouped");
}

int qw_moe_w4a8_tile_m(void) { return qwq4::moe_w4a8_tile_m(); }

size_t qw_moe_w4a8_workspace_size(int T, int topk, int H, int F) {
    if (T < 1 || topk < 1 || H < 1 || F < 1) return 0;
    return qwq4::moe_w4a8_workspace_bytes(T, topk, H, F);
}

int qw_quant_rows_i8(const uint16_t *x, int x_f16, int rows, int K, int ldx, int8_t *q, float *scale, void *stream) {
    REQUIRE(x && q && scale, "qw_quant_rows_i8: null pointer");
    REQUIRE(rows >= 1 && K >= 128 && K % 128 == 0, "qw_quant_rows_i8: rows = %d, K = %d (need K a multiple of 128)",
            rows, K);
    REQUIRE(ldx >= K && ldx % 2 == 0 && aligned(x, 4) && aligned(q, 2) && aligned(scale, 4),
            "qw_quant_rows_i8: row stride %d (>= K, even) or misaligned buffers", ldx);
    qwq4::launch_quant_rows(x, x_f16 != 0, ldx, rows, K, q, scale, st(stream));
    return launched("qw_quant_rows_i8");
}

int qw_moe_experts_w4a8(const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                        const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                        const uint16_t *dz, int E, int H, int F, const int32_t *offsets, const int32_t *pair_tok,
                        const int32_t *tile_e, const int32_t *tile_m0, const int32_t *n_tiles, const uint16_t *x,
                        int x_f16, int T, int topk, uint16_t *h, uint16_t *yp, void *workspace, size_t workspace_bytes,
                        void *stream) {
    if (int r = check_q4("qw_moe_experts_w4a8(gate)", gw, gs, int64_t(E) * F, H)) return r;
    if (int r = check_q4("qw_moe_experts_w4a8(up)", uw, us, int64_t(E) * F, H)) return r;
    if (int r = check_q4("qw_moe_experts_w4a8(down)", dw, ds, int64_t(E) * H, F)) return r;
    REQUIRE(offsets && pair_tok && tile_e && tile_m0 && n_tiles && x && h && yp, "qw_moe_experts_w4a8: null pointer");
    REQUIRE(T >= 1 && topk >= 1 && topk <= E, "qw_moe_experts_w4a8: T = %d, topk = %d", T, topk);
    REQUIRE(int64_t(T) * topk < (int64_t(1) << 30), "qw_moe_experts_w4a8: T * topk too large");
    REQUIRE(F % 128 == 0 && H % 128 == 0, "qw_moe_experts_w4a8: H = %d, F = %d (need multiples of 128)", H, F);
    REQUIRE(aligned(x, 4) && aligned(h, 4) && aligned(yp, 2), "qw_moe_experts_w4a8: misaligned x/h/yp");
    const size_t need = qwq4::moe_w4a8_workspace_bytes(T, topk, H, F);
    REQUIRE(workspace && workspace_bytes >= need && aligned(workspace, 256),
            "qw_moe_experts_w4a8: workspace needs %zu bytes, 256-byte aligned", need);
    qwq4::W8Args a{gw, uw, dw, gs, gz, us, uz, ds, dz, E, H, F, offsets, pair_tok, tile_e, tile_m0, n_tiles, h, yp,
                   workspace, nullptr, nullptr, nullptr, nullptr};
    qwq4::launch_moe_w4a8(a, x, x_f16 != 0, T, topk, st(stream));
    return launched("qw_moe_experts_w4a8");
}

int qw_moe_combine(const void *yp, int yp_f16, const int32_t *tok_slot, const float *tok_w, const void *shared,
                   int shared_f16, int T, int topk, int H, void *out, int out_type, void *stream) {
    REQUIRE(yp && tok_slot && tok_w && out, "qw_moe_combine: null pointer");
    REQUIRE(T >= 1 && topk >= 1 && H >= 4 && H % 4 == 0, "qw_moe_combine: T = %d, topk = %d, H = %d (need H %% 4 == 0)", T,
            topk, H);
    REQUIRE(out_type == QW_T_F32 || out_type == QW_T_BF16 || out_type == QW_T_F16,
            "qw_moe_combine: out_type = %d (0 fp32, 1 bf16, 2 fp16)", out_type);
    REQUIRE(aligned(yp, yp_f16 ? 8 : 16) && (!shared || aligned(shared, shared_f16 ? 8 : 16)) &&
                aligned(out, out_type == QW_T_F32 ? 16 : 8),
            "qw_moe_combine: misaligned yp/shared/out");
    qwq4::launch_combine(yp, yp_f16 != 0, tok_slot, tok_w, shared, shared_f16 != 0, T, topk, H, out, out_type,
                         st(stream));
    return launched("qw_moe_combine");
}

void qw_q4_tiled_size(int64_t N, int64_t K, size_t *wt_bytes, size_t *st_bytes, size_t *zt_bytes) {
    const int64_t G = K / 128, GC = (G + 3) / 4;
    if (wt_bytes) *wt_bytes = size_t(N) * size_t(K) / 2;
    if (st_bytes) *st_bytes = size_t(N / 16) * size_t(GC) * 64 * 2;
    if (zt_bytes) *zt_bytes = size_t(N / 16) * size_t(GC) * 16 * 2;
}

int qw_q4_tile(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, uint32_t *Wt,
               uint16_t *St, uint16_t *Zt, void *stream) {
    if (int r = check_ckpt("qw_q4_tile", W, S, N, K)) return r;
    REQUIRE(N % 16 == 0, "qw_q4_tile: N = %lld must be a multiple of 16", (long long)N);
    REQUIRE(Wt && St && aligned(Wt, 16), "qw_q4_tile: null or misaligned output");
    REQUIRE(!Z || Zt, "qw_q4_tile: zeros given without a Zt output");
    qwq4::launch_tile(W, S, Z, N, K, Wt, St, Zt, st(stream));
    return launched("qw_q4_tile");
}

int qw_q4_untile(const uint32_t *Wt, const uint16_t *St, const uint16_t *Zt, int64_t N, int64_t K, uint32_t *W,
                 uint16_t *S, uint32_t *Z, void *stream) {
    if (int r = check_ckpt("qw_q4_untile", W, S, N, K)) return r;
    REQUIRE(N % 16 == 0, "qw_q4_untile: N = %lld must be a multiple of 16", (long long)N);
    REQUIRE(Wt && St && aligned(Wt, 16), "qw_q4_untile: null or misaligned input");
    REQUIRE(!Zt || Z, "qw_q4_untile: Zt given without a Z output");
    qwq4::launch_untile(Wt, St, Zt, N, K, W, S, Z, st(stream));
    return launched("qw_q4_untile");
}

int qw_q4_unpack(const uint32_t *W, int64_t N, int64_t K, uint8_t *out, void *stream) {
    REQUIRE(W && out && N >= 1 && K >= 8 && K % 8 == 0, "qw_q4_unpack: bad arguments");
    REQUIRE(aligned(out, 8), "qw_q4_unpack: out must be 8-byte aligned");
    qwq4::launch_unpack(W, N, K, out, st(stream));
    return launched("qw_q4_unpack");
}

int qw_q4_dequant(const uint32_t *W, const uint16_t *S, const uint32_t *Z, int64_t N, int64_t K, float *out,
                  void *stream) {
    if (int r = check_ckpt("qw_q4_dequant", W, S, N, K)) return r;
    REQUIRE(out && aligned(out, 16), "qw_q4_dequant: out must be 16-byte aligned");
    qwq4::launch_dequant(W, S, Z, N, K, out, st(stream));
    return launched("qw_q4_dequant");
}

int qw_q4_from_engine_order(const uint32_t *in, uint32_t *out, int64_t n_words, void *stream) {
    REQUIRE(in && out && n_words >= 1, "qw_q4_from_engine_order: bad arguments");
    qwq4::launch_from_engine_order(in, out, n_words, st(stream));
    return launched("qw_q4_from_engine_order");
}

int qw_bf16_to_f16(const uint16_t *in, uint16_t *out, int64_t n, void *stream) {
    REQUIRE(in && out && n >= 0, "qw_bf16_to_f16: bad arguments");
    if (n == 0) return QW_Q4_OK;
    qwq4::launch_bf16_to_f16(in, out, n, st(stream));
    return launched("qw_bf16_to_f16");
}

int qw_read_probe(const void *p, int64_t bytes, void *stream) {
    REQUIRE(bytes >= 0 && bytes % 32768 == 0 && (bytes == 0 || (p && aligned(p, 16))),
            "qw_read_probe: bytes must be a multiple of 32768 and p 16-byte aligned");
    qwq4::launch_read_probe(p, bytes, st(stream));
    return launched("qw_read_probe");
}

int qw_st_open(const char *path, qw_st_file **out) {
    REQUIRE(path && out, "qw_st_open: null argument");
    *out = nullptr;
    auto *f = new qw_st_file;
    std::string err;
    if (!f->f.open(path, err)) {
        delete f;
        return fail("qw_st_open: %s", err.c_str());
    }
    for (auto &kv : f->f.tensors()) f->order.push_back(&kv.second);
    *out = f;
    g_err.clear();
    return QW_Q4_OK;
}

void qw_st_close(qw_st_file *f) { delete f; }

int qw_st_count(const qw_st_file *f) { return f ? int(f->order.size()) : 0; }

const char *qw_st_name(const qw_st_file *f, int i) {
    return f && i >= 0 && i < int(f->order.size()) ? f->order[i]->name.c_str() : nullptr;
}

int qw_st_tensor(const qw_st_file *f, const char *name, char *dtype, int64_t *shape, int *ndim, const void **data,
                 size_t *nbytes) {
    REQUIRE(f && name, "qw_st_tensor: null argument");
    const qwq4::StTensor *t = f->f.find(name);
    REQUIRE(t, "qw_st_tensor: no tensor named %s", name);
    REQUIRE(t->shape.size() <= 8, "qw_st_tensor: %s has more than 8 dimensions", name);
    if (dtype) std::snprintf(dtype, 16, "%s", t->dtype.c_str());
    if (shape)
        for (size_t i = 0; i < t->shape.size(); ++i) shape[i] = t->shape[i];
    if (ndim) *ndim = int(t->shape.size());
    if (data) *data = t->data;
    if (nbytes) *nbytes = t->nbytes;
    g_err.clear();
    return QW_Q4_OK;
}

static size_t round256(size_t b) { return (b + 255) & ~size_t(255); }

size_t qw_q4_load_staging_size(int64_t N, int64_t K) {
    if (N < 1 || K < 128) return 0;
    const size_t G = size_t(K / 128);
    return round256(size_t(N) * size_t(K) / 2) + 2 * round256(size_t(N) * G * 2);
}

void qw_q4_tiled_offset(int64_t row0, int64_t K, size_t *wt_off, size_t *st_off, size_t *zt_off) {
    const int64_t G = K / 128, GC = (G + 3) / 4, sub = row0 / 16;
    if (wt_off) *wt_off = size_t(sub) * size_t(G) * 64 * 16;
    if (st_off) *st_off = size_t(sub) * size_t(GC) * 64 * 2;
    if (zt_off) *zt_off = size_t(sub) * size_t(GC) * 16 * 2;
}

int qw_q4_load(const qw_st_file *f, const char *prefix, int64_t N, int64_t K, uint32_t *Wt, uint16_t *St, void *staging,
               size_t staging_bytes, void *stream) {
    REQUIRE(f && prefix && Wt && St && staging, "qw_q4_load: null argument");
    REQUIRE(N >= 16 && N % 16 == 0 && K >= 128 && K % 128 == 0, "qw_q4_load: N = %lld, K = %lld (need multiples of 16, 128)",
            (long long)N, (long long)K);
    REQUIRE(aligned(Wt, 16) && aligned(St, 8) && aligned(staging, 256), "qw_q4_load: misaligned Wt, St or staging");
    const size_t need = qw_q4_load_staging_size(N, K);
    REQUIRE(staging_bytes >= need, "qw_q4_load: staging needs %zu bytes", need);
    const std::string pw = std::string(prefix) + ".weight_packed", ps = std::string(prefix) + ".weight_scale";
    const qwq4::StTensor *tw = f->f.find(pw), *ts = f->f.find(ps);
    REQUIRE(tw && ts, "qw_q4_load: %s or %s missing", pw.c_str(), ps.c_str());
    const int64_t G = K / 128;
    REQUIRE(tw->dtype == "I32" && tw->shape.size() == 2 && tw->shape[0] == N && tw->shape[1] == K / 8,
            "qw_q4_load: %s must be I32 [%lld][%lld]", pw.c_str(), (long long)N, (long long)(K / 8));
    REQUIRE((ts->dtype == "BF16" || ts->dtype == "F16") && ts->shape.size() == 2 && ts->shape[0] == N &&
                ts->shape[1] == G,
            "qw_q4_load: %s must be BF16 or F16 [%lld][%lld]", ps.c_str(), (long long)N, (long long)G);
    unsigned char *stg = static_cast<unsigned char *>(staging);
    uint32_t *W = reinterpret_cast<uint32_t *>(stg);
    uint16_t *Ssrc = reinterpret_cast<uint16_t *>(stg + round256(tw->nbytes));
    uint16_t *S16 = reinterpret_cast<uint16_t *>(stg + round256(tw->nbytes) + round256(ts->nbytes));
    hipError_t e = hipMemcpyAsync(W, tw->data, tw->nbytes, hipMemcpyHostToDevice, st(stream));
    if (e == hipSuccess) e = hipMemcpyAsync(Ssrc, ts->data, ts->nbytes, hipMemcpyHostToDevice, st(stream));
    if (e != hipSuccess) {
        g_err = std::string("qw_q4_load: copy: ") + hipGetErrorString(e);
        return QW_Q4_ELAUNCH;
    }
    const uint16_t *S = Ssrc;
    if (ts->dtype == "BF16") {
        qwq4::launch_bf16_to_f16(Ssrc, S16, N * G, st(stream));
        S = S16;
    }
    qwq4::launch_tile(W, S, nullptr, N, K, Wt, St, nullptr, st(stream));
    return launched("qw_q4_load");
}

// ---- fused MoE decode block
namespace {
struct DecodeLayout {
    int kl, ksplit, rows;
    size_t part, counts, offsets, pair_tok, active, n_active, rcounter, dcounters, total;
};
DecodeLayout decode_layout(int T, int E, int topk, int H, int F) {
    DecodeLayout L{};
    // router K slices of 512 (128 when H is not a multiple of 512): many
    // blocks stream the fp32 router weights, each stages T x kl activations
    L.kl = H % 512 == 0 ? 512 : 128;
    L.ksplit = H / L.kl;
    L.rows = qwq4::moe_down_row_blocks(H, F);
    auto r = [](size_t b) { return (b + 255) & ~size_t(255); };
    size_t o = 0;
    L.part = o;
    o += r(size_t(L.ksplit) * T * E * 4);
    L.counts = o;
    o += r(size_t(E) * 4);
    L.offsets = o;
    o += r(size_t(E + 1) * 4);
    L.pair_tok = o;
    o += r(size_t(T) * topk * 4);
    L.active = o;
    o += r(size_t(E) * 4);
    L.n_active = o;
    o += 256;
    L.rcounter = o;
    o += r(size_t(1 + (E + 15) / 16) * 4);
    L.dcounters = o;
    o += r(size_t(L.rows) * 4);
    L.total = o;
    return L;
}
}  // namespace

size_t qw_moe_decode_workspace_size(int T, int E, int topk, int H, int F) {
    if (T < 1 || E < 1 || topk < 1 || H < 128 || F < 128) return 0;
    return decode_layout(T, E, topk, H, F).total;
}

}  // extern "C"

namespace {

int moe_decode_check(const char *fn, const void *router_w, const uint16_t *x, int T, int E, int topk,
                     const uint32_t *gw, const uint16_t *gs, const uint32_t *uw, const uint16_t *us,
                     const uint32_t *dw, const uint16_t *ds, int H, int F, const void *out, const float *logits,
                     const int32_t *top_e, const float *top_w, const int32_t *tok_slot, const uint16_t *h,
                     const void *yp, int out_type) {
    if (int r = check_q4(fn, gw, gs, int64_t(E) * F, H)) return r;
    if (int r = check_q4(fn, uw, us, int64_t(E) * F, H)) return r;
    if (int r = check_q4(fn, dw, ds, int64_t(E) * H, F)) return r;
    REQUIRE(router_w && x && out && logits && top_e && top_w && tok_slot && h && yp, "%s: null pointer", fn);
    REQUIRE(T >= 1 && T <= 32, "%s: T = %d outside 1..32", fn, T);
    REQUIRE(E >= 1 && E <= 1024 && topk >= 1 && topk <= E && topk <= 64, "%s: E = %d, topk = %d", fn, E, topk);
    REQUIRE(qwq4::moe_gemv_supported(H, F), "%s: H = %d, F = %d too large", fn, H, F);
    REQUIRE(aligned(router_w, 16) && aligned(x, 16) && aligned(h, 16) && aligned(yp, 4),
            "%s: router_w, x, h must be 16-byte aligned, yp 4-byte", fn);
    REQUIRE(out_type == QW_T_F32 || out_type == QW_T_BF16 || out_type == QW_T_F16,
            "%s: out_type = %d (0 fp32, 1 bf16, 2 fp16)", fn, out_type);
    REQUIRE(aligned(out, out_type == QW_T_F32 ? 16 : 8), "%s: out misaligned", fn);
    return 0;
}

// Router GEMV + routing, the expert GEMVs, and the combine (folded into the
// down projection up to 4 tokens), on the scratch w laid out as L.
void moe_decode_launch(const void *router_w, int router_f16, const uint16_t *x, int x_f16, int T, int E, int topk, const uint32_t *gw,
                       const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us,
                       const uint16_t *uz, const uint32_t *dw, const uint16_t *ds, const uint16_t *dz, int H, int F,
                       const float *shared, void *out, int out_type, float *logits, int32_t *top_e, float *top_w,
                       int32_t *tok_slot, uint16_t *h, void *yp, int yp_f16, unsigned char *w, const DecodeLayout &L,
                       hipStream_t s, const qwq4::ShExpertArgs *sh = nullptr, uint16_t *sh_h = nullptr) {
    auto at = [&](size_t off) { return reinterpret_cast<int32_t *>(w + off); };
    qwq4::RouteArgs ra{logits, T, E, topk, 0, top_e, top_w, at(L.counts), at(L.offsets), tok_slot, at(L.pair_tok),
                       at(L.active), at(L.n_active), nullptr, nullptr, nullptr};
    qwq4::RouterArgs rr{router_w, x, H, L.kl, reinterpret_cast<float *>(w + L.part), logits, at(L.rcounter)};
    rr.x_f16 = x_f16 != 0;
    rr.w_f16 = router_f16 != 0;
    // small batches: the router launch writes the logits only, and the
    // gate/up blocks route the batch themselves (no cross-block hand-off)
    const bool local = qwq4::moe_local_route_ok(T, E, topk) && qwq4::router_logits_ok(T, E, H);
    const bool split = !local && qwq4::router_split_ok(T, E, H);
    // the shared expert: up to 8 tokens its gate/up GEMV shares the router
    // logits launch, and at batch 1 its down GEMV the routed gate/up launch;
    // otherwise its GEMVs run first, as launches of their own
    const bool shl = sh && (local || split) && qwq4::shared_logits_ok(T, H, sh->Fs);
    const bool sh1 = shl && local && T == 1;
    const int nv = sh ? 2 * sh->Fs + 1 : 0;
    // the SwiGLU folded into the down GEMV up to 4 rows (every block forms all
    // of h, which costs more than the separate launch from 8 rows on)
    const bool fold_sh = sh && T <= 4 && qwq4::w16_swiglu_fits(T, sh->Fs, H);
    auto down_gemv = [&] {  // the down GEMV over the SwiGLU rows in sh_h
        qwq4::launch_w16_gemv(qwq4::W16Args{sh->down, sh->Fs, sh_h, sh->Fs, sh->out, H, 0, H, sh->Fs, T, 0, 1, 1}, s);
    };
    auto shared_down = [&] {
        if (fold_sh) {
            qwq4::launch_w16_swiglu(qwq4::W16SwigluArgs{sh->down, sh->v, nv, sh->Fs, sh->out, H, 0, H, T, 0}, s);
        } else {
            qwq4::launch_swiglu_gate(sh->v, nv, sh->Fs, T, sh_h, s);
            down_gemv();
        }
    };
    bool down_pending = false;  // the shared expert's down GEMV over sh_h still to launch
    if (sh) {
        if (!shl) {
            // its own launches; above 4 tokens the down GEMV over the SwiGLU
            // rows rides in the experts' gate/up launch below where it can
            qwq4::launch_w16_gemv(qwq4::W16Args{sh->gu, H, x, H, sh->v, nv, 0, nv, H, T, 0, x_f16 != 0, 1}, s);
            if (fold_sh || local) {
                shared_down();
            } else {
                qwq4::launch_swiglu_gate(sh->v, nv, sh->Fs, T, sh_h, s);
                down_pending = true;
            }
        }
        shared = sh->out;
    }
    if (shl) {
        qwq4::launch_router_logits_shgu(rr, T, E, *sh, s);
        // the shared expert's SwiGLU-down (folded) or SwiGLU rows ride in the
        // routing launch where the shapes allow (the down GEMV over the
        // SwiGLU rows then rides in the gate/up launch below)
        if (split) {
            const bool rode = fold_sh ? qwq4::launch_route_shdown(ra, *sh, H, s)
                                      : qwq4::launch_route_shgate(ra, *sh, sh_h, s);
            if (!rode) {
                qwq4::launch_route(ra, s);
                shared_down();
            } else if (!fold_sh) {
                down_pending = true;
            }
        } else if (!sh1) {
            shared_down();
        }
    } else if (local) {
        qwq4::launch_router_logits(rr, T, E, s);
    } else if (split) {
        // the logits over one block per expert, then the routing launch
        qwq4::launch_router_logits(rr, T, E, s);
        qwq4::launch_route(ra, s);
    } else if (qwq4::router_mfma_ok(T, E, H, L.kl)) {
        // partial logits per K slice on the MFMA, summed by the routing launch
        qwq4::launch_router_mfma(rr, T, E, s);
        qwq4::launch_route_part(ra, rr.part, L.ksplit, logits, s);
    } else {
        qwq4::launch_router_route(ra, rr, s);
    }
    // up to 2 tokens the combine runs in the down projection's last blocks
    // (one launch less); from 3 tokens on its own launch is faster than the
    // serial tail it adds to those blocks
    const bool fold = T <= 2;
    const qwq4::CombineArgs cmb{at(L.dcounters), tok_slot, top_w, shared, out, out_type};
    qwq4::MoeGemvArgs a{gw, gs, gz, uw, us, uz, dw, ds, dz, E, H, F, at(L.offsets), at(L.active), at(L.n_active),
                        at(L.pair_tok), x, T, topk, h, yp, fold ? &cmb : nullptr};
    a.x_f16 = x_f16 != 0;
    a.yp_f16 = yp_f16 != 0;
    if (local) {
        a.route_logits = logits;
        a.top_e = top_e;
        a.top_w = top_w;
        a.tok_slot = tok_slot;
    }
    if (sh1) {
        if (!qwq4::launch_gate_up_routed_shdown(a, *sh, s)) {
            shared_down();
            qwq4::launch_moe_gemv(a, s);
        } else {
            qwq4::launch_moe_down(a, s);
        }
    } else if (down_pending) {
        if (!qwq4::launch_gate_up_shdown(a, *sh, sh_h, s)) {
            down_gemv();
            qwq4::launch_moe_gemv(a, s);
        } else {
            qwq4::launch_moe_down(a, s);
        }
    } else {
        qwq4::launch_moe_gemv(a, s);
    }
    if (!fold) qwq4::launch_combine(yp, yp_f16 != 0, tok_slot, top_w, shared, 0, T, topk, H, out, out_type, s);
}

// ---- the allocation-free variant's scratch: one array per GPU, held until
// the process ends. The completion counters sit at fixed offsets at its
// start (every call leaves them at zero, whatever its shape; the array starts
// zeroed), the rest after them.
constexpr size_t kStaticScratchBytes = size_t(4) << 20;
constexpr size_t kStaticCounterBytes = 16384;  // 1 + E/16 router counters, then the down row counters
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices];

// The device address of the current device's scratch (looked up once per
// device, with that device current; the array's host-side name is not a
// device address).
int static_scratch(void **ptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fail("qw_moe_decode_static: no current device (or more than %d)", kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail("qw_moe_decode_static: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch[dev] = p;
    }
    *ptr = g_scratch[dev];
    return 0;
}

// Zeroes the completion counters at the start of the scratch (a fill
// kernel rather than a memset node, so it is also safe inside graph capture).
__global__ void zero_counters_kernel(uint32_t *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

void reset_static_counters(void *scratch_ptr, hipStream_t s) {
    constexpr int n = int(kStaticCounterBytes / 4);
    zero_counters_kernel<<<(n + 255) / 256, 256, 0, s>>>(static_cast<uint32_t *>(scratch_ptr), n);
}

// The workspace layout with the counters moved to the fixed region.
DecodeLayout static_layout(int T, int E, int topk, int H, int F) {
    DecodeLayout L = decode_layout(T, E, topk, H, F);
    for (size_t *o : {&L.part, &L.counts, &L.offsets, &L.pair_tok, &L.active, &L.n_active}) *o += kStaticCounterBytes;
    L.total += kStaticCounterBytes;
    L.rcounter = 0;
    L.dcounters = 4096;
    return L;
}

}  // namespace

extern "C" {

int qw_moe_decode(const void *router_w, int router_f16, const uint16_t *x, int x_f16, int T, int E, int topk, const uint32_t *gw,
                  const uint16_t *gs, const uint16_t *gz, const uint32_t *uw, const uint16_t *us, const uint16_t *uz,
                  const uint32_t *dw, const uint16_t *ds, const uint16_t *dz, int H, int F, const float *shared,
                  void *out, int out_type, float *logits, int32_t *top_e, float *top_w, int32_t *tok_slot,
                  uint16_t *h, void *yp, int yp_f16, void *workspace, size_t workspace_bytes, void *stream) {
    REQUIRE(router_f16 == 0 || router_f16 == 1, "qw_moe_decode: router_f16 = %d (0: fp32 weights, 1: fp16)", router_f16);
    if (int r = moe_decode_check("qw_moe_decode", router_w, x, T, E, topk, gw, gs, uw, us, dw, ds, H, F, out, logits,
                                 top_e, top_w, tok_slot, h, yp, out_type))
        return r;
    REQUIRE(workspace && aligned(workspace, 256), "qw_moe_decode: workspace null or not 256-byte aligned");
    const DecodeLayout L = decode_layout(T, E, topk, H, F);
    REQUIRE(workspace_bytes >= L.total, "qw_moe_decode: workspace needs %zu bytes", L.total);
    moe_decode_launch(router_w, router_f16, x, x_f16, T, E, topk, gw, gs, gz, uw, us, uz, dw, ds, dz, H, F, shared, out, out_type,
                      logits, top_e, top_w, tok_slot, h, yp, yp_f16, static_cast<unsigned char *>(workspace), L, st(stream));
    return launched("qw_moe_decode");
}

size_t qw_moe_decode_with_shared_workspace_size(int T, int E, int topk, int H, int F, int Fs) {
    const size_t b = qw_moe_decode_workspace_size(T, E, topk, H, F);
    if (b == 0 || Fs < 1) return 0;
    return b + ((size_t(T) * Fs * 2 + 255) & ~size_t(255));
}

int qw_moe_decode_with_shared(const void *router_w, int router_f16, const uint16_t *x, int x_f16, int T, int E,
                              int topk, const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                              const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                              const uint16_t *dz, int H, int F, const void *sh_gu, const void *sh_down, int Fs,
                              float *sh_v, float *sh_out, void *out, int out_type, float *logits, int32_t *top_e,
                              float *top_w, int32_t *tok_slot, uint16_t *h, void *yp, int yp_f16, void *workspace,
                              size_t workspace_bytes, void *stream) {
    const char *fn = "qw_moe_decode_with_shared";
    REQUIRE(router_f16 == 0 || router_f16 == 1, "%s: router_f16 = %d (0: fp32 weights, 1: fp16)", fn, router_f16);
    if (int r = moe_decode_check(fn, router_w, x, T, E, topk, gw, gs, uw, us, dw, ds, H, F, out, logits, top_e, top_w,
                                 tok_slot, h, yp, out_type))
        return r;
    REQUIRE(sh_gu && sh_down && sh_v && sh_out, "%s: null shared-expert pointer", fn);
    REQUIRE(Fs >= 32 && Fs % 32 == 0 && H % 32 == 0, "%s: Fs = %d, H = %d (multiples of 32)", fn, Fs, H);
    REQUIRE(aligned(sh_gu, 16) && aligned(sh_down, 16) && aligned(sh_v, 4) && aligned(sh_out, 4),
            "%s: sh_gu, sh_down must be 16-byte aligned, sh_v, sh_out 4-byte", fn);
    REQUIRE(workspace && aligned(workspace, 256), "%s: workspace null or not 256-byte aligned", fn);
    const size_t need = qw_moe_decode_with_shared_workspace_size(T, E, topk, H, F, Fs);
    REQUIRE(workspace_bytes >= need, "%s: workspace needs %zu bytes", fn, need);
    const DecodeLayout L = decode_layout(T, E, topk, H, F);
    unsigned char *w = static_cast<unsigned char *>(workspace);
    const qwq4::ShExpertArgs sh{static_cast<const uint16_t *>(sh_gu), static_cast<const uint16_t *>(sh_down), Fs, sh_v,
                                sh_out};
    moe_decode_launch(router_w, router_f16, x, x_f16, T, E, topk, gw, gs, gz, uw, us, uz, dw, ds, dz, H, F, nullptr,
                      out, out_type, logits, top_e, top_w, tok_slot, h, yp, yp_f16, w, L, st(stream), &sh,
                      reinterpret_cast<uint16_t *>(w + L.total));
    return launched(fn);
}

size_t qw_moe_decode_static_max_bytes(void) { return kStaticScratchBytes; }

int qw_moe_decode_static(const void *router_w, int router_f16, const uint16_t *x, int x_f16, int T, int E, int topk,
                         const uint32_t *gw, const uint16_t *gs, const uint16_t *gz, const uint32_t *uw,
                         const uint16_t *us, const uint16_t *uz, const uint32_t *dw, const uint16_t *ds,
                         const uint16_t *dz, int H, int F, const float *shared, void *out, int out_type,
                         float *logits, int32_t *top_e, float *top_w, int32_t *tok_slot, uint16_t *h, void *yp,
                         int yp_f16, void *stream) {
    REQUIRE(router_f16 == 0 || router_f16 == 1, "qw_moe_decode_static: router_f16 = %d (0: fp32 weights, 1: fp16)", router_f16);
    if (int r = moe_decode_check("qw_moe_decode_static", router_w, x, T, E, topk, gw, gs, uw, us, dw, ds, H, F, out,
                                 logits, top_e, top_w, tok_slot, h, yp, out_type))
        return r;
    const DecodeLayout L = static_layout(T, E, topk, H, F);
    // Every shape moe_decode_check accepts fits (the largest, T = 32,
    // E = 1024, H = 3840, k = 64, needs about 3.97 MB of the 4 MiB); these
    // checks guard that bound should the limits above change.
    REQUIRE(L.total <= kStaticScratchBytes,
            "qw_moe_decode_static: T = %d, E = %d, k = %d, H = %d needs %zu bytes of scratch, more than the %zu "
            "the library holds (use qw_moe_decode with a workspace)",
            T, E, topk, H, L.total, kStaticScratchBytes);
    REQUIRE(size_t(1 + (E + 15) / 16) * 4 <= 4096 && size_t(L.rows) * 4 <= kStaticCounterBytes - 4096,
            "qw_moe_decode_static: E = %d or H = %d needs more completion counters than the scratch holds", E, H);
    void *w = nullptr;
    if (int r = static_scratch(&w)) return r;
    moe_decode_launch(router_w, router_f16, x, x_f16, T, E, topk, gw, gs, gz, uw, us, uz, dw, ds, dz, H, F, shared, out, out_type,
                      logits, top_e, top_w, tok_slot, h, yp, yp_f16, static_cast<unsigned char *>(w), L, st(stream));
    const int rc = launched("qw_moe_decode_static");
    if (rc != QW_Q4_OK) {
        // a launch failed after others were enqueued: the counters those
        // left behind would misplace the next call's last block, so they are
        // cleared behind them on the same stream
        reset_static_counters(w, st(stream));
        if (hipGetLastError() != hipSuccess)
            g_err += "; clearing the completion counters failed too (call qw_moe_decode_static_reset)";
    }
    return rc;
}

int qw_moe_decode_static_reset(void *stream) {
    void *w = nullptr;
    if (int r = static_scratch(&w)) return r;
    reset_static_counters(w, st(stream));
    return launched("qw_moe_decode_static_reset");
}

}  // extern "C"

// ---- converted-weights cache
int qw_wcache_open(const char *path, uint64_t key, qw_wcache **out, int *mode) {
    REQUIRE(path && out, "qw_wcache_open: null argument");
    *out = nullptr;
    auto *c = new qw_wcache;
    std::string err;
    c->c.open(path, key, err);
    *out = c;
    if (mode) *mode = int(c->c.mode());
    g_err = err;  // why the cache is off, when it is
    return QW_Q4_OK;
}

void qw_wcache_close(qw_wcache *c) { delete c; }

int qw_wcache_put(qw_wcache *c, const void *src, size_t bytes, int on_device, void *stream) {
    REQUIRE(c && (src || bytes == 0), "qw_wcache_put: null argument");
    if (c->c.mode() != qwq4::WCache::RECORD) return QW_Q4_OK;
    const void *h = src;
    if (on_device && bytes) {
        c->host.resize(bytes);
        hipError_t e = hipMemcpyAsync(c->host.data(), src, bytes, hipMemcpyDeviceToHost, st(stream));
        if (e == hipSuccess) e = hipStreamSynchronize(st(stream));
        if (e != hipSuccess) {
            g_err = std::string("qw_wcache_put: ") + hipGetErrorString(e);
            return QW_Q4_ELAUNCH;
        }
        h = c->host.data();
    }
    std::string err;
    if (!c->c.put(h, bytes, err)) g_err = err;  // the recording is dropped; the load goes on
    return QW_Q4_OK;
}

int qw_wcache_get(qw_wcache *c, void *dst, size_t bytes, int on_device, void *stream) {
    REQUIRE(c && (dst || bytes == 0), "qw_wcache_get: null argument");
    std::string err;
    const void *src = c->c.next(bytes, err);
    REQUIRE(src, "qw_wcache_get: %s", err.c_str());
    if (!bytes) return QW_Q4_OK;
    if (!on_device) {
        std::memcpy(dst, src, bytes);
        return QW_Q4_OK;
    }
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(st(stream));
    if (e != hipSuccess) {
        g_err = std::string("qw_wcache_get: ") + hipGetErrorString(e);
        return QW_Q4_ELAUNCH;
    }
    g_err.clear();
    return QW_Q4_OK;
}

int qw_wcache_finish(qw_wcache *c) {
    REQUIRE(c, "qw_wcache_finish: null argument");
    std::string err;
    REQUIRE(c->c.finish(err), "qw_wcache_finish: %s", err.c_str());
    g_err.clear();
    return QW_Q4_OK;
}
