// Dense q4 GEMV entry (bf16 activations here, fp16 ones in
// q4_gemv_f16.hip; the kernel is in q4_gemv_impl.cuh).
#include "q4_gemv_impl.cuh"

namespace qwq4 {

void launch_gemv_fit_f16(const GemvArgs &a, hipStream_t s);

bool gemv_fits(int M, int K) {
    const int MB = M <= 16 ? 1 : 2;
    int KS, SUB, NW;
    dense_split(K / QGROUP, KS, SUB, NW);
    return dense_lds_bytes(M, K, MB, KS * SUB, KS) <= 160 * 1024;
}

static void launch_gemv_fit(const GemvArgs &a, hipStream_t s) {
    if (a.x_f16) launch_gemv_fit_f16(a, s);
    else launch_gemv_fit_t<BF16>(a, s);
}

static void launch_gemv_rows(const GemvArgs &a, hipStream_t s);

// Rows grouped over activation slices (rpg > 0, the reference's
// hyper-connection down projection: row n reads slice n / rpg of x, at
// x + (n / rpg) * K): one launch per slice over the 16-row subtiles its rows
// touch. A subtile that straddles two slices is computed in both launches,
// each storing only its own rows (n_lo, N), so every output row is the
// product of its own slice, with the same arithmetic as an ungrouped row.
void launch_gemv(const GemvArgs &a, hipStream_t s) {
    if (a.rpg <= 0) {
        launch_gemv_rows(a, s);
        return;
    }
    const int G = a.K / QGROUP, GC = (G + 3) / 4;
    const size_t ysz = a.y_bf16 ? 2 : 4;
    for (int r0 = 0, sl = 0; r0 < a.N; r0 += a.rpg, ++sl) {
        const int r1 = r0 + a.rpg < a.N ? r0 + a.rpg : a.N, sub0 = r0 / 16, b0 = sub0 * 16;
        GemvArgs b = a;
        b.rpg = 0;
        b.W = a.W + int64_t(sub0) * G * 256;
        b.S = a.S + int64_t(sub0) * GC * 64;
        b.Z = a.Z ? a.Z + int64_t(sub0) * GC * 16 : nullptr;
        b.x = a.x + int64_t(sl) * a.K;
        b.y = static_cast<char *>(a.y) + int64_t(b0) * ysz;
        b.N = r1 - b0;
        b.n_lo = r0 - b0;
        launch_gemv_rows(b, s);
    }
}

// Batches whose activations exceed LDS run as several launches of fewer rows.
static void launch_gemv_rows(const GemvArgs &a, hipStream_t s) {
    if (gemv_fits(a.M, a.K)) {
        launch_gemv_fit(a, s);
        return;
    }
    int mc = 16;
    while (mc > 1 && !gemv_fits(mc, a.K)) --mc;
    const size_t ysz = a.y_bf16 ? 2 : 4;
    for (int m0 = 0; m0 < a.M; m0 += mc) {
        GemvArgs b = a;
        b.M = a.M - m0 < mc ? a.M - m0 : mc;
        b.x = a.x + int64_t(m0) * a.xs;
        b.y = static_cast<char *>(a.y) + int64_t(m0) * a.ys * ysz;
        launch_gemv_fit(b, s);
    }
}

}  // namespace qwq4
