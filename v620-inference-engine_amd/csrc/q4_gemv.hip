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

// Batches whose activations exceed LDS run as several launches of fewer rows.
void launch_gemv(const GemvArgs &a, hipStream_t s) {
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
