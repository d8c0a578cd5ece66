// Dense q4 GEMV for fp16 activation rows (the reference engine's decode rows,
// src/kernels/gemv.hpp:11-14): the instantiations of q4_gemv_impl.cuh for
// fp16 MFMA operands, in a translation unit of their own (built in parallel
// with the bf16 ones).
#include "q4_gemv_impl.cuh"

namespace qwq4 {

void launch_gemv_fit_f16(const GemvArgs &a, hipStream_t s) { launch_gemv_fit_t<F16>(a, s); }

}  // namespace qwq4
