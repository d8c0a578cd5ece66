// C-ABI wrappers around the reference's own conversion code, compiled from the
// reference sources where they lie (see oracle/Makefile, target `ref`). Test
// infrastructure only: used to pin the oracle's restatements of
// src/core/common.hpp:34-99 and src/engine/weight_convert.cpp:19-26,61-108.
#include <cstddef>
#include <cstdint>
#include <vector>

#include "core/common.hpp"
#include "engine/weight_convert.hpp"

extern "C" {
float ref_bf16_to_f32(uint16_t v) { return qw::bf16_to_f32(v); }
float ref_f16_to_f32(uint16_t v) { return qw::f16_to_f32(v); }
uint16_t ref_f32_to_f16(float f) { return qw::f32_to_f16(f); }
uint16_t ref_bf16_to_f16(uint16_t b) { return qw::bf16_to_f16(b); }
void ref_pack_int4_words(const int32_t *ct, uint32_t *out, size_t n) { qw::pack_int4_words(ct, out, n); }
void ref_quantize_int4_g128(const uint16_t *src, size_t n_groups, int32_t *ct, uint16_t *scales) {
    qw::quantize_int4_g128(src, n_groups, ct, scales);
}
void ref_quantize_rows_i8(const uint16_t *fp16, int64_t N, int64_t K, int8_t *q, float *scale, int64_t group) {
    const std::vector<uint16_t> in(fp16, fp16 + N * K);
    std::vector<int8_t> qv;
    std::vector<float> sv;
    qw::quantize_rows_i8(in, N, K, qv, sv, group);
    for (size_t i = 0; i < qv.size(); ++i) q[i] = qv[i];
    for (size_t i = 0; i < sv.size(); ++i) scale[i] = sv[i];
}
}
