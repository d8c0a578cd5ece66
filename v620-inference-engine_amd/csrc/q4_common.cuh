// Device helpers shared by the q4 kernels (CDNA4 / gfx950, wave64).
//
// Weight format (the checkpoint's compressed-tensors order, kept as is on the
// device; docs/MODEL.md:34-37 of the reference):
//   W  uint32 [N][K/8]        element 8c+i of row n at bits 4i of word c
//   S  fp16   [N][K/128]      scale of each 128-element group along K
//   Z  uint32 [N][ceil(G/8)]  4-bit zero of group g at bits 4(g%8) of word g/8,
//                             or null for the reference's fixed zero of 8
//   w = (q - z) * s.
//
// How a nibble reaches an MFMA operand exactly. For a 32-bit word holding
// elements e0..e7 and a group zero z:
//   lo = (w      & 0x0F0F0F0F) + (16 - z) * 0x01010101   bytes e0,e2,e4,e6
//   hi = (w >> 4 & 0x0F0F0F0F) + (16 - z) * 0x01010101   bytes e1,e3,e5,e7
// Each byte is v = 16 + q - z in [1, 31] (no carry between bytes). One
// v_perm_b32 against a constant then places a byte under a high byte of 0x43
// (bf16) or 0x64 (fp16): 0x43vv is the bf16 number 128 + v and 0x64vv the
// fp16 number 1024 + v, both exact. So the operand holds BIAS + (q - z) with
// BIAS = 144 (bf16) or 1040 (fp16), and the MFMA accumulator is started at
// -BIAS * sum(x) over the group (itself one MFMA against a splat of -BIAS),
// leaving sum x * (q - z) with every product exact in fp32. The group scale
// is applied once per group, in fp32, on the accumulator.
//
// The eight operand elements of one lane therefore come in the order
// e0,e2,e4,e6,e1,e3,e5,e7 ("operand order"). Activations are permuted into the
// same order (act_perm), or stored in it by the kernel that writes them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qwq4 {

constexpr int WAVE = 64;
constexpr int QGROUP = 128;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Operand type traits: bf16 activations (dense paths, expert gate/up) and fp16
// (the expert down projection, whose input h is kept in fp16).
struct BF16 {
    static constexpr uint32_t HI = 0x43434343u;    // high byte of 128 + v
    static constexpr uint32_t NEG_BIAS = 0xC310C310u;  // two bf16 -144
    typedef bf16x8 vec;
};
struct F16 {
    static constexpr uint32_t HI = 0x64646464u;    // high byte of 1024 + v
    static constexpr uint32_t NEG_BIAS = 0xE410E410u;  // two fp16 -1040
    typedef f16x8 vec;
};

template <typename T>
__device__ __forceinline__ f32x4 mfma16(const uint4 &a, const uint4 &b, const f32x4 &c) {
    if constexpr (__is_same(T, BF16))
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
}

template <typename T>
__device__ __forceinline__ f32x16 mfma32(const uint4 &a, const uint4 &b, const f32x16 &c) {
    if constexpr (__is_same(T, BF16))
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
}

// (16 - z) in every byte.
__device__ __forceinline__ uint32_t zero_bytes(uint32_t z) { return (16u - z) * 0x01010101u; }

// One packed word (8 nibbles) -> 8 operand elements BIAS + (q - z), operand order.
template <typename T>
__device__ __forceinline__ uint4 unpack8(uint32_t w, uint32_t zb) {
    const uint32_t lo = (w & 0x0F0F0F0Fu) + zb;
    const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) + zb;
    uint4 r;
    // byte selectors: 0-3 pick from the second source (lo/hi), 4 picks a byte of T::HI
    r.x = __builtin_amdgcn_perm(T::HI, lo, 0x04010400u);  // e0, e2
    r.y = __builtin_amdgcn_perm(T::HI, lo, 0x04030402u);  // e4, e6
    r.z = __builtin_amdgcn_perm(T::HI, hi, 0x04010400u);  // e1, e3
    r.w = __builtin_amdgcn_perm(T::HI, hi, 0x04030402u);  // e5, e7
    return r;
}

// Eight activations in natural order (x0..x7 as four 16-bit pairs) -> operand order.
__device__ __forceinline__ uint4 act_perm(const uint4 &v) {
    uint4 r;
    r.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);  // x0, x2
    r.y = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);  // x4, x6
    r.z = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);  // x1, x3
    r.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);  // x5, x7
    return r;
}

// Position of natural element e (0..7) inside an operand-ordered 8-chunk.
__host__ __device__ constexpr int op_pos(int e) { return (e >> 1) + 4 * (e & 1); }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

// fp32 -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __builtin_bit_cast(float, uint32_t(b) << 16); }

__device__ __forceinline__ int group_zero(const uint32_t *Z, int64_t row, int zw, int g) {
    return Z ? int((Z[row * zw + (g >> 3)] >> (4 * (g & 7))) & 0xfu) : 8;
}

}  // namespace qwq4
