// Device helpers shared by the q4 kernels (CDNA4 / gfx950, wave64).
//
// Device weight format ("tiled"; written once at load time by qw_q4_tile
// from the checkpoint's compressed-tensors order, the role the reference's
// pack_int4_words plays, src/engine/weight_convert.cpp:61-71):
//   Wt  uint4 [N/16][G][4][16]   entry (sub, g, q, n) holds the 16 bytes of
//       row 16 sub + n that cover K elements g*128 + 32q .. +32, i.e. exactly
//       what lane 16q + n of a wave feeds the 16x16x32 MFMA for group g. One
//       wave-wide load is 1 KB of contiguous HBM. Inside each 32-bit word the
//       nibbles are reordered: element j (j < 4) at bits 8j, element j + 4 at
//       bits 8j + 4.
//   St  fp16  [N/16][ceil(G/4)][16][4]   scales, the 4 groups of a chunk per row
//   Zt  u16   [N/16][ceil(G/4)][16]      4-bit zeros, group 4gc + j at bits 4j
//       (absent: the reference's fixed zero of 8)
//   w = (q - z) * s;  G = K / 128.
//
// How a nibble reaches an MFMA operand exactly. For a (reordered) word w and
// a group zero z:
//   lo = (w      & 0x0F0F0F0F) + (16 - z) * 0x01010101   bytes e0 e1 e2 e3
//   hi = (w >> 4 & 0x0F0F0F0F) + (16 - z) * 0x01010101   bytes e4 e5 e6 e7
// Each byte is v = 16 + q - z in [1, 31] (no carry between bytes). One
// v_perm_b32 against a constant places two bytes under a high byte of 0x43
// (bf16) or 0x64 (fp16): 0x43vv is the bf16 number 128 + v and 0x64vv the fp16
// number 1024 + v, both exact. The operand thus holds BIAS + (q - z) with
// BIAS = 144 (bf16) or 1040 (fp16), elements in natural K order, and the MFMA
// accumulator is started at -BIAS * sum(x) over the group, leaving
// sum x * (q - z) with every product exact in fp32. The group scale is
// applied once per group, in fp32, on the accumulator.
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
    static constexpr uint32_t ONE = 0x3F803F80u;       // two bf16 1.0
    // unpack8_q operands: BASE + UNIT * q
    static constexpr float BASE = 128.f, UNIT = 1.f;
    typedef bf16x8 vec;
};
struct F16 {
    static constexpr uint32_t HI = 0x64646464u;    // high byte of 1024 + v
    static constexpr uint32_t ONE = 0x3C003C00u;       // two fp16 1.0
    static constexpr float BASE = 1024.f, UNIT = 16.f;
    typedef f16x8 vec;
};

// Waits until at most N vector-memory loads of this wave are in flight
// (loads complete in order: everything issued before the last N is done),
// without waiting on LDS or scalar traffic. For direct-to-LDS loads followed
// by loads that must stay in flight: a fence would wait for all of them.
template <int N>
__device__ __forceinline__ void wait_vm_below() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS-only barrier: orders this block's LDS traffic without draining the
// global-memory loads in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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

// One reordered word (8 nibbles) -> 8 operand elements BIAS + (q - z), K order.
template <typename T>
__device__ __forceinline__ uint4 unpack8(uint32_t w, uint32_t zb) {
    const uint32_t lo = (w & 0x0F0F0F0Fu) + zb;
    const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) + zb;
    uint4 r;
    // byte selectors: 0-3 pick from the second source (lo/hi), 4 picks a byte of T::HI
    r.x = __builtin_amdgcn_perm(T::HI, lo, 0x04010400u);  // e0, e1
    r.y = __builtin_amdgcn_perm(T::HI, lo, 0x04030402u);  // e2, e3
    r.z = __builtin_amdgcn_perm(T::HI, hi, 0x04010400u);  // e4, e5
    r.w = __builtin_amdgcn_perm(T::HI, hi, 0x04030402u);  // e6, e7
    return r;
}

// One reordered word (8 nibbles) -> 8 operand elements BASE + UNIT * q, K
// order (the zero point is left to the accumulator's starting value): the
// unpack8 scheme without the per-byte zero add. bf16: 128 + q (q in the low
// mantissa bits, the most a 7-bit mantissa allows). fp16: 1024 + 16 q (q in
// mantissa bits 4-7 of 10): the product's cancelling part, BASE / UNIT = 64
// times the wanted one, is 16 times smaller than with 1024 + q, at the same
// instruction count.
template <typename T>
__device__ __forceinline__ uint4 unpack8_q(uint32_t w) {
    uint32_t lo, hi;
    if constexpr (__is_same(T, F16)) {
        lo = (w << 4) & 0xF0F0F0F0u;
        hi = w & 0xF0F0F0F0u;
    } else {
        lo = w & 0x0F0F0F0Fu;
        hi = (w >> 4) & 0x0F0F0F0Fu;
    }
    uint4 r;
    r.x = __builtin_amdgcn_perm(T::HI, lo, 0x04010400u);  // e0, e1
    r.y = __builtin_amdgcn_perm(T::HI, lo, 0x04030402u);  // e2, e3
    r.z = __builtin_amdgcn_perm(T::HI, hi, 0x04010400u);  // e4, e5
    r.w = __builtin_amdgcn_perm(T::HI, hi, 0x04030402u);  // e6, e7
    return r;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

// fp32 -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

// fp32 -> fp16 for the fp16 MFMA operands and intermediates: finite values
// beyond the fp16 range saturate to +-65504 (the reference's bf16_to_f16
// rule, src/engine/weight_convert.cpp:19-26); infinities and NaN pass
// through, so a diverging activation stays visible in the output.
__device__ __forceinline__ _Float16 f32_to_f16_satfinite(float v) {
    const bool finite = __builtin_isfinite(v);
    return _Float16(finite ? fminf(fmaxf(v, -65504.f), 65504.f) : v);
}

// The reference's activation functions (src/kernels/common.cuh:94-99):
// sigmoid(x) = 1 / (1 + exp(-x)) with the fast exp, silu(x) = x * sigmoid(x)
// (a multiply by the reciprocal, not a division: the two can differ in the
// last bit). Every SwiGLU of this library uses these two.
__device__ __forceinline__ float sigmoid_ref(float x) { return 1.f / (1.f + __expf(-x)); }
__device__ __forceinline__ float silu_ref(float x) { return x * sigmoid_ref(x); }

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __builtin_bit_cast(float, uint32_t(b) << 16); }

__device__ __forceinline__ int group_zero(const uint32_t *Z, int64_t row, int zw, int g) {
    return Z ? int((Z[row * zw + (g >> 3)] >> (4 * (g & 7))) & 0xfu) : 8;
}

// Tiled-format addressing of one 16-row subtile.
struct Q4Tile {
    const uint4 *w;     // Wt + sub * G * 64
    const uint16_t *s;  // St + sub * GC * 64
    const uint16_t *z;  // Zt + sub * GC * 16, or null
    __device__ __forceinline__ Q4Tile(const uint32_t *Wt, const uint16_t *St, const uint16_t *Zt, int64_t sub, int G) {
        const int GC = (G + 3) / 4;
        w = reinterpret_cast<const uint4 *>(Wt) + sub * G * 64;
        s = St + sub * GC * 64;
        z = Zt ? Zt + sub * GC * 16 : nullptr;
    }
    // lane's 16 bytes of group g, its row's scale and zero
    __device__ __forceinline__ uint4 word4(int g, int lane) const { return w[g * 64 + lane]; }
    // the same as a streaming (non-temporal) load: weights are read once per
    // launch, so they should not displace the activations (read by every
    // block) from the caches
    __device__ __forceinline__ uint4 word4_stream(int g, int lane) const {
        typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w + g * 64 + lane));
        return make_uint4(v[0], v[1], v[2], v[3]);
    }
    __device__ __forceinline__ uint16_t scale(int g, int n) const { return s[(g >> 2) * 64 + n * 4 + (g & 3)]; }
    // the 16-bit zero word holding group g's zero (z must be non-null); the
    // zero itself is zero_of(word, g)
    __device__ __forceinline__ uint32_t zero_word(int g, int n) const { return z[(g >> 2) * 16 + n]; }
    __device__ __forceinline__ static uint32_t zero_of(uint32_t word, int g) { return (word >> (4 * (g & 3))) & 0xfu; }
};

// Hand-off between the blocks of one launch ("the last block to finish a
// range also reduces it"). Each XCD has its own L2, so an agent-scope fence
// writes back or invalidates the whole L2 of the executing XCD; done by
// thousands of producer blocks that costs more than the kernel itself.
// Instead only the handed-off values are coherent at agent scope: producers
// store them as agent-scope atomics (written through the XCD's L2), wait for
// those stores to complete, and then count the block on an agent-scope atomic
// counter; the block that counts last reads the values with agent-scope
// atomic loads (served past its L2).
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u32(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent_u32(const uint32_t *p) {
    return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Counts the calling block on *counter; true in every thread of the block
// that counted total-th. Every thread's earlier st_agent stores are complete
// before the count. The last block resets the counter to zero.
__device__ __forceinline__ bool count_last_block(int *counter, int total) {
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
        if (s_last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return s_last;
}

// Tile lists over an expert's contiguous slots (routing with tile_m != 0).
// tile_m > 0: tiles of tile_m rows. tile_m = -g: mixed tiles; the tile that
// starts rem slots before the end of the expert's range has 4g rows when
// rem > 5g, else rem rounded up to a multiple of g (g to 5g): whole 4g tiles,
// then one tile for the rest, a rest of at most g joining the last whole
// tile. Each tile of an expert's range dequantises the expert's weights once:
// the fewest tiles at the least padding.
__device__ __forceinline__ int tile_rows(int rem, int tile_m) {
    if (tile_m > 0) return tile_m;
    const int g = -tile_m;
    return rem > 5 * g ? 4 * g : (rem + g - 1) / g * g;
}

// Number of tiles over c slots.
__device__ __forceinline__ int tile_count(int c, int tile_m) {
    if (tile_m > 0) return (c + tile_m - 1) / tile_m;
    int n = 0;
    for (int m0 = 0; m0 < c; m0 += tile_rows(c - m0, tile_m)) ++n;
    return n;
}

}  // namespace qwq4
