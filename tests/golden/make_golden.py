"""Writes tests/golden/ref_vectors.npz from the reference's own conversion code.

Runs in the build container only: it loads oracle/_ref/libqwref.so, which
oracle/Makefile (`make -C oracle ref`) compiles from the reference sources
src/engine/weight_convert.cpp and src/core/{common.hpp,safetensors,json}.
The output holds inputs and the reference's outputs only:
  f16_all      uint16 [65536]      every fp16 pattern
  f16_all_f32  float32             ref f16_to_f32 of each
  f32_in       float32             edge cases + random values
  f32_to_f16   uint16              ref f32_to_f16 of each
  bf16_in      uint16              bf16 patterns (edges + random)
  bf16_to_f16  uint16              ref bf16_to_f16 (saturating) of each
  words_in     uint32 [4096]       random checkpoint-order words
  words_eng    uint32              ref pack_int4_words of them
  qsrc         uint16 [groups*128] bf16 weights (random + edge groups)
  q_words      uint32              ref quantize_int4_g128 words
  q_scales     uint16              ref quantize_int4_g128 fp16 scales
  i8_src       uint16 [12][256]    fp16 weights (random + edge rows) for quantize_rows_i8
  i8_q32, i8_s32                   ref quantize_rows_i8 (group 32): int8 [12][256], fp32 [12][8]
  i8_q16, i8_s16                   the same with group 16
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def main():
    L = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libqwref.so"))
    L.ref_f16_to_f32.restype = ctypes.c_float
    L.ref_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.ref_f32_to_f16.restype = ctypes.c_uint16
    L.ref_f32_to_f16.argtypes = [ctypes.c_float]
    L.ref_bf16_to_f16.restype = ctypes.c_uint16
    L.ref_bf16_to_f16.argtypes = [ctypes.c_uint16]
    rng = np.random.default_rng(20261201)

    f16_all = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f16_all_f32 = np.array([L.ref_f16_to_f32(int(v)) for v in f16_all], np.float32)

    edges = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.99, 1e9, -1e9, np.inf, -np.inf, np.nan,
                      6.1035156e-05, 6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-10,
                      1.0009766, 1.0004883, 1.0014648, 2049.0, 2051.0, 0.33333334], np.float32)
    f32_in = np.concatenate([edges, rng.normal(0, 1, 6000).astype(np.float32),
                             (rng.normal(0, 1, 4000) * 10.0 ** rng.uniform(-9, 5, 4000)).astype(np.float32),
                             rng.integers(0, 2**32, 4000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    f32_in = f32_in[~np.isnan(f32_in) | (np.arange(f32_in.size) == 11)]
    f32_to_f16 = np.array([L.ref_f32_to_f16(float(v)) for v in f32_in], np.uint16)

    bf16_in = np.concatenate([np.array([0x0000, 0x8000, 0x3F80, 0x477F, 0x4780, 0xC780, 0x7F80, 0xFF80, 0x7FC0,
                                        0x0001, 0x3380, 0x3300], np.uint16),
                              rng.integers(0, 65536, 4000, dtype=np.uint32).astype(np.uint16)])
    bf16_to_f16 = np.array([L.ref_bf16_to_f16(int(v)) for v in bf16_in], np.uint16)

    words_in = rng.integers(0, 2**32, 4096, dtype=np.uint64).astype(np.uint32)
    words_eng = np.empty_like(words_in)
    L.ref_pack_int4_words(words_in.ctypes.data_as(ctypes.c_void_p), words_eng.ctypes.data_as(ctypes.c_void_p),
                          ctypes.c_size_t(words_in.size))

    groups = [rng.normal(0, 0.02, 128) for _ in range(60)]
    groups.append(np.zeros(128))                                   # amax 0 -> scale 0
    groups.append(np.full(128, 3.0))                               # constant
    groups.append(np.linspace(-1, 1, 128))                         # exact ties at +-0.5 steps
    groups.append(np.concatenate([[1000.0], rng.normal(0, 1e-3, 127)]))  # one outlier
    src = np.concatenate(groups).astype(np.float32)
    ub = src.view(np.uint32).astype(np.uint64)
    qsrc = ((ub + 0x7FFF + ((ub >> 16) & 1)) >> 16).astype(np.uint16)
    ng = len(groups)
    q_words = np.empty(ng * 16, np.uint32)
    q_scales = np.empty(ng, np.uint16)
    L.ref_quantize_int4_g128(qsrc.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(ng),
                             q_words.ctypes.data_as(ctypes.c_void_p), q_scales.ctypes.data_as(ctypes.c_void_p))

    # int8 rows (quantize_rows_i8, weight_convert.cpp:92-108): fp16 weights,
    # random rows plus a zero group, a constant group, a symmetric ramp (ties
    # of w / s at half steps), an outlier row and large magnitudes
    rows = [rng.normal(0, 0.05, 256) for _ in range(6)]
    r = rng.normal(0, 1, 256)
    r[32:64] = 0.0
    r[64:96] = -2.5
    rows.append(r)
    rows.append(np.tile(np.linspace(-127, 127, 32), 8) * 0.01)
    r = rng.normal(0, 1e-3, 256)
    r[5] = 300.0
    rows.append(r)
    rows.append(rng.normal(0, 1, 256) * 1e4)
    rows.append(rng.uniform(-1, 1, 256))
    rows.append(-np.abs(rng.normal(0, 1, 256)))
    i8_f32 = np.stack(rows).astype(np.float32)
    i8_src = np.array([L.ref_f32_to_f16(float(v)) for v in i8_f32.ravel()], np.uint16).reshape(i8_f32.shape)
    N8, K8 = i8_src.shape
    L.ref_quantize_rows_i8.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_int64]
    i8 = {}
    for g in (32, 16):
        q = np.empty((N8, K8), np.int8)
        sc = np.empty((N8, K8 // g), np.float32)
        L.ref_quantize_rows_i8(i8_src.ctypes.data, N8, K8, q.ctypes.data, sc.ctypes.data, g)
        i8[f"i8_q{g}"], i8[f"i8_s{g}"] = q, sc

    out = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(out, f16_all=f16_all, f16_all_f32=f16_all_f32, f32_in=f32_in, f32_to_f16=f32_to_f16,
                        bf16_in=bf16_in, bf16_to_f16=bf16_to_f16, words_in=words_in, words_eng=words_eng, qsrc=qsrc,
                        q_words=q_words, q_scales=q_scales, i8_src=i8_src, **i8)
    print(out, os.path.getsize(out))


if __name__ == "__main__":
    main()
