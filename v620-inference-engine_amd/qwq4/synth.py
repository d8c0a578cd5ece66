"""Seeded synthetic tensors of the benchmark configurations (numpy, host).

Every tensor has its own generator seeded from (seed, name), so shapes can be
added without changing the other tensors' values.
  q4 weights: nibbles uniform 0..15, 8 per uint32 along K (checkpoint order);
              fp16 scales f16(|N(0, 0.02)|) per 128-group; 4-bit zeros
              uniform 0..15 per group (or None: the reference's fixed 8)
  activations: bf16(N(0, 1)) (round to nearest even)
"""
import zlib

import numpy as np

QGROUP = 128


def rng(seed, name):
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def bf16_bits(a):
    """float32 array -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_zeros(z):
    """z uint8 [..., G] in 0..15 -> uint32 [..., ceil(G/8)], group g at bits 4(g%8)."""
    z = np.asarray(z, np.uint32)
    G = z.shape[-1]
    zw = (G + 7) // 8
    pad = np.zeros(z.shape[:-1] + (zw * 8,), np.uint32)
    pad[..., :G] = z
    pad = pad.reshape(z.shape[:-1] + (zw, 8))
    return np.bitwise_or.reduce(pad << (4 * np.arange(8, dtype=np.uint32)), axis=-1).astype(np.uint32)


def unpack_zeros(Zw, G):
    Zw = np.asarray(Zw, np.uint32)
    z = (Zw[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF
    return z.reshape(Zw.shape[:-1] + (-1,))[..., :G].astype(np.uint8)


def q4_weights(seed, name, N, K, zeros=True, lead=()):
    """(W uint32 [*lead, N, K/8], S uint16 fp16 bits [*lead, N, G], Z uint32 or None)."""
    G = K // QGROUP
    r = rng(seed, name)
    W = r.integers(0, 2**32, size=lead + (N, K // 8), dtype=np.uint64).astype(np.uint32)
    S = np.abs(r.normal(0.0, 0.02, size=lead + (N, G))).astype(np.float16).view(np.uint16)
    Z = pack_zeros(r.integers(0, 16, size=lead + (N, G), dtype=np.uint8)) if zeros else None
    return W, S, Z


def acts(seed, name, M, K):
    """bf16 bits [M, K] of N(0,1) and their exact float32 values."""
    b = bf16_bits(rng(seed, name).normal(0.0, 1.0, size=(M, K)).astype(np.float32))
    return b, bf16_to_f32(b)


def router_logits(seed, name, T, E, bias_sigma=0.0):
    r = rng(seed, name)
    l = r.normal(0.0, 1.0, size=(T, E)).astype(np.float32)
    if bias_sigma:
        l += rng(seed, name + ".bias").normal(0.0, bias_sigma, size=(1, E)).astype(np.float32)
    return l


def experts(seed, E, H, F, zeros=True, name="experts"):
    gate = q4_weights(seed, name + ".gate", F, H, zeros, lead=(E,))
    up = q4_weights(seed, name + ".up", F, H, zeros, lead=(E,))
    down = q4_weights(seed, name + ".down", H, F, zeros, lead=(E,))
    return gate, up, down


def q4_bytes(N, K):
    """Algorithmic bytes of a q4 matrix: 0.5 B per weight + fp16 scale and 4-bit zero per group."""
    return N * K // 2 + N * (K // QGROUP) * 2 + N * (K // QGROUP) // 2
