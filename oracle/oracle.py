"""numpy/ctypes front end of the CPU oracle (oracle/q4_oracle.c).

Test infrastructure only: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, as the checker. The product library never loads
it. Reference citations for each routine are in q4_oracle.c.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C")
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "liboq4.so"], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboq4.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.o_q4_unpack.argtypes = [_u32p, _i64, _i64, _u8p]
        L.o_q4_dequant.argtypes = [_u32p, _u16p, _vp, _i64, _i64, _f32p]
        L.o_q4_linear.argtypes = [_u32p, _u16p, _vp, _i64, _i64, _f32p, _int, _int, _f32p, _int, _int]
        L.o_q4_linear_f64.argtypes = [_u32p, _u16p, _vp, _i64, _i64, _f32p, _int, _int, _f64p, _int, _int]
        L.o_pack_engine_order.argtypes = [_u32p, _u32p, _i64]
        L.o_unpack_engine_order.argtypes = [_u32p, _u32p, _i64]
        L.o_quantize_g128.argtypes = [_u16p, _i64, _u32p, _u16p]
        L.o_route.argtypes = [_f32p, _int, _int, _int, _i32p, _f32p]
        L.o_moe_slots.argtypes = [_i32p, _int, _int, _int, _i32p, _i32p, _i32p, _i32p]
        L.o_q4_tile.argtypes = [_u32p, _u16p, _vp, _i64, _i64, _u32p, _u16p, _vp]
        L.o_moe.argtypes = [_f32p, _int, _int, _int, _int, _int, _f32p] + [_u32p, _u16p, _vp] * 3 + [_f32p, _vp, _vp, _int]
        L.o_linear_w16.argtypes = [_u16p, _int, _i64, _i64, _i64, _f32p, _int, _int, _f32p, _int, _int]
        L.o_swiglu_gate.argtypes = [_f32p, _int, _int, _int, _f32p]
        L.o_quantize_rows_i8.argtypes = [_u16p, _i64, _i64, _i64, _vp, _f32p]
        L.o_i8_linear_f64.argtypes = [_vp, _f32p, _i64, _i64, _int, _u16p, _int, _int, _int, _f64p, _int, _int]
        L.o_quant_rows_i8.argtypes = [_u16p, _int, _i64, _i64, _i64, _vp, _f32p]
        L.o_w4a8_linear.argtypes = [_vp, _f32p, _vp, _i64, _i64, _u32p, _u16p, _vp, _i64, _f32p, _int]
        for n in ("o_bf16_to_f32", "o_f16_to_f32"):
            getattr(L, n).argtypes = [ctypes.c_uint16]
            getattr(L, n).restype = ctypes.c_float
        L.o_bf16_to_f16.argtypes = [ctypes.c_uint16]
        L.o_bf16_to_f16.restype = ctypes.c_uint16
        for n in ("o_f32_to_f16", "o_f32_to_bf16"):
            getattr(L, n).argtypes = [ctypes.c_float]
            getattr(L, n).restype = ctypes.c_uint16
        _LIB = L
    return _LIB


def _zp(Z):
    return None if Z is None else Z.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def nthreads():
    return os.cpu_count() or 1


# ---- numbers (vectorised by looping in C over a numpy array would be nicer;
# these are exact helpers for small arrays and for golden checks)
def f16_to_f32(h):
    h = np.asarray(h, np.uint16)
    return np.array([lib().o_f16_to_f32(int(v)) for v in h.ravel()], np.float32).reshape(h.shape)


def f32_to_f16(x):
    x = np.asarray(x, np.float32)
    return np.array([lib().o_f32_to_f16(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def f32_to_bf16(x):
    x = np.asarray(x, np.float32)
    return np.array([lib().o_f32_to_bf16(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def bf16_to_f16(b):
    """weight_convert.cpp:19-26: saturating bf16 -> fp16 bits."""
    b = np.asarray(b, np.uint16)
    return np.array([lib().o_bf16_to_f16(int(v)) for v in b.ravel()], np.uint16).reshape(b.shape)


def bf16_to_f32(b):
    b = np.asarray(b, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---- q4 format
def q4_unpack(W, N, K):
    out = np.empty((N, K), np.uint8)
    lib().o_q4_unpack(_c(W, np.uint32), N, K, out)
    return out


def q4_dequant(W, S, Z, N, K):
    out = np.empty((N, K), np.float32)
    W, S = _c(W, np.uint32), _c(S, np.uint16)
    Z = None if Z is None else _c(Z, np.uint32)
    lib().o_q4_dequant(W, S, _zp(Z), N, K, out)
    return out


def _row_slices(N, K, x, rpg):
    """Rows grouped over activation slices as gpu::gemv_rows groups them
    (src/kernels/gemv.hip:16-17: row n reads x + (n / rpg) * K): yields
    (r0, r1, x slice [T][K]) per slice of x [T][slices * K]."""
    T = x.shape[0]
    for s, r0 in enumerate(range(0, N, rpg)):
        yield r0, min(N, r0 + rpg), np.ascontiguousarray(x[:, s * K:(s + 1) * K]).reshape(T, K)


def q4_linear(W, S, Z, N, K, x, threads=None, rpg=0):
    """y[t][n] = sum_k deq(W)[n][k] x[t][off(n) + k]; x fp32 [T][K] (or [T][slices * K] with
    rpg > 0, off(n) = (n // rpg) * K) -> y fp32 [T][N]."""
    if rpg:
        x = _c(x, np.float32)
        x = x.reshape(x.shape[0] if x.ndim > 1 else 1, -1)
        y = np.empty((x.shape[0], N), np.float32)
        W, S = np.asarray(W).reshape(N, -1), np.asarray(S).reshape(N, -1)
        Z = None if Z is None else np.asarray(Z).reshape(N, -1)
        for r0, r1, xs in _row_slices(N, K, x, rpg):
            y[:, r0:r1] = q4_linear(W[r0:r1], S[r0:r1], None if Z is None else Z[r0:r1], r1 - r0, K, xs, threads)
        return y
    x = _c(x, np.float32).reshape(-1, K)
    T = x.shape[0]
    y = np.empty((T, N), np.float32)
    W, S = _c(W, np.uint32), _c(S, np.uint16)
    Z = None if Z is None else _c(Z, np.uint32)
    lib().o_q4_linear(W, S, _zp(Z), N, K, x, T, K, y, N, threads or nthreads())
    return y


def q4_linear_f64(W, S, Z, N, K, x, threads=None):
    x = _c(x, np.float32).reshape(-1, K)
    T = x.shape[0]
    y = np.empty((T, N), np.float64)
    W, S = _c(W, np.uint32), _c(S, np.uint16)
    Z = None if Z is None else _c(Z, np.uint32)
    lib().o_q4_linear_f64(W, S, _zp(Z), N, K, x, T, K, y, N, threads or nthreads())
    return y


def pack_engine_order(words):
    w = _c(words, np.uint32).ravel()
    out = np.empty_like(w)
    lib().o_pack_engine_order(w, out, w.size)
    return out.reshape(np.shape(words))


def unpack_engine_order(words):
    w = _c(words, np.uint32).ravel()
    out = np.empty_like(w)
    lib().o_unpack_engine_order(w, out, w.size)
    return out.reshape(np.shape(words))


def quantize_g128(src_bf16):
    s = _c(src_bf16, np.uint16).ravel()
    ng = s.size // 128
    words = np.empty(ng * 16, np.uint32)
    scales = np.empty(ng, np.uint16)
    lib().o_quantize_g128(s, ng, words, scales)
    return words, scales


# ---- routing / MoE
def route(logits, topk):
    logits = _c(logits, np.float32)
    T, E = logits.shape
    top_e = np.empty((T, topk), np.int32)
    top_w = np.empty((T, topk), np.float32)
    lib().o_route(logits, T, E, topk, top_e, top_w)
    return top_e, top_w


def moe_slots(top_e, E):
    top_e = _c(top_e, np.int32)
    T, k = top_e.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    tok_slot = np.empty((T, k), np.int32)
    pair_tok = np.empty(T * k, np.int32)
    lib().o_moe_slots(top_e, T, E, k, counts, offsets, tok_slot, pair_tok)
    return counts, offsets, tok_slot, pair_tok


def moe(x, logits, topk, gate, up, down, threads=None, want_parts=False):
    """gate/up/down: (W, S, Z) with W [E][rows][K/8], S [E][rows][G], Z or None."""
    x = _c(x, np.float32)
    logits = _c(logits, np.float32)
    T, H = x.shape
    E = logits.shape[1]
    F = gate[0].shape[1]
    out = np.empty((T, H), np.float32)
    h = np.empty((T * topk, F), np.float32) if want_parts else None
    yp = np.empty((T * topk, H), np.float32) if want_parts else None
    args = []
    for W, S, Z in (gate, up, down):
        args += [_c(W, np.uint32), _c(S, np.uint16), None if Z is None else _c(Z, np.uint32)]
    keep = args[:]
    cargs = []
    for i, a in enumerate(args):
        cargs.append(_zp(a) if i % 3 == 2 else a)
    lib().o_moe(x, T, H, F, E, topk, logits, *cargs, out,
                None if h is None else h.ctypes.data_as(ctypes.c_void_p),
                None if yp is None else yp.ctypes.data_as(ctypes.c_void_p), threads or nthreads())
    del keep
    if want_parts:
        return out, h, yp
    return out


def linear_w16(W, x, f16=False, threads=None, rpg=0):
    """y[t][o] = sum_i W[o][i] x[t][off(o) + i], W 16-bit bits [N][K] (bf16, or fp16 with f16)
    widened to fp32 (ref::Model::linear, src/ref/ref_model.cpp:86-97); rows grouped over
    activation slices with rpg > 0 as gpu::gemv_rows does (off(o) = (o // rpg) * K)."""
    W = _c(W, np.uint16)
    N, K = W.shape
    if rpg:
        x = _c(x, np.float32)
        x = x.reshape(x.shape[0] if x.ndim > 1 else 1, -1)
        y = np.empty((x.shape[0], N), np.float32)
        for r0, r1, xs in _row_slices(N, K, x, rpg):
            y[:, r0:r1] = linear_w16(W[r0:r1], xs, f16, threads)
        return y
    x = _c(x, np.float32).reshape(-1, K)
    T = x.shape[0]
    y = np.empty((T, N), np.float32)
    lib().o_linear_w16(W, int(f16), N, K, K, x, T, K, y, N, threads or nthreads())
    return y


def swiglu_gate(v, n):
    """h[t][j] = silu(v[t][j]) * v[t][n + j] * sigmoid(v[t][2n]) for v [T][>= 2n + 1]."""
    v = _c(v, np.float32)
    T, ldv = v.shape
    h = np.empty((T, n), np.float32)
    lib().o_swiglu_gate(v, ldv, n, T, h)
    return h


def quantize_rows_i8(w16, group=32):
    """fp16 weight bits [N][K] -> (int8 [N][K], fp32 scales [N][K/group]) as
    quantize_rows_i8 (src/engine/weight_convert.cpp:92-108)."""
    w16 = _c(w16, np.uint16)
    N, K = w16.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N, K // group), np.float32)
    lib().o_quantize_rows_i8(w16, N, K, group, q.ctypes.data, s)
    return q, s


def i8_linear_f64(W8, scale, x16, M, xs=None, rpg=0, group=32, threads=None):
    """fp64 y [M][N] of gemv_rows_i8 (src/kernels/gemv.hip:75-136): int8 W8 [N][K] times
    its group scales times fp16 rows x16 (stride xs; row n reads block n // rpg when rpg)."""
    W8 = np.ascontiguousarray(W8, np.int8)
    N, K = W8.shape
    x16 = _c(x16, np.uint16).ravel()
    xs = xs or K
    y = np.empty((M, N), np.float64)
    lib().o_i8_linear_f64(W8.ctypes.data, _c(scale, np.float32), N, K, group, x16, xs, M, rpg, y, N,
                          threads or nthreads())
    return y


def shared_expert(x, w_gu, w_down, f16_gu=False, f16_down=False):
    """The shared expert's term of ref_model.cpp:465-478: w_gu [2n + 1][H] holds the gate
    rows, the up rows and the gate-logit row (the engine's concatenation, decode.hip:99),
    w_down [H][n]; returns sigmoid(gate logit) * down(silu(gate x) * up x), [T][H]."""
    n = (w_gu.shape[0] - 1) // 2
    v = linear_w16(w_gu, x, f16_gu)
    return linear_w16(w_down, swiglu_gate(v, n), f16_down)


def q4_tile(W, S, Z, N, K):
    """Checkpoint-order q4 -> the kernels' tiled format (Wt, St, Zt or None)."""
    G = K // 128
    GC = (G + 3) // 4
    Wt = np.empty(N * K // 8, np.uint32)
    St = np.empty(N // 16 * GC * 64, np.uint16)
    Zt = np.empty(N // 16 * GC * 16, np.uint16) if Z is not None else None
    W, S = _c(W, np.uint32), _c(S, np.uint16)
    Zc = None if Z is None else _c(Z, np.uint32)
    lib().o_q4_tile(W, S, _zp(Zc), N, K, Wt, St, None if Zt is None else Zt.ctypes.data_as(ctypes.c_void_p))
    return Wt, St, Zt


# ---- W4A8 (the reference's opt-in int8-activation expert GEMMs)
def quant_rows_i8(x16, f16=True):
    """16-bit rows [R][K] (fp16 bits when f16, else bf16) -> (int8 [R][K], fp32 [R][K/128])
    as moe_w4a8.hip's quant_rows_kernel (src/kernels/moe_w4a8.hip:17-36)."""
    x16 = _c(x16, np.uint16)
    R, K = x16.shape
    q = np.empty((R, K), np.int8)
    sc = np.empty((R, K // 128), np.float32)
    lib().o_quant_rows_i8(x16, int(f16), R, K, K, q.ctypes.data, sc)
    return q, sc


def w4a8_linear(q8, sx, W, S, Z, N, rowmap=None, threads=None):
    """y[p][n]: the W4A8 product of quantised rows q8[rowmap[p]] (or q8[p]) with q4 weight
    rows (moe_w4a8.hip:62-183): int32 per 64-wide K step, rescaled per step in fp32."""
    q8 = np.ascontiguousarray(q8, np.int8)
    R, K = q8.shape
    rm = None if rowmap is None else _c(rowmap, np.int32)
    P = R if rm is None else rm.size
    y = np.empty((P, N), np.float32)
    W, S = _c(W, np.uint32).reshape(N, K // 8), _c(S, np.uint16).reshape(N, K // 128)
    Z = None if Z is None else _c(Z, np.uint32).reshape(N, -1)
    lib().o_w4a8_linear(q8.ctypes.data, _c(sx, np.float32), None if rm is None else rm.ctypes.data, P, K, W, S, _zp(Z),
                        N, y, threads or nthreads())
    return y


def _silu(g):
    g = np.asarray(g, np.float32)
    return g * (np.float32(1) / (np.float32(1) + np.exp(-g)))


def moe_w4a8(x16, f16, gate, up, down, offsets, pair_tok, E, slots=None):
    """The reference's W4A8 routed experts (gpu::moe_experts_w4a8,
    src/kernels/moe_w4a8.hip:186-215) over the slots of qw_moe_route: x rows quantised
    per 128-group; per expert e and slot p of it, h[p] = fp16(silu(g) * u) with g, u the
    W4A8 products of x[pair_tok[p]]; h rows quantised; yp[p] = fp16(down W4A8 product).
    gate/up/down: (W [E][rows][K/8], S, Z or None). slots: the slots to form (default
    all). Returns h, yp as fp32 arrays of the fp16 values, rows = slots."""
    qx, sx = quant_rows_i8(x16, f16)
    F, H = gate[0].shape[1], gate[0].shape[2] * 8
    P = int(offsets[E])
    slots = np.arange(P) if slots is None else np.asarray(slots)
    h = np.zeros((P, F), np.float16)
    need = np.zeros(P, bool)
    need[slots] = True
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        ps = np.arange(lo, hi)[need[lo:hi]]
        if ps.size == 0:
            continue
        Zg = None if gate[2] is None else gate[2][e]
        Zu = None if up[2] is None else up[2][e]
        g = w4a8_linear(qx, sx, gate[0][e], gate[1][e], Zg, F, rowmap=pair_tok[ps])
        u = w4a8_linear(qx, sx, up[0][e], up[1][e], Zu, F, rowmap=pair_tok[ps])
        h[ps] = (_silu(g) * u).astype(np.float16)
    qh, sh = quant_rows_i8(h.view(np.uint16), True)
    yp = np.zeros((P, H), np.float16)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        ps = np.arange(lo, hi)[need[lo:hi]]
        if ps.size == 0:
            continue
        Zd = None if down[2] is None else down[2][e]
        yp[ps] = w4a8_linear(qh, sh, down[0][e], down[1][e], Zd, H, rowmap=ps).astype(np.float16)
    return h[slots].astype(np.float32), yp[slots].astype(np.float32)
