"""Python binding of libqwq4.so (include/qw/q4ops.h) over ctypes.

Device memory and streams come from PyTorch; every call goes through the C ABI
to the HIP kernels. There is no fallback: if the library is missing or a call
fails, a RuntimeError is raised.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libqwq4.so")
_lib = None

# every symbol include/qw/q4ops.h declares (checked by the CPU tests)
SYMBOLS = (
    "qw_q4_abi_version", "qw_q4_last_error", "qw_q4_gemv", "qw_q4_gemm_workspace_size", "qw_q4_gemm",
    "qw_moe_route", "qw_moe_experts_gemv", "qw_moe_experts_grouped", "qw_moe_grouped_workspace_size", "qw_moe_grouped_tile_m",
    "qw_moe_combine", "qw_q4_unpack", "qw_q4_dequant", "qw_q4_from_engine_order",
    "qw_q4_tiled_size", "qw_q4_tile", "qw_q4_untile", "qw_bf16_to_f16", "qw_read_probe",
    "qw_st_open", "qw_st_close", "qw_st_count", "qw_st_name", "qw_st_tensor",
    "qw_q4_load_staging_size", "qw_q4_load", "qw_q4_tiled_offset",
    "qw_moe_decode_workspace_size", "qw_moe_decode", "qw_moe_decode_static_max_bytes", "qw_moe_decode_static",
    "qw_moe_decode_static_reset", "qw_moe_decode_with_shared_workspace_size", "qw_moe_decode_with_shared",
    "qw_w16_gemv", "qw_w16_tiled_size", "qw_w16_tile", "qw_w16_gemv_tiled", "qw_w16_swiglu_gemv_tiled", "qw_i8_gemv", "qw_i8_tiled_size", "qw_i8_tile",
    "qw_moe_w4a8_tile_m", "qw_moe_w4a8_workspace_size", "qw_moe_experts_w4a8", "qw_quant_rows_i8", "qw_swiglu_gate",
    "qw_wcache_open", "qw_wcache_put", "qw_wcache_get", "qw_wcache_finish", "qw_wcache_close",
)

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

_SIGS = {
    "qw_q4_abi_version": ([], _I),
    "qw_q4_last_error": ([], ctypes.c_char_p),
    "qw_q4_gemv": ([_P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "qw_q4_gemm_workspace_size": ([_I, _I], _SZ),
    "qw_q4_gemm": ([_P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _I, _I, _P, _SZ, _P], _I),
    "qw_moe_route": ([_P, _I, _I, _I, _I] + [_P] * 11 + [_P], _I),
    "qw_moe_experts_gemv": ([_P] * 9 + [_I, _I, _I] + [_P] * 5 + [_I, _I, _I, _P, _P, _I, _P], _I),
    "qw_moe_grouped_workspace_size": ([_I, _I, _I, _I, _I], _SZ),
    "qw_moe_experts_grouped": ([_P] * 9 + [_I, _I, _I] + [_P] * 6 + [_I, _I, _I, _P, _P, _I, _P, _SZ, _P], _I),
    "qw_moe_grouped_tile_m": ([], _I),
    "qw_moe_combine": ([_P, _I, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P], _I),
    "qw_q4_tiled_size": ([_I64, _I64, _P, _P, _P], None),
    "qw_q4_tile": ([_P, _P, _P, _I64, _I64, _P, _P, _P, _P], _I),
    "qw_q4_untile": ([_P, _P, _P, _I64, _I64, _P, _P, _P, _P], _I),
    "qw_q4_unpack": ([_P, _I64, _I64, _P, _P], _I),
    "qw_q4_dequant": ([_P, _P, _P, _I64, _I64, _P, _P], _I),
    "qw_q4_from_engine_order": ([_P, _P, _I64, _P], _I),
    "qw_bf16_to_f16": ([_P, _P, _I64, _P], _I),
    "qw_read_probe": ([_P, _I64, _P], _I),
    "qw_moe_decode_workspace_size": ([_I, _I, _I, _I, _I], _SZ),
    "qw_moe_decode": ([_P, _I, _P, _I, _I, _I, _I] + [_P] * 9 + [_I, _I, _P, _P, _I] + [_P] * 6 + [_I, _P, _SZ, _P], _I),
    "qw_moe_decode_static_max_bytes": ([], _SZ),
    "qw_w16_gemv": ([_P, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "qw_w16_tiled_size": ([_I, _I], _SZ),
    "qw_w16_tile": ([_P, _I, _I, _I, _P, _P], _I),
    "qw_w16_gemv_tiled": ([_P, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "qw_w16_swiglu_gemv_tiled": ([_P, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P], _I),
    "qw_i8_gemv": ([_P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "qw_i8_tiled_size": ([_I, _I, _I, _P, _P], None),
    "qw_i8_tile": ([_P, _P, _I, _I, _I, _P, _P, _P], _I),
    "qw_moe_w4a8_tile_m": ([], _I),
    "qw_moe_w4a8_workspace_size": ([_I, _I, _I, _I], _SZ),
    "qw_moe_experts_w4a8": ([_P] * 9 + [_I, _I, _I] + [_P] * 6 + [_I, _I, _I, _P, _P, _P, _SZ, _P], _I),
    "qw_quant_rows_i8": ([_P, _I, _I, _I, _I, _P, _P, _P], _I),
    "qw_swiglu_gate": ([_P, _I, _I, _I, _P, _P], _I),
    "qw_moe_decode_static": ([_P, _I, _P, _I, _I, _I, _I] + [_P] * 9 + [_I, _I, _P, _P, _I] + [_P] * 6 + [_I, _P], _I),
    "qw_moe_decode_with_shared_workspace_size": ([_I, _I, _I, _I, _I, _I], _SZ),
    "qw_moe_decode_with_shared": ([_P, _I, _P, _I, _I, _I, _I] + [_P] * 9 + [_I, _I, _P, _P, _I, _P, _P, _P, _I]
                                  + [_P] * 6 + [_I, _P, _SZ, _P], _I),
    "qw_moe_decode_static_reset": ([_P], _I),
    "qw_st_open": ([ctypes.c_char_p, _P], _I),
    "qw_st_close": ([_P], None),
    "qw_wcache_open": ([ctypes.c_char_p, ctypes.c_uint64, _P, _P], _I),
    "qw_wcache_put": ([_P, _P, ctypes.c_size_t, _I, _P], _I),
    "qw_wcache_get": ([_P, _P, ctypes.c_size_t, _I, _P], _I),
    "qw_wcache_finish": ([_P], _I),
    "qw_wcache_close": ([_P], None),
    "qw_st_count": ([_P], _I),
    "qw_st_name": ([_P, _I], ctypes.c_char_p),
    "qw_st_tensor": ([_P, ctypes.c_char_p, _P, _P, _P, _P, _P], _I),
    "qw_q4_load_staging_size": ([_I64, _I64], _SZ),
    "qw_q4_load": ([_P, ctypes.c_char_p, _I64, _I64, _P, _P, _P, _SZ, _P], _I),
    "qw_q4_tiled_offset": ([_I64, _I64, _P, _P, _P], None),
}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with v620-inference-engine_amd/build.py")
        # torch first: its HIP runtime (same soname as the one the library
        # links) is then the only one in the process, so streams and device
        # pointers from torch are the library's own
        import torch  # noqa: F401
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(rc, fn):
    if rc != 0:
        raise RuntimeError(f"{fn} failed ({rc}): {lib().qw_q4_last_error().decode()}")


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("qwq4: all tensors must be on the GPU")


# ------------------------------------------------------------ weight format
def tiled_size(N, K):
    a, b, c = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    lib().qw_q4_tiled_size(N, K, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    return a.value, b.value, c.value


def tile(W, S, Z, N, K):
    """Checkpoint-order (W, S, Z) device tensors -> tiled (Wt, St, Zt or None)."""
    import torch
    wb, sb, zb = tiled_size(N, K)
    Wt = torch.empty(wb // 4, dtype=torch.int32, device=W.device)
    St = torch.empty(sb // 2, dtype=torch.int16, device=W.device)
    Zt = torch.empty(zb // 2, dtype=torch.int16, device=W.device) if Z is not None else None
    _dev(W, S, Z)
    _check(lib().qw_q4_tile(_ptr(W), _ptr(S), _ptr(Z), N, K, _ptr(Wt), _ptr(St), _ptr(Zt), _stream()), "qw_q4_tile")
    return Wt, St, Zt


def untile(Wt, St, Zt, N, K):
    import torch
    G = K // 128
    W = torch.empty((N, K // 8), dtype=torch.int32, device=Wt.device)
    S = torch.empty((N, G), dtype=torch.int16, device=Wt.device)
    Z = torch.empty((N, (G + 7) // 8), dtype=torch.int32, device=Wt.device) if Zt is not None else None
    _check(lib().qw_q4_untile(_ptr(Wt), _ptr(St), _ptr(Zt), N, K, _ptr(W), _ptr(S), _ptr(Z), _stream()),
           "qw_q4_untile")
    return W, S, Z


def tile_experts(W, S, Z, rows, K):
    """[E][rows][...] checkpoint-order expert stacks -> one tiled [E*rows][K] matrix."""
    E = W.shape[0]
    return tile(W.reshape(E * rows, -1), S.reshape(E * rows, -1), None if Z is None else Z.reshape(E * rows, -1),
                E * rows, K)


# ---------------------------------------------------------------- operators
# element-type codes of the *_type arguments (QW_T_F32, QW_T_BF16, QW_T_F16)
T_F32, T_BF16, T_F16 = 0, 1, 2


def _tcode(t):
    """QW_T_* code of a tensor's dtype (float32, bfloat16, float16)."""
    import torch
    codes = {torch.float32: T_F32, torch.bfloat16: T_BF16, torch.float16: T_F16}
    if t.dtype not in codes:
        raise TypeError(f"unsupported element type {t.dtype}")
    return codes[t.dtype]


def _tdtype(code):
    import torch
    return {T_F32: torch.float32, T_BF16: torch.bfloat16, T_F16: torch.float16}[code]


def _is_f16(x, x_f16):
    """x_f16 given, else from the tensor: float16 -> fp16 rows, anything else
    (bfloat16, or int16 bit patterns) -> bf16 rows."""
    import torch
    return bool(x_f16) if x_f16 is not None else x.dtype == torch.float16


def gemv(W, S, Z, x, N, K, M=None, y=None, y_bf16=False, accumulate=False, xs=None, ys=None, x_f16=None, rpg=0):
    """y[m][n] (+)= sum_k deq(W)[n][k] x[m][off(n) + k], off(n) = (n // rpg) * K when rpg (row
    slices, gpu::gemv_rows). x: bf16 rows (bfloat16, or int16 bit patterns) or fp16 rows (float16,
    or x_f16=True with int16 bit patterns)."""
    import torch
    M = M if M is not None else x.shape[0]
    xs = xs if xs is not None else x.stride(0) if x.dim() == 2 else K
    if y is None:
        y = torch.zeros((M, N), dtype=torch.bfloat16 if y_bf16 else torch.float32, device=x.device)
    ys = ys if ys is not None else (y.stride(0) if y.dim() == 2 else N)
    _dev(W, S, Z, x, y)
    rc = lib().qw_q4_gemv(_ptr(W), _ptr(S), _ptr(Z), _ptr(x), int(_is_f16(x, x_f16)), xs, _ptr(y), ys, int(y_bf16),
                          N, K, M, rpg, int(accumulate), _stream())
    _check(rc, "qw_q4_gemv")
    return y


def gemv_w16(W, x, M=None, y=None, y_bf16=False, accumulate=False, f16=None, xs=None, ys=None, rpg=0):
    """y[m][n] (+)= sum_k W[n][k] x[m][k] for 16-bit W [N][K] (row-major, stride W.stride(0)):
    fp16 W with fp16 x (f16 True, the default for float16 tensors) or bf16 with bf16."""
    import torch
    N, K = W.shape
    M = M if M is not None else x.shape[0]
    f16 = _is_f16(x, f16)
    xs = xs if xs is not None else x.stride(0) if x.dim() == 2 else K
    if y is None:
        y = torch.zeros((M, N), dtype=torch.bfloat16 if y_bf16 else torch.float32, device=x.device)
    ys = ys if ys is not None else (y.stride(0) if y.dim() == 2 else N)
    _dev(W, x, y)
    rc = lib().qw_w16_gemv(_ptr(W), W.stride(0), _ptr(x), xs, int(f16), _ptr(y), ys, int(y_bf16), N, K, M, rpg,
                           int(accumulate), _stream())
    _check(rc, "qw_w16_gemv")
    return y


def w16_tile(W):
    """16-bit W [N][K] (row-major, stride W.stride(0)) -> the tiled layout qw_w16_gemv_tiled
    reads (a flat tensor of W's dtype, rows padded to a multiple of 16)."""
    import torch
    N, K = W.shape
    Wt = torch.empty(lib().qw_w16_tiled_size(N, K) // 2, dtype=W.dtype, device=W.device)
    _dev(W)
    _check(lib().qw_w16_tile(_ptr(W), W.stride(0), N, K, _ptr(Wt), _stream()), "qw_w16_tile")
    return Wt


def gemv_w16_tiled(Wt, N, K, x, M=None, y=None, y_bf16=False, accumulate=False, f16=None, xs=None, ys=None, rpg=0):
    """gemv_w16 on the tiled layout (w16_tile) of a 16-bit [N][K] matrix."""
    import torch
    M = M if M is not None else x.shape[0]
    f16 = _is_f16(x, f16)
    xs = xs if xs is not None else x.stride(0) if x.dim() == 2 else K
    if y is None:
        y = torch.zeros((M, N), dtype=torch.bfloat16 if y_bf16 else torch.float32, device=x.device)
    ys = ys if ys is not None else (y.stride(0) if y.dim() == 2 else N)
    _dev(Wt, x, y)
    rc = lib().qw_w16_gemv_tiled(_ptr(Wt), _ptr(x), xs, int(f16), _ptr(y), ys, int(y_bf16), N, K, M, rpg,
                                 int(accumulate), _stream())
    _check(rc, "qw_w16_gemv_tiled")
    return y


def swiglu_gemv_w16_tiled(Wt, N, v, n, M=None, y=None, y_bf16=False, accumulate=False, ldv=None, ys=None):
    """y = W h with h = fp16(silu(v[:, :n]) v[:, n:2n] sigmoid(v[:, 2n])) (swiglu_gate followed by
    gemv_w16_tiled, in one launch); Wt: fp16 [N][n] tiled by w16_tile, v fp32 [M][>= 2n + 1]."""
    import torch
    M = M if M is not None else v.shape[0]
    ldv = ldv if ldv is not None else v.stride(0) if v.dim() == 2 else 2 * n + 1
    if y is None:
        y = torch.zeros((M, N), dtype=torch.bfloat16 if y_bf16 else torch.float32, device=v.device)
    ys = ys if ys is not None else (y.stride(0) if y.dim() == 2 else N)
    _dev(Wt, v, y)
    rc = lib().qw_w16_swiglu_gemv_tiled(_ptr(Wt), _ptr(v), ldv, n, _ptr(y), ys, int(y_bf16), N, M, int(accumulate),
                                        _stream())
    _check(rc, "qw_w16_swiglu_gemv_tiled")
    return y


def i8_tile(W8, scale, group=32):
    """int8 W8 [N][K] and fp32 scale [N][K/group] (row-major, as quantize_rows_i8 writes
    them) -> the kernel format (Wt uint8 bytes, St fp32) qw_i8_gemv reads."""
    import torch
    N, K = W8.shape
    wb, sb = ctypes.c_size_t(), ctypes.c_size_t()
    lib().qw_i8_tiled_size(N, K, group, ctypes.byref(wb), ctypes.byref(sb))
    Wt = torch.empty(wb.value, dtype=torch.uint8, device=W8.device)
    St = torch.empty(sb.value // 4, dtype=torch.float32, device=W8.device)
    _dev(W8, scale)
    _check(lib().qw_i8_tile(_ptr(W8), _ptr(scale), N, K, group, _ptr(Wt), _ptr(St), _stream()), "qw_i8_tile")
    return Wt, St


def gemv_i8(Wt, St, N, K, x, M=None, group=32, rpg=0, y=None, y_bf16=False, accumulate=False, xs=None, ys=None):
    """y[m][n] (+)= sum_g scale[n][g] sum_{k in g} W8[n][k] x[m][off(n) + k] (gpu::gemv_rows_i8) on
    the kernel format (i8_tile) of an int8 [N][K] matrix; fp16 rows x (row n reads slice
    n // rpg when rpg)."""
    import torch
    M = M if M is not None else x.shape[0]
    xs = xs if xs is not None else x.stride(0) if x.dim() == 2 else K
    if y is None:
        y = torch.zeros((M, N), dtype=torch.bfloat16 if y_bf16 else torch.float32, device=x.device)
    ys = ys if ys is not None else (y.stride(0) if y.dim() == 2 else N)
    _dev(Wt, St, x, y)
    rc = lib().qw_i8_gemv(_ptr(Wt), _ptr(St), group, _ptr(x), xs, _ptr(y), ys, int(y_bf16), N, K, M, rpg,
                          int(accumulate), _stream())
    _check(rc, "qw_i8_gemv")
    return y


def swiglu_gate(v, n, h=None):
    """h[t][j] = fp16(silu(v[t][j]) * v[t][n + j] * sigmoid(v[t][2n])); v fp32 [T][>= 2n + 1]."""
    import torch
    T = v.shape[0]
    if h is None:
        h = torch.empty((T, n), dtype=torch.float16, device=v.device)
    _dev(v, h)
    _check(lib().qw_swiglu_gate(_ptr(v), v.stride(0), n, T, _ptr(h), _stream()), "qw_swiglu_gate")
    return h


def gemm_workspace_size(T, K):
    return lib().qw_q4_gemm_workspace_size(T, K)


def gemm(W, S, Z, X, N, K, Y=None, y_bf16=False, workspace=None, x_f16=None, y_dtype=None):
    """Y[t][n] = sum_k X[t][k] deq(W)[n][k]; Y fp32, bf16 (y_bf16) or any of float32 / bfloat16 /
    float16 (y_dtype, or the dtype of a given Y; float16 is the reference's f16_out)."""
    import torch
    T = X.shape[0]
    f16 = _is_f16(X, x_f16)
    if Y is None:
        dt = y_dtype if y_dtype is not None else torch.bfloat16 if y_bf16 else torch.float32
        Y = torch.empty((T, N), dtype=dt, device=X.device)
    if workspace is None and not f16:
        workspace = torch.empty(gemm_workspace_size(T, K), dtype=torch.uint8, device=X.device)
    _dev(W, S, Z, X, Y, workspace)
    rc = lib().qw_q4_gemm(_ptr(W), _ptr(S), _ptr(Z), _ptr(X), int(f16), X.stride(0), T, _ptr(Y), Y.stride(0),
                          _tcode(Y), N, K, _ptr(workspace), 0 if workspace is None else workspace.numel(), _stream())
    _check(rc, "qw_q4_gemm")
    return Y


class Route:
    """Device outputs of qw_moe_route."""

    def __init__(self, T, E, topk, device, tile_m=0):
        import torch
        i32 = dict(dtype=torch.int32, device=device)
        self.T, self.E, self.topk, self.tile_m = T, E, topk, tile_m
        self.top_e = torch.empty((T, topk), **i32)
        self.top_w = torch.empty((T, topk), dtype=torch.float32, device=device)
        self.counts = torch.empty(E, **i32)
        self.offsets = torch.empty(E + 1, **i32)
        self.tok_slot = torch.empty((T, topk), **i32)
        self.pair_tok = torch.empty(T * topk, **i32)
        self.active = torch.empty(E, **i32)
        self.n_active = torch.empty(1, **i32)
        nt = (T * topk) // abs(tile_m) + E if tile_m else 0
        self.tile_e = torch.empty(max(nt, 1), **i32) if tile_m else None
        self.tile_m0 = torch.empty(max(nt, 1), **i32) if tile_m else None
        self.n_tiles = torch.empty(1, **i32) if tile_m else None


def moe_route(logits, topk, tile_m=0, out=None):
    T, E = logits.shape
    r = out if out is not None else Route(T, E, topk, logits.device, tile_m)
    _dev(logits)
    rc = lib().qw_moe_route(_ptr(logits), T, E, topk, tile_m, _ptr(r.top_e), _ptr(r.top_w), _ptr(r.counts),
                            _ptr(r.offsets), _ptr(r.tok_slot), _ptr(r.pair_tok), _ptr(r.active), _ptr(r.n_active),
                            _ptr(r.tile_e), _ptr(r.tile_m0), _ptr(r.n_tiles), _stream())
    _check(rc, "qw_moe_route")
    return r


def moe_experts_gemv(gate, up, down, route, x, E, F, h=None, yp=None, x_f16=None, yp_f16=False):
    """gate/up/down: tiled (Wt, St, Zt) of the stacked experts; returns (h fp16, yp fp32, or fp16
    with yp_f16 or an fp16 yp tensor)."""
    import torch
    H = x.shape[1]
    T, topk = route.T, route.topk
    if h is None:
        h = torch.empty((T * topk, F), dtype=torch.float16, device=x.device)
    if yp is None:
        yp = torch.empty((T * topk, H), dtype=torch.float16 if yp_f16 else torch.float32, device=x.device)
    _dev(x, h, yp, *gate, *up, *down)
    rc = lib().qw_moe_experts_gemv(*[_ptr(t) for t in (*gate, *up, *down)], E, H, F, _ptr(route.offsets),
                                   _ptr(route.active), _ptr(route.n_active), _ptr(route.pair_tok), _ptr(x),
                                   int(_is_f16(x, x_f16)), T, topk, _ptr(h), _ptr(yp),
                                   int(yp.dtype == torch.float16), _stream())
    _check(rc, "qw_moe_experts_gemv")
    return h, yp


def moe_grouped_tile_m():
    return lib().qw_moe_grouped_tile_m()


def moe_grouped_workspace_size(T, topk, E, H, F):
    return lib().qw_moe_grouped_workspace_size(T, topk, E, H, F)


def moe_experts_grouped(gate, up, down, route, x, E, F, h=None, yp=None, workspace=None, x_f16=None, yp_f16=False):
    """Grouped expert GEMMs; yp fp32, or fp16 (yp_f16, or an fp16 yp tensor)."""
    import torch
    T, H = x.shape
    topk = route.topk
    if h is None:
        h = torch.empty((T * topk, F), dtype=torch.float16, device=x.device)
    if yp is None:
        yp = torch.empty((T * topk, H), dtype=torch.float16 if yp_f16 else torch.float32, device=x.device)
    f16 = _is_f16(x, x_f16)
    if workspace is None and not f16:
        workspace = torch.empty(max(moe_grouped_workspace_size(T, topk, E, H, F), 1), dtype=torch.uint8,
                                device=x.device)
    _dev(x, h, yp, workspace, *gate, *up, *down)
    rc = lib().qw_moe_experts_grouped(*[_ptr(t) for t in (*gate, *up, *down)], E, H, F, _ptr(route.offsets),
                                      _ptr(route.pair_tok), _ptr(route.tile_e), _ptr(route.tile_m0),
                                      _ptr(route.n_tiles), _ptr(x), int(f16), T, topk, _ptr(h), _ptr(yp),
                                      int(yp.dtype == torch.float16), _ptr(workspace),
                                      0 if workspace is None else workspace.numel(), _stream())
    _check(rc, "qw_moe_experts_grouped")
    return h, yp


def moe_w4a8_tile_m():
    return lib().qw_moe_w4a8_tile_m()


def quant_rows_i8(x, x_f16=None):
    """16-bit rows [R][K] -> (int8 [R][K], fp32 scales [R][K/128]) (the W4A8 quantiser)."""
    import torch
    R, K = x.shape
    q = torch.empty((R, K), dtype=torch.int8, device=x.device)
    sc = torch.empty((R, K // 128), dtype=torch.float32, device=x.device)
    _dev(x)
    _check(lib().qw_quant_rows_i8(_ptr(x), int(_is_f16(x, x_f16)), R, K, x.stride(0), _ptr(q), _ptr(sc), _stream()),
           "qw_quant_rows_i8")
    return q, sc


def moe_experts_w4a8(gate, up, down, route, x, E, F, h=None, yp=None, workspace=None, x_f16=None):
    """The W4A8 grouped expert GEMMs (route made with tile_m = moe_w4a8_tile_m());
    returns (h fp16 [T*k][F], yp fp16 [T*k][H])."""
    import torch
    T, H = x.shape
    topk = route.topk
    if h is None:
        h = torch.empty((T * topk, F), dtype=torch.float16, device=x.device)
    if yp is None:
        yp = torch.empty((T * topk, H), dtype=torch.float16, device=x.device)
    if workspace is None:
        workspace = torch.empty(lib().qw_moe_w4a8_workspace_size(T, topk, H, F), dtype=torch.uint8, device=x.device)
    _dev(x, h, yp, workspace, *gate, *up, *down)
    rc = lib().qw_moe_experts_w4a8(*[_ptr(t) for t in (*gate, *up, *down)], E, H, F, _ptr(route.offsets),
                                   _ptr(route.pair_tok), _ptr(route.tile_e), _ptr(route.tile_m0), _ptr(route.n_tiles),
                                   _ptr(x), int(_is_f16(x, x_f16)), T, topk, _ptr(h), _ptr(yp), _ptr(workspace),
                                   workspace.numel(), _stream())
    _check(rc, "qw_moe_experts_w4a8")
    return h, yp


def moe_combine(yp, route, H, shared=None, out=None, out_bf16=True, out_dtype=None):
    """out = shared + sum_i w_i yp[slot_i]; yp and shared fp32 or float16 (by dtype), out bf16
    (out_bf16), fp32, or the dtype given (out_dtype, or that of a given out)."""
    import torch
    T, topk = route.T, route.topk
    if out is None:
        dt = out_dtype if out_dtype is not None else torch.bfloat16 if out_bf16 else torch.float32
        out = torch.empty((T, H), dtype=dt, device=yp.device)
    _dev(yp, shared, out)
    rc = lib().qw_moe_combine(_ptr(yp), int(yp.dtype == torch.float16), _ptr(route.tok_slot), _ptr(route.top_w),
                              _ptr(shared), int(shared is not None and shared.dtype == torch.float16), T, topk, H,
                              _ptr(out), _tcode(out), _stream())
    _check(rc, "qw_moe_combine")
    return out


def unpack(W, N, K):
    import torch
    out = torch.empty((N, K), dtype=torch.uint8, device=W.device)
    _check(lib().qw_q4_unpack(_ptr(W), N, K, _ptr(out), _stream()), "qw_q4_unpack")
    return out


def dequant(W, S, Z, N, K):
    import torch
    out = torch.empty((N, K), dtype=torch.float32, device=W.device)
    _check(lib().qw_q4_dequant(_ptr(W), _ptr(S), _ptr(Z), N, K, _ptr(out), _stream()), "qw_q4_dequant")
    return out


def from_engine_order(words):
    import torch
    out = torch.empty_like(words)
    _check(lib().qw_q4_from_engine_order(_ptr(words), _ptr(out), words.numel(), _stream()), "qw_q4_from_engine_order")
    return out


class MoeDecode:
    """Buffers of the fused decode block (qw_moe_decode) for T tokens."""

    def __init__(self, T, E, topk, H, F, device, yp_f16=False, Fs=0):
        """Fs > 0: also the shared expert's rows (sh_v [T][2 Fs + 1], sh_out [T][H], fp32) and the
        workspace of qw_moe_decode_with_shared."""
        import torch
        i32 = dict(dtype=torch.int32, device=device)
        self.T, self.E, self.topk, self.H, self.F, self.Fs = T, E, topk, H, F, Fs
        self.logits = torch.empty((T, E), dtype=torch.float32, device=device)
        self.top_e = torch.empty((T, topk), **i32)
        self.top_w = torch.empty((T, topk), dtype=torch.float32, device=device)
        self.tok_slot = torch.empty((T, topk), **i32)
        self.h = torch.empty((T * topk, F), dtype=torch.float16, device=device)
        self.yp = torch.empty((T * topk, H), dtype=torch.float16 if yp_f16 else torch.float32, device=device)
        # zero once: holds completion counters every call leaves at zero
        self.ws = torch.zeros(lib().qw_moe_decode_workspace_size(T, E, topk, H, F), dtype=torch.uint8, device=device)
        if Fs:
            self.sh_v = torch.empty((T, 2 * Fs + 1), dtype=torch.float32, device=device)
            self.sh_out = torch.empty((T, H), dtype=torch.float32, device=device)
            self.ws_sh = torch.zeros(lib().qw_moe_decode_with_shared_workspace_size(T, E, topk, H, F, Fs),
                                     dtype=torch.uint8, device=device)


def moe_decode(router_w, x, topk, gate, up, down, E, F, buf=None, shared=None, out=None, out_bf16=True, x_f16=None,
               out_dtype=None, yp_f16=False):
    """Router GEMV + routing + experts + combine for a decode batch (3 to 5 launches).
    router_w [E][H] float32, or float16 (the engine's router weights). out bf16 (out_bf16), fp32, or
    out_dtype / the dtype of a given out; yp fp32, or fp16 with yp_f16 (or a buf whose yp is float16)."""
    import torch
    T, H = x.shape
    buf = buf if buf is not None else MoeDecode(T, E, topk, H, F, x.device, yp_f16=yp_f16)
    if out is None:
        dt = out_dtype if out_dtype is not None else torch.bfloat16 if out_bf16 else torch.float32
        out = torch.empty((T, H), dtype=dt, device=x.device)
    _dev(router_w, x, shared, out, *gate, *up, *down)
    if router_w.dtype not in (torch.float32, torch.float16):
        raise TypeError(f"moe_decode: router_w must be float32 or float16, not {router_w.dtype}")
    rc = lib().qw_moe_decode(_ptr(router_w), int(router_w.dtype == torch.float16), _ptr(x), int(_is_f16(x, x_f16)), T, E, topk, *map(_ptr, gate), *map(_ptr, up), *map(_ptr, down),
                             H, F, _ptr(shared), _ptr(out), _tcode(out), _ptr(buf.logits), _ptr(buf.top_e),
                             _ptr(buf.top_w), _ptr(buf.tok_slot), _ptr(buf.h), _ptr(buf.yp),
                             int(buf.yp.dtype == torch.float16), _ptr(buf.ws), buf.ws.numel(), _stream())
    _check(rc, "qw_moe_decode")
    return out, buf


def moe_decode_with_shared(router_w, x, topk, gate, up, down, E, F, sh_gu, sh_down, Fs, buf=None, out=None,
                           out_bf16=True, x_f16=None, yp_f16=False):
    """moe_decode with the shared expert: sh_gu [2 Fs + 1][H] tiled 16-bit (w16_tile) of x's type,
    sh_down [H][Fs] tiled fp16. Returns (out, buf, sh_v, sh_out): the shared expert's gate/up/gate-logit
    rows and output rows (fp32) beside the block's output."""
    import torch
    T, H = x.shape
    buf = buf if buf is not None else MoeDecode(T, E, topk, H, F, x.device, yp_f16=yp_f16, Fs=Fs)
    if buf.Fs != Fs:
        raise ValueError(f"moe_decode_with_shared: buf was made for Fs = {buf.Fs}, not {Fs}")
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16 if out_bf16 else torch.float32, device=x.device)
    if router_w.dtype not in (torch.float32, torch.float16):
        raise TypeError(f"moe_decode_with_shared: router_w must be float32 or float16, not {router_w.dtype}")
    sh_v, sh_out, ws = buf.sh_v, buf.sh_out, buf.ws_sh
    _dev(router_w, x, out, sh_gu, sh_down, *gate, *up, *down)
    rc = lib().qw_moe_decode_with_shared(
        _ptr(router_w), int(router_w.dtype == torch.float16), _ptr(x), int(_is_f16(x, x_f16)), T, E, topk,
        *map(_ptr, gate), *map(_ptr, up), *map(_ptr, down), H, F, _ptr(sh_gu), _ptr(sh_down), Fs, _ptr(sh_v),
        _ptr(sh_out), _ptr(out), _tcode(out), _ptr(buf.logits), _ptr(buf.top_e), _ptr(buf.top_w), _ptr(buf.tok_slot),
        _ptr(buf.h), _ptr(buf.yp), int(buf.yp.dtype == torch.float16), _ptr(ws), ws.numel(), _stream())
    _check(rc, "qw_moe_decode_with_shared")
    return out, buf, sh_v, sh_out


# -------------------------------------------------------- checkpoint loading
def bf16_to_f16(x, out=None):
    """bf16 bits (int16/uint16 or bfloat16 tensor) -> fp16 bits, saturating as
    the reference converts scales at load."""
    import torch
    out = out if out is not None else torch.empty(x.shape, dtype=torch.int16, device=x.device)
    _dev(x, out)
    _check(lib().qw_bf16_to_f16(_ptr(x), _ptr(out), x.numel(), _stream()), "qw_bf16_to_f16")
    return out


def read_probe(t=None):
    """Measurement aid: read tensor t's bytes (a multiple of 32768) with the
    dense GEMV's load shape and nothing else; t=None launches one empty block."""
    if t is None:
        _check(lib().qw_read_probe(None, 0, _stream()), "qw_read_probe")
        return
    _dev(t)
    _check(lib().qw_read_probe(_ptr(t), t.numel() * t.element_size(), _stream()), "qw_read_probe")


class StFile:
    """A safetensors file mapped by the library (host side)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        _check(lib().qw_st_open(os.fsencode(path), ctypes.byref(h)), "qw_st_open")
        self._h = h

    def close(self):
        if self._h:
            lib().qw_st_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def names(self):
        return [lib().qw_st_name(self._h, i).decode() for i in range(lib().qw_st_count(self._h))]

    def info(self, name):
        """(dtype, shape, nbytes) of one tensor."""
        dt = ctypes.create_string_buffer(16)
        shape = (ctypes.c_int64 * 8)()
        nd, nb, data = ctypes.c_int(), ctypes.c_size_t(), ctypes.c_void_p()
        _check(lib().qw_st_tensor(self._h, name.encode(), dt, shape, ctypes.byref(nd), ctypes.byref(data),
                                  ctypes.byref(nb)), "qw_st_tensor")
        return dt.value.decode(), tuple(shape[i] for i in range(nd.value)), nb.value


def tiled_offset(row0, K):
    a, b, c = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    lib().qw_q4_tiled_offset(row0, K, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    return a.value, b.value, c.value


def load_q4(st, prefix, N, K, out=None, row0=0, device=None, cache=None):
    """Loads "<prefix>.weight_packed/.weight_scale" of an StFile into tiled
    device tensors (Wt, St, None). With out=(Wt, St, Zt) of a larger tiled
    matrix, writes rows row0 .. row0 + N - 1 of it (stacked experts).
    With a WCache: replaying, the rows come from the cache (st may be None);
    recording, they are converted and appended to it."""
    import torch
    device = device or torch.device("cuda", torch.cuda.current_device())
    if out is None:
        wb, sb, _ = tiled_size(N, K)
        out = (torch.empty(wb // 4, dtype=torch.int32, device=device),
               torch.empty(sb // 2, dtype=torch.int16, device=device), None)
    Wt, St_ = out[0], out[1]
    _dev(Wt, St_)
    ow, os_, _ = tiled_offset(row0, K)
    nw, ns, _ = tiled_size(N, K)
    if ow + nw > Wt.numel() * Wt.element_size() or os_ + ns > St_.numel() * St_.element_size():
        raise ValueError("load_q4: rows beyond the output tensors")
    wp, sp = Wt.data_ptr() + ow, St_.data_ptr() + os_
    if cache is not None and cache.mode == "replay":
        cache.get_ptr(wp, nw)
        cache.get_ptr(sp, ns)
        return out
    staging = torch.empty(lib().qw_q4_load_staging_size(N, K), dtype=torch.uint8, device=Wt.device)
    rc = lib().qw_q4_load(st._h, prefix.encode(), N, K, ctypes.c_void_p(wp), ctypes.c_void_p(sp), _ptr(staging),
                          staging.numel(), _stream())
    _check(rc, "qw_q4_load")
    torch.cuda.current_stream().synchronize()  # staging is freed on return
    if cache is not None:
        cache.put_ptr(wp, nw)
        cache.put_ptr(sp, ns)
    return out


def checkpoint_key(paths, options=""):
    """A 64-bit cache key for a checkpoint: names, sizes and modification
    times of its files plus the caller's conversion options."""
    import hashlib
    h = hashlib.blake2b(digest_size=8)
    for p in sorted(os.fspath(x) for x in paths):
        st = os.stat(p)
        h.update(f"{os.path.basename(p)}\0{st.st_size}\0{st.st_mtime_ns}\0".encode())
    h.update(options.encode())
    return int.from_bytes(h.digest(), "little")


class WCache:
    """Converted-weights cache file (qw_wcache_*). mode is "replay" when the
    file is a complete cache for `key`, "record" while writing it (completed
    by finish()), or "off" (reason in `why`)."""

    _MODES = {0: "off", 1: "record", 2: "replay"}

    def __init__(self, path, key):
        h, m = ctypes.c_void_p(), ctypes.c_int()
        _check(lib().qw_wcache_open(os.fsencode(path), ctypes.c_uint64(key), ctypes.byref(h), ctypes.byref(m)),
               "qw_wcache_open")
        self._h, self.mode = h, self._MODES[m.value]
        self.why = lib().qw_q4_last_error().decode() if self.mode == "off" else ""

    def put_ptr(self, ptr, nbytes, on_device=True):
        _check(lib().qw_wcache_put(self._h, ctypes.c_void_p(ptr), nbytes, int(on_device),
                                   _stream() if on_device else None), "qw_wcache_put")

    def get_ptr(self, ptr, nbytes, on_device=True):
        _check(lib().qw_wcache_get(self._h, ctypes.c_void_p(ptr), nbytes, int(on_device),
                                   _stream() if on_device else None), "qw_wcache_get")

    def put(self, t):
        """Appends a contiguous tensor (device or host) while recording."""
        if not t.is_contiguous():
            raise ValueError("WCache.put: tensor must be contiguous")
        self.put_ptr(t.data_ptr(), t.numel() * t.element_size(), t.is_cuda)

    def get(self, t):
        """Fills a contiguous tensor (device or host) with the next piece."""
        if not t.is_contiguous():
            raise ValueError("WCache.get: tensor must be contiguous")
        self.get_ptr(t.data_ptr(), t.numel() * t.element_size(), t.is_cuda)

    def finish(self):
        _check(lib().qw_wcache_finish(self._h), "qw_wcache_finish")
        if self.mode == "record":
            self.mode = "off"

    def close(self):
        if self._h:
            lib().qw_wcache_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
