"""Helpers of the GPU parity tests."""
import numpy as np

# fp outputs: max|y - r| / max|r| against the fp32 oracle (BASELINE tolerance)
TOL = 2e-3
# bf16 outputs add their own rounding: at most half an ulp, 2^-8 of |r|
BF16_HALF_ULP = 2.0**-8


def to_dev(a, dev):
    import torch
    if a is None:
        return None
    a = np.ascontiguousarray(a)
    view = {np.dtype(np.uint32): np.int32, np.dtype(np.uint16): np.int16}.get(a.dtype)
    t = torch.from_numpy(a.view(view) if view else a)
    return t.to(dev)


def host(t, dtype=None):
    a = t.detach().cpu()
    import torch
    if a.dtype == torch.bfloat16:
        return (a.view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    a = a.numpy()
    return a.view(dtype) if dtype is not None else a


def rel_err(y, r):
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - r)) / max(np.max(np.abs(r)), 1e-30))


def bf16_err_ok(y, r):
    """|y - r| <= TOL * max|r| + half an ulp of bf16 at |r|."""
    r = np.asarray(r, np.float64)
    bound = TOL * np.max(np.abs(r)) + BF16_HALF_ULP * np.abs(r)
    return bool(np.all(np.abs(np.asarray(y, np.float64) - r) <= bound))
