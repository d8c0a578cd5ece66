"""qw_moe_decode_static (the entry point that allocates nothing: library-held
scratch per GPU) against qw_moe_decode with a caller workspace, through the
C-ABI: two calls in a row, the second with fewer tokens (the scratch keeps
the first call's contents), outputs bit for bit equal."""
import ctypes

import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import host, to_dev

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _static_call(L, Wr, x, T, E, k, g, u, d, H, F, shared, outs):
    out, logits, top_e, top_w, tok_slot, h, yp = outs
    import torch
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return L.qw_moe_decode_static(_ptr(Wr), 0, _ptr(x), 0, T, E, k, *map(_ptr, g), *map(_ptr, u), *map(_ptr, d), H, F,
                                  _ptr(shared), _ptr(out), 0, _ptr(logits), _ptr(top_e), _ptr(top_w), _ptr(tok_slot),
                                  _ptr(h), _ptr(yp), int(yp.dtype == torch.float16), s)


@pytest.mark.parametrize("E,H,F,k,Ts,yp16", [(64, 1024, 256, 4, (8, 3), False), (256, 4096, 1536, 8, (4, 1), False),
                                             (256, 4096, 1536, 8, (2, 1), True)])
def test_static_matches_workspace_entry(gpu, E, H, F, k, Ts, yp16):
    import torch
    L = qwq4.lib()
    assert L.qw_moe_decode_static_max_bytes() == 4 << 20
    ex = synth.experts(71, E, H, F)
    from test_moe_gpu import _experts_dev
    (g, u, d), _, _ = _experts_dev(gpu, ex)
    Wr = to_dev((np.random.default_rng(71).standard_normal((E, H)) * 0.05).astype(np.float32), gpu)
    for T in Ts:   # the second call has fewer tokens
        print(f"moe_decode_static E={E} H={H} T={T}", flush=True)
        xb, _ = synth.acts(72 + T, "sx", T, H)
        x = to_dev(xb, gpu)
        shared = to_dev(np.random.default_rng(T).standard_normal((T, H)).astype(np.float32), gpu)
        want, buf = qwq4.moe_decode(Wr, x, k, g, u, d, E, F, shared=shared, out_bf16=False, yp_f16=yp16)
        outs = (torch.empty((T, H), dtype=torch.float32, device=gpu), torch.empty((T, E), dtype=torch.float32, device=gpu),
                torch.empty((T, k), dtype=torch.int32, device=gpu), torch.empty((T, k), dtype=torch.float32, device=gpu),
                torch.empty((T, k), dtype=torch.int32, device=gpu),
                torch.empty((T * k, F), dtype=torch.float16, device=gpu),
                torch.empty((T * k, H), dtype=torch.float16 if yp16 else torch.float32, device=gpu))
        rc = _static_call(L, Wr, x, T, E, k, g, u, d, H, F, shared, outs)
        assert rc == 0, L.qw_q4_last_error().decode()
        torch.cuda.synchronize()
        assert np.array_equal(host(outs[0]).view(np.uint32), host(want).view(np.uint32))
        assert np.array_equal(host(outs[2]), host(buf.top_e))
        assert np.array_equal(host(outs[3]).view(np.uint32), host(buf.top_w).view(np.uint32))
        assert np.array_equal(host(outs[6]).view(np.uint8), host(buf.yp).view(np.uint8))


def test_static_rejects_unsupported_shapes(gpu):
    """Shapes outside the decode limits are refused before anything is
    launched, with a message. (Every accepted shape fits the library's
    array, so no accepted shape is refused for its scratch.)"""
    L = qwq4.lib()
    p = ctypes.c_void_p(1 << 20)
    rc = L.qw_moe_decode_static(p, 0, p, 0, 33, 256, 8, *([p] * 9), 4096, 1536, None, p, 0, *([p] * 6), 0, None)
    assert rc == -1 and b"outside 1..32" in L.qw_q4_last_error()
    rc = L.qw_moe_decode_static(p, 0, p, 0, 32, 1024, 8, *([p] * 9), 65536, 1536, None, p, 0, *([p] * 6), 0, None)
    assert rc == -1 and b"too large" in L.qw_q4_last_error()


def test_static_reset_then_call(gpu):
    """qw_moe_decode_static_reset clears the counters (one kernel, no
    allocation); a call after it still matches the workspace entry point."""
    import torch
    L = qwq4.lib()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.qw_moe_decode_static_reset(s) == 0, L.qw_q4_last_error().decode()
    test_static_matches_workspace_entry(gpu, 64, 1024, 256, 4, (2,), False)
