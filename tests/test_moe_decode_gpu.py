"""Fused MoE decode block (qw_moe_decode): fp32 router GEMV, routing, gathered
experts and the combine folded into the down projection, against the oracle.

Routing is checked on the block's own logits (the oracle routes the same
fp32 values, so the selection must match bit for bit); the logits themselves
against an fp64 product; the output against the oracle's MoE on those logits.
"""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, bf16_err_ok, host, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _case(gpu, seed, T, E, H, F, k, with_shared, zeros=True):
    ex = synth.experts(seed, E, H, F, zeros=zeros)
    xb, xf = synth.acts(seed, "dx", T, H)
    r = np.random.default_rng(seed)
    Wr = (r.standard_normal((E, H)) * 0.05).astype(np.float32)
    shared = r.standard_normal((T, H)).astype(np.float32) if with_shared else None
    from test_moe_gpu import _experts_dev
    (g, u, d), _, _ = _experts_dev(gpu, ex)
    return ex, xb, xf, Wr, shared, (g, u, d)


@pytest.mark.parametrize("T,E,H,F,k,shared,bf16", [(1, 64, 1024, 256, 4, False, False), (5, 64, 1024, 256, 4, True, False),
                                                   (32, 32, 512, 384, 6, True, True), (8, 256, 4096, 1536, 8, True, True),
                                                   (3, 64, 1024, 512, 4, False, False),
                                                   (16, 64, 2048, 1536, 6, True, True),
                                                   # config 3's full size at batches 1, 2 (combine folded
                                                   # into the down projection), 4, 16 and 32 (separate combine)
                                                   (1, 256, 4096, 1536, 8, True, True),
                                                   (2, 256, 4096, 1536, 8, True, False),
                                                   (4, 256, 4096, 1536, 8, False, False),
                                                   (16, 256, 4096, 1536, 8, True, True),
                                                   (32, 256, 4096, 1536, 8, True, True),
                                                   # the MFMA router (9-32 tokens): experts not a multiple
                                                   # of 16, 16 K slices (H 8192), one slice (H 512) with a
                                                   # partial second token tile, 1024 experts
                                                   (9, 40, 8192, 256, 4, True, False),
                                                   (17, 48, 512, 128, 8, False, False),
                                                   (24, 1024, 1024, 128, 8, True, False)])
def test_moe_decode_matches_oracle(gpu, oracle, T, E, H, F, k, shared, bf16):
    print(f"moe_decode T={T} E={E} H={H} F={F} k={k}", flush=True)
    ex, xb, xf, Wr, sh, (g, u, d) = _case(gpu, 40 + T, T, E, H, F, k, shared)
    buf = qwq4.MoeDecode(T, E, k, H, F, gpu)
    outs = []
    for _ in range(3):   # repeated calls: counters left at zero, identical results
        out, _ = qwq4.moe_decode(to_dev(Wr, gpu), to_dev(xb, gpu), k, g, u, d, E, F, buf=buf,
                                 shared=to_dev(sh, gpu), out_bf16=bf16)
        outs.append(host(out))
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    logits = host(buf.logits)
    ref_l = xf.astype(np.float64) @ Wr.astype(np.float64).T
    assert rel_err(logits, ref_l) <= 1e-5
    te, tw = oracle.route(logits, k)
    assert np.array_equal(host(buf.top_e), te)
    assert np.array_equal(host(buf.top_w).view(np.uint32), tw.view(np.uint32))
    ref = oracle.moe(xf, logits, k, *ex)
    if sh is not None:
        ref = ref + sh
    if bf16:
        assert bf16_err_ok(outs[0], ref)
    else:
        assert rel_err(outs[0], ref) <= TOL


@pytest.mark.parametrize("T,E,H,F,k", [(1, 64, 1024, 256, 4), (2, 64, 1024, 256, 4), (2, 16, 1024, 256, 8),
                                       (1, 4, 1024, 256, 2), (2, 4, 1024, 256, 3), (2, 8, 1024, 256, 8),
                                       (3, 64, 1024, 512, 4), (4, 64, 1024, 256, 4),
                                       (6, 64, 1024, 256, 4), (6, 64, 1024, 512, 4), (1, 256, 4096, 1536, 8),
                                       (2, 256, 4096, 1536, 8), (4, 256, 4096, 1536, 8), (16, 256, 4096, 1536, 8),
                                       (1, 64, 2048, 512, 6), (1, 32, 4096, 2048, 8), (1, 512, 2048, 256, 8)])
@pytest.mark.parametrize("yp16", [False, True])
def test_moe_decode_matches_unfused_path(gpu, T, E, H, F, k, yp16):
    """The block against routing + experts + combine as separate calls, with
    fp32 and fp16 yp (the combine then adds the fp16 values): yp and out
    bit-identical, on both sides of the switch that folds the combine into
    the down projection (up to 2 tokens; batch 1 in one block per 16 output
    rows), with experts chosen by both tokens (E = 16, k = 8; E = 8, k = 8:
    every expert twice), fewer experts than the kernels' waves (E = 4), and at
    config 3's full size (down projection with 6 groups per wave), and batch 1
    at H 2048 / 4096 with down K halves of 2 to 8 groups and E up to 512 (the
    gate/up blocks' own routing over 1 to 8 logits per lane)."""
    print(f"moe_decode vs unfused T={T} E={E} H={H} F={F} yp16={yp16}", flush=True)
    ex, xb, xf, Wr, sh, (g, u, d) = _case(gpu, 77 + T, T, E, H, F, k, True)
    out, buf = qwq4.moe_decode(to_dev(Wr, gpu), to_dev(xb, gpu), k, g, u, d, E, F, shared=to_dev(sh, gpu),
                               out_bf16=False, yp_f16=yp16)
    r = qwq4.moe_route(buf.logits, k)
    h, yp = qwq4.moe_experts_gemv(g, u, d, r, to_dev(xb, gpu), E, F, yp_f16=yp16)
    o2 = qwq4.moe_combine(yp, r, H, shared=to_dev(sh, gpu), out_bf16=False)
    assert np.array_equal(host(r.top_e), host(buf.top_e))
    assert np.array_equal(host(yp).view(np.uint8), host(buf.yp).view(np.uint8))
    assert np.array_equal(host(out).view(np.uint32), host(o2).view(np.uint32))


@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_moe_decode_f16_out(gpu, T):
    """fp16 output rows (QW_T_F16): the fp32 output of the same call rounded
    to nearest even, bit for bit, with the combine folded into the down
    projection (T <= 2) and as its own launch (T = 4, 8)."""
    import torch
    E, H, F, k = 64, 1024, 256, 4
    ex, xb, xf, Wr, sh, (g, u, d) = _case(gpu, 130 + T, T, E, H, F, k, True)
    o32, _ = qwq4.moe_decode(to_dev(Wr, gpu), to_dev(xb, gpu), k, g, u, d, E, F, shared=to_dev(sh, gpu),
                             out_bf16=False, yp_f16=True)
    o16, _ = qwq4.moe_decode(to_dev(Wr, gpu), to_dev(xb, gpu), k, g, u, d, E, F, shared=to_dev(sh, gpu),
                             out_dtype=torch.float16, yp_f16=True)
    want = np.clip(host(o32), -65504, 65504).astype(np.float16)
    assert np.array_equal(host(o16).view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_moe_decode_symmetric_experts(gpu, oracle, T):
    """Symmetric experts (no zero points: zero 8 for every group, the
    reference's format, ref_model.cpp:114) through the fused block at config
    3's full size: against the oracle, and bit for bit against the unfused
    calls (the batch-1 routed gate/up and the batch-1 / batch-2 down kernels
    without zeros)."""
    E, H, F, k = 256, 4096, 1536, 8
    print(f"moe_decode symmetric T={T}", flush=True)
    ex, xb, xf, Wr, sh, (g, u, d) = _case(gpu, 170 + T, T, E, H, F, k, True, zeros=False)
    assert g[2] is None and d[2] is None
    out, buf = qwq4.moe_decode(to_dev(Wr, gpu), to_dev(xb, gpu), k, g, u, d, E, F, shared=to_dev(sh, gpu),
                               out_bf16=False, yp_f16=True)
    r = qwq4.moe_route(buf.logits, k)
    h, yp = qwq4.moe_experts_gemv(g, u, d, r, to_dev(xb, gpu), E, F, yp_f16=True)
    o2 = qwq4.moe_combine(yp, r, H, shared=to_dev(sh, gpu), out_bf16=False)
    assert np.array_equal(host(out).view(np.uint32), host(o2).view(np.uint32))
    ref = oracle.moe(xf, host(buf.logits), k, *ex) + sh
    assert rel_err(host(out), ref) <= TOL


@pytest.mark.parametrize("T,k", [(1, 6), (4, 6), (16, 6), (1, 10)])
def test_moe_decode_fp16_router(gpu, T, k):
    """The engine's fp16 router weights (router_f16 = 1, decode.hip:101's w.router)
    against fp32 weights holding the same values: logits, routing and output bit
    for bit, through every router path: the logits launch (batch 1, routed in the
    gate/up blocks; batch 4, then a routing launch), the K-sliced router with the
    routing in its last block (batch 16), and the full-K router with the routing in
    its last block (batch 1 with k > 8)."""
    import torch
    E, H, F = 64, 2048, 256
    print(f"moe_decode fp16 router T={T} k={k}", flush=True)
    ex, xb, xf, Wr, sh, (g, u, d) = _case(gpu, 150 + T, T, E, H, F, k, True)
    w16 = to_dev(Wr.astype(np.float16), gpu)
    w32 = w16.float()
    o16, b16 = qwq4.moe_decode(w16, to_dev(xb, gpu), k, g, u, d, E, F, shared=to_dev(sh, gpu), out_bf16=False)
    o32, b32 = qwq4.moe_decode(w32, to_dev(xb, gpu), k, g, u, d, E, F, shared=to_dev(sh, gpu), out_bf16=False)
    assert np.array_equal(host(b16.logits).view(np.uint32), host(b32.logits).view(np.uint32))
    assert np.array_equal(host(b16.top_e), host(b32.top_e))
    assert np.array_equal(host(o16).view(np.uint32), host(o32).view(np.uint32))
    with pytest.raises(TypeError):
        qwq4.moe_decode(w32.to(torch.bfloat16), to_dev(xb, gpu), k, g, u, d, E, F)


@pytest.mark.parametrize("T,E", [(6, 64), (8, 64), (8, 256)])
def test_moe_decode_router_lds_limit(gpu, oracle, T, E):
    """H = 8192: the full-K router kernels stage the token rows (T x 16 KB) in
    LDS (the routing variant beside its static arrays). T = 6 and 8 at E = 64
    fit the CU's 160 KiB (the second within 2 KB) and take the logits launch
    then the routing launch; T = 8 at E = 256 does not fit and takes the
    K-sliced router. Logits against the fp64 product, routing bit-exact with
    the oracle, output bit-identical to the unfused calls."""
    H, F, k = 8192, 128, 8
    print(f"moe_decode router LDS T={T} E={E} H={H}", flush=True)
    ex, xb, xf, Wr, sh, (g, u, d) = _case(gpu, 95 + T + E, T, E, H, F, k, True)
    out, buf = qwq4.moe_decode(to_dev(Wr, gpu), to_dev(xb, gpu), k, g, u, d, E, F, shared=to_dev(sh, gpu),
                               out_bf16=False)
    logits = host(buf.logits)
    assert rel_err(logits, xf.astype(np.float64) @ Wr.astype(np.float64).T) <= 1e-5
    te, tw = oracle.route(logits, k)
    assert np.array_equal(host(buf.top_e), te)
    assert np.array_equal(host(buf.top_w).view(np.uint32), tw.view(np.uint32))
    r = qwq4.moe_route(buf.logits, k)
    h, yp = qwq4.moe_experts_gemv(g, u, d, r, to_dev(xb, gpu), E, F)
    o2 = qwq4.moe_combine(yp, r, H, shared=to_dev(sh, gpu), out_bf16=False)
    assert np.array_equal(host(out).view(np.uint32), host(o2).view(np.uint32))


def _random_moe(n, seed):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = 8 * int(r.integers(2, 33))
        out.append((int(r.integers(1, 3)), E, 1024 * int(r.integers(1, 5)), 128 * int(r.integers(1, 17)),
                    int(r.integers(1, min(E, 10) + 1))))
    return out


@pytest.mark.parametrize("T,E,H,F,k", _random_moe(10, 2033))
def test_moe_decode_random_small_batches(gpu, T, E, H, F, k):
    """Seeded random shapes at batches 1 and 2 (E 16-256, H 1024-4096, F
    128-2048, k 1-10): the fused block (one-block-per-row-range down kernels
    where they apply, the folded combine elsewhere) against the unfused calls,
    bit for bit."""
    print(f"moe_decode random T={T} E={E} H={H} F={F} k={k}", flush=True)
    ex, xb, xf, Wr, sh, (g, u, d) = _case(gpu, 300 + T + E + F, T, E, H, F, k, True)
    out, buf = qwq4.moe_decode(to_dev(Wr, gpu), to_dev(xb, gpu), k, g, u, d, E, F, shared=to_dev(sh, gpu),
                               out_bf16=False)
    r = qwq4.moe_route(buf.logits, k)
    h, yp = qwq4.moe_experts_gemv(g, u, d, r, to_dev(xb, gpu), E, F)
    o2 = qwq4.moe_combine(yp, r, H, shared=to_dev(sh, gpu), out_bf16=False)
    assert np.array_equal(host(yp), host(buf.yp))
    assert np.array_equal(host(out).view(np.uint32), host(o2).view(np.uint32))
