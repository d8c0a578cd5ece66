"""HIP-graph capture of a decode layer's q4 calls (the reference records its
whole decode step into a graph, src/engine/decode.hip:166-181).

One decode layer: QKV projection, routing, gathered experts, combine and the
down projection, the fused MoE block (router GEMV, routing, experts and the
combine, whose cross-block counters must be left at zero by every call) at
batches 4 and 1, the shared expert on tiled fp16 weights (SwiGLU x gate folded
into the down GEMV, and as two launches), the fused block with the shared
expert merged into its launches at batches 4 and 1, plus a prefill GEMM, captured once and replayed several times with the program's own eager work and synchronisations in between.
Every replay must reproduce the eager results bit for bit (all kernels are
deterministic), and the eager results must match the oracle.
"""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, bf16_err_ok, host, rel_err, to_dev

pytestmark = pytest.mark.gpu


def test_decode_layer_graph_replays(gpu, oracle):
    import torch
    M, H, QKV, E, F, k = 4, 1024, 1536, 32, 256, 4
    print(f"graph decode layer M={M} H={H} E={E} F={F} k={k}", flush=True)
    Wq = synth.q4_weights(71, "gq", QKV, H)
    Wd = synth.q4_weights(71, "gd", H, F * 2)
    ex = synth.experts(71, E, H, F)
    xb, xf = synth.acts(71, "gx", M, H)
    hb, hf = synth.acts(71, "gh", M, F * 2)
    l = synth.router_logits(71, "gl", M, E)
    T = 256
    Xb, Xf = synth.acts(71, "gX", T, H)

    dq = qwq4.tile(*(to_dev(a, gpu) for a in Wq), QKV, H)
    dd = qwq4.tile(*(to_dev(a, gpu) for a in Wd), H, F * 2)
    from test_moe_gpu import _experts_dev
    (eg, eu, ed), _, _ = _experts_dev(gpu, ex)
    x, h2, logits, X = to_dev(xb, gpu), to_dev(hb, gpu), to_dev(l, gpu), to_dev(Xb, gpu)

    # preallocated outputs: nothing is allocated inside the capture
    yq = torch.empty((M, QKV), dtype=torch.bfloat16, device=gpu)
    yd = torch.empty((M, H), dtype=torch.float32, device=gpu)
    r = qwq4.Route(M, E, k, gpu)
    h = torch.empty((M * k, F), dtype=torch.float16, device=gpu)
    yp = torch.empty((M * k, H), dtype=torch.float32, device=gpu)
    out = torch.empty((M, H), dtype=torch.float32, device=gpu)
    Y = torch.empty((T, QKV), dtype=torch.float32, device=gpu)
    ws = torch.empty(qwq4.gemm_workspace_size(T, H), dtype=torch.uint8, device=gpu)
    Wr = (np.random.default_rng(71).standard_normal((E, H)) * 0.05).astype(np.float32)
    router_w = to_dev(Wr, gpu)
    mdb = qwq4.MoeDecode(M, E, k, H, F, gpu)
    mout = torch.empty((M, H), dtype=torch.bfloat16, device=gpu)
    # batch 1 of the fused block (down projection and combine in one kernel)
    x1 = x[:1].contiguous()
    mdb1 = qwq4.MoeDecode(1, E, k, H, F, gpu)
    mout1 = torch.empty((1, H), dtype=torch.float32, device=gpu)
    # the shared expert on fp16 weights tiled at load: gate/up/gate-logit GEMV,
    # then the SwiGLU x gate folded into the down GEMV, and as two launches
    SF = 256
    gu16 = (torch.randn((2 * SF + 1, H), generator=torch.Generator(device=gpu).manual_seed(72), device=gpu) * 0.05).half()
    dn16 = (torch.randn((H, SF), generator=torch.Generator(device=gpu).manual_seed(73), device=gpu) * 0.05).half()
    gu16t, dn16t = qwq4.w16_tile(gu16), qwq4.w16_tile(dn16)
    xh = to_dev(xf.astype(np.float16), gpu)  # x's values as fp16 rows (x holds bf16 bits)
    v = torch.empty((M, 2 * SF + 1), dtype=torch.float32, device=gpu)
    hs16 = torch.empty((M, SF), dtype=torch.float16, device=gpu)
    sh = torch.empty((M, H), dtype=torch.float32, device=gpu)
    sh3 = torch.empty((M, H), dtype=torch.float32, device=gpu)
    # the fused block with the shared expert (its GEMVs inside the block's
    # router, routing and gate/up launches) at batches 4 and 1, fp16 rows
    msb, msb1 = qwq4.MoeDecode(M, E, k, H, F, gpu, Fs=SF), qwq4.MoeDecode(1, E, k, H, F, gpu, Fs=SF)
    msout = torch.empty((M, H), dtype=torch.float32, device=gpu)
    msout1 = torch.empty((1, H), dtype=torch.float32, device=gpu)
    xh1 = xh[:1].contiguous()

    def layer():
        qwq4.gemv(*dq, x, QKV, H, M, y=yq, y_bf16=True)
        qwq4.moe_route(logits, k, out=r)
        qwq4.moe_experts_gemv(eg, eu, ed, r, x, E, F, h=h, yp=yp)
        qwq4.moe_combine(yp, r, H, out=out, out_bf16=False)
        qwq4.gemv(*dd, h2, H, F * 2, M, y=yd)
        qwq4.gemm(*dq, X, QKV, H, Y=Y, workspace=ws)
        qwq4.moe_decode(router_w, x, k, eg, eu, ed, E, F, buf=mdb, out=mout)
        qwq4.moe_decode(router_w, x1, k, eg, eu, ed, E, F, buf=mdb1, out=mout1, out_bf16=False)
        qwq4.gemv_w16_tiled(gu16t, 2 * SF + 1, H, xh, M, y=v)
        qwq4.swiglu_gemv_w16_tiled(dn16t, H, v, SF, M, y=sh)
        qwq4.swiglu_gate(v, SF, h=hs16)
        qwq4.gemv_w16_tiled(dn16t, H, SF, hs16, M, y=sh3)
        qwq4.moe_decode_with_shared(router_w, xh, k, eg, eu, ed, E, F, gu16t, dn16t, SF, buf=msb, out=msout,
                                    out_bf16=False)
        qwq4.moe_decode_with_shared(router_w, xh1, k, eg, eu, ed, E, F, gu16t, dn16t, SF, buf=msb1, out=msout1,
                                    out_bf16=False)

    outs = (yq, yd, out, Y, r.top_e, r.pair_tok, h, mout, mdb.logits, mdb.top_e, mout1, mdb1.top_e, v, hs16, sh, sh3,
            msout, msb.sh_out, msb.top_e, msout1, msb1.sh_out, msb1.top_e)
    layer()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]

    # eager results against the oracle
    assert bf16_err_ok(host(yq), oracle.q4_linear(*Wq, QKV, H, xf))
    assert rel_err(host(yd), oracle.q4_linear(*Wd, H, F * 2, hf)) <= TOL
    assert rel_err(host(out), oracle.moe(xf, l, k, *ex)) <= TOL
    assert rel_err(host(Y), oracle.q4_linear(*Wq, QKV, H, Xf)) <= TOL
    ml = host(mdb.logits)
    assert bf16_err_ok(host(mout), oracle.moe(xf, ml, k, *ex))
    assert rel_err(host(mout1), oracle.moe(xf[:1], host(mdb1.logits), k, *ex)) <= TOL
    assert torch.equal(sh.view(torch.uint8), sh3.view(torch.uint8))
    hsb = host(hs16.view(torch.int16)).view(np.uint16)
    assert rel_err(host(sh), oracle.linear_w16(host(dn16.view(torch.int16)).view(np.uint16),
                                               hsb.view(np.float16).astype(np.float32), True)) <= TOL

    xhf = xf.astype(np.float16).astype(np.float32)
    assert torch.equal(msb.sh_out.view(torch.uint8), sh.view(torch.uint8))
    assert rel_err(host(msout), oracle.moe(xhf, host(msb.logits), k, *ex) + host(sh)) <= TOL
    assert rel_err(host(msb1.sh_out), host(sh)[:1]) <= TOL
    assert rel_err(host(msout1), oracle.moe(xhf[:1], host(msb1.logits), k, *ex) + host(msb1.sh_out)) <= TOL

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            layer()
    torch.cuda.synchronize()
    for rep in range(4):
        for o in outs:
            o.zero_()        # eager work between replays, on torch's stream
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.view(torch.uint8), e.view(torch.uint8)), f"replay {rep}"
