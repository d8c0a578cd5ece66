"""Benchmark of the q4 matmul path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|gemv|moe|shared|i8|gemm|moe_prefill]

Prints ONE JSON line. The headline (`value`) is the q4 decode GEMV of
a "step" is one decode pass over the dense projections of
L_LAYERS layers (fused QKV/gate-up 4096->12288 and down 6144->4096, every layer
its own weights) plus the LM head 4096->151936, at batch M; the step is run for
M in {1, 2, 4, 6, 8}. value = algorithmic bytes / time over all timed steps of
the sweep (GB/s). The weight pool (1.26 GB) is ~5x the 256 MB Infinity Cache,
so each launch streams its weights from HBM. Inputs are resident in HBM when the
timed region starts.

The other configs are measured too and reported under "workloads": the routed
MoE decode (config 3), the 4096-token q4 prefill GEMM (config 4) and the grouped
MoE prefill (config 5).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "v620-inference-engine_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
L_LAYERS = 24
BATCHES = (1, 2, 4, 6, 8)
DOM_BATCHES = BATCHES
# name prefix of the dominant launches' instantiations (every batch: 8-wave
# blocks, one 16-row tile of tokens, zero points, whole 4-group chunks)
DOM_KERNEL = "q4_gemv_block_kernel<qwq4::BF16, 8, 1, true, true"
H, QKV, FFN_DOWN_K, VOCAB = 4096, 12288, 6144, 151936


def q4_bytes(N, K, zeros=True):
    return N * K // 2 + N * (K // 128) * 2 + (N * (K // 128) // 2 if zeros else 0)


def gen_q4(torch, dev, N, K, zeros=True, lead=(), seed=0):
    """Seeded q4 weights generated in checkpoint order on the GPU, then tiled
    (qw_q4_tile) into the device format the kernels read; lead = (E,) stacks
    experts as one [E*N][K] matrix."""
    import qwq4
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    G = K // 128
    R = N * (lead[0] if lead else 1)
    W = torch.randint(-2**31, 2**31 - 1, (R, K // 8), generator=g, device=dev, dtype=torch.int32)
    S = (torch.randn((R, G), generator=g, device=dev) * 0.02).abs().to(torch.float16)
    Z = torch.randint(-2**31, 2**31 - 1, (R, (G + 7) // 8), generator=g, device=dev,
                      dtype=torch.int32) if zeros else None
    t = qwq4.tile(W, S, Z, R, K)
    del W, S, Z
    return t


def gen_x(torch, dev, M, K, seed=1):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)


def graphed(torch, fn):
    """Capture fn's launches into a HIP graph (the way the reference engine
    replays its decode step, src/engine/decode.hip:166-181); returns replay."""
    fn()  # warm: first-call set-up (kernel attributes) stays out of the graph
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            fn()
    torch.cuda.synchronize()
    return g.replay


class Timer:
    """HIP events on torch's current stream, the stream every qwq4 call launches on."""

    def __init__(self, torch):
        self.torch = torch
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.torch.cuda.synchronize()
        self.a.record()
        return self

    def __exit__(self, *exc):
        self.b.record()
        self.torch.cuda.synchronize()
        self.ms = self.a.elapsed_time(self.b)


# ---------------------------------------------------------------- config 2
def time_dominant(torch, qwq4, wqs, x, y, M, steps, warmup):
    """The dominant kernel alone: the 4096->12288 projection, launched back to
    back over the 24 layers' weights (a 627 MB pool, beyond the Infinity
    Cache) in one graph; average launch duration (us) from HIP events on the
    launching stream."""
    def dom():
        for wq in wqs:
            qwq4.gemv(*wq, x, QKV, H, M, y=y, y_bf16=True, xs=x.stride(0), ys=y.stride(0))

    dstep = graphed(torch, dom)
    for _ in range(warmup):
        dstep()
    with Timer(torch) as td:
        for _ in range(steps):
            dstep()
    return td.ms * 1e3 / (steps * len(wqs))


def launch_ceiling(torch, qwq4, wqs, steps, warmup):
    """What one launch can reach at all: the graph-launched per-kernel floor
    (an empty one-block kernel) and a kernel that only reads the dominant
    launch's weight bytes with the GEMV's load shape (qw_read_probe), both back
    to back over the same 24-layer pool as the dominant launches."""
    def timed(fn):
        g = graphed(torch, fn)
        for _ in range(warmup):
            g()
        with Timer(torch) as t:
            for _ in range(steps):
                g()
        return t.ms * 1e3 / (steps * len(wqs))

    empty_us = timed(lambda: [qwq4.read_probe() for _ in wqs])
    read_us = timed(lambda: [qwq4.read_probe(wq[0]) for wq in wqs])
    wb = wqs[0][0].numel() * wqs[0][0].element_size()
    return {"empty_launch_us": round(empty_us, 3), "read_only_us": round(read_us, 3), "read_bytes": wb,
            "read_only_GB_s": round(wb / (read_us * 1e-6) / 1e9, 1),
            "read_only_frac": round(wb / (read_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_dominant(torch, qwq4, dev, steps, warmup):
    """Only the dominant launches (the command whose kernel trace is compared
    with the bench line's roofline figures)."""
    wqs = [gen_q4(torch, dev, QKV, H, seed=2 * l) for l in range(L_LAYERS)]
    us = {}
    for M in DOM_BATCHES:
        x = gen_x(torch, dev, M, H, seed=M)
        y = torch.empty((M, QKV), dtype=torch.bfloat16, device=dev)
        us[M] = time_dominant(torch, qwq4, wqs, x, y, M, steps, warmup)
    return {"per_batch_us": us, "avg_launch_us": sum(us.values()) / len(us)}


def bench_gemv(torch, qwq4, dev, steps, warmup):
    layers = []
    for l in range(L_LAYERS):
        layers.append((gen_q4(torch, dev, QKV, H, seed=2 * l), gen_q4(torch, dev, H, FFN_DOWN_K, seed=2 * l + 1)))
    head = gen_q4(torch, dev, VOCAB, H, seed=999)
    step_bytes_w = L_LAYERS * (q4_bytes(QKV, H) + q4_bytes(H, FFN_DOWN_K)) + q4_bytes(VOCAB, H)
    per_m = {}
    tot_bytes = tot_ms = 0.0
    dom_us, dom_bytes = [], []
    for M in BATCHES:
        x = gen_x(torch, dev, M, FFN_DOWN_K, seed=M)
        y = torch.empty((M, VOCAB), dtype=torch.bfloat16, device=dev)

        def launches():
            for (wq, wd) in layers:
                qwq4.gemv(*wq, x, QKV, H, M, y=y, y_bf16=True, xs=x.stride(0), ys=y.stride(0))
                qwq4.gemv(*wd, x, H, FFN_DOWN_K, M, y=y, y_bf16=True, xs=x.stride(0), ys=y.stride(0))
            qwq4.gemv(*head, x, VOCAB, H, M, y=y, y_bf16=True, xs=x.stride(0), ys=y.stride(0))

        step = graphed(torch, launches)

        for _ in range(warmup):
            step()
        with Timer(torch) as t:
            for _ in range(steps):
                step()
        act = L_LAYERS * (M * H * 2 + M * QKV * 2 + M * FFN_DOWN_K * 2 + M * H * 2) + M * H * 2 + M * VOCAB * 2
        b = (step_bytes_w + act) * steps
        per_m[M] = {"GB_s": b / (t.ms * 1e-3) / 1e9, "ms_per_step": t.ms / steps,
                    "tokens_s": M * steps / (t.ms * 1e-3)}
        tot_bytes += b
        tot_ms += t.ms

        dom_us.append(time_dominant(torch, qwq4, [wq for (wq, _) in layers], x, y, M, steps, warmup))
        dom_bytes.append(q4_bytes(QKV, H) + M * H * 2 + M * QKV * 2)
    ceiling = launch_ceiling(torch, qwq4, [wq for (wq, _) in layers], steps, warmup)
    return {
        "GB_s": tot_bytes / (tot_ms * 1e-3) / 1e9,
        "ms_per_step": tot_ms / (steps * len(BATCHES)),
        "per_batch": per_m,
        "bytes_per_step_weights": step_bytes_w,
        "launches_per_step": 2 * L_LAYERS + 1,
        # roofline over every batch of the sweep
        "dominant": {"shape": f"{H}->{QKV}", "batches": list(DOM_BATCHES),
                     "avg_launch_us": sum(dom_us[BATCHES.index(m)] for m in DOM_BATCHES) / len(DOM_BATCHES),
                     "avg_bytes_per_launch": sum(dom_bytes[BATCHES.index(m)] for m in DOM_BATCHES) / len(DOM_BATCHES),
                     "per_batch_us": dict(zip(BATCHES, dom_us)), "launch_ceiling": ceiling},
    }


# ---------------------------------------------------------------- config 3
MOE_LAYERS = 8  # routing sets per step: successive blocks read different experts, as in a model's layers


def bench_moe(torch, qwq4, dev, steps, warmup, batches=(1, 2, 4, 8, 16, 32)):
    """Config 3: each step runs MOE_LAYERS MoE blocks over one 256-expert pool,
    each with its own activations, router logits (router weights for the
    fused block) and so its own experts; bytes are the distinct experts each
    block reads. Between two reads of one expert the step streams the other
    blocks' experts (>= 8 x 9.4 MB at batch 1, past the 256 MB Infinity
    Cache), so the weights come from HBM. The experts are symmetric (group-128
    fp16 scales, no zero points: config 3's format and the reference's,
    ref_model.cpp:114); the fused block is also timed at batch 1 on experts
    with zero points (block_zero_points) and, at batches 1-8, with a 16-bit shared expert, merged
    into its launches (qw_moe_decode_with_shared) and as separate launches
    (block_with_shared_expert; bytes add the shared expert's weights)."""
    E, F, k, L = 256, 1536, 8, MOE_LAYERS
    gate = gen_q4(torch, dev, F, H, zeros=False, lead=(E,), seed=10)
    up = gen_q4(torch, dev, F, H, zeros=False, lead=(E,), seed=11)
    down = gen_q4(torch, dev, H, F, zeros=False, lead=(E,), seed=12)
    per_expert = q4_bytes(F, H, False) * 2 + q4_bytes(H, F, False)
    gr = torch.Generator(device=dev)
    gr.manual_seed(13)
    router_w = [torch.randn((E, H), generator=gr, device=dev) * 0.02 for _ in range(L)]
    out = {}
    for B in batches:
        xs = [gen_x(torch, dev, B, H, seed=100 + 16 * B + l) for l in range(L)]
        g = torch.Generator(device=dev)
        g.manual_seed(200 + B)
        logits = [torch.randn((B, E), generator=g, device=dev) for _ in range(L)]
        r = qwq4.Route(B, E, k, dev)
        h = torch.empty((B * k, F), dtype=torch.float16, device=dev)
        yp = torch.empty((B * k, H), dtype=torch.float32, device=dev)
        o = torch.empty((B, H), dtype=torch.bfloat16, device=dev)
        U = 0
        for l in range(L):
            qwq4.moe_route(logits[l], k, out=r)
            U += int(r.n_active.item())

        def launches():
            for l in range(L):
                qwq4.moe_route(logits[l], k, out=r)
                qwq4.moe_experts_gemv(gate, up, down, r, xs[l], E, F, h=h, yp=yp)
                qwq4.moe_combine(yp, r, H, out=o)

        step = graphed(torch, launches)

        for _ in range(warmup):
            step()
        with Timer(torch) as t:
            for _ in range(steps):
                step()
        b = U * per_expert
        out[B] = {"distinct_experts": U / L, "GB_s": b * steps / (t.ms * 1e-3) / 1e9,
                  "us_per_block": t.ms * 1e3 / (steps * L), "tokens_s": B * L * steps / (t.ms * 1e-3)}

        # the fused block (qw_moe_decode): fp32 router GEMV + routing, experts,
        # combine inside the down projection; bytes add the router weights
        buf = qwq4.MoeDecode(B, E, k, H, F, dev)
        ob = torch.empty((B, H), dtype=torch.bfloat16, device=dev)
        Uf = 0
        for l in range(L):
            qwq4.moe_decode(router_w[l], xs[l], k, gate, up, down, E, F, buf=buf, out=ob)
            Uf += int(torch.unique(buf.top_e).numel())

        def fused():
            for l in range(L):
                qwq4.moe_decode(router_w[l], xs[l], k, gate, up, down, E, F, buf=buf, out=ob)

        fstep = graphed(torch, fused)
        for _ in range(warmup):
            fstep()
        with Timer(torch) as tf:
            for _ in range(steps):
                fstep()
        bf = Uf * per_expert + L * E * H * 4
        out[B]["block"] = {"distinct_experts": Uf / L, "GB_s": bf * steps / (tf.ms * 1e-3) / 1e9,
                           "us_per_block": tf.ms * 1e3 / (steps * L)}
        if B == 1:
            # the same block on experts with a 4-bit zero point per group
            zg = gen_q4(torch, dev, F, H, lead=(E,), seed=20)
            zu = gen_q4(torch, dev, F, H, lead=(E,), seed=21)
            zd = gen_q4(torch, dev, H, F, lead=(E,), seed=22)

            def fused_z():
                for l in range(L):
                    qwq4.moe_decode(router_w[l], xs[l], k, zg, zu, zd, E, F, buf=buf, out=ob)

            zstep = graphed(torch, fused_z)
            for _ in range(warmup):
                zstep()
            with Timer(torch) as tz:
                for _ in range(steps):
                    zstep()
            bz = Uf * (q4_bytes(F, H) * 2 + q4_bytes(H, F)) + L * E * H * 4
            out[B]["block_zero_points"] = {"GB_s": bz * steps / (tz.ms * 1e-3) / 1e9,
                                           "us_per_block": tz.ms * 1e3 / (steps * L)}
            del zg, zu, zd

        if B <= 8:
            # the block with the shared expert (16-bit, SH_FFN wide, weights of its own per
            # block): qw_moe_decode_with_shared against the shared expert's own launches
            # (two up to 4 rows, three above, as bench_shared picks them) followed by
            # qw_moe_decode (the form the engine runs, src/engine/decode.hip:99-105)
            gs = torch.Generator(device=dev)
            gs.manual_seed(23)
            sgu = [qwq4.w16_tile((torch.randn((2 * SH_FFN + 1, H), generator=gs, device=dev) * 0.05).half())
                   for _ in range(L)]
            sdn = [qwq4.w16_tile((torch.randn((H, SH_FFN), generator=gs, device=dev) * 0.05).half())
                   for _ in range(L)]
            sbuf = qwq4.MoeDecode(B, E, k, H, F, dev, Fs=SH_FFN)
            xh = [x.half() if x.dtype != torch.float16 else x for x in xs]
            sv = torch.empty((B, 2 * SH_FFN + 1), dtype=torch.float32, device=dev)
            so = torch.empty((B, H), dtype=torch.float32, device=dev)
            sh16 = torch.empty((B, SH_FFN), dtype=torch.float16, device=dev)

            def with_shared():
                for l in range(L):
                    qwq4.moe_decode_with_shared(router_w[l], xh[l], k, gate, up, down, E, F, sgu[l], sdn[l],
                                                SH_FFN, buf=sbuf, out=ob)

            def separate():
                for l in range(L):
                    qwq4.gemv_w16_tiled(sgu[l], 2 * SH_FFN + 1, H, xh[l], B, y=sv, f16=True)
                    if B <= 4:
                        qwq4.swiglu_gemv_w16_tiled(sdn[l], H, sv, SH_FFN, B, y=so)
                    else:
                        qwq4.swiglu_gate(sv, SH_FFN, h=sh16)
                        qwq4.gemv_w16_tiled(sdn[l], H, SH_FFN, sh16, B, y=so)
                    qwq4.moe_decode(router_w[l], xh[l], k, gate, up, down, E, F, buf=sbuf, shared=so, out=ob)

            sb = Uf * per_expert + L * E * H * 4 + L * ((2 * SH_FFN + 1) * H + H * SH_FFN) * 2
            rs = {}
            for name, fn in (("merged", with_shared), ("separate", separate)):
                st = graphed(torch, fn)
                for _ in range(warmup):
                    st()
                with Timer(torch) as ts:
                    for _ in range(steps):
                        st()
                rs[name] = {"GB_s": sb * steps / (ts.ms * 1e-3) / 1e9, "us_per_block": ts.ms * 1e3 / (steps * L)}
            out[B]["block_with_shared_expert"] = rs
            del sgu, sdn
    return out


# ------------------------------------------------- shared expert (16-bit)
SH_LAYERS, SH_FFN = 8, 1536


def bench_shared(torch, qwq4, dev, steps, warmup, batches=(1, 2, 4, 8)):
    """The shared expert as the engine runs it (src/engine/decode.hip:99-101):
    fused gate/up/gate-logit GEMV [2F+1][H] on fp16 weights, SwiGLU x sigmoid
    gate folded into the down GEMV [H][F] on fp16 weights (and, for comparison,
    as the reference's separate swiglu_T launch); SH_LAYERS layers of their own
    weights (302 MB, past the Infinity Cache), tiled once at load (qw_w16_tile,
    outside the timed region). Bytes: the 16-bit weights."""
    g = torch.Generator(device=dev)
    g.manual_seed(500)
    gu = [(torch.randn((2 * SH_FFN + 1, H), generator=g, device=dev) * 0.05).half() for _ in range(SH_LAYERS)]
    dn = [(torch.randn((H, SH_FFN), generator=g, device=dev) * 0.05).half() for _ in range(SH_LAYERS)]
    wbytes = SH_LAYERS * (gu[0].numel() + dn[0].numel()) * 2
    gu = [qwq4.w16_tile(w) for w in gu]
    dn = [qwq4.w16_tile(w) for w in dn]
    out = {}
    for M in batches:
        x = torch.randn((M, H), generator=g, device=dev).half()
        v = torch.empty((M, 2 * SH_FFN + 1), dtype=torch.float32, device=dev)
        hs = torch.empty((M, SH_FFN), dtype=torch.float16, device=dev)
        y = torch.empty((M, H), dtype=torch.float32, device=dev)

        def launches(fused):
            for l in range(SH_LAYERS):
                qwq4.gemv_w16_tiled(gu[l], 2 * SH_FFN + 1, H, x, M, y=v)
                if fused:  # swiglu_T folded into the down projection (two launches per layer)
                    qwq4.swiglu_gemv_w16_tiled(dn[l], H, v, SH_FFN, M, y=y)
                else:      # the reference's three launches
                    qwq4.swiglu_gate(v, SH_FFN, h=hs)
                    qwq4.gemv_w16_tiled(dn[l], H, SH_FFN, hs, M, y=y)

        # the form the header recommends for M rows (the SwiGLU folded into the
        # down GEMV up to 4 rows, else the three launches) is the headline
        # figure; the other is reported beside it
        best = M <= 4
        for fused in (best, not best):
            step = graphed(torch, lambda: launches(fused))
            for _ in range(warmup):
                step()
            with Timer(torch) as t:
                for _ in range(steps):
                    step()
            r = {"GB_s": wbytes * steps / (t.ms * 1e-3) / 1e9, "us_per_layer": t.ms * 1e3 / (steps * SH_LAYERS),
                 "form": "swiglu folded into the down GEMV" if fused else "three launches"}
            if fused == best:
                out[M] = r
            else:
                out[M]["other_form"] = r
    return out


def bench_i8(torch, qwq4, dev, steps, warmup, batches=(1, 2, 4, 8)):
    """The int8 dense GEMV (the engine's QW_INT8_DENSE copy, gpu::gemv_rows_i8,
    src/engine/decode.hip:64-70) on config 2's decode projections: L_LAYERS x
    (4096->12288, 6144->4096), int8 weights with an fp32 scale per 32 along K
    (1.125 B a weight, 2.04 GB of layers, past the Infinity Cache), fp16 rows,
    fp32 out, one graph per step, weights tiled at load (qw_i8_tile). Bytes:
    weights + scales + rows in and out."""
    g = torch.Generator(device=dev)
    g.manual_seed(600)
    shapes = ((QKV, H), (H, FFN_DOWN_K))
    ws = [[qwq4.i8_tile(torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8),
                        torch.rand((N, K // 32), generator=g, device=dev) * 1e-3) for N, K in shapes]
          for _ in range(L_LAYERS)]
    out = {}
    for M in batches:
        xs = {K: torch.randn((M, K), generator=g, device=dev).half() for _, K in shapes}
        ys = {N: torch.empty((M, N), dtype=torch.float32, device=dev) for N, _ in shapes}
        nbytes = L_LAYERS * sum(N * K * 1.125 + M * K * 2 + M * N * 4 for N, K in shapes)

        def launches():
            for layer in ws:
                for (Wt, St), (N, K) in zip(layer, shapes):
                    qwq4.gemv_i8(Wt, St, N, K, xs[K], M, y=ys[N])

        step = graphed(torch, launches)
        for _ in range(warmup):
            step()
        with Timer(torch) as t:
            for _ in range(steps):
                step()
        out[M] = {"GB_s": nbytes * steps / (t.ms * 1e-3) / 1e9,
                  "us_per_launch": t.ms * 1e3 / (steps * L_LAYERS * len(shapes))}
    return out


# ---------------------------------------------------------------- config 4
def bench_gemm(torch, qwq4, dev, steps, warmup):
    T = 4096
    res = {}
    for (N, K) in ((QKV, H), (H, FFN_DOWN_K)):
        W = gen_q4(torch, dev, N, K, seed=300 + N)
        X = gen_x(torch, dev, T, K, seed=301)
        Y = torch.empty((T, N), dtype=torch.bfloat16, device=dev)
        ws = torch.empty(qwq4.gemm_workspace_size(T, K), dtype=torch.uint8, device=dev)
        Yh = torch.empty((T // 2, N), dtype=torch.bfloat16, device=dev)
        wsh = torch.empty(qwq4.gemm_workspace_size(T // 2, K), dtype=torch.uint8, device=dev)
        # one HIP graph per step (the activation conversion and the GEMM, as a
        # prefill step would record them); warm up for >= 1 s so the timed
        # region runs at steady clocks
        full = graphed(torch, lambda: qwq4.gemm(*W, X, N, K, Y=Y, y_bf16=True, workspace=ws))
        halves = graphed(torch, lambda: [qwq4.gemm(*W, X[half * (T // 2):(half + 1) * (T // 2)], N, K, Y=Yh,
                                                   y_bf16=True, workspace=wsh) for half in range(2)])
        t_end = time.perf_counter() + 1.0
        while time.perf_counter() < t_end or warmup > 0:
            full()
            halves()
            torch.cuda.synchronize()
            warmup -= 1
        with Timer(torch) as t:
            for _ in range(steps):
                full()
        with Timer(torch) as t2:
            for _ in range(steps):
                halves()
        flops = 2.0 * T * N * K
        res[f"{K}x{N}"] = {"TFLOP_s": flops * steps / (t.ms * 1e-3) / 1e12, "us": t.ms * 1e3 / steps,
                           "TFLOP_s_2x2048": flops * steps / (t2.ms * 1e-3) / 1e12,
                           "tokens_s": T * steps / (t.ms * 1e-3)}
    return res


class SmiSampler:
    """Samples the GPU's own telemetry (amdsmi gpu_metrics) from a thread while
    kernels run: the graphics clock of every XCD, the socket power, and the
    residency counters of the package power limit (PPT)."""

    def __init__(self, period_s=0.01):
        import amdsmi
        self.smi = amdsmi
        amdsmi.amdsmi_init()
        self.h = amdsmi.amdsmi_get_processor_handles()[0]
        self.period = period_s
        self.samples = []

    def read(self):
        m = self.smi.amdsmi_get_gpu_metrics_info(self.h)
        clk = [c for c in m.get("current_gfxclks", []) if isinstance(c, (int, float))]
        return {"clk": sum(clk) / len(clk) if clk else float("nan"), "power": m.get("current_socket_power"),
                "ppt": m.get("ppt_residency_acc"), "acc": m.get("accumulation_counter")}

    def __enter__(self):
        import threading
        self.samples = []
        self.stop = threading.Event()
        self.first = self.read()

        def loop():
            while not self.stop.is_set():
                self.samples.append(self.read())
                time.sleep(self.period)
        self.t = threading.Thread(target=loop, daemon=True)
        self.t.start()
        return self

    def __exit__(self, *exc):
        self.stop.set()
        self.t.join()
        self.last = self.read()

    def summary(self):
        import statistics
        clk = [s["clk"] for s in self.samples]
        pw = [s["power"] for s in self.samples if isinstance(s["power"], (int, float))]
        out = {"samples": len(self.samples), "gfxclk_mhz_median": statistics.median(clk),
               "gfxclk_mhz_min": min(clk), "gfxclk_mhz_max": max(clk),
               "socket_power_w_median": statistics.median(pw) if pw else None}
        try:
            out["ppt_limit_residency"] = (self.last["ppt"] - self.first["ppt"]) / (self.last["acc"] - self.first["acc"])
        except (TypeError, ZeroDivisionError):
            out["ppt_limit_residency"] = None
        return out


def bench_gemm_power(torch, qwq4, dev, seconds=1.5):
    """Clock and power of the q4 prefill GEMM beside hipBLASLt (torch.matmul)
    on the same contraction with plain fp16 weights (the dequantised q4
    weights), one process, interleaved: 4096 tokens x 4096 -> 12288, fp16
    rows, fp16 out. Each leg replays its HIP graph for `seconds` after a 1 s
    warm-up while SmiSampler reads the GPU's telemetry."""
    T, N, K = 4096, QKV, H
    W = gen_q4(torch, dev, N, K, seed=300 + N)
    X = gen_x(torch, dev, T, K, seed=301).view(torch.bfloat16).float().half()
    Wc = qwq4.untile(*W, N, K)
    Wf = qwq4.dequant(*Wc, N, K).half()
    del Wc
    Y = torch.empty((T, N), dtype=torch.float16, device=dev)
    legs = {"q4_gemm": graphed(torch, lambda: qwq4.gemm(*W, X, N, K, Y=Y)),
            "hipblaslt_fp16": graphed(torch, lambda: torch.matmul(X, Wf.t(), out=Y))}
    flops = 2.0 * T * N * K
    res = {}
    for rep in range(2):
        for name, fn in legs.items():
            t_end = time.perf_counter() + 1.0
            while time.perf_counter() < t_end:
                for _ in range(50):
                    fn()
                torch.cuda.synchronize()
            n = 0
            with SmiSampler() as smi, Timer(torch) as t:
                t_end = time.perf_counter() + seconds
                while time.perf_counter() < t_end:
                    for _ in range(20):
                        fn()
                    n += 20
                    torch.cuda.synchronize()
            r = {"TFLOP_s": flops * n / (t.ms * 1e-3) / 1e12, "us": t.ms * 1e3 / n}
            r.update(smi.summary())
            res[f"{name}#{rep}"] = r
            print(f"# {name} rep {rep}: {json.dumps(r)}", file=sys.stderr, flush=True)
    return res


# ---------------------------------------------------------------- config 5
def bench_moe_prefill(torch, qwq4, dev, steps, warmup):
    """Config 5: one 4096-token chunk through the config-3 experts (symmetric:
    group-128 fp16 scales, no zero points); also timed on experts with zero
    points (zero_points) and through the opt-in W4A8 path."""
    E, F, k, T = 256, 1536, 8, 4096
    gate = gen_q4(torch, dev, F, H, zeros=False, lead=(E,), seed=10)
    up = gen_q4(torch, dev, F, H, zeros=False, lead=(E,), seed=11)
    down = gen_q4(torch, dev, H, F, zeros=False, lead=(E,), seed=12)
    x = gen_x(torch, dev, T, H, seed=400)
    g = torch.Generator(device=dev)
    g.manual_seed(401)
    logits = torch.randn((T, E), generator=g, device=dev) + torch.randn((1, E), generator=g, device=dev) * 0.5
    tm = qwq4.moe_grouped_tile_m()
    r = qwq4.Route(T, E, k, dev, tile_m=tm)
    h = torch.empty((T * k, F), dtype=torch.float16, device=dev)
    yp = torch.empty((T * k, H), dtype=torch.float16, device=dev)  # fp16 per-slot rows, as the reference keeps them
    o = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(max(qwq4.moe_grouped_workspace_size(T, k, E, H, F), 1), dtype=torch.uint8, device=dev)

    def timed(g_, u_, d_, warm):
        def step():
            qwq4.moe_route(logits, k, tile_m=tm, out=r)
            qwq4.moe_experts_grouped(g_, u_, d_, r, x, E, F, h=h, yp=yp, workspace=ws)
            qwq4.moe_combine(yp, r, H, out=o)

        gstep = graphed(torch, step)  # one HIP graph per step, warmed for >= 1 s (steady clocks)
        t_end = time.perf_counter() + 1.0
        while time.perf_counter() < t_end or warm > 0:
            gstep()
            torch.cuda.synchronize()
            warm -= 1
        with Timer(torch) as t:
            for _ in range(steps):
                gstep()
        return t.ms

    flops = 2.0 * (k * T) * (2 * F * H + H * F)
    ms = timed(gate, up, down, warmup)
    res = {"TFLOP_s": flops * steps / (ms * 1e-3) / 1e12, "us_per_step": ms * 1e3 / steps,
           "tokens_s": T * steps / (ms * 1e-3)}
    zg = gen_q4(torch, dev, F, H, lead=(E,), seed=20)
    zu = gen_q4(torch, dev, F, H, lead=(E,), seed=21)
    zd = gen_q4(torch, dev, H, F, lead=(E,), seed=22)
    msz = timed(zg, zu, zd, warmup)
    res["zero_points"] = {"TFLOP_s": flops * steps / (msz * 1e-3) / 1e12, "us_per_step": msz * 1e3 / steps}
    del zg, zu, zd

    # the reference's opt-in W4A8 path (int8 activations, lossy) on the same
    # experts and routing: 64-slot tiles, fp16 rows as the engine passes them
    tm8 = qwq4.moe_w4a8_tile_m()
    r8 = qwq4.Route(T, E, k, dev, tile_m=tm8)
    xh = x.half()
    ws8 = torch.empty(qwq4.lib().qw_moe_w4a8_workspace_size(T, k, H, F), dtype=torch.uint8, device=dev)

    def step8():
        qwq4.moe_route(logits, k, tile_m=tm8, out=r8)
        qwq4.moe_experts_w4a8(gate, up, down, r8, xh, E, F, h=h, yp=yp, workspace=ws8)
        qwq4.moe_combine(yp, r8, H, out=o)

    g8 = graphed(torch, step8)
    t_end = time.perf_counter() + 1.0
    while time.perf_counter() < t_end:
        g8()
        torch.cuda.synchronize()
    with Timer(torch) as t8:
        for _ in range(steps):
            g8()
    res["w4a8"] = {"TOP_s": flops * steps / (t8.ms * 1e-3) / 1e12, "us_per_step": t8.ms * 1e3 / steps,
                   "note": "int8 activations per (row, 128-group), int8 MFMA, lossy (the reference's opt-in path)"}
    return res


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    PMC summary (FETCH_SIZE and WRITE_SIZE, each scaled by the copy-kernel
    calibration recorded there); None when absent."""
    path = os.path.join(ROOT, "profiles", "gemv_4096x12288_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


# ------------------------------------------------------------ CPU baseline
def host_cores():
    """CPUs this process may run on: the affinity mask, capped by the cgroup
    CPU quota when one is set (a GPU box grants each GPU's job a share of the
    host, whatever the machine-wide count says)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return n


def cpu_baseline(runs=5):
    """The C oracle (oracle/q4_oracle.c, the reference's expert_linear scheme,
    threaded over N with a grain of 16 rows like src/core/threadpool.hpp:38-58)
    on every host core this job has: one warm-up, then the median of `runs`
    timed passes of (a) the decode step at M=1 on a 2-layer + LM-head sample
    and (b) config 1 (4096x4096, M=1, fp32 x)."""
    import statistics
    from oracle import oracle as o
    from qwq4 import synth
    threads = host_cores()
    mats = [(QKV, H), (H, FFN_DOWN_K)] * 2 + [(VOCAB, H)]
    ws = [synth.q4_weights(7, f"cpu{i}", N, K) for i, (N, K) in enumerate(mats)]
    xs = {K: synth.acts(7, f"cx{K}", 1, K)[1] for K in (H, FFN_DOWN_K)}
    nbytes = sum(q4_bytes(N, K) for N, K in mats)

    def one_step():
        for (N, K), (W, S, Z) in zip(mats, ws):
            o.q4_linear(W, S, Z, N, K, xs[K], threads=threads)

    t0 = time.perf_counter()
    one_step()
    reps = max(1, int(2.0 / max(time.perf_counter() - t0, 1e-4)))  # ~2 s per timed run

    def step_pass():
        for _ in range(reps):
            one_step()

    W1, S1, Z1 = synth.q4_weights(7, "config1", H, H)
    x1 = np.random.default_rng(7).standard_normal((1, H)).astype(np.float32)

    def c1_pass():
        for _ in range(200):
            o.q4_linear(W1, S1, Z1, H, H, x1, threads=threads)

    def median_s(fn):
        fn()  # warm-up
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    t_step = median_s(step_pass) / reps
    t_c1 = median_s(c1_pass) / 200
    return {"value": nbytes / t_step / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"oracle q4_linear on {threads} threads, M=1: one pass over 2 layers (4096->12288, "
                      f"6144->4096) + LM head 4096->151936 ({nbytes / 1e6:.0f} MB of q4 weights); median of "
                      f"{runs} runs of {reps} passes after 1 warm-up",
            "config1": {"us": t_c1 * 1e6, "GB_s": q4_bytes(H, H) / t_c1 / 1e9,
                        "sample": "4096x4096 q4 with zero points, M=1, fp32 x; median of "
                                  f"{runs} runs of 200 calls after 1 warm-up"}}


# ------------------------------------------------ HBM traffic (rocprofv3 PMC)
COPY_BYTES = 512 << 20


def traffic_probe(torch, qwq4, dev):
    """Launches for the PMC runs: the dominant kernel (4096->12288 over the
    24-layer weight pool, each batch of DOM_BATCHES once per layer) and a plain
    copy of COPY_BYTES, whose counter readings calibrate the byte counters."""
    layers = [gen_q4(torch, dev, QKV, H, seed=2 * l) for l in range(L_LAYERS)]
    for M in DOM_BATCHES:
        x = gen_x(torch, dev, M, H, seed=M)
        y = torch.empty((M, QKV), dtype=torch.bfloat16, device=dev)
        for wq in layers:
            qwq4.gemv(*wq, x, QKV, H, M, y=y, y_bf16=True)
    torch.cuda.synchronize()
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def parse_pmc(fetch_dir, write_dir, out_path):
    """Reduces two rocprofv3 --pmc runs of `--workload traffic` (FETCH_SIZE,
    then WRITE_SIZE; KiB per dispatch) to HBM bytes per launch of the dominant
    kernel, each counter scaled by copy bytes / its reading for the copy."""
    import csv
    import glob

    def per_kernel(d, counter):
        gemv, copies = [], []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r.get("Counter_Name") != counter:
                    continue
                v = float(r["Counter_Value"]) * 1024.0
                if DOM_KERNEL in r["Kernel_Name"]:
                    gemv.append(v)
                elif "copy" in r["Kernel_Name"].lower():
                    copies.append((int(r["Grid_Size"]), v))
        big = max(g for g, _ in copies)  # the COPY_BYTES copies, not torch's small casts
        cv = [v for g, v in copies if g == big]
        return {"gemv": sum(gemv) / len(gemv), "copy": sum(cv) / len(cv)}

    fe, wr = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    kf, kw = COPY_BYTES / fe["copy"], COPY_BYTES / wr["copy"]
    res = {"kernel": "q4_gemv_block_kernel (4096->12288), batches " + ",".join(map(str, DOM_BATCHES)),
           "fetch_raw_bytes": fe["gemv"], "write_raw_bytes": wr["gemv"],
           "copy_fetch_raw_bytes": fe["copy"], "copy_write_raw_bytes": wr["copy"],
           "fetch_scale": kf, "write_scale": kw,
           "traffic_bytes_per_launch": int(fe["gemv"] * kf + wr["gemv"] * kw),
           "algorithmic_bytes_per_launch": int(q4_bytes(QKV, H) + sum(M * (H + QKV) * 2 for M in DOM_BATCHES) /
                                               len(DOM_BATCHES))}
    with open(out_path, "w") as f:
        json.dump(res, f, indent=1)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="all", help="all, or a comma list of gemv, moe, shared, i8, gemm, moe_prefill; or traffic (launches for PMC runs), or dominant (the roofline kernel's launches alone), or gemm_power (clock and power of the prefill GEMM beside hipBLASLt)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--moe-batches", default="1,2,4,8,16,32",
                    help="decode batches of the moe workload (comma list), e.g. one batch for a per-launch trace")
    ap.add_argument("--parse-pmc", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "OUT_JSON"),
                    help="reduce two rocprofv3 --pmc runs of --workload traffic to bytes per launch")
    a = ap.parse_args()
    if a.parse_pmc:
        print(json.dumps(parse_pmc(*a.parse_pmc)))
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: --gpus must be 1 (no collectives, "
                                   "no multi-GPU path)"}))
        sys.exit(2)
    import torch
    import qwq4
    dev = torch.device("cuda:0")
    qwq4.lib()
    if a.workload == "traffic":
        traffic_probe(torch, qwq4, dev)
        return
    if a.workload == "gemm_power":
        print(json.dumps(bench_gemm_power(torch, qwq4, dev)))
        return
    if a.workload == "dominant":
        print(json.dumps(bench_dominant(torch, qwq4, dev, a.steps, a.warmup)))
        return
    wl = set(a.workload.split(","))
    if "all" in wl:
        wl = {"gemv", "moe", "shared", "i8", "gemm", "moe_prefill"}
    res = {}
    if "gemv" in wl:
        res["gemv"] = bench_gemv(torch, qwq4, dev, a.steps, a.warmup)
        print(f"# gemv {res['gemv']['GB_s']:.1f} GB/s", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    if "moe" in wl:
        res["moe_decode"] = bench_moe(torch, qwq4, dev, a.steps, a.warmup,
                                      batches=tuple(int(b) for b in a.moe_batches.split(",")))
        print("# moe decode done", file=sys.stderr, flush=True)
    if "shared" in wl:
        res["shared_expert"] = bench_shared(torch, qwq4, dev, a.steps, a.warmup)
        print("# shared expert done", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    if "i8" in wl:
        res["i8_gemv"] = bench_i8(torch, qwq4, dev, a.steps, a.warmup)
        print("# int8 gemv done", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    if "gemm" in wl:
        res["prefill_gemm"] = bench_gemm(torch, qwq4, dev, max(4, a.steps), 1)
        print("# gemm done", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    if "moe_prefill" in wl:
        res["moe_prefill"] = bench_moe_prefill(torch, qwq4, dev, max(4, a.steps // 2), 1)
        print("# moe prefill done", file=sys.stderr, flush=True)
    line = {
        "metric": "q4 GEMV HBM GB/s (% of peak) at batch 1-8; q4 prefill GEMM TFLOP/s (% MFMA)",
        "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "q4 weights, bf16 x, fp32 acc",
        "data": "synthetic (seeded): uniform nibbles, |N(0,0.02)| fp16 scales, uniform 4-bit zeros, N(0,1) bf16 x",
        "config": {"workload": f"decode dense q4 GEMV, {L_LAYERS} layers x (4096->12288, 6144->4096) + LM head "
                               f"4096->151936, batch 1/2/4/6/8, bf16 out, one HIP graph per step",
                   "batches": list(BATCHES)},
    }
    if "gemv" in res:
        g = res["gemv"]
        line["value"] = round(g["GB_s"], 1)
        line["ms_per_step"] = round(g["ms_per_step"], 4)
        d = g["dominant"]
        ach = d["avg_bytes_per_launch"] / (d["avg_launch_us"] * 1e-6) / 1e9
        line["roofline"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                            "kernel": DOM_KERNEL + ", ...> (4096->12288, every batch of the sweep)",
                            "avg_launch_us": round(d["avg_launch_us"], 3),
                            "algorithmic_bytes_per_launch": int(d["avg_bytes_per_launch"]),
                            "launch_ceiling": d["launch_ceiling"]}
    line["workloads"] = res
    if not a.no_cpu and "gemv" in wl:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
