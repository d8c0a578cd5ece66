"""The shared expert and the dense 16-bit linear: qw_w16_gemv (fp16 weights
with fp16 rows, as the engine's gemv_rows; bf16 with bf16, as the reference's
Model::linear) and qw_swiglu_gate (the engine's swiglu_T) against the oracle,
and the whole MoE block (routed experts + shared expert, ref_model.cpp:406-478)
composed from the entry points."""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, bf16_err_ok, host, rel_err, to_dev

pytestmark = pytest.mark.gpu


def w16(seed, name, N, K, f16, scale=0.05):
    """16-bit weight bits [N][K] and their exact fp32 values."""
    w = (synth.rng(seed, name).normal(0.0, scale, size=(N, K))).astype(np.float32)
    if f16:
        b = w.astype(np.float16).view(np.uint16)
        return b, b.view(np.float16).astype(np.float32)
    b = synth.bf16_bits(w)
    return b, synth.bf16_to_f32(b)


def rows(seed, name, M, K, f16):
    v = synth.rng(seed, name).normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    if f16:
        b = v.astype(np.float16).view(np.uint16)
        return b, b.view(np.float16).astype(np.float32)
    b = synth.bf16_bits(v)
    return b, synth.bf16_to_f32(b)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("N,K,M", [(3073, 4096, 1), (3073, 4096, 4), (3073, 4096, 8), (4096, 1536, 1), (4096, 1536, 8),
                                   (100, 320, 3), (1024, 2048, 17), (256, 4096, 32)])
def test_w16_gemv(gpu, oracle, f16, N, K, M):
    print(f"w16 gemv f16={f16} N={N} K={K} M={M}", flush=True)
    Wb, _ = w16(81, f"w{N}x{K}", N, K, f16)
    xb, xf = rows(81, f"x{M}x{K}", M, K, f16)
    y = host(qwq4.gemv_w16(to_dev(Wb, gpu), to_dev(xb, gpu), M, f16=f16))
    assert rel_err(y, oracle.linear_w16(Wb, xf, f16)) <= TOL


@pytest.mark.parametrize("N,K,rpg,M", [(1296, 1024, 324, 1), (1296, 1024, 324, 4), (1296, 1024, 324, 8),
                                        (4096, 2048, 1024, 2), (1000, 512, 130, 3)])
def test_w16_gemv_row_slices(gpu, oracle, N, K, rpg, M):
    """gemv_rows' row grouping (rpg: row n reads activation slice n // rpg,
    src/kernels/gemv.hip:16-17) on fp16 weights, row-major and tiled at
    load: the engine's hyper-connection down projection (4 streams of 324
    rows, decode.hip:55-59; 324 is not a multiple of 16, so tiles straddle
    two slices) and others, strided rows covering every slice, accumulating
    into y. Against the oracle; the two layouts bit for bit; rows past N
    untouched."""
    import torch
    print(f"w16 gemv rpg N={N} K={K} rpg={rpg} M={M}", flush=True)
    ns = (N + rpg - 1) // rpg
    Wb, _ = w16(84, f"r{N}x{K}", N, K, True)
    xs = ns * K + 8
    xb, xf = rows(84, f"rx{M}", M, xs, True)
    dW, dx = to_dev(Wb, gpu), to_dev(xb, gpu)
    ref = oracle.linear_w16(Wb, xf[:, :ns * K], True, rpg=rpg) + 0.25
    y = torch.full((M, N + 16), 0.25, dtype=torch.float32, device=gpu)
    qwq4.gemv_w16(dW, dx, M, y=y, accumulate=True, f16=True, xs=xs, ys=N + 16, rpg=rpg)
    yh = host(y)
    assert np.all(yh[:, N:] == 0.25)
    assert rel_err(yh[:, :N], ref) <= TOL
    Wt = qwq4.w16_tile(dW)
    yt = torch.full((M, N + 16), 0.25, dtype=torch.float32, device=gpu)
    qwq4.gemv_w16_tiled(Wt, N, K, dx, M, y=yt, accumulate=True, f16=True, xs=xs, ys=N + 16, rpg=rpg)
    assert np.array_equal(host(yt).view(np.uint32), yh.view(np.uint32))


def test_w16_gemv_strides_bf16_out_and_accumulate(gpu, oracle):
    import torch
    N, K, M = 500, 1024, 5
    Wb, _ = w16(82, "ws", N, K, True)
    xb, xf = rows(82, "xs", M, K, True)
    Wp = torch.zeros((N, K + 64), dtype=torch.int16, device=gpu)
    Wp[:, :K] = to_dev(Wb, gpu)
    y = torch.full((M, N + 8), 0.5, dtype=torch.float32, device=gpu)
    qwq4.gemv_w16(Wp[:, :K], to_dev(xb, gpu), M, y=y, accumulate=True, f16=True, ys=N + 8)
    yh = host(y)
    assert np.all(yh[:, N:] == 0.5)
    assert rel_err(yh[:, :N], oracle.linear_w16(Wb, xf, True) + 0.5) <= TOL
    yb = host(qwq4.gemv_w16(to_dev(Wb, gpu), to_dev(xb, gpu), M, y_bf16=True, f16=True))
    assert bf16_err_ok(yb, oracle.linear_w16(Wb, xf, True))


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("N,K,M", [(3073, 4096, 1), (3073, 4096, 8), (4096, 1536, 4), (100, 320, 3), (1024, 2048, 17),
                                   (256, 4096, 32), (40, 32, 2)])
def test_w16_gemv_tiled(gpu, oracle, f16, N, K, M):
    """The tiled layout gives the row-major GEMV's results bit for bit (the same
    products summed in the same order), and the oracle's."""
    print(f"w16 gemv tiled f16={f16} N={N} K={K} M={M}", flush=True)
    Wb, _ = w16(87, f"wt{N}x{K}", N, K, f16)
    xb, xf = rows(87, f"xt{M}x{K}", M, K, f16)
    W, x = to_dev(Wb, gpu), to_dev(xb, gpu)
    y = host(qwq4.gemv_w16_tiled(qwq4.w16_tile(W), N, K, x, M, f16=f16))
    assert np.array_equal(y.view(np.uint32), host(qwq4.gemv_w16(W, x, M, f16=f16)).view(np.uint32))
    assert rel_err(y, oracle.linear_w16(Wb, xf, f16)) <= TOL


def test_w16_gemv_tiled_strides_bf16_out_and_accumulate(gpu, oracle):
    import torch
    N, K, M = 500, 1024, 5
    Wb, _ = w16(88, "wts", N, K, True)
    xb, xf = rows(88, "xts", M, K, True)
    Wp = torch.zeros((N, K + 64), dtype=torch.int16, device=gpu)
    Wp[:, :K] = to_dev(Wb, gpu)
    Wt = qwq4.w16_tile(Wp[:, :K])  # from a padded row stride
    xp = torch.zeros((M, K + 32), dtype=torch.int16, device=gpu)
    xp[:, :K] = to_dev(xb, gpu)
    y = torch.full((M, N + 8), 0.5, dtype=torch.float32, device=gpu)
    qwq4.gemv_w16_tiled(Wt, N, K, xp, M, y=y, accumulate=True, f16=True, xs=K + 32, ys=N + 8)
    yh = host(y)
    assert np.all(yh[:, N:] == 0.5)
    assert rel_err(yh[:, :N], oracle.linear_w16(Wb, xf, True) + 0.5) <= TOL
    yb = host(qwq4.gemv_w16_tiled(Wt, N, K, to_dev(xb, gpu), M, y_bf16=True, f16=True))
    assert bf16_err_ok(yb, oracle.linear_w16(Wb, xf, True))


def test_w16_tile_layout(gpu):
    """qw_w16_tile against a numpy restatement of the layout: entry (sub, s, 16 q + n)
    = row 16 sub + n, K 32 s + 8 q .. +8; rows past N zero (ragged last tile)."""
    rng = np.random.default_rng(89)
    N, K = 37, 96
    Wb = rng.integers(0, 1 << 16, size=(N, K), dtype=np.uint16)
    Wt = host(qwq4.w16_tile(to_dev(Wb, gpu))).view(np.uint16)
    tiles = (N + 15) // 16
    Wp = np.zeros((tiles * 16, K), np.uint16)
    Wp[:N] = Wb
    want = Wp.reshape(tiles, 16, K // 32, 4, 8).transpose(0, 2, 3, 1, 4)  # [sub][s][q][n][8]
    assert np.array_equal(Wt.reshape(want.shape), want)


@pytest.mark.parametrize("N,n,M", [(4096, 1536, 1), (4096, 1536, 2), (4096, 1536, 3), (4096, 1536, 5),
                                   (4096, 1536, 8), (4096, 1536, 10), (4096, 1536, 11), (4096, 1536, 32), (100, 64, 4),
                                   (1024, 512, 17), (40, 32, 1)])
def test_w16_swiglu_gemv_tiled(gpu, N, n, M):
    """The SwiGLU x gate folded into the down GEMV gives, bit for bit, what
    qw_swiglu_gate followed by qw_w16_gemv_tiled gives (register staging up to two
    pieces per thread, the staging loop beyond); v scaled so that some h values
    saturate at the fp16 limit."""
    import torch
    print(f"w16 swiglu gemv N={N} n={n} M={M}", flush=True)
    Wb, _ = w16(90, f"dn{N}x{n}", N, n, True)
    v = (np.random.default_rng(91 + M).standard_normal((M, 2 * n + 1)) * 3).astype(np.float32)
    v[:, : n // 8] *= 200.0  # silu(g) * u beyond 65504 for some
    Wt = qwq4.w16_tile(to_dev(Wb, gpu))
    dv = to_dev(v, gpu)
    y = host(qwq4.swiglu_gemv_w16_tiled(Wt, N, dv, n, M))
    h = qwq4.swiglu_gate(dv, n)
    ref = host(qwq4.gemv_w16_tiled(Wt, N, n, h, M, f16=True))
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    assert np.all(np.isfinite(y))


def test_w16_swiglu_gemv_tiled_strides_bf16_out_and_accumulate(gpu, oracle):
    import torch
    N, n, M = 300, 256, 6
    Wb, _ = w16(92, "dns", N, n, True)
    v = (np.random.default_rng(92).standard_normal((M, 2 * n + 7)) * 2).astype(np.float32)  # ldv = 2n + 7
    Wt = qwq4.w16_tile(to_dev(Wb, gpu))
    dv = to_dev(v, gpu)
    h = oracle.swiglu_gate(np.ascontiguousarray(v[:, : 2 * n + 1]), n)
    ref = oracle.linear_w16(Wb, h, True)
    y = torch.full((M, N + 8), 0.5, dtype=torch.float32, device=gpu)
    qwq4.swiglu_gemv_w16_tiled(Wt, N, dv, n, M, y=y, accumulate=True, ys=N + 8)
    yh = host(y)
    assert np.all(yh[:, N:] == 0.5)
    assert rel_err(yh[:, :N], ref + 0.5) <= TOL
    yb = host(qwq4.swiglu_gemv_w16_tiled(Wt, N, dv, n, M, y_bf16=True))
    assert bf16_err_ok(yb, ref)


def test_swiglu_gate(gpu, oracle):
    n, T = 1536, 6
    v = (np.random.default_rng(83).standard_normal((T, 2 * n + 1)) * 2).astype(np.float32)
    h = host(qwq4.swiglu_gate(to_dev(v, gpu), n)).astype(np.float32)
    r = oracle.swiglu_gate(v, n)
    # fp16 output: the oracle's value rounded to fp16, within an ulp
    assert np.all(np.abs(h - r) <= 2.0**-10 * np.abs(r) + 2.0**-24)


@pytest.mark.parametrize("T,tiled", [(1, False), (4, False), (8, False), (1, True), (8, True), (1, "fused"),
                                     (4, "fused"), (8, "fused")])
def test_moe_block_with_shared_expert(gpu, oracle, T, tiled):
    """The engine's decode MoE block (decode.hip:99-111): shared expert
    (fused gate/up/gate-logit GEMV on bf16 weights, SwiGLU x sigmoid gate,
    down GEMV on fp16 weights) into the routed block's combine; against the
    oracle's routed experts plus its shared expert (ref_model.cpp:406-478)."""
    E, H, F, k, SF = 64, 1024, 256, 4, 512
    print(f"moe block + shared expert T={T}", flush=True)
    ex = synth.experts(84, E, H, F)
    xb, xf = synth.acts(84, f"bx{T}", T, H)
    Wr = (np.random.default_rng(84).standard_normal((E, H)) * 0.05).astype(np.float32)
    gu_b, _ = w16(85, "gu", 2 * SF + 1, H, False)
    dn_b, _ = w16(86, "dn", H, SF, True)
    from test_moe_gpu import _experts_dev
    (g, u, d), _, _ = _experts_dev(gpu, ex)
    dx = to_dev(xb, gpu)
    if tiled == "fused":  # tiled weights, SwiGLU x gate folded into the down GEMV
        v = qwq4.gemv_w16_tiled(qwq4.w16_tile(to_dev(gu_b, gpu)), 2 * SF + 1, H, dx, T, f16=False)
        sh = qwq4.swiglu_gemv_w16_tiled(qwq4.w16_tile(to_dev(dn_b, gpu)), H, v, SF, T)
    elif tiled:  # weights tiled at load (qw_w16_tile)
        v = qwq4.gemv_w16_tiled(qwq4.w16_tile(to_dev(gu_b, gpu)), 2 * SF + 1, H, dx, T, f16=False)
        hs = qwq4.swiglu_gate(v, SF)
        sh = qwq4.gemv_w16_tiled(qwq4.w16_tile(to_dev(dn_b, gpu)), H, SF, hs, T, f16=True)
    else:
        v = qwq4.gemv_w16(to_dev(gu_b, gpu), dx, T, f16=False)          # [T][2 SF + 1] fp32
        hs = qwq4.swiglu_gate(v, SF)                                     # [T][SF] fp16
        sh = qwq4.gemv_w16(to_dev(dn_b, gpu), hs, T, f16=True)           # [T][H] fp32
    out, buf = qwq4.moe_decode(to_dev(Wr, gpu), dx, k, g, u, d, E, F, shared=sh, out_bf16=False)
    logits = host(buf.logits)
    ref = oracle.moe(xf, logits, k, *ex) + oracle.shared_expert(xf, gu_b, dn_b, f16_gu=False, f16_down=True)
    assert rel_err(host(out), ref) <= TOL


def _random_w16(n, seed):
    r = np.random.default_rng(seed)
    return [(int(r.integers(1, 5000)), 32 * int(r.integers(1, 257)), int(r.integers(1, 33)), bool(r.integers(0, 2)))
            for _ in range(n)]


@pytest.mark.parametrize("N,K,M,f16", _random_w16(12, 2031))
def test_w16_gemv_tiled_random_shapes(gpu, oracle, N, K, M, f16):
    """Seeded random shapes (any N, K a multiple of 32 up to 8192, batch 1-32,
    fp16 or bf16): the tiled GEMV equals the row-major one bit for bit (every
    launch-shape choice: K split, steps in flight, register or direct staging,
    row-split launches) and the oracle."""
    print(f"w16 tiled random N={N} K={K} M={M} f16={f16}", flush=True)
    Wb, _ = w16(N + K, f"wr{N}x{K}", N, K, f16)
    xb, xf = rows(N + K, f"xr{M}x{K}", M, K, f16)
    W, x = to_dev(Wb, gpu), to_dev(xb, gpu)
    y = host(qwq4.gemv_w16_tiled(qwq4.w16_tile(W), N, K, x, M, f16=f16))
    assert np.array_equal(y.view(np.uint32), host(qwq4.gemv_w16(W, x, M, f16=f16)).view(np.uint32))
    assert rel_err(y, oracle.linear_w16(Wb, xf, f16)) <= TOL


def _random_swiglu(n, seed):
    r = np.random.default_rng(seed)
    return [(int(r.integers(1, 5000)), 32 * int(r.integers(1, 129)), int(r.integers(1, 33))) for _ in range(n)]


@pytest.mark.parametrize("N,n,M", _random_swiglu(12, 2032))
def test_w16_swiglu_gemv_tiled_random_shapes(gpu, N, n, M):
    """Seeded random shapes (any N, n a multiple of 32 up to 4096, batch 1-32): the
    SwiGLU x gate folded into the down GEMV equals qw_swiglu_gate followed by
    qw_w16_gemv_tiled bit for bit, or is rejected when the rows exceed the staging
    LDS (as the two-launch form, which splits them, is not)."""
    print(f"w16 swiglu random N={N} n={n} M={M}", flush=True)
    Wb, _ = w16(N + n, f"dr{N}x{n}", N, n, True)
    v = (np.random.default_rng(N + n + M).standard_normal((M, 2 * n + 1)) * 2).astype(np.float32)
    Wt = qwq4.w16_tile(to_dev(Wb, gpu))
    dv = to_dev(v, gpu)
    ref = host(qwq4.gemv_w16_tiled(Wt, N, n, qwq4.swiglu_gate(dv, n), M, f16=True))
    try:
        y = host(qwq4.swiglu_gemv_w16_tiled(Wt, N, dv, n, M))
    except RuntimeError as err:
        assert "staging LDS" in str(err) and M * n * 2 > 96 * 1024
        return
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("T,E,H,F,k,SF,f16,zeros", [(1, 256, 4096, 1536, 8, 1536, True, False),
                                                    (1, 64, 2048, 512, 6, 512, False, False),
                                                    (1, 64, 1024, 256, 4, 320, True, False),
                                                    (2, 256, 4096, 1536, 8, 1536, True, False),
                                                    (4, 64, 1024, 256, 4, 512, False, False),
                                                    (8, 64, 2048, 512, 6, 1536, True, False),
                                                    (3, 256, 4096, 1536, 8, 1536, False, False),
                                                    (8, 256, 4096, 1536, 8, 1536, False, False),
                                                    (5, 128, 4096, 512, 6, 1024, True, True),
                                                    (6, 64, 4096, 256, 8, 512, False, False),
                                                    (7, 32, 4096, 256, 8, 1536, True, False),
                                                    (12, 64, 2048, 256, 6, 512, True, False),
                                                    (24, 128, 4096, 256, 8, 1024, False, True),
                                                    (32, 256, 4096, 1536, 8, 1536, True, False),
                                                    (20, 64, 4096, 256, 8, 256, True, True)])
def test_moe_decode_with_shared(gpu, oracle, T, E, H, F, k, SF, f16, zeros):
    """qw_moe_decode_with_shared against its parts as separate calls (the
    shared expert's tiled gate/up/gate-logit GEMV and SwiGLU-down GEMV, then
    qw_moe_decode with their output as the shared rows): the shared rows, the
    gate/up rows and the block's output bit for bit, and against the oracle.
    With Fs a multiple of 256 the gate/up GEMV runs inside the router-logits
    launch (batches 1-8: one, two and four rows per MFMA pass, every staging
    width up to the looped one at 8 rows of 4096), the down GEMV at batch 1
    inside the routed gate/up launch and at batches 2-4 inside the routing
    launch, and at batches 5-8 the routing launch forms the SwiGLU rows and, at
    H 2048 and 4096, the down GEMV over them rides in the gate/up launch (experts with
    more than the 4 staged rows at batches 5-7; zero points at 5) (fp16 rows
    and weights at config 3's size, bf16 at H 2048 and at batches 3, 6 and 8).
    Above 8 tokens the shared GEMVs take their own launches, except the down
    GEMV, which rides in the gate/up launch where its LDS leaves the gate/up
    blocks per CU unchanged (batch 12, and 20 with Fs 256: two row tiles;
    batches 24 and 32 take its own launch); Fs = 320 takes their own launches."""
    print(f"moe decode with shared T={T} E={E} H={H} F={F} k={k} Fs={SF} f16={f16} zeros={zeros}", flush=True)
    ex = synth.experts(95 + T, E, H, F, zeros=zeros)
    xb, xf = rows(96, f"sx{T}x{H}", T, H, f16)
    Wr = (np.random.default_rng(97 + T).standard_normal((E, H)) * 0.05).astype(np.float32)
    gu_b, _ = w16(98, f"sgu{SF}x{H}", 2 * SF + 1, H, f16)
    dn_b, _ = w16(99, f"sdn{H}x{SF}", H, SF, True)
    from test_moe_gpu import _experts_dev
    (g, u, d), _, _ = _experts_dev(gpu, ex)
    gut, dnt = qwq4.w16_tile(to_dev(gu_b, gpu)), qwq4.w16_tile(to_dev(dn_b, gpu))
    dx, dr = to_dev(xb, gpu), to_dev(Wr, gpu)
    out, buf, sv, so = qwq4.moe_decode_with_shared(dr, dx, k, g, u, d, E, F, gut, dnt, SF, out_bf16=False,
                                                   x_f16=f16, yp_f16=True)
    v = qwq4.gemv_w16_tiled(gut, 2 * SF + 1, H, dx, T, f16=f16)
    sh = qwq4.swiglu_gemv_w16_tiled(dnt, H, v, SF, T)
    o2, _ = qwq4.moe_decode(dr, dx, k, g, u, d, E, F, shared=sh, out_bf16=False, x_f16=f16, yp_f16=True)
    assert np.array_equal(host(sv).view(np.uint32), host(v).view(np.uint32))
    assert np.array_equal(host(so).view(np.uint32), host(sh).view(np.uint32))
    assert np.array_equal(host(out).view(np.uint32), host(o2).view(np.uint32))
    ref = oracle.moe(xf, host(buf.logits), k, *ex) + oracle.shared_expert(xf, gu_b, dn_b, f16_gu=f16, f16_down=True)
    assert rel_err(host(out), ref) <= TOL


def _random_block(n, seed):
    """Seeded (T, E, H, F, k, Fs, f16, zeros) within the decode block's limits and a
    few hundred MB of host experts: every router, routing and shared-expert path
    (merged at T = 1, routing launch at 2-4 and 5-8, own launches above 8 or for Fs
    not a multiple of 256)."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        T = int(r.choice([1, 1, 2, 3, 4, 5, 6, 8, 12, 16]))
        E = int(r.choice([8, 16, 48, 64, 128, 256]))
        H = int(r.choice([512, 768, 1024, 1536, 2048, 3072, 4096]))
        F = int(r.choice([128, 256, 384, 512, 768, 1536]))
        if E * F * H > 256 * 1536 * 1024:
            continue
        k = int(r.integers(1, min(8, E) + 1))
        Fs = int(r.choice([256, 512, 1024, 1536, 32 * int(r.integers(1, 49))]))
        out.append((T, E, H, F, k, Fs, bool(r.integers(0, 2)), bool(r.integers(0, 2))))
    return out


@pytest.mark.parametrize("T,E,H,F,k,SF,f16,zeros", _random_block(12, 2036))
def test_moe_decode_with_shared_random_shapes(gpu, T, E, H, F, k, SF, f16, zeros):
    """qw_moe_decode_with_shared over seeded random shapes against its parts as
    separate calls (shared gate/up GEMV, SwiGLU-down GEMV, then qw_moe_decode with
    their output as the shared rows): routing, shared rows and output bit for bit."""
    print(f"moe decode with shared random T={T} E={E} H={H} F={F} k={k} Fs={SF} f16={f16} zeros={zeros}", flush=True)
    ex = synth.experts(3000 + T + E, E, H, F, zeros=zeros)
    xb, _ = rows(3001, f"rx{T}x{H}", T, H, f16)
    Wr = (np.random.default_rng(3002 + E).standard_normal((E, H)) * 0.05).astype(np.float32)
    gu_b, _ = w16(3003, f"rgu{SF}x{H}", 2 * SF + 1, H, f16)
    dn_b, _ = w16(3004, f"rdn{H}x{SF}", H, SF, True)
    from test_moe_gpu import _experts_dev
    (g, u, d), _, _ = _experts_dev(gpu, ex)
    gut, dnt = qwq4.w16_tile(to_dev(gu_b, gpu)), qwq4.w16_tile(to_dev(dn_b, gpu))
    dx, dr = to_dev(xb, gpu), to_dev(Wr, gpu)
    out, buf, sv, so = qwq4.moe_decode_with_shared(dr, dx, k, g, u, d, E, F, gut, dnt, SF, out_bf16=False,
                                                   x_f16=f16, yp_f16=True)
    v = qwq4.gemv_w16_tiled(gut, 2 * SF + 1, H, dx, T, f16=f16)
    if T <= 4:
        sh = qwq4.swiglu_gemv_w16_tiled(dnt, H, v, SF, T)
    else:
        sh = qwq4.gemv_w16_tiled(dnt, H, SF, qwq4.swiglu_gate(v, SF), T)
    o2, b2 = qwq4.moe_decode(dr, dx, k, g, u, d, E, F, shared=sh, out_bf16=False, x_f16=f16, yp_f16=True)
    assert np.array_equal(host(buf.top_e), host(b2.top_e))
    assert np.array_equal(host(buf.top_w).view(np.uint32), host(b2.top_w).view(np.uint32))
    assert np.array_equal(host(sv).view(np.uint32), host(v).view(np.uint32))
    assert np.array_equal(host(so).view(np.uint32), host(sh).view(np.uint32))
    assert np.array_equal(host(out).view(np.uint32), host(o2).view(np.uint32))
