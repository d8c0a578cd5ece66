"""q4 prefill GEMM (qw_q4_gemm) and the grouped expert GEMM against the oracle."""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, bf16_err_ok, host, rel_err, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,N,K", [(1, 256, 512), (200, 384, 1024), (512, 1024, 4096), (333, 4096, 6144)])
def test_gemm_small_full_check(gpu, oracle, T, N, K):
    print(f"gemm T={T} N={N} K={K}", flush=True)
    W, S, Z = synth.q4_weights(51, f"g{N}x{K}", N, K)
    xb, xf = synth.acts(51, f"x{T}x{K}", T, K)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    Y = host(qwq4.gemm(dW, dS, dZ, to_dev(xb, gpu), N, K))
    assert rel_err(Y, oracle.q4_linear(W, S, Z, N, K, xf)) <= TOL


@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 6144)])
@pytest.mark.parametrize("T", [4096, 2048])
def test_gemm_prefill_chunk_sampled(gpu, oracle, N, K, T):
    """4096-token chunk (256 x 256 tiles) and a 2048-token micro-batch (256 x
    256 tiles and 256 x 128 halves, or 256 x 128 only for 6144->4096), bf16 out; checked on sampled tokens and rows
    (fp64 oracle), first and last included."""
    print(f"gemm sampled T={T} N={N} K={K}", flush=True)
    W, S, Z = synth.q4_weights(52, f"p{N}x{K}", N, K)
    xb, xf = synth.acts(52, f"px{K}", T, K)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    Y = host(qwq4.gemm(dW, dS, dZ, to_dev(xb, gpu), N, K, y_bf16=True))
    r = np.random.default_rng(0)
    toks = np.sort(np.unique(np.r_[0, T - 1, r.choice(T, 48, replace=False)]))
    rows = np.sort(np.unique(np.r_[0, N - 1, r.choice(N, 512, replace=False)]))
    ref = oracle.q4_linear(W[rows], S[rows], Z[rows], len(rows), K, xf[toks])
    assert bf16_err_ok(Y[np.ix_(toks, rows)], ref)


@pytest.mark.parametrize("T", [2048, 3072, 2304])
def test_gemm_tile_shapes_bit_identical(gpu, T):
    """A token row's result does not depend on the tile shape that computed it:
    2048 and 3072 tokens of 4096->12288 (whole 256 x 256 rounds plus 256 x 128
    halves in one launch) and 2304 (128 x 256 tiles) against the same rows of a
    4096-token run (256 x 256 tiles only), bit for bit."""
    N, K = 12288, 4096
    print(f"gemm tile shapes T={T}", flush=True)
    W, S, Z = synth.q4_weights(53, f"m{N}x{K}", N, K)
    xb, _ = synth.acts(53, f"mx{K}", 4096, K)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    X = to_dev(xb, gpu)
    Y4 = host(qwq4.gemm(dW, dS, dZ, X, N, K))
    YT = host(qwq4.gemm(dW, dS, dZ, X[:T].contiguous(), N, K))
    assert np.array_equal(YT.view(np.uint32), Y4[:T].view(np.uint32))


def test_gemm_microbatch_fp32_out(gpu, oracle):
    """2048-token micro-batch (256 tokens x 128 weight rows per block) with
    fp32 output, symmetric weights; sampled tokens and rows, first and last
    included."""
    N, K, T = 12288, 4096, 2048
    print("gemm micro-batch fp32 out", flush=True)
    W, S, _ = synth.q4_weights(53, f"m{N}x{K}", N, K, zeros=False)
    xb, xf = synth.acts(53, f"mx{K}", T, K)
    dW, dS, _ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), None, N, K)
    Y = host(qwq4.gemm(dW, dS, None, to_dev(xb, gpu), N, K, y_bf16=False))
    r = np.random.default_rng(1)
    toks = np.sort(np.unique(np.r_[0, T - 1, r.choice(T, 32, replace=False)]))
    rows = np.sort(np.unique(np.r_[0, N - 1, r.choice(N, 512, replace=False)]))
    ref = oracle.q4_linear(W[rows], S[rows], None, len(rows), K, xf[toks])
    assert rel_err(Y[np.ix_(toks, rows)], ref) <= TOL


def _f16_sat(y32):
    """fp32 -> fp16 round to nearest even, finite values beyond +-65504 saturated."""
    y = np.asarray(y32, np.float32)
    fin = np.isfinite(y)
    return np.where(fin, np.clip(y, -65504.0, 65504.0), y).astype(np.float16)


@pytest.mark.parametrize("N,K,T", [(12288, 4096, 4096), (4096, 6144, 2048), (384, 1024, 200)])
def test_gemm_f16_out(gpu, oracle, N, K, T):
    """fp16 Y (the reference's gemm(..., f16_out = true), which the engine's
    prefill passes for most projections): the fp16 rows are the fp32 results
    rounded to nearest even, bit for bit, on fp16 activation rows (the
    engine's) at config-4 sizes, and within the tolerance of the oracle
    (plus fp16's half ulp) on sampled tokens and rows."""
    import torch
    print(f"gemm f16 out T={T} N={N} K={K}", flush=True)
    W, S, Z = synth.q4_weights(54, f"h{N}x{K}", N, K)
    xb, xf = synth.acts(54, f"hx{K}", T, K)
    x16 = xf.astype(np.float16)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    X = torch.from_numpy(x16).to(gpu)
    Y32 = host(qwq4.gemm(dW, dS, dZ, X, N, K))
    Y16 = host(qwq4.gemm(dW, dS, dZ, X, N, K, y_dtype=torch.float16))
    assert Y16.dtype == np.float16
    assert np.array_equal(Y16.view(np.uint16), _f16_sat(Y32).view(np.uint16))
    r = np.random.default_rng(2)
    toks = np.sort(np.unique(np.r_[0, T - 1, r.choice(T, min(T, 32), replace=False)]))
    rows = np.sort(np.unique(np.r_[0, N - 1, r.choice(N, min(N, 512), replace=False)]))
    ref = oracle.q4_linear(W[rows], S[rows], Z[rows], len(rows), K, x16.astype(np.float32)[toks])
    got = Y16[np.ix_(toks, rows)].astype(np.float64)
    bound = TOL * np.max(np.abs(ref)) + 2.0**-11 * np.abs(ref)
    assert np.all(np.abs(got - ref) <= bound)


def test_gemm_f16_out_saturates(gpu):
    """fp16 Y beyond the fp16 range saturates to +-65504 (no infinities)."""
    import torch
    N, K, T = 256, 512, 64
    W, S, Z = synth.q4_weights(55, "sat", N, K)
    S = np.full_like(S, np.float16(60.0).view(np.uint16))
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    X = torch.full((T, K), 100.0, dtype=torch.float16, device=gpu)
    Y32 = host(qwq4.gemm(dW, dS, dZ, X, N, K))
    Y16 = host(qwq4.gemm(dW, dS, dZ, X, N, K, y_dtype=torch.float16))
    assert np.max(np.abs(Y32)) > 65504.0
    assert np.all(np.isfinite(Y16.astype(np.float32)))
    assert np.array_equal(Y16.view(np.uint16), _f16_sat(Y32).view(np.uint16))


# (E, H, F, k, T, zeros, bias): few tokens per expert (one partial tile each,
# some experts empty); many per expert (several tiles, ragged last tile, F
# not a multiple of 256); symmetric weights (no zero tensor).
@pytest.mark.parametrize("yp16", [False, True])
@pytest.mark.parametrize("E,H,F,k,T,zeros,bias", [(16, 512, 256, 4, 300, True, 0.5),
                                                  (8, 256, 384, 2, 1100, True, 1.0),
                                                  (64, 384, 128, 6, 40, False, 0.0)])
def test_grouped_matches_oracle_small(gpu, oracle, E, H, F, k, T, zeros, bias, yp16):
    print(f"grouped E={E} H={H} F={F} k={k} T={T} zeros={zeros} yp16={yp16}", flush=True)
    ex = synth.experts(61, E, H, F, zeros=zeros)
    xb, xf = synth.acts(61, "x", T, H)
    l = synth.router_logits(61, "l", T, E, bias_sigma=bias)
    out, h_ref, yp_ref = oracle.moe(xf, l, k, *ex, want_parts=True)
    from test_moe_gpu import _experts_dev
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    r = qwq4.moe_route(to_dev(l, gpu), k, tile_m=qwq4.moe_grouped_tile_m())
    h, yp = qwq4.moe_experts_grouped(dg, du, dd, r, to_dev(xb, gpu), E, F, yp_f16=yp16)
    assert rel_err(host(h).astype(np.float32), h_ref) <= TOL
    assert rel_err(host(yp).astype(np.float32), yp_ref) <= TOL
    o = host(qwq4.moe_combine(yp, r, H, out_bf16=False))
    assert rel_err(o, out) <= TOL


def test_grouped_full_config_sampled(gpu, oracle):
    """The MoE prefill configuration at full size: 4096 tokens, 256 experts
    (H 4096, F 1536), top-8, router logits with a per-expert bias N(0, 0.5).
    The whole chunk runs on the device (mixed tiles of 32 to 160 slots); 32
    sampled tokens, first and last among them, are checked against the oracle
    (a token's output depends only on its own routing and activation row)."""
    E, H, F, k, T = 256, 4096, 1536, 8, 4096
    print("grouped full config T=4096", flush=True)
    ex = synth.experts(42, E, H, F)
    xb, xf = synth.acts(62, "x", T, H)
    l = synth.router_logits(62, "l", T, E, bias_sigma=0.5)
    from test_moe_gpu import _experts_dev
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    g = -qwq4.moe_grouped_tile_m()
    r = qwq4.moe_route(to_dev(l, gpu), k, tile_m=-g)
    _, yp = qwq4.moe_experts_grouped(dg, du, dd, r, to_dev(xb, gpu), E, F, yp_f16=True)   # as the benchmark runs it
    o = host(qwq4.moe_combine(yp, r, H, out_bf16=False))
    counts = host(r.counts)
    last = [int(c) - 4 * g * max(0, (int(c) - g - 1) // (4 * g)) for c in counts if c > 0]  # last tile's slots
    assert all(any(lo < x <= lo + g for x in last) for lo in (0, g, 2 * g, 3 * g, 4 * g))  # every height occurs
    idx = np.random.default_rng(5).choice(T, 32, replace=False)
    idx[:2] = [0, T - 1]
    ref = oracle.moe(xf[idx], l[idx], k, *ex)
    assert rel_err(o[idx], ref) <= TOL


def _random_gemm_shapes(n, seed=77):
    r = np.random.default_rng(seed)
    return [(int(r.integers(1, 4097)), 16 * int(r.integers(1, 769)), 128 * int(r.integers(1, 49)),
             bool(r.integers(0, 2)), bool(r.integers(0, 2))) for _ in range(n)]


@pytest.mark.parametrize("T,N,K,zeros,y_bf16", _random_gemm_shapes(10))
def test_gemm_random_shapes(gpu, oracle, T, N, K, zeros, y_bf16):
    """Seeded random shapes (T up to 4096, N a multiple of 16 up to 12288, K a
    multiple of 128 up to 6144, with and without zeros, fp32 or bf16 out):
    the tile-shape choice and ragged tile edges, on sampled tokens and rows
    (first and last included)."""
    print(f"gemm random T={T} N={N} K={K} zeros={zeros} bf16={y_bf16}", flush=True)
    W, S, Z = synth.q4_weights(T + N, f"r{N}x{K}", N, K, zeros)
    xb, xf = synth.acts(T + K, f"rx{T}x{K}", T, K)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    Y = host(qwq4.gemm(dW, dS, dZ, to_dev(xb, gpu), N, K, y_bf16=y_bf16))
    r = np.random.default_rng(T)
    toks = np.sort(np.unique(np.r_[0, T - 1, r.choice(T, min(T, 24), replace=False)]))
    rows = np.sort(np.unique(np.r_[0, N - 1, r.choice(N, min(N, 256), replace=False)]))
    ref = oracle.q4_linear(W[rows], S[rows], Z[rows] if zeros else None, len(rows), K, xf[toks])
    got = Y[np.ix_(toks, rows)]
    if y_bf16:
        assert bf16_err_ok(got, ref)
    else:
        assert rel_err(got, ref) <= TOL


def test_gemm_saturation_and_nonfinite(gpu, oracle):
    """Stated behaviour of the fp16 activation path: finite |x| > 65504
    saturates to +-65504 (output equals the oracle on the clipped x), and NaN
    or infinity in a row is carried into that row's outputs, not replaced."""
    T, N, K = 8, 256, 512
    W, S, Z = synth.q4_weights(57, "sat", N, K)
    xf = np.random.default_rng(57).standard_normal((T, K)).astype(np.float32)
    xf[1, 3] = 1.0e6
    xf[2, 100] = -3.0e5
    xb = synth.bf16_bits(xf)
    xf = synth.bf16_to_f32(xb)
    xb_bad = xb.copy()
    xb_bad[5, 7] = 0x7fc0          # NaN
    xb_bad[6, 9] = 0x7f80          # +inf
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    Y = host(qwq4.gemm(dW, dS, dZ, to_dev(xb_bad, gpu), N, K))
    clipped = np.clip(xf, -65504.0, 65504.0)
    ok = [0, 1, 2, 3, 4, 7]
    ref = oracle.q4_linear(W, S, Z, N, K, clipped[ok])
    assert rel_err(Y[ok], ref) <= TOL
    assert np.all(np.isnan(Y[5]))
    assert np.all(~np.isfinite(Y[6]))
