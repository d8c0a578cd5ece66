"""fp16 activation rows (x_f16): the reference engine's decode and prefill rows
are fp16 (src/kernels/gemv.hpp:11-14, src/engine/decode.hip:65-70), so every
product entry point takes them as they are. Checked against the oracle on the
exact fp32 values of the fp16 inputs."""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, bf16_err_ok, host, rel_err, to_dev

pytestmark = pytest.mark.gpu


def f16_acts(seed, name, M, K, scale=1.0):
    """fp16 bits [M, K] of N(0, scale^2) and their exact fp32 values."""
    v = (synth.rng(seed, name).normal(0.0, scale, size=(M, K))).astype(np.float16)
    return v.view(np.uint16), v.astype(np.float32)


@pytest.mark.parametrize("N,K,M,zeros", [(4096, 4096, 1, True), (4096, 4096, 2, True), (4096, 4096, 4, False),
                                         (4096, 4096, 8, True), (12288, 4096, 1, True), (12288, 4096, 6, True),
                                         (4096, 6144, 4, True), (1024, 2048, 17, True), (1008, 640, 3, False)])
def test_gemv_fp16_rows(gpu, oracle, N, K, M, zeros):
    print(f"gemv fp16 N={N} K={K} M={M}", flush=True)
    W, S, Z = synth.q4_weights(91, f"h{N}x{K}", N, K, zeros)
    xh, xf = f16_acts(91, f"hx{M}x{K}", M, K)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    y = host(qwq4.gemv(dW, dS, dZ, to_dev(xh, gpu), N, K, M, x_f16=True))
    assert rel_err(y, oracle.q4_linear(W, S, Z, N, K, xf)) <= TOL


def test_gemv_fp16_large_magnitudes(gpu, oracle):
    """fp16 rows near the top of the fp16 range: every product stays exact
    (fp16 x times 1024 + 16 q), sums in fp32."""
    N, K, M = 2048, 4096, 2
    W, S, Z = synth.q4_weights(92, "hl", N, K)
    xh, xf = f16_acts(92, "hlx", M, K, scale=4000.0)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    y = host(qwq4.gemv(dW, dS, dZ, to_dev(xh, gpu), N, K, M, x_f16=True))
    assert rel_err(y, oracle.q4_linear(W, S, Z, N, K, xf)) <= TOL


@pytest.mark.parametrize("T,N,K", [(333, 4096, 6144), (4096, 12288, 4096)])
def test_gemm_fp16_rows(gpu, oracle, T, N, K):
    """fp16 rows go to the MFMAs without the pre-pass (no workspace)."""
    print(f"gemm fp16 T={T} N={N} K={K}", flush=True)
    W, S, Z = synth.q4_weights(93, f"gh{N}x{K}", N, K)
    xh, xf = f16_acts(93, f"ghx{T}x{K}", T, K)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    Y = host(qwq4.gemm(dW, dS, dZ, to_dev(xh, gpu), N, K, y_bf16=True, x_f16=True))
    r = np.random.default_rng(1)
    toks = np.sort(np.unique(np.r_[0, T - 1, r.choice(T, min(T, 40), replace=False)]))
    rows = np.sort(np.unique(np.r_[0, N - 1, r.choice(N, 384, replace=False)]))
    ref = oracle.q4_linear(W[rows], S[rows], Z[rows], len(rows), K, xf[toks])
    assert bf16_err_ok(Y[np.ix_(toks, rows)], ref)


@pytest.mark.parametrize("T", [1, 5, 32])
def test_moe_experts_gemv_fp16_rows(gpu, oracle, T):
    E, H, F, k = 64, 1024, 512, 8
    print(f"moe gemv fp16 T={T}", flush=True)
    ex = synth.experts(94, E, H, F)
    xh, xf = f16_acts(94, f"mx{T}", T, H)
    l = synth.router_logits(94, f"ml{T}", T, E)
    out, h_ref, yp_ref = oracle.moe(xf, l, k, *ex, want_parts=True)
    from test_moe_gpu import _experts_dev
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    r = qwq4.moe_route(to_dev(l, gpu), k)
    h, yp = qwq4.moe_experts_gemv(dg, du, dd, r, to_dev(xh, gpu), E, F, x_f16=True)
    assert rel_err(host(h).astype(np.float32), h_ref) <= TOL
    assert rel_err(host(yp), yp_ref) <= TOL


def test_moe_grouped_fp16_rows(gpu, oracle):
    E, H, F, k, T = 16, 512, 256, 4, 300
    ex = synth.experts(95, E, H, F)
    xh, xf = f16_acts(95, "gx", T, H)
    l = synth.router_logits(95, "gl", T, E, bias_sigma=0.5)
    out, h_ref, yp_ref = oracle.moe(xf, l, k, *ex, want_parts=True)
    from test_moe_gpu import _experts_dev
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    r = qwq4.moe_route(to_dev(l, gpu), k, tile_m=qwq4.moe_grouped_tile_m())
    h, yp = qwq4.moe_experts_grouped(dg, du, dd, r, to_dev(xh, gpu), E, F, x_f16=True)
    assert rel_err(host(h).astype(np.float32), h_ref) <= TOL
    assert rel_err(host(yp), yp_ref) <= TOL


@pytest.mark.parametrize("T", [1, 6])
def test_moe_decode_fp16_rows(gpu, oracle, T):
    E, H, F, k = 64, 1024, 256, 4
    print(f"moe decode fp16 T={T}", flush=True)
    ex = synth.experts(96, E, H, F)
    xh, xf = f16_acts(96, f"dx{T}", T, H)
    Wr = (np.random.default_rng(96).standard_normal((E, H)) * 0.05).astype(np.float32)
    from test_moe_gpu import _experts_dev
    (g, u, d), _, _ = _experts_dev(gpu, ex)
    out, buf = qwq4.moe_decode(to_dev(Wr, gpu), to_dev(xh, gpu), k, g, u, d, E, F, out_bf16=False, x_f16=True)
    logits = host(buf.logits)
    assert rel_err(logits, xf.astype(np.float64) @ Wr.astype(np.float64).T) <= 1e-5
    te, _ = oracle.route(logits, k)
    assert np.array_equal(host(buf.top_e), te)
    assert rel_err(host(out), oracle.moe(xf, logits, k, *ex)) <= TOL
