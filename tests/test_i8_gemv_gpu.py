"""qw_i8_gemv (the role of gpu::gemv_rows_i8, src/kernels/gemv.hip:75-136) against
the oracle: weights quantised by the oracle's quantize_rows_i8 (pinned to the
reference's own quantiser by tests/test_oracle.py), outputs against the fp64
product (the reference's own check, tests/gpu/test_gemv.hip:93-104), integer
cases bit-exact, grouped rows (rpg) as the engine's hyper-connection down
projection uses them (src/engine/decode.hip:52-58)."""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, bf16_err_ok, host, rel_err, to_dev

pytestmark = pytest.mark.gpu


def quantised(oracle, seed, N, K, group):
    w = synth.rng(seed, f"i8w{N}x{K}").normal(0.0, 0.05, size=(N, K)).astype(np.float16)
    return oracle.quantize_rows_i8(w.view(np.uint16), group)


def f16_rows(seed, name, M, K):
    return synth.rng(seed, name).normal(0.0, 1.0, size=(M, K)).astype(np.float16).view(np.uint16)


def run(gpu, W8, S, x16, M, group, rpg=0, xs=None, **kw):
    N, K = W8.shape
    Wt, St = qwq4.i8_tile(to_dev(W8, gpu), to_dev(S, gpu), group)
    return host(qwq4.gemv_i8(Wt, St, N, K, to_dev(x16, gpu), M, group=group, rpg=rpg, xs=xs, **kw))


@pytest.mark.parametrize("group", [32, 16])
@pytest.mark.parametrize("N,K,M", [(4096, 4096, 1), (4096, 4096, 2), (4096, 4096, 4), (4096, 4096, 8),
                                   (1024, 6144, 3), (100, 64, 5), (333, 1024, 16), (512, 2048, 17), (256, 4096, 32)])
def test_i8_gemv(gpu, oracle, group, N, K, M):
    print(f"i8 gemv group={group} N={N} K={K} M={M}", flush=True)
    W8, S = quantised(oracle, 91, N, K, group)
    x16 = f16_rows(91, f"x{M}x{K}", M, K)
    y = run(gpu, W8, S, x16, M, group)
    assert rel_err(y, oracle.i8_linear_f64(W8, S, x16, M, group=group)) <= TOL


@pytest.mark.parametrize("group", [32, 16])
def test_i8_gemv_integer_exact(gpu, group):
    """Integer activations and power-of-two scales: every product and partial sum is
    an exact fp32 integer, so any pairing of a weight with the wrong activation, or a
    group with the wrong scale, changes the result; the output is bit-exact."""
    rng = np.random.default_rng(5)
    N, K, M = 272, 1024, 6
    W8 = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
    S = np.ldexp(1.0, rng.integers(-3, 4, size=(N, K // group))).astype(np.float32)
    x = rng.integers(-8, 9, size=(M, K)).astype(np.float16)
    y = run(gpu, W8, S, x.view(np.uint16), M, group)
    ref = np.einsum("nk,mk->mn", (W8.astype(np.float64) * np.repeat(S, group, axis=1)), x.astype(np.float64))
    assert np.array_equal(y, ref.astype(np.float32))


@pytest.mark.parametrize("group", [32, 16])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_i8_gemv_grouped_rows(gpu, oracle, group, M):
    """rpg = 324 rows per activation slice (the engine's HC_DOWN): 16-row tiles that
    straddle two slices; and rpg = 64 (whole tiles)."""
    HC, SH = 4, 1024
    for rpg in (324, 64):
        N = HC * rpg
        print(f"i8 gemv grouped group={group} M={M} rpg={rpg}", flush=True)
        W8, S = quantised(oracle, 92, N, SH, group)
        x16 = f16_rows(92, f"xg{M}", M, HC * SH)
        y = run(gpu, W8, S, x16, M, group, rpg=rpg, xs=HC * SH)
        assert rel_err(y, oracle.i8_linear_f64(W8, S, x16, M, xs=HC * SH, rpg=rpg, group=group)) <= TOL


def test_i8_gemv_rows_independent(gpu, oracle):
    """A token row's result does not depend on the batch it is in (bit for bit)."""
    N, K = 1000, 4096
    W8, S = quantised(oracle, 93, N, K, 32)
    x16 = f16_rows(93, "xr", 8, K)
    y8 = run(gpu, W8, S, x16, 8, 32)
    for m in (0, 5, 7):
        y1 = run(gpu, W8, S, np.ascontiguousarray(x16[m:m + 1]), 1, 32)
        assert np.array_equal(y1[0].view(np.uint32), y8[m].view(np.uint32))


def test_i8_gemv_strides_bf16_out_and_accumulate(gpu, oracle):
    import torch
    N, K, M = 500, 1024, 5
    W8, S = quantised(oracle, 94, N, K, 32)
    x16 = f16_rows(94, "xs", M, K)
    ref = oracle.i8_linear_f64(W8, S, x16, M, group=32)
    xp = np.zeros((M, K + 64), np.uint16)
    xp[:, :K] = x16
    y = torch.full((M, N + 8), 0.5, dtype=torch.float32, device=gpu)
    Wt, St = qwq4.i8_tile(to_dev(W8, gpu), to_dev(S, gpu), 32)
    qwq4.gemv_i8(Wt, St, N, K, to_dev(xp, gpu), M, y=y, accumulate=True, xs=K + 64, ys=N + 8)
    yh = host(y)
    assert np.all(yh[:, N:] == 0.5)
    assert rel_err(yh[:, :N], ref + 0.5) <= TOL
    yb = run(gpu, W8, S, x16, M, 32, y_bf16=True)
    assert bf16_err_ok(yb, ref)




@pytest.mark.parametrize("group", [32, 16])
def test_i8_tile_layout(gpu, group):
    """The kernel format against a numpy restatement of its definition (qw_i8_tile's
    comment in i8_gemv.hip), with a ragged last tile (rows past N zero)."""
    rng = np.random.default_rng(7)
    N, K = 37, 192
    W8 = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
    S = rng.random((N, K // group), dtype=np.float32)
    Wt, St = qwq4.i8_tile(to_dev(W8, gpu), to_dev(S, gpu), group)
    tiles, steps = (N + 15) // 16, K // 64
    Wp = np.zeros((tiles * 16, K), np.int8)
    Wp[:N] = W8
    Sp = np.zeros((tiles * 16, K // group), np.float32)
    Sp[:N] = S
    r = Wp.reshape(tiles, 16, steps, 64)  # [tile][n][step][k]
    if group == 32:
        q = np.arange(4)
        a = np.stack([r[:, :, :, 8 * j:8 * j + 8] for j in q], axis=2)  # [tile][n][q][step][8]
        b = np.stack([r[:, :, :, 32 + 8 * j:40 + 8 * j] for j in q], axis=2)
        e = np.concatenate([a, b], axis=-1)  # [tile][n][q][step][16]
    else:
        e = np.stack([np.concatenate([r[:, :, :, 16 * g + 4 * j:16 * g + 4 * j + 4] for g in range(4)], axis=-1)
                      for j in range(4)], axis=2)
    want = e.transpose(0, 3, 2, 1, 4)  # [tile][step][q][n][16] = lane 16 q + n
    assert np.array_equal(host(Wt).view(np.int8).reshape(want.shape), want)
    sps = 64 // group
    ws = Sp.reshape(tiles, 16, steps, sps).transpose(0, 2, 1, 3)
    assert np.array_equal(host(St).reshape(ws.shape), ws)
