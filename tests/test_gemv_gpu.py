"""q4 GEMV (qw_q4_gemv) against the CPU oracle (decode projections, LM head)."""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, bf16_err_ok, host, rel_err, to_dev

pytestmark = pytest.mark.gpu

SHAPES = [(256, 512), (384, 128), (4096, 4096), (12288, 4096), (4096, 6144), (1536, 4096), (4096, 1536)]


def _setup(dev, N, K, M, zeros=True, seed=11):
    W, S, Z = synth.q4_weights(seed, f"w{N}x{K}", N, K, zeros)
    xb, xf = synth.acts(seed, f"x{M}x{K}", M, K)
    dW, dS, dZ = qwq4.tile(to_dev(W, dev), to_dev(S, dev), to_dev(Z, dev), N, K)
    return (W, S, Z, xb, xf), (dW, dS, dZ, to_dev(xb, dev))


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 2, 4, 6, 8])
def test_gemv_fp32(gpu, oracle, N, K, M):
    print(f"gemv N={N} K={K} M={M}", flush=True)
    (W, S, Z, xb, xf), (dW, dS, dZ, dx) = _setup(gpu, N, K, M)
    y = host(qwq4.gemv(dW, dS, dZ, dx, N, K, M))
    r = oracle.q4_linear(W, S, Z, N, K, xf)
    assert rel_err(y, r) <= TOL


@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 6144)])
@pytest.mark.parametrize("M", [3, 5, 7])
def test_gemv_odd_batches(gpu, oracle, N, K, M):
    """Batches between the benchmarked ones (packed corrections with clamped
    rows, register or direct activation staging)."""
    print(f"gemv odd N={N} K={K} M={M}", flush=True)
    (W, S, Z, xb, xf), (dW, dS, dZ, dx) = _setup(gpu, N, K, M, seed=13)
    y = host(qwq4.gemv(dW, dS, dZ, dx, N, K, M))
    r = oracle.q4_linear(W, S, Z, N, K, xf)
    assert rel_err(y, r) <= TOL


@pytest.mark.parametrize("M,K", [(1, 2048), (8, 2048), (16, 2048), (17, 2048), (32, 2048), (32, 6144), (13, 640)])
def test_gemv_symmetric_and_wide(gpu, oracle, M, K):
    N = 1024
    (W, S, Z, xb, xf), (dW, dS, dZ, dx) = _setup(gpu, N, K, M, zeros=False)
    y = host(qwq4.gemv(dW, dS, dZ, dx, N, K, M))
    r = oracle.q4_linear(W, S, None, N, K, xf)
    assert rel_err(y, r) <= TOL


def test_gemv_bf16_out_is_rne_of_fp32(gpu, oracle):
    N, K, M = 4096, 4096, 4
    (W, S, Z, xb, xf), (dW, dS, dZ, dx) = _setup(gpu, N, K, M)
    y32 = host(qwq4.gemv(dW, dS, dZ, dx, N, K, M))
    y16 = qwq4.gemv(dW, dS, dZ, dx, N, K, M, y_bf16=True)
    bits = host(y16).view(np.uint32) >> 16
    assert np.array_equal(bits.astype(np.uint16), synth.bf16_bits(y32))
    assert bf16_err_ok(host(y16), oracle.q4_linear(W, S, Z, N, K, xf))


@pytest.mark.parametrize("M", [1, 2, 4, 6, 8])
def test_gemv_lm_head(gpu, oracle, M):
    """The LM head at every benchmarked batch: batches 4-8 run the persistent
    prefetching kernel (blocks take items grid-stride), 1-2 one item per
    block over many rounds."""
    N, K = 151936, 4096
    print(f"gemv lm head M={M}", flush=True)
    (W, S, Z, xb, xf), (dW, dS, dZ, dx) = _setup(gpu, N, K, M)
    y = host(qwq4.gemv(dW, dS, dZ, dx, N, K, M, y_bf16=True))
    r = oracle.q4_linear(W, S, Z, N, K, xf)
    assert bf16_err_ok(y, r)


@pytest.mark.parametrize("N,K,rpg,M", [(1296, 1024, 324, 1), (1296, 1024, 324, 8), (12288, 4096, 3076, 1),
                                        (12288, 4096, 3076, 8), (4096, 6144, 2048, 4), (2000, 512, 130, 3),
                                        (4096, 4096, 64, 32)])
def test_gemv_row_slices(gpu, oracle, N, K, rpg, M):
    """gemv_rows' row grouping (rpg: row n reads activation slice n // rpg,
    src/kernels/gemv.hip:16-17) on q4 weights: the engine's hyper-connection
    shape (4 slices of 324 rows: tiles straddle two slices), config 2's
    4096->12288 in 4 slices of 3076 rows (not a multiple of 16) at batches 1
    and 8, slices of whole tiles, and 64 slices at batch 32 (two launches
    per slice). Rows strided over every slice, accumulated into y; against
    the oracle; rows past N untouched; each row equal, bit for bit, to the
    ungrouped GEMV of its own slice."""
    import torch
    print(f"gemv rpg N={N} K={K} rpg={rpg} M={M}", flush=True)
    ns = (N + rpg - 1) // rpg
    W, S, Z = synth.q4_weights(15, f"r{N}x{K}", N, K)
    xs = ns * K + 8
    xb, xf = synth.acts(15, f"rx{M}x{xs}", M, xs)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    dx = to_dev(xb, gpu)
    y = torch.full((M, N + 16), 0.5, dtype=torch.float32, device=gpu)
    qwq4.gemv(dW, dS, dZ, dx, N, K, M, y=y, accumulate=True, xs=xs, ys=N + 16, rpg=rpg)
    yh = host(y)
    assert np.all(yh[:, N:] == 0.5)
    ref = oracle.q4_linear(W, S, Z, N, K, xf[:, :ns * K], rpg=rpg) + 0.5
    assert rel_err(yh[:, :N], ref) <= TOL
    # each slice's rows equal the plain GEMV of that slice (same arithmetic)
    for sl in sorted({0, ns - 1, ns // 2}):
        y1 = host(qwq4.gemv(dW, dS, dZ, dx[:, sl * K:].contiguous(), N, K, M))
        r0, r1 = sl * rpg, min(N, (sl + 1) * rpg)
        assert np.array_equal((y1[:, r0:r1] + np.float32(0.5)).view(np.uint32), yh[:, r0:r1].view(np.uint32))


def test_gemv_rows_independent_bit_exact(gpu):
    N, K, M = 2048, 4096, 8
    (W, S, Z, xb, xf), (dW, dS, dZ, dx) = _setup(gpu, N, K, M)
    y8 = host(qwq4.gemv(dW, dS, dZ, dx, N, K, M))
    for m in (0, 5, 7):
        y1 = host(qwq4.gemv(dW, dS, dZ, dx[m:m + 1].contiguous(), N, K, 1))
        assert np.array_equal(y1[0].view(np.uint32), y8[m].view(np.uint32))


def test_gemv_strides_accumulate_and_guard(gpu, oracle):
    import torch
    N, K, M = 1008, 1024, 3   # N not a multiple of 128
    (W, S, Z, xb, xf), (dW, dS, dZ, dx) = _setup(gpu, N, K, M)
    xs = K + 64
    xpad = torch.zeros((M, xs), dtype=torch.int16, device=gpu)
    xpad[:, :K] = dx
    ys = N + 24
    y = torch.full((M, ys), 12345.0, device=gpu)
    y[:, :N] = 1.5
    qwq4.gemv(dW, dS, dZ, xpad, N, K, M, y=y, accumulate=True, xs=xs, ys=ys)
    yh = host(y)
    assert np.all(yh[:, N:] == 12345.0)  # no stray writes past N
    r = oracle.q4_linear(W, S, Z, N, K, xf) + 1.5
    assert rel_err(yh[:, :N], r) <= TOL


def test_gemv_special_inputs(gpu, oracle):
    import torch
    N, K = 512, 1024
    W, S, Z = synth.q4_weights(12, "sp", N, K)
    dW, dS, dZ = qwq4.tile(to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu), N, K)
    x = np.zeros((2, K), np.float32)
    x[1, 777] = 1.0
    y = host(qwq4.gemv(dW, dS, dZ, to_dev(synth.bf16_bits(x), gpu), N, K, 2))
    assert np.all(y[0] == 0)
    deq = oracle.q4_dequant(W, S, Z, N, K)
    assert np.array_equal(y[1], deq[:, 777])  # one-hot: a column, exactly


def _random_shapes(n, seed=2024):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        out.append((16 * int(r.integers(1, 641)), 128 * int(r.integers(1, 65)), int(r.integers(1, 33)),
                    bool(r.integers(0, 2)), bool(r.integers(0, 2))))
    return out


@pytest.mark.parametrize("N,K,M,zeros,y_bf16", _random_shapes(16))
def test_gemv_random_shapes(gpu, oracle, N, K, M, zeros, y_bf16):
    """Seeded random shapes (N a multiple of 16 up to 10240, K a multiple of
    128 up to 8192, batch 1-32, with and without zeros, fp32 or bf16 out):
    exercises the launch-shape choices (K split, block width, register or
    direct staging, one round or persistent, row-split launches) against
    the oracle."""
    print(f"gemv random N={N} K={K} M={M} zeros={zeros} bf16={y_bf16}", flush=True)
    (W, S, Z, xb, xf), (dW, dS, dZ, dx) = _setup(gpu, N, K, M, zeros=zeros, seed=N + K + M)
    y = host(qwq4.gemv(dW, dS, dZ, dx, N, K, M, y_bf16=y_bf16))
    r = oracle.q4_linear(W, S, Z if zeros else None, N, K, xf)
    if y_bf16:
        assert bf16_err_ok(y, r)
    else:
        assert rel_err(y, r) <= TOL


@pytest.mark.gpu
def test_read_probe_runs():
    """The measurement aid the bench times beside the GEMV: launches and
    rejects sizes that are not whole 32 KB blocks."""
    import torch
    t = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    qwq4.read_probe(t)
    qwq4.read_probe()
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError):
        qwq4.read_probe(t[:1000])
