"""Bit-exact format surface: unpack, dequant, engine-order conversion."""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import host, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("zeros", [False, True])
def test_unpack_and_dequant_bit_exact(gpu, oracle, zeros):
    N, K = 777, 1536
    W, S, Z = synth.q4_weights(21, "f", N, K, zeros)
    dW = to_dev(W, gpu)
    assert np.array_equal(host(qwq4.unpack(dW, N, K)), oracle.q4_unpack(W, N, K))
    d = host(qwq4.dequant(dW, to_dev(S, gpu), to_dev(Z, gpu), N, K))
    assert np.array_equal(d.view(np.uint32), oracle.q4_dequant(W, S, Z, N, K).view(np.uint32))


def test_from_engine_order(gpu, oracle):
    import os
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
    got = host(qwq4.from_engine_order(to_dev(gold["words_eng"], gpu)), np.uint32)
    assert np.array_equal(got, gold["words_in"])


@pytest.mark.parametrize("N,K,zeros", [(16, 128, True), (48, 640, True), (1024, 4096, False), (272, 6144, True)])
def test_tile_matches_oracle_and_round_trips(gpu, oracle, N, K, zeros):
    W, S, Z = synth.q4_weights(22, f"t{N}x{K}", N, K, zeros)
    dW, dS, dZ = to_dev(W, gpu), to_dev(S, gpu), to_dev(Z, gpu)
    Wt, St, Zt = qwq4.tile(dW, dS, dZ, N, K)
    oW, oS, oZ = oracle.q4_tile(W, S, Z, N, K)
    assert np.array_equal(host(Wt, np.uint32), oW)
    assert np.array_equal(host(St, np.uint16), oS)
    if zeros:
        assert np.array_equal(host(Zt, np.uint16), oZ)
    bW, bS, bZ = qwq4.untile(Wt, St, Zt, N, K)
    assert np.array_equal(host(bW, np.uint32), W)
    assert np.array_equal(host(bS, np.uint16), S)
    if zeros:
        assert np.array_equal(host(bZ, np.uint32), Z)
