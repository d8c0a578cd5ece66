"""The W4A8 grouped expert GEMMs (qw_moe_experts_w4a8, the role of the reference's
opt-in gpu::moe_experts_w4a8, src/kernels/moe_w4a8.hip:13-215) and their activation
quantiser (qw_quant_rows_i8) against the oracle's restatement of that algorithm:
the quantised rows bit for bit, h and yp within the tolerance (the per-step int32
sums and their fp32 rescale are the oracle's own operations; silu's exp and the fp16
roundings of h and yp can differ by an ulp)."""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, host, rel_err, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("pad", [0, 2])
def test_quant_rows_bit_exact(gpu, oracle, f16, pad):
    """Rows of stride K (16-byte loads, four groups per wave; 444 groups: a partly
    used last block) and of stride K + 2 (the two-elements-per-lane kernel)."""
    r = np.random.default_rng(21)
    R, K = 37, 1536
    v = (r.standard_normal((R, K)) * 4).astype(np.float32)
    v[3, :128] = 0.0
    v[5, 128:256] = 1e-4
    bits = v.astype(np.float16).view(np.uint16) if f16 else synth.bf16_bits(v)
    wide = np.zeros((R, K + pad), np.uint16)
    wide[:, :K] = bits
    q, sc = qwq4.quant_rows_i8(to_dev(wide, gpu)[:, :K], x_f16=f16)
    qr, sr = oracle.quant_rows_i8(bits, f16)
    assert np.array_equal(host(q), qr)
    assert np.array_equal(host(sc).view(np.uint32), sr.view(np.uint32))


def _run(gpu, oracle, E, H, F, k, T, zeros, f16, seed, bias=0.0, slots=None):
    ex = synth.experts(seed, E, H, F, zeros=zeros)
    v = synth.rng(seed, "x").normal(0.0, 1.0, size=(T, H)).astype(np.float32)
    xb = v.astype(np.float16).view(np.uint16) if f16 else synth.bf16_bits(v)
    l = synth.router_logits(seed, "l", T, E, bias_sigma=bias)
    from test_moe_gpu import _experts_dev
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    r = qwq4.moe_route(to_dev(l, gpu), k, tile_m=qwq4.moe_w4a8_tile_m())
    h, yp = qwq4.moe_experts_w4a8(dg, du, dd, r, to_dev(xb, gpu), E, F, x_f16=f16)
    offsets, pair_tok = host(r.offsets), host(r.pair_tok)
    h_ref, yp_ref = oracle.moe_w4a8(xb, f16, *ex, offsets, pair_tok, E, slots=slots)
    hs, ys = host(h).astype(np.float32), host(yp).astype(np.float32)
    if slots is not None:
        hs, ys = hs[slots], ys[slots]
    return hs, ys, h_ref, yp_ref, r


@pytest.mark.parametrize("E,H,F,k,T,zeros,f16", [(8, 256, 128, 2, 12, True, True), (16, 512, 256, 4, 100, False, True),
                                                 (16, 512, 256, 4, 100, True, False), (4, 1024, 512, 1, 300, True, True)])
def test_w4a8_matches_oracle(gpu, oracle, E, H, F, k, T, zeros, f16):
    print(f"w4a8 E={E} H={H} F={F} k={k} T={T} zeros={zeros} f16={f16}", flush=True)
    h, yp, h_ref, yp_ref, r = _run(gpu, oracle, E, H, F, k, T, zeros, f16, 71)
    assert rel_err(h, h_ref) <= TOL
    assert rel_err(yp, yp_ref) <= TOL
    # most h values agree bit for bit (only silu's exp and one fp16 rounding differ)
    assert np.mean(h == h_ref) > 0.9
    counts = host(r.counts)
    assert any(c % 64 for c in counts if c)  # a ragged last tile occurs


def test_w4a8_full_config_sampled(gpu, oracle):
    """Config 5 (4096 tokens, 256 experts, H 4096, F 1536, top-8, biased router) run
    whole on the device; 64 sampled slots (first and last included) against the oracle."""
    E, H, F, k, T = 256, 4096, 1536, 8, 4096
    print("w4a8 full config T=4096", flush=True)
    slots = np.random.default_rng(3).choice(T * k, 64, replace=False)
    slots[:2] = [0, T * k - 1]
    h, yp, h_ref, yp_ref, _ = _run(gpu, oracle, E, H, F, k, T, False, True, 42, bias=0.5, slots=np.sort(slots))
    assert rel_err(h, h_ref) <= TOL
    assert rel_err(yp, yp_ref) <= TOL
