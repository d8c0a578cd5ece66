"""MoE decode path: routing (bit-exact), gathered expert GEMVs, combine."""
import numpy as np
import pytest

import qwq4
from qwq4 import synth
from _gpu_util import TOL, bf16_err_ok, host, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _experts_dev(dev, ex):
    gate, up, down = ex
    E, F, H = gate[0].shape[0], gate[0].shape[1], gate[0].shape[2] * 8
    out = []
    for (W, S, Z), rows, K in ((gate, F, H), (up, F, H), (down, H, F)):
        out.append(qwq4.tile_experts(to_dev(W, dev), to_dev(S, dev), to_dev(Z, dev), rows, K))
    return out, E, F


@pytest.mark.parametrize("T,E,k", [(1, 256, 8), (7, 256, 8), (32, 256, 8), (64, 128, 4), (100, 512, 10),
                                   (4096, 256, 8), (9001, 256, 8), (130, 1024, 64)])
def test_route_bit_exact(gpu, oracle, T, E, k):
    print(f"route T={T} E={E} k={k}", flush=True)
    l = synth.router_logits(31, f"l{T}", T, E, bias_sigma=0.5 if T > 64 else 0.0)
    if T == 7:
        l[2, :] = 0.0          # all-equal logits: ties to the lower index
        l[3, [5, 9, 200]] = 9.0
    r = qwq4.moe_route(to_dev(l, gpu), k, tile_m=32 if T > 64 else 0)
    te, tw = oracle.route(l, k)
    assert np.array_equal(host(r.top_e), te)
    # the device evaluates the C library's expf algorithm: weights bit-exact
    assert np.array_equal(host(r.top_w).view(np.uint32), tw.view(np.uint32))
    counts, offsets, tok_slot, pair_tok = oracle.moe_slots(te, E)
    assert np.array_equal(host(r.counts), counts)
    assert np.array_equal(host(r.offsets), offsets)
    assert np.array_equal(host(r.tok_slot), tok_slot)
    assert np.array_equal(host(r.pair_tok), pair_tok)
    na = int(host(r.n_active)[0])
    assert np.array_equal(host(r.active)[:na], np.nonzero(counts)[0])
    if T > 64:
        nt = int(host(r.n_tiles)[0])
        want = [(e, m0) for e in range(E) for m0 in range(0, counts[e], 32)]
        got = list(zip(host(r.tile_e)[:nt], host(r.tile_m0)[:nt]))
        assert got == want


# Adjacent floats (d_small, d_large) = bit patterns (u, u - 1) in [-1, 0)
# where the C library's expf and the correctly rounded exp disagree on
# whether exp(d_small) == exp(d_large): a tie under one rounding and not under
# the other, so the (p desc, index asc) order differs. An exhaustive
# comparison of the two over [-4, 0) finds 127,332 such pairs, none below -1;
# these are the first two of each binade from 2^-6 up (the tie flag is
# glibc's). tests/test_oracle.py checks them against the host's expf.
EXPF_TIE_PAIRS = [
    (0xbc8000bf, True), (0xbc8000c0, False), (0xbd000aa1, True), (0xbd000aa2, False),
    (0xbd801976, True), (0xbd801977, False), (0xbe0000d8, True), (0xbe0000d9, False),
    (0xbe801e5d, True), (0xbe801e5e, False), (0xbf001f30, True), (0xbf001f31, False),
]


def _f32(u):
    return np.array([u], np.uint32).view(np.float32)[0]


@pytest.mark.parametrize("k", [2, 3])
def test_route_expf_tie_order(gpu, oracle, k):
    """Adversarial routing: the larger of two logits sits at the higher
    index, and the two exponentials tie under the C library's expf but not
    under the correctly rounded exp (or the reverse). The reference orders by
    (p desc, index asc), so the pick depends on that rounding: the device must
    choose what the CPU path (glibc's expf) chooses."""
    rows = []
    for u, _ in EXPF_TIE_PAIRS:
        for lead in (0.0, 0.25):
            row = np.full(16, -8.0, np.float32)
            row[0] = lead            # the maximum (lead 0: d exact; 0.25: shifted copies)
            row[5] = lead + _f32(u)        # d_small, lower index
            row[9] = lead + _f32(u - 1)    # d_large, higher index
            row[12] = lead + _f32(u)       # a third copy of d_small
            rows.append(row)
    l = np.stack(rows)
    r = qwq4.moe_route(to_dev(l, gpu), k)
    te, tw = oracle.route(l, k)
    assert np.array_equal(host(r.top_e), te)
    assert np.array_equal(host(r.top_w).view(np.uint32), tw.view(np.uint32))


def test_route_weights_bit_exact_dense(gpu, oracle):
    """Every expert selected (k = E) over logits near the maximum, where most
    exponentials are computed: the weights p / sum p equal the CPU path's bit
    for bit, so every p does."""
    T, E = 512, 64
    r0 = np.random.default_rng(5)
    l = (r0.uniform(-4.0, 0.0, size=(T, E)) + r0.normal(0.0, 0.001, size=(T, 1))).astype(np.float32)
    r = qwq4.moe_route(to_dev(l, gpu), E)
    te, tw = oracle.route(l, E)
    assert np.array_equal(host(r.top_e), te)
    assert np.array_equal(host(r.top_w).view(np.uint32), tw.view(np.uint32))


def _mixed_tiles(counts, g):
    """(expert, m0) of a mixed tile list (tile_m = -g) over per-expert counts."""
    out = []
    for e, c in enumerate(counts):
        m0 = 0
        while m0 < c:
            out.append((e, m0))
            rem = c - m0
            m0 += 4 * g if rem > 5 * g else -(-rem // g) * g
    return out


@pytest.mark.parametrize("T,E,k", [(300, 16, 4), (1100, 8, 2), (4096, 256, 8)])
def test_route_mixed_tiles(gpu, T, E, k):
    print(f"route mixed tiles T={T} E={E} k={k}", flush=True)
    l = synth.router_logits(33, f"m{T}", T, E, bias_sigma=1.0)
    g = -qwq4.moe_grouped_tile_m()
    r = qwq4.moe_route(to_dev(l, gpu), k, tile_m=-g)
    counts = host(r.counts)
    want = _mixed_tiles(counts, g)
    nt = int(host(r.n_tiles)[0])
    assert nt <= T * k // g + E
    got = list(zip(host(r.tile_e)[:nt].tolist(), host(r.tile_m0)[:nt].tolist()))
    assert got == want
    # the heights cover every remainder class at these sizes
    rems = {int(counts[e]) - m0 for e, m0 in want}
    heights = {(x - 1) // g for x in rems if x <= 5 * g}  # the last tiles' height classes
    assert len(heights) == 5 if T >= 4096 else len(heights) >= 3  # every height at full size


@pytest.mark.parametrize("T,zeros", [(1, True), (2, True), (4, False), (8, True), (16, True), (17, False),
                                     (32, True)])
def test_experts_gemv_and_combine(gpu, oracle, T, zeros):
    E, H, F, k = 64, 1024, 512, 8
    print(f"moe gemv T={T}", flush=True)
    ex = synth.experts(41, E, H, F, zeros=zeros)
    xb, xf = synth.acts(41, f"x{T}", T, H)
    l = synth.router_logits(41, f"l{T}", T, E)
    out, h_ref, yp_ref = oracle.moe(xf, l, k, *ex, want_parts=True)
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    dx = to_dev(xb, gpu)
    r = qwq4.moe_route(to_dev(l, gpu), k)
    h, yp = qwq4.moe_experts_gemv(dg, du, dd, r, dx, E, F)
    hh = host(h).astype(np.float32)
    assert rel_err(hh, h_ref) <= TOL
    assert rel_err(host(yp), yp_ref) <= TOL
    o32 = host(qwq4.moe_combine(yp, r, H, out_bf16=False))
    assert rel_err(o32, out) <= TOL
    o16 = host(qwq4.moe_combine(yp, r, H, out_bf16=True))
    assert bf16_err_ok(o16, out)


def test_experts_full_config(gpu, oracle):
    """256 experts, H=4096, F=1536, top-8, batch 8, symmetric and zero-point weights."""
    E, H, F, k, T = 256, 4096, 1536, 8, 8
    ex = synth.experts(42, E, H, F)
    xb, xf = synth.acts(42, "x", T, H)
    l = synth.router_logits(42, "l", T, E)
    out = oracle.moe(xf, l, k, *ex)
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    r = qwq4.moe_route(to_dev(l, gpu), k)
    h, yp = qwq4.moe_experts_gemv(dg, du, dd, r, to_dev(xb, gpu), E, F)
    o = host(qwq4.moe_combine(yp, r, H, out_bf16=False))
    assert rel_err(o, out) <= TOL


def test_combine_with_shared(gpu):
    import torch
    T, k, H = 3, 2, 64
    yp = torch.arange(T * k * H, dtype=torch.float32, device=gpu).reshape(T * k, H) / 100
    r = qwq4.Route(T, 8, k, gpu)
    r.tok_slot.copy_(torch.tensor([[1, 0], [3, 2], [5, 4]], dtype=torch.int32))
    r.top_w.copy_(torch.tensor([[0.25, 0.75], [0.5, 0.5], [1.0, 0.0]]))
    shared = torch.ones((T, H), device=gpu)
    o = host(qwq4.moe_combine(yp, r, H, shared=shared, out_bf16=False))
    y = host(yp)
    want = np.stack([1 + 0.25 * y[1] + 0.75 * y[0], 1 + 0.5 * y[3] + 0.5 * y[2], 1 + y[5] + 0 * y[4]])
    assert np.allclose(o, want, rtol=1e-6)


def _f16_sat(y32):
    y = np.asarray(y32, np.float32)
    return np.where(np.isfinite(y), np.clip(y, -65504.0, 65504.0), y).astype(np.float16)


@pytest.mark.parametrize("T,E,H,F", [(1, 64, 1024, 512), (2, 64, 1024, 512), (8, 64, 1024, 512), (32, 64, 1024, 512),
                                     (8, 256, 4096, 1536)])
def test_experts_gemv_yp_f16(gpu, oracle, T, E, H, F):
    """fp16 yp (the reference's moe_experts_P output, moe.hpp:35-37): the
    fp32 sums rounded to nearest even, bit for bit against the fp32 yp of the
    same kernels, h unchanged; the combine of the fp16 rows within the
    tolerance of the oracle's MoE."""
    k = 8
    print(f"moe gemv yp16 T={T} E={E} H={H} F={F}", flush=True)
    ex = synth.experts(44, E, H, F)
    xb, xf = synth.acts(44, f"x{T}", T, H)
    l = synth.router_logits(44, f"l{T}", T, E)
    out = oracle.moe(xf, l, k, *ex)
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    dx = to_dev(xb, gpu)
    r = qwq4.moe_route(to_dev(l, gpu), k)
    h32, yp32 = qwq4.moe_experts_gemv(dg, du, dd, r, dx, E, F)
    h16, yp16 = qwq4.moe_experts_gemv(dg, du, dd, r, dx, E, F, yp_f16=True)
    assert host(yp16).dtype == np.float16
    assert np.array_equal(host(h16).view(np.uint16), host(h32).view(np.uint16))
    assert np.array_equal(host(yp16).view(np.uint16), _f16_sat(host(yp32)).view(np.uint16))
    o = host(qwq4.moe_combine(yp16, r, H, out_bf16=False))
    assert rel_err(o, out) <= TOL


@pytest.mark.parametrize("H", [64, 4096, 100])
def test_combine_fp16_rows_and_foreign_slots(gpu, H):
    """moe_combine_T's types (fp16 yp, fp16 shared, fp16 out, moe.hpp:42-43)
    and moe_combine_B's (fp16 yp, fp32 shared and out): out = shared + the
    weighted rows in selection order, against an fp64 sum of the same fp16
    values; a negative slot (a selection another rank holds) adds nothing,
    as in the reference (moe_route.hip:174-175)."""
    import torch
    T, k = 5, 4
    rng = np.random.default_rng(H)
    yp = torch.from_numpy(rng.standard_normal((T * k, H)).astype(np.float16)).to(gpu)
    r = qwq4.Route(T, 8, k, gpu)
    slots = rng.permutation(T * k).reshape(T, k).astype(np.int32)
    slots[1, 2] = -1
    slots[3, 0] = -1
    w = rng.random((T, k)).astype(np.float32)
    r.tok_slot.copy_(torch.from_numpy(slots))
    r.top_w.copy_(torch.from_numpy(w))
    sh16 = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16)).to(gpu)
    y = host(yp).astype(np.float64)
    want = host(sh16).astype(np.float64)
    for t in range(T):
        for i in range(k):
            if slots[t, i] >= 0:
                want[t] += float(w[t, i]) * y[slots[t, i]]
    o32 = host(qwq4.moe_combine(yp, r, H, shared=sh16, out_dtype=torch.float32))
    assert np.max(np.abs(o32 - want)) <= 1e-5 * np.max(np.abs(want))
    o16 = host(qwq4.moe_combine(yp, r, H, shared=sh16, out_dtype=torch.float16))
    assert o16.dtype == np.float16
    assert np.array_equal(o16.view(np.uint16), _f16_sat(o32).view(np.uint16))
    sh32 = sh16.float()
    ob = host(qwq4.moe_combine(yp, r, H, shared=sh32, out_bf16=False))
    assert np.array_equal(ob.view(np.uint32), o32.view(np.uint32))


@pytest.mark.parametrize("T", [8, 32])
def test_decode_and_prefill_experts_agree(gpu, oracle, T):
    """The decode path (gathered GEMVs, bf16 operands) and the prefill path
    (grouped GEMM on fp16-dequantised weights) on the same routing agree
    within 1% of max|y| (the reference's P-vs-T check, test_moe.hip), each
    within the 2e-3 bar of the oracle."""
    E, H, F, k = 32, 1024, 384, 4
    print(f"moe decode vs prefill T={T}", flush=True)
    ex = synth.experts(43, E, H, F)
    xb, xf = synth.acts(43, f"x{T}", T, H)
    l = synth.router_logits(43, f"l{T}", T, E, bias_sigma=0.5)
    out = oracle.moe(xf, l, k, *ex)
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    dx, dl = to_dev(xb, gpu), to_dev(l, gpu)
    r1 = qwq4.moe_route(dl, k)
    _, yp1 = qwq4.moe_experts_gemv(dg, du, dd, r1, dx, E, F)
    o1 = host(qwq4.moe_combine(yp1, r1, H, out_bf16=False))
    r2 = qwq4.moe_route(dl, k, tile_m=qwq4.moe_grouped_tile_m())
    _, yp2 = qwq4.moe_experts_grouped(dg, du, dd, r2, dx, E, F)
    o2 = host(qwq4.moe_combine(yp2, r2, H, out_bf16=False))
    assert np.array_equal(host(r1.tok_slot), host(r2.tok_slot))
    assert np.max(np.abs(o1 - o2)) <= 0.01 * np.max(np.abs(o1))
    assert rel_err(o1, out) <= TOL and rel_err(o2, out) <= TOL


def _random_moe(n, seed=99):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(r.integers(2, 65))
        out.append((E, int(r.integers(1, min(E, 8) + 1)), 128 * int(r.integers(1, 17)), 128 * int(r.integers(1, 13)),
                    int(r.integers(1, 33)), int(r.integers(33, 700)), bool(r.integers(0, 2))))
    return out


@pytest.mark.parametrize("E,k,H,F,Td,Tp,zeros", _random_moe(6))
def test_moe_random_shapes(gpu, oracle, E, k, H, F, Td, Tp, zeros):
    """Seeded random expert counts, top-k, H, F, with and without zeros: a
    decode batch (gathered GEMVs) and a prefill chunk (grouped GEMMs over
    mixed tiles, skewed routing) against the oracle; routing bit-exact."""
    print(f"moe random E={E} k={k} H={H} F={F} Td={Td} Tp={Tp} zeros={zeros}", flush=True)
    ex = synth.experts(E + H + F, E, H, F, zeros=zeros)
    (dg, du, dd), E, F = _experts_dev(gpu, ex)
    for T, tm in ((Td, 0), (Tp, qwq4.moe_grouped_tile_m())):
        xb, xf = synth.acts(T + E, f"rx{T}", T, H)
        l = synth.router_logits(T + k, f"rl{T}", T, E, bias_sigma=0.5 if tm else 0.0)
        out = oracle.moe(xf, l, k, *ex)
        r = qwq4.moe_route(to_dev(l, gpu), k, tile_m=tm)
        te, _ = oracle.route(l, k)
        assert np.array_equal(host(r.top_e), te)
        if tm:
            _, yp = qwq4.moe_experts_grouped(dg, du, dd, r, to_dev(xb, gpu), E, F)
        else:
            _, yp = qwq4.moe_experts_gemv(dg, du, dd, r, to_dev(xb, gpu), E, F)
        o = host(qwq4.moe_combine(yp, r, H, out_bf16=False))
        assert rel_err(o, out) <= TOL
