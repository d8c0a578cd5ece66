"""CPU oracle pinned against the reference's own code (golden vectors from
oracle/_ref, see tests/golden/make_golden.py), independent library routines
(numpy, torch) and closed forms."""
import os

import numpy as np
import pytest

from qwq4 import synth

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---------------------------------------------------------------- numbers
def test_f16_to_f32_matches_reference_on_every_pattern(oracle):
    got = np.array([oracle.lib().o_f16_to_f32(int(v)) for v in GOLD["f16_all"]], np.float32)
    assert np.array_equal(got.view(np.uint32), GOLD["f16_all_f32"].view(np.uint32))
    # and numpy's own fp16 widening agrees wherever it is not NaN
    npv = GOLD["f16_all"].view(np.float16).astype(np.float32)
    ok = ~np.isnan(npv)
    assert np.array_equal(npv[ok].view(np.uint32), got[ok].view(np.uint32))


def test_f32_to_f16_matches_reference(oracle):
    got = oracle.f32_to_f16(GOLD["f32_in"])
    assert np.array_equal(got, GOLD["f32_to_f16"])
    x = GOLD["f32_in"]
    ok = ~np.isnan(x)
    assert np.array_equal(x[ok].astype(np.float16).view(np.uint16), got[ok])


def test_bf16_to_f16_matches_reference(oracle):
    got = oracle.bf16_to_f16(GOLD["bf16_in"])
    assert np.array_equal(got, GOLD["bf16_to_f16"])
    # independent: numpy's fp16 cast of the clipped value (NaN aside)
    f = oracle.bf16_to_f32(GOLD["bf16_in"])
    ok = ~np.isnan(f)
    ref = np.clip(f[ok], -65504, 65504).astype(np.float16).view(np.uint16)
    assert np.array_equal(got[ok], ref)


def test_f32_to_bf16_is_round_to_nearest_even(oracle):
    import torch
    r = np.random.default_rng(5)
    x = np.concatenate([r.normal(0, 1, 3000), r.normal(0, 1, 1000) * 1e30,
                        [1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 0.0, -0.0, 3.3895314e38, np.inf]]).astype(np.float32)
    got = oracle.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(synth.bf16_bits(x), want)
    assert got[-7] == 0x3F80 and got[-6] == 0x3F82  # ties to even


# ------------------------------------------------------------ q4 format
def test_engine_order_matches_reference(oracle):
    assert np.array_equal(oracle.pack_engine_order(GOLD["words_in"]), GOLD["words_eng"])
    assert np.array_equal(oracle.unpack_engine_order(GOLD["words_eng"]), GOLD["words_in"])


def test_quantizer_matches_reference(oracle):
    words, scales = oracle.quantize_g128(GOLD["qsrc"])
    assert np.array_equal(words, GOLD["q_words"])
    assert np.array_equal(scales, GOLD["q_scales"])


def test_unpack_against_byte_view(oracle):
    W, _, _ = synth.q4_weights(1, "u", 24, 512)
    got = oracle.q4_unpack(W, 24, 512)
    b = W.view(np.uint8).reshape(24, 256)  # little-endian: byte j holds elements 2j (low) and 2j+1 (high)
    want = np.stack([b & 0xF, b >> 4], axis=-1).reshape(24, 512)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("zeros", [False, True])
def test_dequant_closed_form(oracle, zeros):
    N, K = 16, 384
    W, S, Z = synth.q4_weights(2, "d", N, K, zeros)
    got = oracle.q4_dequant(W, S, Z, N, K)
    q = oracle.q4_unpack(W, N, K).astype(np.int32)
    z = synth.unpack_zeros(Z, K // 128).astype(np.int32) if zeros else np.full((N, K // 128), 8, np.int32)
    s = S.view(np.float16).astype(np.float32)
    want = ((q - np.repeat(z, 128, axis=1)).astype(np.float32) * np.repeat(s, 128, axis=1)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_special_cases(oracle):
    N, K = 8, 256
    W, S, Z = synth.q4_weights(3, "s", N, K)
    S[:, 0] = 0                                   # scale 0 -> exact zeros
    q = oracle.q4_unpack(W, N, K)
    z = np.zeros((N, 2), np.uint8)
    z[:, 1] = q[:, 128]                           # zero equal to one element's nibble
    Zp = synth.pack_zeros(z)
    d = oracle.q4_dequant(W, S, Zp, N, K)
    assert np.all(d[:, :128] == 0)
    assert np.all(d[:, 128] == 0)


def test_linear_vs_fp64_and_numpy(oracle):
    N, K, T = 96, 1024, 3
    W, S, Z = synth.q4_weights(4, "l", N, K)
    _, x = synth.acts(4, "x", T, K)
    y = oracle.q4_linear(W, S, Z, N, K, x)
    y64 = oracle.q4_linear_f64(W, S, Z, N, K, x)
    deq = oracle.q4_dequant(W, S, Z, N, K).astype(np.float64)
    ref = x.astype(np.float64) @ deq.T
    assert np.max(np.abs(y64 - ref)) <= 1e-9 * np.max(np.abs(ref))
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_linear_exact_cases(oracle):
    N, K = 32, 512
    W, S, Z = synth.q4_weights(5, "e", N, K)
    # one-hot x picks column k exactly: s * (q - z)
    x = np.zeros((1, K), np.float32)
    x[0, 300] = 1.0
    y = oracle.q4_linear(W, S, Z, N, K, x)
    deq = oracle.q4_dequant(W, S, Z, N, K)
    assert np.array_equal(y[0], deq[:, 300])
    # integer activations with unit scales: every partial sum is an exact integer
    S1 = np.full_like(S, 0x3C00)  # fp16 1.0
    xi = np.random.default_rng(0).integers(-8, 9, size=(2, K)).astype(np.float32)
    yi = oracle.q4_linear(W, S1, Z, N, K, xi)
    q = oracle.q4_unpack(W, N, K).astype(np.int64) - np.repeat(synth.unpack_zeros(Z, K // 128).astype(np.int64), 128, 1)
    assert np.array_equal(yi.astype(np.int64), xi.astype(np.int64) @ q.T)
    # zero activations
    assert np.all(oracle.q4_linear(W, S, Z, N, K, np.zeros((1, K), np.float32)) == 0)


@pytest.mark.parametrize("rpg", [20, 32, 324])
def test_linear_row_slices_one_hot(oracle, rpg):
    """Rows grouped over activation slices (gpu::gemv_rows' rpg,
    src/kernels/gemv.hip:16-17: row n reads slice n // rpg): with x one-hot
    at column k of slice s, row n gives deq[n][k] exactly when n // rpg == s
    and 0 otherwise, for the q4 and the 16-bit linear; the one-hot sum over
    all slices gives every row's column k."""
    N, K = 48 if rpg < 64 else 660, 256
    W, S, Z = synth.q4_weights(9, "rs", N, K)
    deq = oracle.q4_dequant(W, S, Z, N, K)
    ns = (N + rpg - 1) // rpg
    r = np.random.default_rng(rpg)
    W16 = (r.standard_normal((N, K)) * 0.05).astype(np.float16)
    for sl in range(ns):
        x = np.zeros((1, ns * K), np.float32)
        x[0, sl * K + 77] = 1.0
        y = oracle.q4_linear(W, S, Z, N, K, x, rpg=rpg)
        yw = oracle.linear_w16(W16.view(np.uint16), x, True, rpg=rpg)
        rows = (np.arange(N) // rpg) == sl
        assert np.array_equal(y[0][rows], deq[rows, 77]) and np.all(y[0][~rows] == 0)
        assert np.array_equal(yw[0][rows], W16[rows, 77].astype(np.float32)) and np.all(yw[0][~rows] == 0)
    x = np.zeros((1, ns * K), np.float32)
    x[0, [s * K + 5 for s in range(ns)]] = 1.0
    assert np.array_equal(oracle.q4_linear(W, S, Z, N, K, x, rpg=rpg)[0], deq[:, 5])


# ------------------------------------------------------------- routing
def test_route_order_and_weights(oracle):
    T, E, k = 64, 256, 8
    l = synth.router_logits(6, "r", T, E)
    te, tw = oracle.route(l, k)
    # exp is monotone: with no two selected probabilities equal, the order is
    # the logits' order (ties to the lower index)
    order = np.lexsort((np.arange(E)[None, :].repeat(T, 0), -l), axis=1)[:, :k]
    assert np.array_equal(te, order)
    p = np.exp((l - l.max(1, keepdims=True)).astype(np.float64))
    sel = np.take_along_axis(p, te, 1)
    assert np.allclose(tw, sel / sel.sum(1, keepdims=True), rtol=1e-6, atol=0)
    assert np.allclose(tw.astype(np.float64).sum(1), 1.0, atol=1e-6)


def test_route_ties_to_lower_index(oracle):
    l = np.zeros((2, 16), np.float32)
    l[0, [3, 7, 11]] = 2.0
    te, tw = oracle.route(l, 4)
    assert list(te[0]) == [3, 7, 11, 0]
    assert list(te[1]) == [0, 1, 2, 3]
    assert np.all(tw[1] == np.float32(0.25))


def test_slots_invariants(oracle):
    T, E, k = 40, 32, 4
    te, _ = oracle.route(synth.router_logits(7, "s", T, E), k)
    counts, offsets, tok_slot, pair_tok = oracle.moe_slots(te, E)
    assert np.array_equal(counts, np.bincount(te.ravel(), minlength=E))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
    assert np.array_equal(np.sort(tok_slot.ravel()), np.arange(T * k))
    for t in range(T):
        for j in range(k):
            s = tok_slot[t, j]
            assert pair_tok[s] == t and offsets[te[t, j]] <= s < offsets[te[t, j] + 1]
    for e in range(E):  # tokens ascending within an expert
        seg = pair_tok[offsets[e]:offsets[e + 1]]
        assert np.all(np.diff(seg) > 0)


def test_moe_vs_dense_numpy(oracle):
    T, E, H, F, k = 5, 8, 256, 256, 2
    gate, up, down = synth.experts(8, E, H, F)
    _, x = synth.acts(8, "x", T, H)
    l = synth.router_logits(8, "l", T, E)
    out = oracle.moe(x, l, k, gate, up, down)
    te, tw = oracle.route(l, k)
    deq = lambda w, n, kk: oracle.q4_dequant(w[0][e], w[1][e], w[2][e], n, kk).astype(np.float64)
    ref = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            e = te[t, j]
            g = deq(gate, F, H) @ x[t]
            u = deq(up, F, H) @ x[t]
            h = g / (1 + np.exp(-g)) * u
            ref[t] += tw[t, j] * (deq(down, H, F) @ h)
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("N,K,zeros", [(32, 384, True), (16, 640, False)])
def test_tile_against_numpy_restatement(oracle, N, K, zeros):
    """The tiled format from reshapes: tile (sub, g, q, n) = row 16 sub + n,
    words 16 g + 4 q .. +4, nibbles of each word reordered (j, j+4) per byte."""
    W, S, Z = synth.q4_weights(9, "t", N, K, zeros)
    Wt, St, Zt = oracle.q4_tile(W, S, Z, N, K)
    G = K // 128
    q = oracle.q4_unpack(W, N, K).reshape(N, K // 8, 2, 4)       # [row][word][half][j]
    byte = q[:, :, 0, :] | (q[:, :, 1, :] << 4)                     # byte j = e_j | e_{j+4} << 4
    words = byte.astype(np.uint32) @ (np.uint32(1) << (8 * np.arange(4, dtype=np.uint32)))
    want = words.reshape(N // 16, 16, G, 4, 4).transpose(0, 2, 3, 1, 4).reshape(-1)
    assert np.array_equal(Wt, want.astype(np.uint32))
    GC = (G + 3) // 4
    Sp = np.zeros((N, GC * 4), np.uint16)
    Sp[:, :G] = S
    assert np.array_equal(St, Sp.reshape(N // 16, 16, GC, 4).transpose(0, 2, 1, 3).reshape(-1))
    if zeros:
        z = np.zeros((N, GC * 4), np.uint16)
        z[:, :G] = synth.unpack_zeros(Z, G)
        zt = (z.reshape(N, GC, 4) << (4 * np.arange(4, dtype=np.uint16))).sum(-1).astype(np.uint16)
        assert np.array_equal(Zt, zt.reshape(N // 16, 16, GC).transpose(0, 2, 1).reshape(-1))


def _libm_expf():
    import ctypes
    import ctypes.util
    m = ctypes.CDLL(ctypes.util.find_library("m"))
    m.expf.argtypes = [ctypes.c_float]
    m.expf.restype = ctypes.c_float
    return m.expf


def test_expf_tie_pairs_are_rounding_conflicts():
    """The adversarial routing pairs (test_moe_gpu.EXPF_TIE_PAIRS) really are
    pairs of adjacent floats whose exponentials tie under the C library's
    expf (what the reference's std::exp on a float calls) and not under the
    correctly rounded exp, or the reverse."""
    from test_moe_gpu import EXPF_TIE_PAIRS
    expf = _libm_expf()
    for u, glibc_tie in EXPF_TIE_PAIRS:
        d_small, d_large = np.array([u, u - 1], np.uint32).view(np.float32)
        g = (np.float32(expf(float(d_small))), np.float32(expf(float(d_large))))
        c = (np.float32(np.exp(np.float64(d_small))), np.float32(np.exp(np.float64(d_large))))
        assert (g[0] == g[1]) == glibc_tie
        assert (c[0] == c[1]) != glibc_tie


def test_device_expf_table_is_nearest_powers_of_two():
    """The 32-entry table of the device's expf (csrc/route_core.cuh) holds the
    doubles nearest 2^(i/32), i << 47 subtracted from their bits."""
    import re
    import struct
    from decimal import Decimal, getcontext
    src = open(os.path.join(ROOT, "v620-inference-engine_amd", "csrc", "route_core.cuh")).read()
    body = src[src.index("kExp2Tab32[32] = {"):]
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", body[:body.index("};")])]
    assert len(vals) == 32
    getcontext().prec = 60
    for i, v in enumerate(vals):
        exact = float(Decimal(2) ** (Decimal(i) / Decimal(32)))
        assert (v + (i << 47)) & (2**64 - 1) == struct.unpack("<Q", struct.pack("<d", exact))[0]


@pytest.mark.parametrize("f16", [False, True])
def test_linear_w16_vs_fp64(oracle, f16):
    """The 16-bit-weight linear (ref_model.cpp:86-97) against an fp64 numpy
    product of the same widened weights, and exactly on integer data."""
    r = np.random.default_rng(3)
    W = (r.standard_normal((37, 384)) * 0.05).astype(np.float32)
    bits = W.astype(np.float16).view(np.uint16) if f16 else synth.bf16_bits(W)
    Wf = bits.view(np.float16).astype(np.float32) if f16 else synth.bf16_to_f32(bits)
    x = r.standard_normal((3, 384)).astype(np.float32)
    y = oracle.linear_w16(bits, x, f16)
    ref = x.astype(np.float64) @ Wf.astype(np.float64).T
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    Wi = r.integers(-8, 8, size=(16, 256)).astype(np.float32)
    xi = r.integers(-8, 8, size=(2, 256)).astype(np.float32)
    bi = Wi.astype(np.float16).view(np.uint16) if f16 else synth.bf16_bits(Wi)
    assert np.array_equal(oracle.linear_w16(bi, xi, f16), xi @ Wi.T)


def test_swiglu_gate_vs_torch(oracle):
    """h = silu(g) * u * sigmoid(gate logit), against torch's own silu and
    sigmoid in fp64."""
    import torch
    r = np.random.default_rng(4)
    n, T = 96, 5
    v = (r.standard_normal((T, 2 * n + 3)) * 3).astype(np.float32)
    h = oracle.swiglu_gate(v, n)
    vt = torch.from_numpy(v.astype(np.float64))
    ref = (torch.nn.functional.silu(vt[:, :n]) * vt[:, n:2 * n] * torch.sigmoid(vt[:, 2 * n:2 * n + 1])).numpy()
    assert np.max(np.abs(h - ref)) <= 1e-6 * np.max(np.abs(ref))


def test_shared_expert_vs_dense_numpy(oracle):
    """The shared expert's term (ref_model.cpp:465-478) against a dense fp64
    numpy evaluation of the same formula from the widened weights."""
    r = np.random.default_rng(6)
    H, n, T = 256, 128, 4
    gu = synth.bf16_bits((r.standard_normal((2 * n + 1, H)) * 0.05).astype(np.float32))
    dn = synth.bf16_bits((r.standard_normal((H, n)) * 0.05).astype(np.float32))
    x = r.standard_normal((T, H)).astype(np.float32)
    got = oracle.shared_expert(x, gu, dn)
    v = x.astype(np.float64) @ synth.bf16_to_f32(gu).astype(np.float64).T
    g, u, s = v[:, :n], v[:, n:2 * n], v[:, 2 * n:2 * n + 1]
    h = g / (1 + np.exp(-g)) * u / (1 + np.exp(-s))
    ref = h @ synth.bf16_to_f32(dn).astype(np.float64).T
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("group", [32, 16])
def test_quantize_rows_i8_matches_reference(oracle, group):
    """The int8 row quantiser against the reference's own quantize_rows_i8
    (weight_convert.cpp:92-108, run from oracle/_ref): int8 values and fp32
    scales bit for bit, over random rows, a zero group, a constant group, a
    symmetric ramp, an outlier and large magnitudes."""
    q, s = oracle.quantize_rows_i8(GOLD["i8_src"], group)
    assert np.array_equal(q, GOLD[f"i8_q{group}"])
    assert np.array_equal(s.view(np.uint32), GOLD[f"i8_s{group}"].view(np.uint32))


def test_i8_linear_vs_numpy_and_one_hot(oracle):
    """The int8 GEMV's oracle against a numpy fp64 restatement (with row groups
    over activation blocks, rpg) and the closed form of a one-hot row."""
    r = np.random.default_rng(8)
    N, K, M, rpg, g = 50, 160, 3, 20, 32
    W8 = r.integers(-127, 128, size=(N, K)).astype(np.int8)
    S = np.abs(r.standard_normal((N, K // g))).astype(np.float32) * 0.01
    nb = (N + rpg - 1) // rpg
    xs = nb * K + 8
    x = r.standard_normal((M, xs)).astype(np.float16)
    y = oracle.i8_linear_f64(W8, S, x.view(np.uint16), M, xs=xs, rpg=rpg, group=g)
    Wf = W8.astype(np.float64) * np.repeat(S.astype(np.float64), g, axis=1)
    ref = np.empty((M, N))
    for n in range(N):
        blk = x[:, (n // rpg) * K:(n // rpg) * K + K].astype(np.float64)
        ref[:, n] = blk @ Wf[n]
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)
    oh = np.zeros((1, K), np.float16)
    oh[0, 37] = 1.0
    y1 = oracle.i8_linear_f64(W8, S, oh.view(np.uint16), 1, group=g)
    assert np.array_equal(y1[0], W8[:, 37].astype(np.float64) * S[:, 37 // g].astype(np.float64))


@pytest.mark.parametrize("f16", [True, False])
def test_quant_rows_i8_properties(oracle, f16):
    """The W4A8 activation quantiser (moe_w4a8.hip:17-36): per 128-group the
    largest magnitude maps to +-127, every value to within half a step of its
    q * scale, an all-zero group to q = 0 with scale 1; and the values agree
    bit for bit with IEEE fp32 numpy arithmetic of the same steps."""
    r = np.random.default_rng(11)
    R, K = 6, 512
    v = r.standard_normal((R, K)).astype(np.float32) * np.float32(3.0)
    v[1, 128:256] = 0.0                    # a zero group
    v[2, 0:128] = 0.0
    v[2, 5] = -1e-3                        # one nonzero value
    v[3, 256:384] = np.linspace(-2, 2, 128, dtype=np.float32)  # symmetric ramp
    bits = v.astype(np.float16).view(np.uint16) if f16 else synth.bf16_bits(v)
    x = bits.view(np.float16).astype(np.float32) if f16 else synth.bf16_to_f32(bits)
    q, sc = oracle.quant_rows_i8(bits, f16)
    xg = x.reshape(R, K // 128, 128)
    qg = q.reshape(R, K // 128, 128).astype(np.int32)
    amax = np.abs(xg).max(-1)
    zero = amax == 0
    assert np.all(sc[zero] == 1.0) and np.all(qg[zero] == 0)
    nz = ~zero
    assert np.all(np.abs(qg).max(-1)[nz] == 127)
    assert np.all(np.abs(qg) <= 127)
    err = np.abs(qg * sc[..., None] - xg)
    assert np.all(err <= sc[..., None] * (0.5 + 1e-5))
    assert q[2, 5] == -127
    # IEEE fp32 steps: scale = amax / 127, inv = 1 / scale, q = rint(x * inv)
    s32 = np.where(zero, np.float32(1), (amax / np.float32(127)).astype(np.float32)).astype(np.float32)
    inv = (np.float32(1) / s32).astype(np.float32)
    ref = np.rint((xg * inv[..., None]).astype(np.float32)).astype(np.int32)
    assert np.array_equal(sc.view(np.uint32), s32.view(np.uint32))
    assert np.array_equal(qg, ref)


def test_w4a8_linear_vs_numpy_and_exact(oracle):
    """The W4A8 product (moe_w4a8.hip:62-183): against numpy (exact int64 dots per
    64-wide K step, fp64 sums of the per-step fp32 terms), and bit-exact where every
    term is exact (power-of-two scales, small values)."""
    r = np.random.default_rng(12)
    N, K, P = 24, 384, 9
    W, S, Z = synth.q4_weights(12, "w4a8", N, K, zeros=True)
    q8 = r.integers(-127, 128, size=(P + 3, K)).astype(np.int8)
    sx = np.abs(r.standard_normal((P + 3, K // 128))).astype(np.float32) * 0.02
    rowmap = r.integers(0, P + 3, size=P).astype(np.int32)
    y = oracle.w4a8_linear(q8, sx, W, S, Z, N, rowmap=rowmap)
    wq = oracle.q4_unpack(W, N, K).astype(np.int64) - np.repeat(synth.unpack_zeros(Z, K // 128), 128, 1)
    sw = S.view(np.float16).astype(np.float32)
    ref = np.zeros((P, N))
    for s in range(K // 64):
        d = q8[rowmap][:, 64 * s:64 * s + 64].astype(np.int64) @ wq[:, 64 * s:64 * s + 64].T
        g = s // 2
        ref += (d.astype(np.float32) * sw[None, :, g]).astype(np.float64) * sx[rowmap][:, g:g + 1]
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    # exact: scales 2^-4 .. 2^-1 and 1, small activations: every term and sum is an exact fp32
    S2 = (np.float16(2.0) ** -r.integers(0, 5, size=(N, K // 128))).astype(np.float16).view(np.uint16)
    q2 = r.integers(-3, 4, size=(P, K)).astype(np.int8)
    sx2 = (np.float32(2.0) ** -r.integers(0, 4, size=(P, K // 128))).astype(np.float32)
    y2 = oracle.w4a8_linear(q2, sx2, W, S2, Z, N)
    w2 = wq.astype(np.float64) * np.repeat(S2.view(np.float16).astype(np.float64), 128, 1)
    a2 = q2.astype(np.float64) * np.repeat(sx2.astype(np.float64), 128, 1)
    assert np.array_equal(y2, (a2 @ w2.T).astype(np.float32))


def test_moe_w4a8_close_to_the_unquantised_moe(oracle):
    """The W4A8 experts (oracle restatement of moe_experts_w4a8) stay close to the
    unquantised fp32 MoE (o_moe) on the same routing: int8 activations cost a few
    1e-3 of max|y| (the reference's documented loss), nothing structural."""
    E, H, F, k, T = 8, 256, 128, 2, 12
    ex = synth.experts(13, E, H, F, zeros=True)
    xb, xf = synth.acts(13, "x", T, H)
    l = synth.router_logits(13, "l", T, E)
    out, h_ref, yp_ref = oracle.moe(xf, l, k, *ex, want_parts=True)
    te, _ = oracle.route(l, k)
    counts, offsets, tok_slot, pair_tok = oracle.moe_slots(te, E)
    h, yp = oracle.moe_w4a8(xb, False, *ex, offsets, pair_tok, E)
    assert np.max(np.abs(h - h_ref)) <= 2e-2 * np.max(np.abs(h_ref))
    assert np.max(np.abs(yp - yp_ref)) <= 3e-2 * np.max(np.abs(yp_ref))
