"""Checkpoint loading: safetensors header parsing (CPU) and q4 projections
loaded straight into the tiled device format (GPU, bit-exact against the
oracle's conversion of the same file).

Files are written by the safetensors library in the layout of the reference's
checkpoint (docs/MODEL.md:34-38): "<p>.weight_packed" int32 [out][in/8],
"<p>.weight_scale" bf16 [out][in/128], symmetric (zero 8).
"""
import os
import struct

import numpy as np
import pytest

import qwq4
from qwq4 import synth


def _write(path, tensors):
    import torch
    from safetensors.torch import save_file
    save_file({k: torch.from_numpy(v) if isinstance(v, np.ndarray) else v for k, v in tensors.items()}, path)


def _q4_tensors(seed, prefix, N, K):
    """Checkpoint tensors of one projection: packed words and bf16 scales
    (drawn so that some exceed the fp16 range and saturate)."""
    import torch
    W, _, _ = synth.q4_weights(seed, prefix, N, K, zeros=False)
    r = np.random.default_rng(seed)
    sc = (np.abs(r.standard_normal((N, K // 128))) * 0.02).astype(np.float32)
    sc[0, 0] = 1e6           # saturates to 65504 in fp16
    sc[1 % N, 0] = 3e-8      # fp16 subnormal range
    sb = torch.from_numpy(sc).to(torch.bfloat16)
    return {f"{prefix}.weight_packed": W.view(np.int32), f"{prefix}.weight_scale": sb}


def test_header_listing_and_info(tmp_path, lib):
    p = str(tmp_path / "m.safetensors")
    t = _q4_tensors(3, "layers.0.mlp.experts.1.up_proj", 32, 256)
    t["norm.weight"] = np.arange(6, dtype=np.float32)
    _write(p, t)
    with qwq4.StFile(p) as f:
        names = f.names()
        assert names == sorted(t)
        assert f.info("layers.0.mlp.experts.1.up_proj.weight_packed") == ("I32", (32, 32), 32 * 32 * 4)
        assert f.info("layers.0.mlp.experts.1.up_proj.weight_scale") == ("BF16", (32, 2), 32 * 2 * 2)
        assert f.info("norm.weight") == ("F32", (6,), 24)
        with pytest.raises(RuntimeError, match="no tensor named"):
            f.info("missing")


def test_bad_files_are_rejected(tmp_path, lib):
    good = str(tmp_path / "g.safetensors")
    _write(good, {"a": np.zeros(4, np.float32)})
    raw = open(good, "rb").read()
    hl = struct.unpack("<Q", raw[:8])[0]
    cases = {
        "short": raw[:5],
        "header_past_end": struct.pack("<Q", len(raw)) + raw[8:],
        "not_json": struct.pack("<Q", 4) + b"nope" + b"\0" * 16,
        "size_mismatch": raw.replace(b'"shape":[4]', b'"shape":[5]'),
        "data_past_end": raw[:8 + hl + 8],
    }
    for name, data in cases.items():
        p = str(tmp_path / f"{name}.safetensors")
        open(p, "wb").write(data)
        with pytest.raises(RuntimeError, match="qw_st_open"):
            qwq4.StFile(p)
    with pytest.raises(RuntimeError, match="cannot open"):
        qwq4.StFile(str(tmp_path / "absent.safetensors"))


@pytest.mark.gpu
def test_load_matches_oracle_and_stacks(tmp_path, gpu, oracle):
    import torch
    from _gpu_util import TOL, host, rel_err, to_dev
    E, N, K = 3, 48, 384
    p = str(tmp_path / "experts.safetensors")
    t = {}
    for e in range(E):
        t.update(_q4_tensors(10 + e, f"layers.2.mlp.experts.{e}.gate_proj", N, K))
    _write(p, t)
    wb, sb, _ = qwq4.tiled_size(E * N, K)
    Wt = torch.empty(wb // 4, dtype=torch.int32, device=gpu)
    St = torch.empty(sb // 2, dtype=torch.int16, device=gpu)
    with qwq4.StFile(p) as f:
        for e in range(E):
            qwq4.load_q4(f, f"layers.2.mlp.experts.{e}.gate_proj", N, K, out=(Wt, St, None), row0=e * N)
    # back to checkpoint order: words bit-exact, scales = the reference's
    # saturating bf16 -> fp16 of the file's scales
    W, S, _ = qwq4.untile(Wt, St, None, E * N, K)
    Wf = np.concatenate([t[f"layers.2.mlp.experts.{e}.gate_proj.weight_packed"].view(np.uint32) for e in range(E)])
    Sb = np.concatenate([t[f"layers.2.mlp.experts.{e}.gate_proj.weight_scale"].view(torch.int16).numpy().view(np.uint16)
                         for e in range(E)])
    S16 = oracle.bf16_to_f16(Sb)
    assert np.array_equal(host(W).view(np.uint32), Wf)
    assert np.array_equal(host(S).view(np.uint16), S16)
    # and the loaded weights multiply like the oracle's
    xb, xf = synth.acts(5, "lx", 2, K)
    y = qwq4.gemv(Wt, St, None, to_dev(xb, gpu), E * N, K, 2)
    ref = oracle.q4_linear(Wf, S16, None, E * N, K, xf)
    assert rel_err(host(y), ref) <= TOL


@pytest.mark.gpu
def test_bf16_to_f16_device_matches_reference(gpu, oracle):
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
    from _gpu_util import host, to_dev
    for b, want in ((gold["bf16_in"], gold["bf16_to_f16"]),
                    (np.arange(65536, dtype=np.uint32).astype(np.uint16), None)):
        got = host(qwq4.bf16_to_f16(to_dev(b, gpu))).view(np.uint16)
        assert np.array_equal(got, oracle.bf16_to_f16(b) if want is None else want)


def _pieces():
    import torch
    g = torch.Generator().manual_seed(7)
    return [torch.randint(0, 256, (n,), dtype=torch.uint8, generator=g) for n in (100, 64, 0, 4097)]


def test_weight_cache_record_then_replay(tmp_path, lib):
    import torch
    p = str(tmp_path / "w.qwc")
    ps = _pieces()
    with qwq4.WCache(p, 1234) as c:
        assert c.mode == "record"
        for t in ps:
            c.put(t)
        assert not os.path.exists(p)       # only the .tmp until finished
        c.finish()
    assert os.path.exists(p) and not os.path.exists(p + ".tmp")
    with qwq4.WCache(p, 1234) as c:
        assert c.mode == "replay"
        for t in ps:
            got = torch.empty_like(t)
            c.get(got)
            assert torch.equal(got, t)
        c.finish()


def test_weight_cache_rejects_stale_and_damaged_files(tmp_path, lib):
    import torch
    p = str(tmp_path / "w.qwc")
    ps = _pieces()
    with qwq4.WCache(p, 5) as c:
        for t in ps:
            c.put(t)
        c.finish()
    good = open(p, "rb").read()
    # another key records afresh (and leaves the old file until finished)
    with qwq4.WCache(p, 6) as c:
        assert c.mode == "record"
    assert open(p, "rb").read() == good    # not finished: nothing replaced
    # truncated, or a count that does not match: recorded afresh
    for bad in (good[:-8], good[:-1], good[:200], good[:-8] + (99).to_bytes(8, "little")):
        open(p, "wb").write(bad)
        with qwq4.WCache(p, 5) as c:
            assert c.mode == "record"
    # replaying: a piece of another size, too many pieces, pieces left over
    open(p, "wb").write(good)
    with qwq4.WCache(p, 5) as c:
        with pytest.raises(RuntimeError, match="expected"):
            c.get(torch.empty(101, dtype=torch.uint8))
    with qwq4.WCache(p, 5) as c:
        c.get(torch.empty(100, dtype=torch.uint8))
        with pytest.raises(RuntimeError, match="left unused"):
            c.finish()
    with qwq4.WCache(p, 5) as c:
        for t in ps:
            c.get(torch.empty_like(t))
        with pytest.raises(RuntimeError, match="more pieces"):
            c.get(torch.empty(1, dtype=torch.uint8))


def test_weight_cache_off_when_unwritable(tmp_path, lib):
    import torch
    c = qwq4.WCache(str(tmp_path / "absent_dir" / "w.qwc"), 1)
    assert c.mode == "off" and "cannot write" in c.why
    c.put(torch.zeros(3, dtype=torch.uint8))   # a no-op
    with pytest.raises(RuntimeError, match="not replaying"):
        c.get(torch.zeros(3, dtype=torch.uint8))
    c.finish()
    c.close()


def test_checkpoint_key_tracks_files(tmp_path):
    a = tmp_path / "a.safetensors"
    a.write_bytes(b"x" * 10)
    k1 = qwq4.checkpoint_key([a])
    assert k1 == qwq4.checkpoint_key([a]) and k1 != qwq4.checkpoint_key([a], "opt")
    a.write_bytes(b"x" * 11)
    assert qwq4.checkpoint_key([a]) != k1


@pytest.mark.gpu
def test_load_through_weight_cache(tmp_path, gpu):
    import torch
    E, N, K = 2, 32, 256
    p = str(tmp_path / "experts.safetensors")
    t = {}
    for e in range(E):
        t.update(_q4_tensors(20 + e, f"e.{e}.up_proj", N, K))
    _write(p, t)
    wb, sb, _ = qwq4.tiled_size(E * N, K)

    def load(cache, st):
        Wt = torch.zeros(wb // 4, dtype=torch.int32, device=gpu)
        St = torch.zeros(sb // 2, dtype=torch.int16, device=gpu)
        for e in range(E):
            qwq4.load_q4(st, f"e.{e}.up_proj", N, K, out=(Wt, St, None), row0=e * N, cache=cache)
        cache.finish()
        return Wt, St

    cp = str(tmp_path / "c.qwc")
    key = qwq4.checkpoint_key([p])
    with qwq4.StFile(p) as f, qwq4.WCache(cp, key) as c:
        assert c.mode == "record"
        W1, S1 = load(c, f)
    with qwq4.WCache(cp, key) as c:
        assert c.mode == "replay"
        W2, S2 = load(c, None)     # no checkpoint read at all
    assert torch.equal(W1, W2) and torch.equal(S1, S2)
