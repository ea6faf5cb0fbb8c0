"""The model-file readers of the host mirror, on small synthetic files
written here from the format description (ane/stories/weights.go:73-153,
ane/stories/ckpt.go:271-712): every tensor is filled with a distinct ramp,
so a tensor read from the wrong offset, a skipped block of the wrong size or
a missing default shows.  CPU only."""
import struct

import numpy as np
import pytest

import ane
from ane import checkpoint as ck

D, H, L, V, NH = 128, 256, 2, 512, 2


def cfg(arch="nanochat"):
    return ane.tiny(arch, dim=D, hidden=H, heads=NH, layers=L, vocab=V)


class Ramp:
    """Distinct float32 values: tensor k holds k * 1e4 + arange."""

    def __init__(self):
        self.k = 0

    def __call__(self, n):
        self.k += 1
        return (np.arange(n, dtype=np.float64) + self.k * 1e4).astype(np.float32) / 1e3


def write_llama2(path, vocab_field=V, dims=(D, H, L)):
    r = Ramp()
    t = {}
    d, h, l = dims
    with open(path, "wb") as f:
        f.write(struct.pack("<7i", d, h, l, NH, NH, vocab_field, 64))

        def put(name, n):
            a = r(n)
            t[name] = a
            f.write(a.tobytes())

        put("embed", abs(vocab_field) * d)
        for i in range(l):
            put(f"rms_att.{i}", d)
        for nm in ("wq", "wk", "wv", "wo"):
            for i in range(l):
                put(f"{nm}.{i}", d * d)
        for i in range(l):
            put(f"rms_ffn.{i}", d)
        for i in range(l):
            put(f"w1.{i}", h * d)
        for i in range(l):
            put(f"w2.{i}", d * h)
        for i in range(l):
            put(f"w3.{i}", h * d)
        put("rms_final", d)
        f.write(r(1000).tobytes())   # trailing data (freq_cis, wcls) is not read
    return t


def test_llama2c_file_into_the_reference_model(tmp_path):
    p = tmp_path / "stories.bin"
    t = write_llama2(p)
    c = cfg("nanochat")
    params, hdr = ck.load_pretrained(str(p), c)
    assert hdr.shared_classifier and hdr.vocab_size == V and hdr.n_kv_heads == NH
    w = ane.views(c, params)
    np.testing.assert_array_equal(w["embed"].reshape(-1), t["embed"])
    for i in range(L):
        for nm in ("wq", "wk", "wv", "wo", "w1", "w2"):
            np.testing.assert_array_equal(w[f"layers.{i}.{nm}"].reshape(-1), t[f"{nm}.{i}"])
    # the reference drops the gains and W3 and sets initLambdasDefault
    np.testing.assert_array_equal(w["resid_lambdas"], 1.0)
    for nm in ("x0_lambdas", "smear_lambda", "backout_lambda", "smear_gate"):
        assert not w[nm].any(), nm
    for i in range(L):
        if ane.is_ve_layer(c, i):
            assert not w[f"layers.{i}.ve_embed"].any() and not w[f"layers.{i}.ve_gate"].any()


def test_llama2c_file_into_the_llama2_variant(tmp_path):
    p = tmp_path / "stories.bin"
    t = write_llama2(p, vocab_field=-V)          # negative: own classifier (not read; tied here)
    c = cfg("llama2")
    params, hdr = ck.load_pretrained(str(p), c)
    assert not hdr.shared_classifier
    w = ane.views(c, params)
    for i in range(L):
        for nm in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
            np.testing.assert_array_equal(w[f"layers.{i}.{nm}"].reshape(-1), t[f"{nm}.{i}"])
        np.testing.assert_array_equal(w[f"layers.{i}.g_att"], t[f"rms_att.{i}"])
        np.testing.assert_array_equal(w[f"layers.{i}.g_ffn"], t[f"rms_ffn.{i}"])
    np.testing.assert_array_equal(w["g_final"], t["rms_final"])


def test_llama2c_errors(tmp_path):
    p = tmp_path / "bad.bin"
    write_llama2(p, dims=(D, H + 64, L))
    with pytest.raises(ValueError, match=rf"config mismatch: got dim={D} hidden={H + 64} layers={L}"):
        ck.load_pretrained(str(p), cfg())
    q = tmp_path / "short.bin"
    q.write_bytes(open(p, "rb").read()[:1000].replace(struct.pack("<i", H + 64), struct.pack("<i", H), 1))
    with pytest.raises(ValueError, match="truncated"):
        ck.load_pretrained(str(q), cfg())


def _header(ver, c):
    return struct.pack("<10i2f3d3i3i", ck.CKPT_MAGIC, ver, 7, 99, c.layers, c.vocab, c.dim, c.hidden, c.heads,
                       c.seq, 1e-3, 2.5, 1.0, 2.0, 3.0, 11, 12, 13, 0, 0, 0)


def write_v4(path, c):
    """Sequential writes in the order loadCheckpointV4V5 reads (isV5 false)."""
    r, t = Ramp(), {}
    with open(path, "wb") as f:
        f.write(_header(4, c))

        def put(name, n):
            a = r(n)
            t[name] = a
            f.write(a.tobytes())

        for i in range(c.layers):
            for nm, n in (("wq", D * D), ("wk", D * D), ("wv", D * D), ("wo", D * D), ("w1", H * D), ("w2", D * H)):
                put(f"{nm}.{i}", n)
            put(f"w3.{i}", H * D)
            if ane.is_ve_layer(c, i):
                put(f"ve_embed.{i}", V * D)
                put(f"old_ve_gate.{i}", D)
        for i in range(c.layers):
            for nm, n in (("wq", D * D), ("wk", D * D), ("wv", D * D), ("wo", D * D), ("w1", H * D), ("w2", D * H)):
                put(f"m.{nm}.{i}", n)
                put(f"v.{nm}.{i}", n)
            put(f"m.w3.{i}", H * D)
            put(f"v.w3.{i}", H * D)
            if ane.is_ve_layer(c, i):
                put(f"m.ve_embed.{i}", V * D)
                put(f"v.ve_embed.{i}", V * D)
                put(f"m.old_ve_gate.{i}", D)
                put(f"v.old_ve_gate.{i}", D)
        for nm, n in (("embed", V * D), ("resid_lambdas", L), ("x0_lambdas", L), ("smear_gate", D * D),
                      ("smear_lambda", 1), ("backout_lambda", 1)):
            put(nm, n)
            put("m." + nm, n)
            put("v." + nm, n)
    return t


def write_v3(path, c, ver):
    r, t = Ramp(), {}
    with open(path, "wb") as f:
        f.write(_header(ver, c))

        def put(name, n):
            a = r(n)
            t[name] = a
            f.write(a.tobytes())

        mats = (("wq", D * D), ("wk", D * D), ("wv", D * D), ("wo", D * D), ("w1", H * D), ("w2", D * H))
        for i in range(c.layers):
            for nm, n in mats:
                put(f"{nm}.{i}", n)
            put(f"w3.{i}", H * D)
            put(f"rms_att.{i}", D)
            put(f"rms_ffn.{i}", D)
        for i in range(c.layers):
            for nm, n in mats:
                put(f"m.{nm}.{i}", n)
                put(f"v.{nm}.{i}", n)
            put(f"mv.w3.{i}", 2 * H * D)
            put(f"mv.rms.{i}", 4 * D)
        put("rms_final", D)
        put("mv.rms_final", 2 * D)
        put("embed", V * D)
        put("m.embed", V * D)
        put("v.embed", V * D)
    return t


def test_v4_checkpoint(tmp_path):
    c = cfg()
    p = tmp_path / "v4.ckpt"
    t = write_v4(p, c)
    base = ane.init_params(c, seed=3)
    meta, params, m, v, trailer = ck.read_checkpoint(str(p), c, base=base)
    assert (meta.Step, meta.TotalSteps, meta.CumSteps, meta.CumBatches, meta.AdamT) == (7, 99, 11, 12, 13)
    assert trailer is None
    w, wm, wv, wb = (ane.views(c, a) for a in (params, m, v, base))
    for i in range(L):
        for nm in ("wq", "wk", "wv", "wo", "w1", "w2"):
            np.testing.assert_array_equal(w[f"layers.{i}.{nm}"].reshape(-1), t[f"{nm}.{i}"])
            np.testing.assert_array_equal(wm[f"layers.{i}.{nm}"].reshape(-1), t[f"m.{nm}.{i}"])
            np.testing.assert_array_equal(wv[f"layers.{i}.{nm}"].reshape(-1), t[f"v.{nm}.{i}"])
        if ane.is_ve_layer(c, i):
            np.testing.assert_array_equal(w[f"layers.{i}.ve_embed"].reshape(-1), t[f"ve_embed.{i}"])
            np.testing.assert_array_equal(wm[f"layers.{i}.ve_embed"].reshape(-1), t[f"m.ve_embed.{i}"])
            # the old dim-sized gate is skipped: the gate keeps its value, its moments are zero
            np.testing.assert_array_equal(w[f"layers.{i}.ve_gate"], wb[f"layers.{i}.ve_gate"])
            assert not wm[f"layers.{i}.ve_gate"].any()
    for nm in ("embed", "resid_lambdas", "x0_lambdas", "smear_gate", "smear_lambda", "backout_lambda"):
        np.testing.assert_array_equal(w[nm].reshape(-1), t[nm])
        np.testing.assert_array_equal(wv[nm].reshape(-1), t["v." + nm])


@pytest.mark.parametrize("ver", [2, 3])
def test_v2_v3_checkpoints(tmp_path, ver):
    c = cfg()
    p = tmp_path / f"v{ver}.ckpt"
    t = write_v3(p, c, ver)
    base = ane.init_params(c, seed=4)
    with open(p, "ab") as f:          # bytes after the body that are not a trailer at the V5 offset
        f.write(b"XXXX" * 16)
    meta, params, m, v, trailer = ck.read_checkpoint(str(p), c, base=base)
    assert trailer is None and meta.AdamT == 13
    w, wm, wb = (ane.views(c, a) for a in (params, m, base))
    for i in range(L):
        for nm in ("wq", "wk", "wv", "wo", "w1", "w2"):
            np.testing.assert_array_equal(w[f"layers.{i}.{nm}"].reshape(-1), t[f"{nm}.{i}"])
            if ver == 3:
                np.testing.assert_array_equal(wm[f"layers.{i}.{nm}"].reshape(-1), t[f"m.{nm}.{i}"])
            else:
                assert not wm[f"layers.{i}.{nm}"].any()
        if ane.is_ve_layer(c, i):   # V2 / V3 have no value embeddings: prior values stay
            np.testing.assert_array_equal(w[f"layers.{i}.ve_embed"], wb[f"layers.{i}.ve_embed"])
    np.testing.assert_array_equal(w["embed"].reshape(-1), t["embed"])
    np.testing.assert_array_equal(wm["embed"].reshape(-1), t["m.embed"])
    # initLambdasDefault; x0 lambdas and the smear gate keep their values
    np.testing.assert_array_equal(w["resid_lambdas"], 1.0)
    assert w["smear_lambda"][0] == 0.0 and w["backout_lambda"][0] == 0.0
    np.testing.assert_array_equal(w["x0_lambdas"], wb["x0_lambdas"])
    np.testing.assert_array_equal(w["smear_gate"], wb["smear_gate"])


def test_bad_version_and_v5_round_trip(tmp_path):
    c = cfg()
    p = tmp_path / "bad.ckpt"
    p.write_bytes(_header(6, c) + b"\0" * 64)
    with pytest.raises(ValueError, match="bad checkpoint header magic=424c5a54 version=6"):
        ck.read_checkpoint(str(p), c)
    prm = ane.init_params(c, seed=5)
    r = np.random.default_rng(6)
    m = r.standard_normal(prm.size).astype(np.float32)
    v = r.random(prm.size).astype(np.float32)
    acc = r.standard_normal(prm.size).astype(np.float32)
    q = tmp_path / "v5.ckpt"
    ck.write_checkpoint(str(q), c, ck.TrainMeta(Step=3, AdamT=2), prm, m, v, token_pos=77, pending=2, accum=acc)
    meta, p2, m2, v2, tr = ck.read_checkpoint(str(q), c)
    assert meta.Step == 3 and tr["token_pos"] == 77 and tr["pending"] == 2
    for a, b in ((prm, p2), (m, m2), (v, v2), (acc, tr["accum"])):
        np.testing.assert_array_equal(a, b)
