"""SaveCheckpoint / LoadCheckpoint through the device engine (V5 file + SANE
trailer): weights, Adam moments, counters, LR and the pending accumulated
gradient survive the round trip, and two engines resumed from the same file
continue identically."""
import numpy as np
import pytest

import ane
from ane.checkpoint import TrainMeta, read_checkpoint

pytestmark = pytest.mark.gpu


def _engine(cfg, p, stream):
    return ane.Open(ane.Options(Config=cfg, Params=p, MaxBatch=1, Tokens=stream, AccumSteps=2, LR=1e-3, Seed=5))


def test_checkpoint_round_trip(tmp_path):
    cfg = ane.tiny("nanochat")
    p = ane.init_params(cfg, seed=3, std=0.08)
    stream = np.random.default_rng(4).integers(0, cfg.vocab, 20 * (cfg.seq + 1)).astype(np.uint16)
    path = str(tmp_path / "ck.bin")
    a = _engine(cfg, p, stream)
    try:
        for _ in range(3):          # one AdamW update + one pending step
            a.Step()
        st = a.State()
        assert st.adam_t == 1 and st.pending_steps == 1
        a.SetLR(7e-4)
        a.SaveCheckpoint(path, TrainMeta(Step=3, TotalSteps=10))
        pa, (ma, va), ga = a.Params(), a.OptState(), a.AccumGrads()
    finally:
        a.Destroy()
    meta, pf, mf, vf, tr = read_checkpoint(path, cfg)
    assert meta.Step == 3 and meta.AdamT == 1 and abs(meta.LR - 7e-4) < 1e-9
    np.testing.assert_array_equal(pf, pa)
    np.testing.assert_array_equal(mf, ma)
    assert tr["pending"] == 1 and np.abs(tr["accum"]).max() > 0

    losses, params = [], []
    for _ in range(2):
        b = _engine(cfg, ane.init_params(cfg, seed=99), stream)
        try:
            meta = b.LoadCheckpoint(path)
            np.testing.assert_array_equal(b.Params(), pa)
            mb, vb = b.OptState()
            np.testing.assert_array_equal(mb, ma)
            np.testing.assert_array_equal(vb, va)
            np.testing.assert_array_equal(b.AccumGrads(), ga)
            s = b.State()
            assert (s.adam_t, s.pending_steps, s.cum_steps) == (1, 1, st.cum_steps)
            assert abs(b.LR() - 7e-4) < 1e-9
            r = b.Step()              # completes the pending accumulation -> AdamW update 2
            assert b.State().adam_t == 2
            losses.append(r.loss)
            params.append(b.Params())
        finally:
            b.Destroy()
    assert losses[0] == losses[1]
    np.testing.assert_allclose(params[0], params[1], rtol=1e-6, atol=1e-7)


def test_open_from_model_files(tmp_path):
    """Open(ModelPath=...) as the reference's Open (ane/engine.go:240-248):
    a llama2.c file (LoadPretrained) for both architectures, and a training
    checkpoint, whose Adam moments come along when the engine trains; the
    device then computes exactly what it computes from the same weights
    passed directly."""
    import struct
    from ane import checkpoint as ck
    for arch in ("llama2", "nanochat"):
        cfg = ane.tiny(arch)
        p = ane.init_params(cfg, seed=8, std=0.08)
        w = ane.views(cfg, p)
        path = tmp_path / f"{arch}.bin"
        with open(path, "wb") as f:
            f.write(struct.pack("<7i", cfg.dim, cfg.hidden, cfg.layers, cfg.heads, cfg.heads, cfg.vocab, cfg.seq))
            f.write(w["embed"].tobytes())
            ones = np.ones(cfg.dim, np.float32)
            for l in range(cfg.layers):
                f.write((w[f"layers.{l}.g_att"] if arch == "llama2" else ones).tobytes())
            for nm in ("wq", "wk", "wv", "wo"):
                for l in range(cfg.layers):
                    f.write(w[f"layers.{l}.{nm}"].tobytes())
            for l in range(cfg.layers):
                f.write((w[f"layers.{l}.g_ffn"] if arch == "llama2" else ones).tobytes())
            for nm in ("w1", "w2"):
                for l in range(cfg.layers):
                    f.write(w[f"layers.{l}.{nm}"].tobytes())
            for l in range(cfg.layers):
                f.write((w[f"layers.{l}.w3"] if arch == "llama2" else np.zeros(cfg.hidden * cfg.dim, np.float32))
                        .tobytes())
            f.write((w["g_final"] if arch == "llama2" else ones).tobytes())
        want, _ = ck.load_pretrained(str(path), cfg)
        tok, tgt = ane.make_tokens(cfg, 2, seed=9)
        a = ane.Open(ane.Options(Config=cfg, ModelPath=str(path), MaxBatch=2))
        b = ane.Open(ane.Options(Config=cfg, Params=want, MaxBatch=2))
        try:
            np.testing.assert_array_equal(a.Params(), want)
            np.testing.assert_array_equal(a.EvalLoss(tok, tgt)[1], b.EvalLoss(tok, tgt)[1])
        finally:
            a.Destroy()
            b.Destroy()
        if arch == "llama2":   # the file held every llama2 tensor: the model is the one written
            np.testing.assert_array_equal(want, p)
    cfg = ane.tiny("nanochat")
    p = ane.init_params(cfg, seed=10, std=0.08)
    r = np.random.default_rng(11)
    m = r.standard_normal(p.size).astype(np.float32)
    v = r.random(p.size).astype(np.float32)
    cp = tmp_path / "train.ckpt"
    ck.write_checkpoint(str(cp), cfg, ck.TrainMeta(Step=2, AdamT=1), p, m, v)
    stream = r.integers(0, cfg.vocab, 500).astype(np.uint16)
    e = ane.Open(ane.Options(Config=cfg, ModelPath=str(cp), MaxBatch=1, Tokens=stream))
    try:
        np.testing.assert_array_equal(e.Params(), p)
        m2, v2 = e.OptState()
        np.testing.assert_array_equal(m2, m)
        np.testing.assert_array_equal(v2, v)
        assert e.State().adam_t == 0          # Open keeps fresh counters, as the reference's
    finally:
        e.Destroy()
    with pytest.raises(ane.EngineError, match="storiesane open: load model: "):
        ane.Open(ane.Options(Config=cfg, ModelPath=str(tmp_path / "missing.bin")))
