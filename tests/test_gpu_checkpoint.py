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
