"""Eval harness (ane/harness.py) on the CPU with an oracle-backed stand-in
engine: token files, the reference's windowing (39 windows of 256 at stride
255 over the last 10,000 tokens), target alignment, and the reference's
vocab-major-as-position-major loss reproduced against a direct restatement."""
import math

import numpy as np
import pytest

import ane
import oracle
from ane import harness


class OracleEngine:
    """EvalLoss / EvalLogits with the engine's signatures, computed by the oracle."""

    def __init__(self, cfg, params, max_batch=8):
        self.cfg, self.p, self.max_batch = cfg, params, max_batch
        self.calls = 0

    def EvalLoss(self, tok, tgt):
        self.calls += 1
        mean, per, _ = oracle.forward_loss(self.cfg, self.p, tok, tgt)
        return mean, per

    def EvalLogits(self, window):
        _, _, lg = oracle.forward_loss(self.cfg, self.p, np.asarray(window)[None], np.asarray(window)[None],
                                       want_logits=True)
        return lg[0].reshape(-1)


def test_load_tokens(tmp_path):
    ids = np.array([0, 1, 31999, 65535, 7], np.uint16)
    p = tmp_path / "t.bin"
    p.write_bytes(ids.astype("<u2").tobytes())
    np.testing.assert_array_equal(harness.LoadTokens(str(p)), ids)
    p.write_bytes(b"\x01\x02\x03")
    with pytest.raises(ValueError, match="not even"):
        harness.LoadTokens(str(p))


def test_reference_windowing():
    val, starts = harness.eval_windows(np.zeros(12_000, np.uint16))
    assert len(val) == 10_000 and len(starts) == 39
    assert starts[:3] == [0, 255, 510] and starts[-1] + 256 < 10_000
    with pytest.raises(ValueError, match="need at least"):
        harness.eval_windows(np.zeros(10_100, np.uint16))


def test_eval_loss_matches_direct_cross_entropy():
    cfg = ane.tiny("llama2", vocab=128)
    p = ane.init_params(cfg, seed=1, std=0.1)
    toks = np.random.default_rng(2).integers(0, cfg.vocab, 1_000).astype(np.uint16)
    eng = OracleEngine(cfg, p, max_batch=4)
    got = harness.EvalLoss(eng, toks, eval_tokens=600)
    val, starts = harness.eval_windows(toks, 600, cfg.seq)
    total, n = 0.0, 0
    for s in starts:
        w = val[s:s + cfg.seq]
        lg = eng.EvalLogits(w).reshape(cfg.vocab, cfg.seq).astype(np.float64)
        for t in range(cfg.seq - 1):
            col = lg[:, t]
            total += math.log(np.exp(col - col.max()).sum()) + col.max() - col[w[t + 1]]
            n += 1
    assert n == len(starts) * (cfg.seq - 1)
    assert abs(got - total / n) < 1e-5
    assert eng.calls == math.ceil(len(starts) / 4)
    assert abs(harness.ValBPB(got) - got / math.log(2) / 3.7) < 1e-12


def test_reference_layout_loss_reproduced():
    cfg = ane.tiny("nanochat", vocab=128)
    p = ane.init_params(cfg, seed=3, std=0.1)
    toks = np.random.default_rng(4).integers(0, cfg.vocab, 400).astype(np.uint16)
    eng = OracleEngine(cfg, p)
    got = harness.ReferenceEvalLoss(eng, toks, eval_tokens=300)
    val, starts = harness.eval_windows(toks, 300, cfg.seq)
    total, n = 0.0, 0
    for s in starts:
        w = val[s:s + cfg.seq]
        flat = eng.EvalLogits(w).astype(np.float64)     # vocab-major [V * seq]
        for i in range(cfg.seq - 1):
            row = flat[i * cfg.vocab:(i + 1) * cfg.vocab]  # the reference's slice
            m = max(row.max(), 5e-324)
            total -= row[w[i + 1]] - m - math.log(np.exp(row - m).sum())
            n += 1
    assert abs(got - total / n) < 1e-9
    # and it differs from the true cross-entropy
    assert abs(got - harness.EvalLoss(eng, toks, eval_tokens=300)) > 1e-3
