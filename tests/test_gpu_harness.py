"""Eval harness on the device engine against the same harness over the
oracle (tests/test_harness.py's OracleEngine): validation loss within the
contract's 1e-3 nats."""
import numpy as np
import pytest

import ane
from ane import harness
from test_harness import OracleEngine

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("arch", ["llama2", "nanochat"])
def test_eval_loss_matches_oracle(arch):
    cfg = ane.tiny(arch, vocab=512)
    p = ane.init_params(cfg, seed=5, std=0.08)
    toks = np.random.default_rng(6).integers(0, cfg.vocab, 3_000).astype(np.uint16)
    eng = ane.Open(ane.Options(Config=cfg, Params=p, MaxBatch=16))
    try:
        got = harness.EvalLoss(eng, toks, eval_tokens=2_000)
        got_ref = harness.ReferenceEvalLoss(eng, toks, eval_tokens=600)
    finally:
        eng.Destroy()
    orc = OracleEngine(cfg, p, max_batch=16)
    want = harness.EvalLoss(orc, toks, eval_tokens=2_000)
    want_ref = harness.ReferenceEvalLoss(orc, toks, eval_tokens=600)
    print(f"{arch}: val loss gpu {got:.6f} oracle {want:.6f}; reference-layout {got_ref:.6f} / {want_ref:.6f}")
    assert abs(got - want) <= 1e-3
    assert abs(got_ref - want_ref) <= 2e-2
