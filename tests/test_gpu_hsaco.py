"""The llama2 eval forward + loss run over the gfx950 code objects alone
(hipModuleLoad / hipModuleGetFunction / hipModuleLaunchKernel through
ctypes, as a purego host would), against the library's EvalLoss
(ane/engine.go:464-482) on the same weights and windows."""
import numpy as np
import pytest

import ane
from ane import hsaco

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nseq", [16, 32])
def test_code_objects_alone_give_the_eval_loss(nseq):
    cfg = ane.stories110m("llama2")
    p = ane.init_params(cfg, seed=7, std=0.02)
    tok, tgt = ane.make_tokens(cfg, nseq, seed=8 + nseq)
    tgt[0, 5] = 65535  # an excluded target counts in neither path
    eng = ane.Open(ane.Options(Config=cfg, Params=p, MaxBatch=nseq))
    try:
        _, per = eng.EvalLoss(tok, tgt)
    finally:
        eng.Destroy()
    got = hsaco.eval_loss(cfg, p, tok, tgt)
    print("max rel diff", float(np.max(np.abs(got - per) / np.abs(per))), "bit-equal", bool(np.array_equal(got, per)))
    # the same kernels with the same arguments; the RoPE tables are built on
    # the host by each side (libm against numpy cos / sin)
    np.testing.assert_allclose(got, per, rtol=2e-6, atol=0)


def test_code_objects_refuse_other_shapes():
    cfg = ane.tiny("llama2")
    p = ane.init_params(cfg, seed=1)
    tok, tgt = ane.make_tokens(cfg, 2, seed=2)
    with pytest.raises(ValueError):
        hsaco.eval_loss(cfg, p, tok, tgt)
