"""The device engine, decoder and MoE layer against the committed golden
fixtures (tests/golden) at the contract's tolerances; no oracle call at run
time."""
import numpy as np
import pytest

import ane
from ane.moe import MoeConfig, MoeLayer, init_moe_params
from golden_io import load

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("arch", ["llama2", "nanochat"])
def test_forward_matches_fixture(arch):
    cfg = ane.tiny(arch)
    p = ane.init_params(cfg, seed=0, std=0.08)
    tok, _ = load(f"forward_{arch}_tokens")
    _, tgt = ane.make_tokens(cfg, 1, seed=1)
    ref_lg, tol = load(f"forward_{arch}_logits")
    ref_loss, ltol = load(f"forward_{arch}_loss")
    eng = ane.Open(ane.Options(Config=cfg, Params=p, MaxBatch=1))
    try:
        lg = eng.EvalLogits(tok[0]).reshape(cfg.vocab, cfg.seq)
        mean, _ = eng.EvalLoss(tok, tgt)
    finally:
        eng.Destroy()
    assert np.abs(lg - ref_lg).max() <= tol
    assert abs(mean - float(ref_loss[0])) <= ltol


@pytest.mark.parametrize("arch,mode", [("llama2", "true"), ("nanochat", "compat")])
def test_grads_match_fixture(arch, mode):
    cfg = ane.tiny(arch, grad_mode=mode)
    p = ane.init_params(cfg, seed=21, std=0.08)
    tok, tgt = ane.make_tokens(cfg, 2, seed=22)
    eng = ane.Open(ane.Options(Config=cfg, Params=p, MaxBatch=2))
    try:
        loss, g = eng.Grads(tok, tgt)
    finally:
        eng.Destroy()
    ref_norms, tol = load(f"grads_{arch}_{mode}_norms")
    ref_loss, ltol = load(f"grads_{arch}_{mode}_loss")
    norms = [np.linalg.norm(g[off:off + int(np.prod(s))].astype(np.float64)) for _, off, s in ane.param_layout(cfg)]
    scalar = [n.split(".")[-1] in ("resid_lambdas", "x0_lambdas", "smear_lambda", "backout_lambda", "ve_gate")
              for n, _, _ in ane.param_layout(cfg)]
    for n, r, sc in zip(norms, ref_norms, scalar):
        assert abs(n - r) <= (5e-2 if sc else tol) * max(r, 1e-12)
    assert abs(loss - float(ref_loss[0])) <= ltol


def test_decode_matches_fixture():
    cfg = ane.tiny_decode()
    p = ane.init_params(cfg, seed=61, std=0.05)
    prefix, _ = load("decode_gqa_prefix")
    forced, _ = load("decode_gqa_forced")
    ref_lg, tol = load("decode_gqa_logits")
    dec = ane.Decoder(cfg, p, max_batch=2, max_ctx=128)
    try:
        _, lg0 = dec.Prefill(prefix, want_logits=True)
        lgs = [lg0] + [dec.Step(forced[:, i], want_logits=True)[1] for i in range(2)]
    finally:
        dec.Close()
    assert np.abs(np.stack(lgs, 1) - ref_lg).max() <= tol


def test_moe_matches_fixture():
    cfg = MoeConfig(dim=64, hidden=128, experts=8)
    x, _ = load("moe_small_x")
    layer = MoeLayer(cfg, init_moe_params(cfg, seed=71, std=0.1), max_tokens=16)
    try:
        out, idx, w = layer.Forward(x)
    finally:
        layer.Close()
    np.testing.assert_array_equal(idx, load("moe_small_experts")[0])
    ref, tol = load("moe_small_out")
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) <= tol
