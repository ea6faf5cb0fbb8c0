"""Forward + loss parity of the device engine against the CPU oracle.

Config-1 shape (stories110M, B1 x 256) for both architectures: logits
max-abs error <= 2e-2 and mean loss within 1e-3 nats (the tolerances of the
benchmark contract: fp16 activations and weights, fp32 accumulation).
Smaller models cover batching, edge cases and the error behaviour of the
reference API (ane/engine.go:449-455, 567).
"""
import numpy as np
import pytest

import ane
import oracle

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
LOSS_TOL = 1e-3


def open_engine(cfg, params, max_batch=1, tokens=None):
    return ane.Open(ane.Options(Config=cfg, Params=params, MaxBatch=max_batch, Tokens=tokens))


@pytest.fixture(scope="module", params=["llama2", "nanochat"])
def full(request):
    cfg = ane.stories110m(request.param)
    p = ane.init_params(cfg, seed=0)
    eng = open_engine(cfg, p, max_batch=2)
    yield cfg, p, eng
    eng.Destroy()


def test_config1_logits_and_loss(full):
    cfg, p, eng = full
    tok, tgt = ane.make_tokens(cfg, 1, seed=1)
    lo, _, lg_ref = oracle.forward_loss(cfg, p, tok, tgt, want_logits=True)
    lg = eng.EvalLogits(tok[0]).reshape(cfg.vocab, cfg.seq)
    err = np.abs(lg - lg_ref[0]).max()
    print(f"{cfg.arch}: logits max-abs err {err:.3e}")
    assert err <= LOGIT_TOL
    mean, per = eng.EvalLoss(tok, tgt)
    print(f"{cfg.arch}: loss gpu {mean:.6f} oracle {lo:.6f}")
    assert abs(mean - lo) <= LOSS_TOL


def test_full_batched_loss_per_sequence(full):
    cfg, p, eng = full
    tok, tgt = ane.make_tokens(cfg, 2, seed=2)
    lo, per_ref, _ = oracle.forward_loss(cfg, p, tok, tgt)
    mean, per = eng.EvalLoss(tok, tgt)
    np.testing.assert_allclose(per, per_ref, atol=LOSS_TOL)
    assert abs(mean - lo) <= LOSS_TOL


@pytest.mark.parametrize("arch", ["llama2", "nanochat"])
def test_tiny_model_batched(arch):
    cfg = ane.tiny(arch, layers=4)
    p = ane.init_params(cfg, seed=3, std=0.08)
    eng = open_engine(cfg, p, max_batch=5)
    tok, tgt = ane.make_tokens(cfg, 5, seed=4)
    lo, per_ref, lg_ref = oracle.forward_loss(cfg, p, tok, tgt, want_logits=True)
    mean, per = eng.EvalLoss(tok, tgt)
    np.testing.assert_allclose(per, per_ref, atol=LOSS_TOL)
    for b in (0, 4):
        lg = eng.EvalLogits(tok[b]).reshape(cfg.vocab, cfg.seq)
        assert np.abs(lg - lg_ref[b]).max() <= LOGIT_TOL
    eng.Destroy()


@pytest.mark.parametrize("seq", [128, 192])
@pytest.mark.parametrize("arch", ["llama2", "nanochat"])
def test_tiny_model_other_sequence_lengths(arch, seq):
    """Sequences of 2 and 3 pairs of 32-query blocks (2 and 3 attention
    waves per block)."""
    cfg = ane.tiny(arch, layers=2, seq=seq)
    p = ane.init_params(cfg, seed=5, std=0.08)
    eng = open_engine(cfg, p, max_batch=3)
    tok, tgt = ane.make_tokens(cfg, 3, seed=6)
    lo, per_ref, lg_ref = oracle.forward_loss(cfg, p, tok, tgt, want_logits=True)
    mean, per = eng.EvalLoss(tok, tgt)
    np.testing.assert_allclose(per, per_ref, atol=LOSS_TOL)
    for b in (0, 2):
        lg = eng.EvalLogits(tok[b]).reshape(cfg.vocab, cfg.seq)
        assert np.abs(lg - lg_ref[b]).max() <= LOGIT_TOL
    eng.Destroy()


@pytest.mark.parametrize("arch", ["llama2", "nanochat"])
def test_out_of_range_tokens_and_targets(arch):
    """Token >= vocab embeds as a zero row (ane/stories/cpu.go:60-64); target
    >= vocab is excluded from the mean (ane/stories/cpu.go:253-257); a
    sequence with no valid target has loss 0."""
    cfg = ane.tiny(arch)
    p = ane.init_params(cfg, seed=5, std=0.08)
    eng = open_engine(cfg, p, max_batch=3)
    tok, tgt = ane.make_tokens(cfg, 3, seed=6)
    tok[0, 3] = 60000
    tok[1, 0] = cfg.vocab
    tgt[0, 5] = 60000
    tgt[2, :] = 65535
    lo, per_ref, _ = oracle.forward_loss(cfg, p, tok, tgt)
    mean, per = eng.EvalLoss(tok, tgt)
    assert per[2] == 0.0 and per_ref[2] == 0.0
    np.testing.assert_allclose(per, per_ref, atol=LOSS_TOL)
    eng.Destroy()


def test_windows_equal_explicit_batch():
    cfg = ane.tiny("nanochat")
    p = ane.init_params(cfg, seed=7, std=0.08)
    stream = np.random.default_rng(8).integers(0, cfg.vocab, 5000).astype(np.uint16)
    eng = open_engine(cfg, p, max_batch=4, tokens=stream)
    pos = np.array([0, 17, 4000, 5000 - cfg.seq - 1], np.uint64)
    m1, per1 = eng.EvalLossWindows(pos)
    tok = np.stack([stream[int(q):int(q) + cfg.seq] for q in pos])
    tgt = np.stack([stream[int(q) + 1:int(q) + 1 + cfg.seq] for q in pos])
    m2, per2 = eng.EvalLoss(tok, tgt)
    np.testing.assert_array_equal(per1, per2)
    with pytest.raises(ane.EngineError):
        eng.EvalLossWindows(np.array([5000 - cfg.seq], np.uint64))  # window runs past the end
    eng.Destroy()


@pytest.mark.parametrize("arch", ["nanochat", "llama2"])
def test_more_windows_than_kernel_arguments_hold(arch):
    """72 windows: past the 64 window starts a launch carries as arguments,
    the starts go to the device first and a separate gather reads them; the
    losses equal the explicit batch bit for bit (both architectures, the
    llama2 one through the deferred-norm forward)."""
    cfg = ane.tiny(arch)
    p = ane.init_params(cfg, seed=9, std=0.08)
    stream = np.random.default_rng(10).integers(0, cfg.vocab, 20000).astype(np.uint16)
    n = 72
    eng = open_engine(cfg, p, max_batch=n, tokens=stream)
    pos = np.random.default_rng(11).integers(0, 20000 - cfg.seq - 1, n).astype(np.uint64)
    m1, per1 = eng.EvalLossWindows(pos)
    tok = np.stack([stream[int(q):int(q) + cfg.seq] for q in pos])
    tgt = np.stack([stream[int(q) + 1:int(q) + 1 + cfg.seq] for q in pos])
    m2, per2 = eng.EvalLoss(tok, tgt)
    np.testing.assert_array_equal(per1, per2)
    eng.Destroy()


def test_error_behaviour():
    cfg = ane.tiny("llama2")
    p = ane.init_params(cfg, seed=9)
    eng = open_engine(cfg, p)
    with pytest.raises(ane.EngineError, match=r"storiesane eval logits: token len=3 want=64"):
        eng.EvalLogits(np.zeros(3, np.uint16))
    with pytest.raises(ane.EngineError, match=r"nseq=2 must be in \[1, 1\]"):
        eng.EvalLoss(np.zeros((2, 64), np.uint16), np.zeros((2, 64), np.uint16))
    eng.Close()
    with pytest.raises(ane.EngineError, match="storiesane eval logits: engine is closed"):
        eng.EvalLogits(np.zeros(64, np.uint16))
    eng.Destroy()


def test_params_round_trip_and_profile():
    cfg = ane.tiny("nanochat")
    p = ane.init_params(cfg, seed=10)
    eng = open_engine(cfg, p, max_batch=2)
    np.testing.assert_array_equal(eng.Params(), p)
    tok, tgt = ane.make_tokens(cfg, 2, seed=11)
    eng.ProfileEnable(True)
    eng.EvalLoss(tok, tgt)
    prof = eng.ProfileRead()
    assert prof["qkv_gemm"]["launches"] == cfg.layers
    assert prof["attention"]["launches"] == cfg.layers
    assert prof["classifier_gemm"]["ms"] > 0
    eng.Destroy()


def test_graph_replay_matches_eager(monkeypatch):
    """With ANE_GRAPHS=1 eval loss replays a captured graph per batch size.
    Every replay must equal the same engine run eagerly (the default), bit
    for bit, across changing windows, batch sizes, new parameters, eager work
    in between (EvalLogits, a training step that allocates its buffers) and
    profiling."""
    cfg = ane.tiny("llama2", layers=4)
    p = ane.init_params(cfg, seed=11, std=0.08)
    stream = np.random.default_rng(12).integers(0, cfg.vocab, 6000).astype(np.uint16)
    monkeypatch.setenv("ANE_GRAPHS", "1")
    eng_g = open_engine(cfg, p, max_batch=4, tokens=stream)
    monkeypatch.delenv("ANE_GRAPHS")
    eng_e = open_engine(cfg, p, max_batch=4, tokens=stream)
    rng = np.random.default_rng(13)

    def check(nseq):
        pos = rng.integers(0, 6000 - cfg.seq - 1, nseq).astype(np.uint64)
        mg, pg = eng_g.EvalLossWindows(pos)
        me, pe = eng_e.EvalLossWindows(pos)
        np.testing.assert_array_equal(pg, pe)
        assert mg == me

    for nseq in (4, 4, 2, 4, 1):
        check(nseq)
        eng_g.EvalLogits(stream[:cfg.seq])
    p2 = ane.init_params(cfg, seed=14, std=0.08)
    eng_g.SetParams(p2)
    eng_e.SetParams(p2)
    check(4)
    eng_g.Step()  # training buffers, split-K workspace, new weights
    eng_e.SetParams(eng_g.Params())
    for nseq in (4, 3, 3):
        check(nseq)
    eng_g.ProfileEnable(True)
    check(2)
    eng_g.ProfileEnable(False)
    check(2)
    eng_g.Destroy()
    eng_e.Destroy()
