"""Backward + optimizer parity of the device engine against the CPU oracle.

Weight gradients are compared per parameter tensor at relative L2 error
<= 1e-2 (the contract's tolerance; fp16 activations and weights, fp32
accumulation).  nanochat is checked in both gradient modes: `compat`
reproduces the reference's backward (scale-1 attention recompute, no RoPE
backward, 1.2^2 QK-norm coefficient, x0 gradient before smear), `true` is the
exact gradient.  Scalar parameters (lambdas) are single sums over the whole
activation tensor; they are held to 5e-2.
"""
import numpy as np
import pytest

import ane
import oracle

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2
SCALAR_TOL = 5e-2
HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=1.0, embed_lr_mult=2.0,
          scalar_lr_mult=0.5, lambda_lr_mult=0.01, lambda_beta1=0.96, lambda_beta2=0.97)


def open_engine(cfg, params, max_batch=1, tokens=None, **kw):
    return ane.Open(ane.Options(Config=cfg, Params=params, MaxBatch=max_batch, Tokens=tokens, **kw))


def seg_errors(cfg, g, ref):
    out = {}
    for name, off, shape in ane.param_layout(cfg):
        n = int(np.prod(shape))
        a, b = g[off:off + n].astype(np.float64), ref[off:off + n].astype(np.float64)
        out[name] = np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)
    return out


def check_grads(cfg, g, ref, overrides=None):
    errs = seg_errors(cfg, g, ref)
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:5]
    print(f"{cfg.arch}/{cfg.grad_mode}: worst rel L2 {[(k, f'{v:.2e}') for k, v in worst]}")
    for name, err in errs.items():
        tol = SCALAR_TOL if name.split(".")[-1] in ("resid_lambdas", "x0_lambdas", "smear_lambda",
                                                     "backout_lambda", "ve_gate") else REL_TOL
        tol = (overrides or {}).get(name, tol)
        assert err <= tol, (name, err)


@pytest.mark.parametrize("arch,mode", [("llama2", "true"), ("nanochat", "compat"), ("nanochat", "true")])
def test_tiny_grads_match_oracle(arch, mode):
    cfg = ane.tiny(arch, layers=4, grad_mode=mode)
    p = ane.init_params(cfg, seed=21, std=0.08)
    tok, tgt = ane.make_tokens(cfg, 3, seed=22)
    loss_ref, g_ref = oracle.grads(cfg, p, tok, tgt)
    eng = open_engine(cfg, p, max_batch=3)
    loss, g = eng.Grads(tok, tgt)
    eng.Destroy()
    assert abs(loss - loss_ref) <= 1e-3
    check_grads(cfg, g, g_ref)


@pytest.mark.parametrize("seq", [128, 192])
@pytest.mark.parametrize("arch,mode", [("llama2", "true"), ("nanochat", "compat")])
def test_tiny_grads_at_other_sequence_lengths(arch, mode, seq):
    """Sequences of 2 and 3 pairs of 32-query blocks: the attention backward
    then runs 2 and 3 waves per block (4 at seq 256, 1 at seq 64)."""
    cfg = ane.tiny(arch, layers=2, grad_mode=mode, seq=seq)
    p = ane.init_params(cfg, seed=23, std=0.08)
    tok, tgt = ane.make_tokens(cfg, 2, seed=24)
    loss_ref, g_ref = oracle.grads(cfg, p, tok, tgt)
    eng = open_engine(cfg, p, max_batch=2)
    loss, g = eng.Grads(tok, tgt)
    eng.Destroy()
    assert abs(loss - loss_ref) <= 1e-3
    check_grads(cfg, g, g_ref)


@pytest.mark.parametrize("arch,mode", [("llama2", "true"), ("nanochat", "compat")])
def test_full_size_grads_match_oracle(arch, mode):
    """BASELINE config 3 shape per sequence (stories110M, seq 256)."""
    cfg = ane.stories110m(arch, grad_mode=mode)
    p = ane.init_params(cfg, seed=0)
    tok, tgt = ane.make_tokens(cfg, 1, seed=3)
    loss_ref, g_ref = oracle.grads(cfg, p, tok, tgt)
    eng = open_engine(cfg, p, max_batch=1)
    loss, g = eng.Grads(tok, tgt)
    eng.Destroy()
    assert abs(loss - loss_ref) <= 1e-3
    # smear_lambda's gradient at this size is one sum over 256 x 768 products
    # that nearly cancels (3.2e-3): two builds of this engine that differ
    # only in the last-bit rounding of fp32 epilogue arithmetic give values
    # 10% apart, while every weight matrix stays within 0.5% of the other
    # build; the oracle's own value moves 1.2% when the parameters are merely
    # rounded to fp16.  Its bound is set by that conditioning, not by the
    # weight-gradient contract; the finite-difference test below pins it.
    check_grads(cfg, g, g_ref, overrides={"smear_lambda": 0.25})


def test_full_size_smear_lambda_gradient_by_finite_difference():
    """smear_lambda's full-size gradient nearly cancels (see above), so it is
    pinned against the device's own loss instead: central differences of
    EvalLoss over smear_lambda +- eps at eps = 1/8 and 1/16, extrapolated
    (Richardson: the eps^2 term cancels; the loss is strongly curved in
    lambda, so a single difference at a larger eps is biased), against
    Grads in the exact gradient mode, one sequence (the same per-token mean
    loss in both)."""
    cfg = ane.stories110m("nanochat", grad_mode="true")
    p = ane.init_params(cfg, seed=0)
    tok, tgt = ane.make_tokens(cfg, 1, seed=3)
    off = {name: o for name, o, _ in ane.param_layout(cfg)}["smear_lambda"]
    eng = open_engine(cfg, p, max_batch=1)
    try:
        _, g = eng.Grads(tok, tgt)
        fd = {}
        for eps in (0.125, 0.0625):
            lp = []
            for sgn in (1.0, -1.0):
                q = p.copy()
                q[off] += np.float32(sgn * eps)
                eng.SetParams(q)
                lp.append(float(eng.EvalLoss(tok, tgt)[0]))
            fd[eps] = (lp[0] - lp[1]) / (2 * eps)
    finally:
        eng.Destroy()
    rich = (4.0 * fd[0.0625] - fd[0.125]) / 3.0
    print(f"smear_lambda grad: device {g[off]:.6e}, central differences {fd}, extrapolated {rich:.6e}")
    assert abs(g[off] - rich) <= 0.05 * abs(rich)


# gradients accumulated by atomic adds (the token-indexed embedding rows and
# the value-embedding tables): their fp32 sums may round differently per run
ATOMIC_SEGMENTS = ("embed", "ve_embed", "ve_gate")


@pytest.mark.parametrize("arch,mode,nseq", [("llama2", "true", 16), ("nanochat", "compat", 4), ("nanochat", "true", 4)])
def test_dw_stream_matches_single_stream(arch, mode, nseq, monkeypatch):
    """The weight-gradient GEMMs on their own stream (the default) give the
    same gradients as the one-stream backward (ANE_DW_ASYNC=0): bit for bit
    except where atomics add in run-dependent order."""
    cfg = ane.stories110m(arch, grad_mode=mode)
    p = ane.init_params(cfg, seed=5)
    tok, tgt = ane.make_tokens(cfg, nseq, seed=6)
    out = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("ANE_DW_ASYNC", flag)
        eng = open_engine(cfg, p, max_batch=nseq)
        try:
            out[flag] = eng.Grads(tok, tgt)
        finally:
            eng.Destroy()
    assert out["0"][0] == out["1"][0]
    g0, g1 = out["0"][1], out["1"][1]
    for name, off, shape in ane.param_layout(cfg):
        n = int(np.prod(shape))
        a, b = g0[off:off + n], g1[off:off + n]
        if name.split(".")[-1] in ATOMIC_SEGMENTS:
            assert np.linalg.norm(a - b) <= 1e-5 * np.linalg.norm(a), name
        else:
            assert np.array_equal(a, b), name


@pytest.mark.parametrize("arch,fused,accum", [("llama2", "1", 1), ("llama2", "1", 2), ("nanochat", "1", 2),
                                              ("llama2", "0", 2)])
def test_flush_shadows_match_a_refresh_from_the_masters(arch, fused, accum, monkeypatch):
    """The flush writes the fp16 weight shadows in its update pass
    (ANE_FUSED_ADAM=1, the default; the transposed ones after it, on the dW
    stream beside the next forward in accumulate mode) or refreshes them
    after it: either way they equal what a refresh from the updated fp32
    masters writes (SetParams(Params())): the same loss and the same
    gradients, bit for bit (atomically summed segments aside)."""
    monkeypatch.setenv("ANE_FUSED_ADAM", fused)
    cfg = ane.tiny(arch, layers=2)
    p = ane.init_params(cfg, seed=71, std=0.05)
    stream = np.random.default_rng(72).integers(0, cfg.vocab, 4000).astype(np.uint16)
    tok, tgt = ane.make_tokens(cfg, 2, seed=73)
    eng = open_engine(cfg, p, max_batch=2, tokens=stream, AccumSteps=accum)
    try:
        for _ in range(2):
            eng.TrainBatch(2)
        assert eng.State().adam_t == 2
        runs = []
        for _ in range(2):
            loss = eng.EvalLoss(tok, tgt)
            runs.append((loss, eng.Grads(tok, tgt)[1]))
            eng.SetParams(eng.Params())
    finally:
        eng.Destroy()
    (la, ga), (lb, gb) = runs
    assert la[0] == lb[0]
    np.testing.assert_array_equal(la[1], lb[1])
    for name, off, shape in ane.param_layout(cfg):
        n = int(np.prod(shape))
        a, b = ga[off:off + n], gb[off:off + n]
        if name.split(".")[-1] in ATOMIC_SEGMENTS:
            assert np.linalg.norm(a - b) <= 1e-5 * np.linalg.norm(a), name
        else:
            assert np.array_equal(a, b), name


@pytest.mark.parametrize("arch", ["llama2", "nanochat"])
def test_flush_matches_oracle_adam(arch):
    """Clip + AdamW with the reference's parameter groups, two flushes."""
    cfg = ane.tiny(arch, layers=2)
    n = ane.param_count(cfg)
    r = np.random.default_rng(30)
    p = ane.init_params(cfg, seed=31, std=0.08)
    eng = open_engine(cfg, p, AccumSteps=2, LR=HP["lr"], AdamBeta1=HP["beta1"], AdamBeta2=HP["beta2"],
                      AdamEps=HP["eps"], WeightDecay=HP["weight_decay"], GradClip=HP["grad_clip"],
                      EmbedLRMult=HP["embed_lr_mult"], ScalarLRMult=HP["scalar_lr_mult"],
                      LambdaLRMult=HP["lambda_lr_mult"], LambdaBeta1=HP["lambda_beta1"],
                      LambdaBeta2=HP["lambda_beta2"])
    w_ref = p.copy()
    m_ref = np.zeros(n, np.float32)
    v_ref = np.zeros(n, np.float32)
    for step in (1, 2):
        raw = (r.standard_normal(n) * 3.0).astype(np.float32)   # loss-scaled sum over 2 pending steps
        eng.SetGrads(raw, pending=2)
        eng.Flush()
        g = raw * np.float32(1.0 / 2.0) / np.float32(256.0)
        oracle.adam_update(cfg, w_ref, g, m_ref, v_ref, step, HP)
        st = eng.State()
        assert st.adam_t == step and st.pending_steps == 0 and st.cum_batches == step
    w = eng.Params()
    m, v = eng.OptState()
    eng.Destroy()
    np.testing.assert_allclose(m, m_ref, rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(v, v_ref, rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(w, w_ref, rtol=1e-5, atol=1e-7)


def drand48_positions(seed, n, limit):
    st = oracle.lib().orc_drand48_seed(seed)
    import ctypes
    s = ctypes.c_uint64(st)
    out = []
    for _ in range(n):
        f = oracle.lib().orc_drand48_next(ctypes.byref(s))
        p = int(f * limit)
        out.append(min(p, limit - 1))
    return out


def test_steps_follow_reference_sampler_and_batch_equivalence():
    """Step draws windows with the reference's drand48 rule; TrainBatch(k)
    equals k Steps; AccumSteps accumulation flushes once per k windows."""
    cfg = ane.tiny("llama2", layers=2)
    p = ane.init_params(cfg, seed=40, std=0.08)
    stream = np.random.default_rng(41).integers(0, cfg.vocab, 3000).astype(np.uint16)
    kw = dict(AccumSteps=4, Seed=7, LR=1e-3, AdamBeta2=0.95, GradClip=1.0)
    a = open_engine(cfg, p, max_batch=4, tokens=stream, **kw)
    b = open_engine(cfg, p, max_batch=4, tokens=stream, **kw)
    limit = len(stream) - cfg.seq - 1
    pos = drand48_positions(7, 8, limit)
    for i in range(4):
        a.Step()
        assert a.State().token_pos == pos[i] + cfg.seq
    sa = a.State()
    assert sa.cum_steps == 4 and sa.adam_t == 1 and sa.pending_steps == 0 and sa.cum_batches == 1
    b.TrainBatch(4)
    sb = b.State()
    assert sb.token_pos == sa.token_pos and sb.adam_t == 1 and sb.cum_steps == 4
    np.testing.assert_allclose(a.Params(), b.Params(), rtol=1e-4, atol=2e-6)
    # the update itself equals oracle grads of those windows + AdamW
    tok = np.stack([stream[q:q + cfg.seq] for q in pos[:4]])
    tgt = np.stack([stream[q + 1:q + 1 + cfg.seq] for q in pos[:4]])
    _, g = oracle.grads(cfg, p, tok, tgt)
    w_ref = p.copy()
    n = ane.param_count(cfg)
    hp = dict(HP, lr=1e-3, beta2=0.95, weight_decay=0.0, grad_clip=1.0, embed_lr_mult=1.0, scalar_lr_mult=1.0,
              lambda_lr_mult=0.01, lambda_beta1=0.9, lambda_beta2=0.95)
    oracle.adam_update(cfg, w_ref, g, np.zeros(n, np.float32), np.zeros(n, np.float32), 1, hp)
    # Adam's first step is lr * g / (|g| + eps) ~ lr * sign(g): coordinates
    # whose gradient is at rounding level may flip, so the check is on sign
    # agreement weighted by the oracle's gradient magnitude.
    dw_ref = w_ref - p
    dw = b.Params() - p
    agree = np.sign(dw) == np.sign(dw_ref)
    wagree = np.abs(g[agree]).sum() / np.abs(g).sum()
    print(f"update sign agreement {agree.mean():.4f}, |g|-weighted {wagree:.6f}")
    assert wagree >= 0.999 and agree.mean() >= 0.95
    a.Destroy()
    b.Destroy()


def test_training_reduces_loss():
    cfg = ane.tiny("nanochat", layers=2)
    p = ane.init_params(cfg, seed=50, std=0.05)
    stream = np.tile(np.random.default_rng(51).integers(0, cfg.vocab, 200).astype(np.uint16), 5)
    eng = open_engine(cfg, p, max_batch=4, tokens=stream, AccumSteps=4, LR=3e-3, AdamBeta2=0.95)
    first = eng.TrainBatch(4).loss
    for _ in range(25):
        last = eng.TrainBatch(4).loss
    eng.Destroy()
    print(f"loss {first:.3f} -> {last:.3f}")
    assert last < first - 0.5


def test_training_error_behaviour():
    cfg = ane.tiny("llama2", layers=2)
    p = ane.init_params(cfg, seed=60)
    eng = open_engine(cfg, p)
    with pytest.raises(ane.EngineError, match="storiesane step: not enough tokens"):
        eng.Step()
    with pytest.raises(ane.EngineError, match="storiesane set lr: lr must be > 0"):
        eng.SetLR(0.0)
    eng.SetLR(1e-3)
    assert abs(eng.LR() - 1e-3) < 1e-9
    eng.Close()
    with pytest.raises(ane.EngineError, match="storiesane step: engine is closed"):
        eng.Step()
    eng.Destroy()


@pytest.mark.parametrize("arch,nseq,accum,calls", [("llama2", 8, 16, 2), ("llama2", 8, 8, 3), ("llama2", 2, 1, 3),
                                                    ("nanochat", 2, 2, 3)])
def test_async_update_matches_update_in_line(arch, nseq, accum, calls, monkeypatch):
    """The update of an accumulate-mode flush on the dW stream, in per-layer
    chunks the next forward waits for (ANE_ASYNC_UPDATE=1, the default),
    gives what the update in line on the main stream gives: the same losses
    call after call and the same weights and optimizer state (bit for bit
    where no atomically summed gradient feeds them).  Reading the weights
    waits for an update still running."""
    cfg = ane.stories110m(arch) if nseq == 8 else ane.tiny(arch, layers=2)
    p = ane.init_params(cfg, seed=81, std=0.05)
    stream = np.random.default_rng(82).integers(0, cfg.vocab, 64 * (cfg.seq + 1)).astype(np.uint16)
    out = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("ANE_ASYNC_UPDATE", flag)
        eng = open_engine(cfg, p, max_batch=nseq, tokens=stream, AccumSteps=accum, LR=1e-3, GradClip=1.0)
        try:
            losses = [eng.TrainBatch(nseq).loss for _ in range(calls)]
            w = eng.Params()
            m, v = eng.OptState()
            out[flag] = (losses, w, m, v, eng.State().adam_t)
        finally:
            eng.Destroy()
    pending, updates = 0, 0
    for _ in range(calls):  # TrainBatch flushes once pending >= AccumSteps
        pending += nseq
        if pending >= accum:
            pending, updates = 0, updates + 1
    assert out["0"][4] == out["1"][4] == updates
    # the atomically summed gradient segments (embedding rows of repeated
    # tokens, nanochat's value embeddings) round differently per run, and so
    # do the updates and losses that follow from them, by a few ulps
    # (the next forward rounds its activations to fp16, which turns such
    # differences into whole-ulp ones in a few activations; two runs of the
    # in-line update differ by ~4e-6 in every weight tensor after 3
    # updates, and by ~2e-4 in the moments, which follow the gradients.  A
    # forward reading a layer before its update would move that layer's
    # weights and gradients by ~lr / |w| ~ 2e-2.)
    np.testing.assert_allclose(out["0"][0], out["1"][0], rtol=1e-6)
    for what, a, b, tol in zip(("w", "m", "v"), out["0"][1:4], out["1"][1:4], (1e-4, 2e-3, 2e-3)):
        for name, off, shape in ane.param_layout(cfg):
            n = int(np.prod(shape))
            x, y = a[off:off + n].astype(np.float64), b[off:off + n].astype(np.float64)
            if updates == 1 and name.split(".")[-1] not in ATOMIC_SEGMENTS:
                assert np.array_equal(x, y), (what, name)
            else:
                assert np.linalg.norm(x - y) <= tol * max(np.linalg.norm(x), 1e-12), (what, name)


@pytest.mark.parametrize("arch,async_update", [("llama2", "1"), ("llama2", "0"), ("nanochat", "1")])
def test_step_result_phase_timers_and_flush_duration(arch, async_update, monkeypatch):
    """StepResult's phase durations (ane/engine.go:416-441) and Flush's
    return value (the weight-refresh time, added to CumTrainMS,
    ane/engine.go:484-496).  With the update asynchronous (the default) a
    flushing call reports the latest update that has completed: the one
    before its own."""
    monkeypatch.setenv("ANE_ASYNC_UPDATE", async_update)
    cfg = ane.tiny(arch, layers=2)
    p = ane.init_params(cfg, seed=61, std=0.05)
    stream = np.random.default_rng(62).integers(0, cfg.vocab, 4000).astype(np.uint16)
    eng = open_engine(cfg, p, max_batch=2, tokens=stream, AccumSteps=3)
    try:
        r1 = eng.TrainBatch(2)           # first call: set-up, no update yet
        assert r1.startup_compile_ns > 0 and r1.compile_ns == r1.startup_compile_ns
        assert r1.weight_refresh_ns == 0 and r1.adam_ns == 0
        for f in ("ane_eval_ns", "final_head_ns", "embed_grad_ns", "dw_gemm_ns"):
            assert getattr(r1, f) > 0, f
        assert (r1.rms_dw_ns > 0) == (arch == "llama2")
        assert r1.dw_gemm_ns + r1.embed_grad_ns < r1.ane_eval_ns <= r1.step_ns
        assert r1.final_head_ns < r1.ane_eval_ns
        # 4 pending >= 3: clip + AdamW; in accumulate mode the refresh runs
        # asynchronously and the step reports none (flushPending returns 0,
        # ane/engine.go:674-682); Flush waits for it and returns its duration
        r2 = eng.TrainBatch(2)
        assert r2.startup_compile_ns == 0
        assert (r2.adam_ns > 0 or async_update == "1") and r2.weight_refresh_ns == 0 and r2.compile_ns == 0
        assert eng.State().pending_steps == 0
        assert eng.Flush() > 0           # nothing pending: the outstanding refresh
        assert eng.Flush() == 0          # nothing pending, nothing outstanding
        eng.TrainBatch(2)                # 2 pending
        r4 = eng.TrainBatch(2)           # 4 pending: the second update
        assert r4.adam_ns > 0            # (asynchronous: the first one's, complete since the Flush)
        assert eng.State().adam_t == 2
        eng.Flush()
        eng.Step()                       # one pending window
        before = eng.State().cum_train_ms
        ns = eng.Flush()
        st = eng.State()
        assert ns > 0 and st.pending_steps == 0 and st.adam_t == 3
        assert abs((st.cum_train_ms - before) - ns / 1e6) < 1e-6
    finally:
        eng.Destroy()
