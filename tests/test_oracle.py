"""Pins the C oracle (oracle/refcpu.c) before anything is checked against it.

The reference ships no golden vectors for this path, so every oracle
function is pinned by closed forms, invariants, textbook routines (torch on
the CPU, libc's drand48) and an independent float64 PyTorch model with
autograd (tests/torch_ref.py) on tiny full models, for both architectures
and both gradient modes.  CPU only.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

import ane
import oracle
import torch_ref


def rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- ops ----
def test_param_layout_matches_python():
    for arch in ("llama2", "nanochat"):
        for cfg in (ane.tiny(arch), ane.stories110m(arch), ane.tiny(arch, layers=3)):
            segs = oracle.param_segments(cfg)
            py = [(off, int(np.prod(shape))) for _, off, shape in ane.param_layout(cfg)]
            assert segs == py
            assert oracle.param_count(cfg) == ane.param_count(cfg)
    assert ane.param_count(ane.stories110m("nanochat")) == 238_683_002
    assert ane.param_count(ane.stories110m("llama2")) == 109_529_856


def test_linear_cf_matches_f64_matmul():
    r = rng(1)
    w = r.standard_normal((96, 80), dtype=np.float32)
    x = r.standard_normal((80, 33), dtype=np.float32)
    out = oracle.linear_cf(w, x)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-4)
    # exact on integers (no rounding anywhere)
    wi = r.integers(-3, 4, (7, 5)).astype(np.float32)
    xi = r.integers(-3, 4, (5, 4)).astype(np.float32)
    assert np.array_equal(oracle.linear_cf(wi, xi), wi @ xi)


def test_rmsnorm_closed_form_and_torch():
    x = np.full((768, 4), 3.0, np.float32)
    out = oracle.rmsnorm_noweight_cf(x)
    np.testing.assert_allclose(out, 3.0 / math.sqrt(9.0 + 1e-5), rtol=1e-6)
    r = rng(2)
    x = r.standard_normal((768, 16), dtype=np.float32) * 5
    g = r.standard_normal(768, dtype=np.float32)
    ref = torch.nn.functional.rms_norm(torch.tensor(x.T, dtype=torch.float64), (768,),
                                       torch.tensor(g, dtype=torch.float64), eps=1e-5).numpy().T
    np.testing.assert_allclose(oracle.rmsnorm_cf(x, g), ref, rtol=1e-5, atol=1e-6)
    ref1 = torch.nn.functional.rms_norm(torch.tensor(x.T, dtype=torch.float64), (768,), eps=1e-5).numpy().T
    np.testing.assert_allclose(oracle.rmsnorm_noweight_cf(x), ref1, rtol=1e-5, atol=1e-6)


def test_rope_identity_at_pos0_and_norm_preserving():
    c, s = oracle.rope_tables(256, 64, 100000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # table values against an independent float64 formula
    i = np.arange(32)
    ang = 255 / (100000.0 ** (2 * i / 64))
    np.testing.assert_allclose(c[255], np.cos(ang), atol=1e-6)
    np.testing.assert_allclose(s[255], np.sin(ang), atol=1e-6)
    x = rng(3).standard_normal((768, 256), dtype=np.float32)
    y = oracle.apply_rope_cf(x, 12, c, s)
    np.testing.assert_array_equal(y[:, 0], x[:, 0])
    pn_x = x[0::2] ** 2 + x[1::2] ** 2
    pn_y = y[0::2] ** 2 + y[1::2] ** 2
    np.testing.assert_allclose(pn_y, pn_x, rtol=1e-4, atol=1e-5)
    # rotation direction: complex multiply by e^{i*ang}
    z = (x[0::2].astype(np.float64) + 1j * x[1::2]) * np.exp(1j * np.tile(
        (np.arange(256)[None, :] / (100000.0 ** (2 * np.arange(32)[:, None] / 64))), (12, 1)))
    np.testing.assert_allclose(y[0::2], z.real, atol=2e-4)
    np.testing.assert_allclose(y[1::2], z.imag, atol=2e-4)


def test_qknorm_rms_closed_form():
    r = rng(4)
    q = r.standard_normal((768, 8), dtype=np.float32) * 3
    k = r.standard_normal((768, 8), dtype=np.float32) * 0.01
    qn, kn = oracle.qknorm_cf(q, k, 12)
    for src, dst in ((q, qn), (k, kn)):
        ms = (src.reshape(12, 64, 8).astype(np.float64) ** 2).mean(1)
        got = np.sqrt((dst.reshape(12, 64, 8).astype(np.float64) ** 2).mean(1))
        np.testing.assert_allclose(got, 1.2 * np.sqrt(ms / (ms + 1e-5)), rtol=1e-5)


def test_attention_special_cases_and_torch():
    r = rng(5)
    D, S, NH = 128, 40, 2
    q = r.standard_normal((D, S), dtype=np.float32)
    k = r.standard_normal((D, S), dtype=np.float32)
    v = r.standard_normal((D, S), dtype=np.float32)
    out = oracle.causal_attention_cf(q, k, v, NH)
    np.testing.assert_allclose(out[:, 0], v[:, 0], rtol=1e-6)       # row 0 = v[:,0]
    q0 = np.zeros_like(q)
    out0 = oracle.causal_attention_cf(q0, k, v, NH)                   # q=0 -> prefix means
    pref = np.cumsum(v.astype(np.float64), 1) / np.arange(1, S + 1)
    np.testing.assert_allclose(out0, pref, rtol=1e-5, atol=1e-6)
    ref = torch_ref.attention(torch.tensor(q.T, dtype=torch.float64), torch.tensor(k.T, dtype=torch.float64),
                              torch.tensor(v.T, dtype=torch.float64), NH, 1 / 8.0).numpy().T
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_softcap_and_cross_entropy():
    x = np.linspace(-100, 100, 1001, dtype=np.float32)
    np.testing.assert_allclose(oracle.softcap(x), 15 * np.tanh(x.astype(np.float64) / 15), rtol=1e-6, atol=1e-6)
    V, S = 32000, 4
    loss, dl = oracle.cross_entropy(np.zeros((V, S), np.float32), np.array([0, 5, 31999, 7], np.uint16))
    assert abs(loss - math.log(32000)) < 1e-5                         # ln 32000 = 10.373491
    r = rng(6)
    lg = r.standard_normal((V, S), dtype=np.float32) * 3
    tg = np.array([1, 2, 3, 4], np.uint16)
    loss, dl = oracle.cross_entropy(lg, tg)
    tl = torch.tensor(lg.T, dtype=torch.float64, requires_grad=True)
    ref = torch.nn.functional.cross_entropy(tl, torch.tensor(tg.astype(np.int64)))
    ref.backward()
    assert abs(loss - ref.item()) < 1e-5
    np.testing.assert_allclose(dl, tl.grad.numpy().T, atol=1e-7)
    # out-of-range targets are excluded from the mean and get zero grad
    tg2 = np.array([1, 40000, 3, 4], np.uint16)
    loss2, dl2 = oracle.cross_entropy(lg, tg2)
    keep = torch.tensor([0, 2, 3])
    ref2 = torch.nn.functional.cross_entropy(torch.tensor(lg.T, dtype=torch.float64)[keep],
                                             torch.tensor(tg2.astype(np.int64))[keep])
    assert abs(loss2 - ref2.item()) < 1e-5
    assert np.all(dl2[:, 1] == 0)


def test_drand48_matches_libc():
    libc = ctypes.CDLL(None)
    libc.drand48.restype = ctypes.c_double
    libc.srand48.argtypes = [ctypes.c_long]
    for seed in (42, 7, 123456789):
        libc.srand48(seed)
        want = [libc.drand48() for _ in range(5)]
        got = oracle.drand48_stream(seed, 5)
        np.testing.assert_array_equal(got, want)


# --------------------------------------------------------- full model ----
def _tiny(arch, grad_mode="true", **kw):
    base = dict(dim=64, hidden=96, heads=2, layers=4, vocab=97, seq=12, arch=arch, grad_mode=grad_mode)
    base.update(kw)
    return ane.Config(**base)


def _setup(cfg, nseq=2, seed=11, std=0.3):
    p = ane.init_params(cfg, seed=seed, std=std)
    tok, tgt = ane.make_tokens(cfg, nseq, seed + 1)
    return p, tok, tgt


@pytest.mark.parametrize("arch", ["llama2", "nanochat"])
def test_forward_matches_torch_f64(arch):
    cfg = _tiny(arch)
    p, tok, tgt = _setup(cfg)
    loss, per, lg = oracle.forward_loss(cfg, p, tok, tgt, want_logits=True)
    P = torch_ref.params_to_torch(cfg, p, requires_grad=False)
    tl, tlog = torch_ref.model_loss(cfg, P, torch.tensor(tok.astype(np.int64)), torch.tensor(tgt.astype(np.int64)))
    assert abs(loss - tl.item()) < 2e-5
    np.testing.assert_allclose(lg.transpose(0, 2, 1), tlog.numpy(), atol=2e-4)


@pytest.mark.parametrize("arch,mode", [("llama2", "true"), ("nanochat", "true"), ("nanochat", "compat")])
def test_grads_match_torch_autograd(arch, mode):
    cfg = _tiny(arch, mode)
    p, tok, tgt = _setup(cfg)
    loss, g = oracle.grads(cfg, p, tok, tgt)
    P = torch_ref.params_to_torch(cfg, p)
    tl, _ = torch_ref.model_loss(cfg, P, torch.tensor(tok.astype(np.int64)),
                                 torch.tensor(tgt.astype(np.int64)), grad_mode=mode)
    tl.backward()
    ref = torch_ref.grads_flat(cfg, P)
    assert abs(loss - tl.item()) < 2e-5
    for name, off, shape in ane.param_layout(cfg):
        n = int(np.prod(shape))
        a, b = g[off:off + n].astype(np.float64), ref[off:off + n]
        err = np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)
        assert err < 2e-4, (name, err)


def test_compat_differs_from_true_grad():
    """The four reference quirks change the nanochat gradient (so the compat
    test above is not vacuous)."""
    p, tok, tgt = _setup(_tiny("nanochat"))
    _, gc = oracle.grads(_tiny("nanochat", "compat"), p, tok, tgt)
    _, gt = oracle.grads(_tiny("nanochat", "true"), p, tok, tgt)
    lay = {n: (o, int(np.prod(s))) for n, o, s in ane.param_layout(_tiny("nanochat"))}
    o, n = lay["layers.0.wq"]
    assert np.linalg.norm(gc[o:o + n] - gt[o:o + n]) > 0.1 * np.linalg.norm(gt[o:o + n])


def test_true_grad_finite_difference():
    cfg = _tiny("llama2", layers=2, seq=6)
    p, tok, tgt = _setup(cfg, nseq=1, std=0.3)
    P = torch_ref.params_to_torch(cfg, p)
    loss, g = oracle.grads(cfg, p, tok, tgt)
    r = rng(9)
    idx = r.choice(p.size, 12, replace=False)
    pd = p.astype(np.float64)
    for i in idx:
        h = 1e-3
        plus, minus = pd.copy(), pd.copy()
        plus[i] += h
        minus[i] -= h
        fp = torch_ref.model_loss(cfg, torch_ref.params_to_torch(cfg, plus, False),
                                  torch.tensor(tok.astype(np.int64)), torch.tensor(tgt.astype(np.int64)))[0].item()
        fm = torch_ref.model_loss(cfg, torch_ref.params_to_torch(cfg, minus, False),
                                  torch.tensor(tok.astype(np.int64)), torch.tensor(tgt.astype(np.int64)))[0].item()
        fd = (fp - fm) / (2 * h)
        assert abs(fd - g[i]) < 1e-4 + 1e-3 * abs(fd), (i, fd, g[i])


def test_out_of_range_tokens_and_targets():
    cfg = _tiny("nanochat")
    p, tok, tgt = _setup(cfg, nseq=1)
    tok = tok.copy()
    tgt = tgt.copy()
    tok[0, 3] = 60000        # embed row -> zeros (ane/stories/cpu.go:60-64)
    tgt[0, 5] = 60000        # excluded from the mean (ane/stories/cpu.go:253-257)
    loss, per, lg = oracle.forward_loss(cfg, p, tok, tgt, want_logits=True)
    P = torch_ref.params_to_torch(cfg, p, requires_grad=False)
    P["embed"] = torch.cat([P["embed"], torch.zeros(60001 - cfg.vocab, cfg.dim, dtype=torch.float64)])
    for name in list(P):
        if name.endswith("ve_embed"):
            P[name] = torch.cat([P[name], torch.zeros(60001 - cfg.vocab, cfg.dim, dtype=torch.float64)])
    tl, tlog = torch_ref.model_loss(cfg, P, torch.tensor(tok.astype(np.int64)), torch.tensor(tgt.astype(np.int64)))
    # torch's logits now include the zero rows appended for the lookup; compare the real vocab only
    np.testing.assert_allclose(lg[0].T, tlog[0, :, :cfg.vocab].numpy(), atol=2e-4)


def test_adam_closed_form_and_groups():
    cfg = _tiny("nanochat")
    n = ane.param_count(cfg)
    r = rng(10)
    w = r.standard_normal(n, dtype=np.float32)
    g = r.standard_normal(n, dtype=np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=0.0,
              embed_lr_mult=2.0, scalar_lr_mult=0.5, lambda_lr_mult=0.01, lambda_beta1=0.96, lambda_beta2=0.95)
    w1 = w.copy()
    oracle.adam_update(cfg, w1, g.copy(), m, v, 1, hp)
    lay = {nm: (o, int(np.prod(s))) for nm, o, s in ane.param_layout(cfg)}
    def upd(name, lr, wd):
        o, k = lay[name]
        return w[o:o + k] - lr * (g[o:o + k] / (np.abs(g[o:o + k]) + 1e-8) + wd * w[o:o + k])
    for name, lr, wd in (("layers.0.wq", 3e-4, 0.1), ("layers.1.ve_embed", 6e-4, 0.0),
                         ("layers.1.ve_gate", 1.5e-4, 0.0), ("embed", 6e-4, 0.0),
                         ("smear_gate", 3e-4, 0.1), ("smear_lambda", 1.5e-4, 0.0),
                         ("resid_lambdas", 1.5e-6, 0.0)):
        o, k = lay[name]
        np.testing.assert_allclose(w1[o:o + k], upd(name, lr, wd), rtol=1e-5, atol=1e-7)
    # clipping: global L2 over layer grads + embed only
    hp["grad_clip"] = 1.0
    g2 = g.copy()
    oracle.adam_update(cfg, w.copy(), g2, np.zeros(n, np.float32), np.zeros(n, np.float32), 1, hp)
    lo, hi = lay["layers.0.wq"][0], lay["embed"][0] + lay["embed"][1]
    norm = np.sqrt((g[lo:hi].astype(np.float64) ** 2).sum())
    np.testing.assert_allclose(g2[lo:hi], g[lo:hi] * (1.0 / norm), rtol=1e-5)
    o, k = lay["smear_gate"]
    np.testing.assert_array_equal(g2[o:o + k], g[o:o + k])


def test_adam_moment_decay_closed_forms():
    """AdamW past the first step, pinned by two closed forms that exercise the
    moment decay and bias correction of every parameter group
    (ane/train_full.go:1107-1150, groups ane/engine.go:659-673):
      (a) a constant gradient g at every step keeps m_hat = g and
          v_hat = g^2, so each step is w -= lr (g / (|g| + eps) + wd w);
      (b) g at step 1 and 0 at step 2 give m_hat = b1 g / (1 + b1) and
          v_hat = b2 g^2 / (1 + b2) at step 2, with each group's own betas
          (the lambdas use lambda_beta1/2)."""
    cfg = _tiny("nanochat")
    n = ane.param_count(cfg)
    r = rng(11)
    w0 = r.standard_normal(n, dtype=np.float32)
    g = r.standard_normal(n, dtype=np.float32)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, grad_clip=0.0,
              embed_lr_mult=2.0, scalar_lr_mult=0.5, lambda_lr_mult=0.01, lambda_beta1=0.8, lambda_beta2=0.7)
    lay = {nm: (o, int(np.prod(s))) for nm, o, s in ane.param_layout(cfg)}
    groups = (("layers.0.wq", 3e-4, 0.1, 0.9, 0.95), ("layers.1.ve_embed", 6e-4, 0.0, 0.9, 0.95),
              ("embed", 6e-4, 0.0, 0.9, 0.95), ("smear_gate", 3e-4, 0.1, 0.9, 0.95),
              ("smear_lambda", 1.5e-4, 0.0, 0.9, 0.95), ("resid_lambdas", 1.5e-6, 0.0, 0.8, 0.7),
              ("x0_lambdas", 1.5e-6, 0.0, 0.8, 0.7))
    # (a) five steps of the same gradient
    w = w0.copy()
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    for t in range(1, 6):
        oracle.adam_update(cfg, w, g.copy(), m, v, t, hp)
    for name, lr, wd, _, _ in groups:
        o, k = lay[name]
        ref = w0[o:o + k].astype(np.float64)
        gg = g[o:o + k].astype(np.float64)
        for _ in range(5):
            ref = ref - lr * (gg / (np.abs(gg) + 1e-8) + wd * ref)
        np.testing.assert_allclose(w[o:o + k], ref, rtol=2e-6, atol=2e-7, err_msg=name)
    # (b) g, then a zero gradient
    w = w0.copy()
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    oracle.adam_update(cfg, w, g.copy(), m, v, 1, hp)
    w1 = w.copy()
    oracle.adam_update(cfg, w, np.zeros(n, np.float32), m, v, 2, hp)
    for name, lr, wd, b1, b2 in groups:
        o, k = lay[name]
        gg = g[o:o + k].astype(np.float64)
        mh = b1 * gg / (1 + b1)
        vh = b2 * gg * gg / (1 + b2)
        ref = w1[o:o + k] - lr * (mh / (np.sqrt(vh) + 1e-8) + wd * w1[o:o + k].astype(np.float64))
        np.testing.assert_allclose(w[o:o + k], ref, rtol=2e-6, atol=2e-7, err_msg=name)
