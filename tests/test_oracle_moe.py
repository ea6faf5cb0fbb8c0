"""Pins the MoE oracle (oracle/refmoe.c) on the CPU: routing by closed forms
(one-hot routers make the logits equal chosen input components, ties go to
the lower expert), the expert FFN and combine against an independent
float64 PyTorch restatement, and token independence (the property the
full-size GPU test relies on to check a sample of tokens)."""
import numpy as np
import torch
import torch.nn.functional as F

import ane
import oracle
from ane.moe import MoeConfig, init_moe_params, make_moe_input, moe_param_layout, moe_param_count


def _cfg():
    return MoeConfig(dim=64, hidden=96, experts=8)


def test_param_layout_count():
    for cfg in (_cfg(), MoeConfig()):
        lay = moe_param_layout(cfg)
        name, off, shape = lay[-1]
        assert off + int(np.prod(shape)) == moe_param_count(cfg) == oracle.moe_param_count(cfg.dim, cfg.hidden,
                                                                                           cfg.experts)
    assert moe_param_count(MoeConfig()) == 8 * 768 + 8 * 3 * 2048 * 768


def test_route_closed_forms_and_ties():
    cfg = _cfg()
    p = init_moe_params(cfg, seed=1)
    router = p[:cfg.experts * cfg.dim].reshape(cfg.experts, cfg.dim)
    router[...] = 0.0
    for e in range(cfg.experts):
        router[e, e] = 1.0  # logit e = x[:, e]
    x = np.zeros((5, cfg.dim), np.float32)
    x[0, :8] = [0.1, 0.9, 0.3, 0.8, 0.0, 0.0, 0.0, 0.0]   # -> 1, 3
    x[1, :8] = [0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5]   # all tied -> 0, 1
    x[2, :8] = [0.0, 0.2, 0.7, 0.2, 0.7, 0.0, 0.0, 0.0]   # tie for first -> 2, 4
    x[3, :8] = [-1, -2, -3, -4, -5, -6, -7, -0.5]         # -> 7, 0
    x[4, :8] = [0.0, 0.3, 0.0, 0.3, 0.0, 0.3, 0.0, 0.0]   # three-way tie -> 1, 3
    idx, w = oracle.moe_route(p, x, cfg.hidden, cfg.experts)
    assert idx.tolist() == [[1, 3], [0, 1], [2, 4], [7, 0], [1, 3]]
    # weights: softmax over the two chosen logits
    np.testing.assert_allclose(w[0], [1 / (1 + np.exp(-0.1)), np.exp(-0.1) / (1 + np.exp(-0.1))], rtol=1e-6)
    np.testing.assert_allclose(w[1], [0.5, 0.5])
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)


def _torch_moe(cfg, p, x):
    D, H, E = cfg.dim, cfg.hidden, cfg.experts
    P = {n: torch.tensor(p[off:off + int(np.prod(s))].reshape(s).astype(np.float64)) for n, off, s in
         moe_param_layout(cfg)}
    xt = torch.tensor(x.astype(np.float64))
    logits = xt @ P["router"].T
    top = torch.topk(logits, 2, dim=-1)
    w = torch.softmax(top.values, -1)
    out = torch.zeros_like(xt)
    for k in range(2):
        for e in range(E):
            m = top.indices[:, k] == e
            if m.any():
                xe = xt[m]
                h = F.silu(xe @ P[f"experts.{e}.w1"].T) * (xe @ P[f"experts.{e}.w3"].T)
                out[m] += w[m, k:k + 1] * (h @ P[f"experts.{e}.w2"].T)
    return out.numpy(), top.indices.numpy(), w.numpy()


def test_forward_matches_torch_f64():
    cfg = _cfg()
    p = init_moe_params(cfg, seed=2, std=0.1)
    x = make_moe_input(cfg, 40, seed=3)
    out, idx, w = oracle.moe_forward(p, x, cfg.hidden, cfg.experts)
    ref, ridx, rw = _torch_moe(cfg, p, x)
    np.testing.assert_array_equal(idx, ridx)  # random logits: no near-ties at this size
    np.testing.assert_allclose(w, rw, rtol=1e-5)
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


def test_tokens_are_independent():
    cfg = _cfg()
    p = init_moe_params(cfg, seed=4)
    x = make_moe_input(cfg, 64, seed=5)
    out, idx, w = oracle.moe_forward(p, x, cfg.hidden, cfg.experts)
    sel = np.array([3, 17, 40, 63])
    o2, i2, w2 = oracle.moe_forward(p, x[sel], cfg.hidden, cfg.experts)
    np.testing.assert_array_equal(o2, out[sel])
    np.testing.assert_array_equal(i2, idx[sel])
