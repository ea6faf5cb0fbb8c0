"""Pins of the seam oracle (oracle/refseam.c): the per-object layer forward,
layer backward and offload functions the reference's accelerator programs
compute, against independent float64 formulations in torch -- RoPE as a
complex rotation, attention by torch's scaled_dot_product_attention, and
every backward as automatic differentiation of the forward it belongs to.
A dropped score scale, a transposed weight or a wrong rotation pair fails
one of them.  CPU only."""
import numpy as np
import pytest
import torch

import oracle

D, H, NH, S, V = 128, 256, 2, 64, 320
HD = D // NH


def weights(rng, scale=0.08):
    shapes = {"wq": (D, D), "wk": (D, D), "wv": (D, D), "wo": (D, D), "w1": (H, D), "w2": (D, H)}
    return {n: (rng.standard_normal(s) * scale).astype(np.float32) for n, s in shapes.items()}


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


def rms64(x):
    return x / torch.sqrt((x * x).mean(dim=0, keepdim=True) + 1e-5)


def rope64(x):
    """Rotate channel pairs (2i, 2i+1) of each head by t / 100000^(2i/64),
    as one complex multiplication per pair."""
    seq = x.shape[1]
    xh = x.reshape(NH, HD // 2, 2, seq)
    z = torch.complex(xh[:, :, 0, :], xh[:, :, 1, :])
    i = torch.arange(HD // 2, dtype=torch.float64)[:, None]
    t = torch.arange(seq, dtype=torch.float64)[None, :]
    z = z * torch.polar(torch.ones_like(t * i), t / torch.pow(100000.0, 2 * i / HD))
    return torch.stack([z.real, z.imag], dim=2).reshape(D, seq)


def attention64(q, k, v):
    """Causal attention of channel-first q, k, v at scale 1/sqrt(head_dim)."""
    seq = q.shape[1]
    heads = lambda a: a.reshape(NH, HD, seq).transpose(1, 2)
    o = torch.nn.functional.scaled_dot_product_attention(heads(q), heads(k), heads(v), is_causal=True)
    return o.transpose(1, 2).reshape(D, seq)


def close(a, b, tol):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    err = np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)
    assert err <= tol, err


def test_layer_forward_and_taps_match_float64():
    rng = np.random.default_rng(1)
    w = weights(rng)
    x = rng.standard_normal((D, S)).astype(np.float32)
    out, taps = oracle.seam_layer_forward(w, NH, x)
    W = {n: t64(a) for n, a in w.items()}
    xn = rms64(t64(x))
    q = rope64(W["wq"] @ xn)
    k = rope64(W["wk"] @ xn)
    v = W["wv"] @ xn
    att = attention64(q, k, v)
    x2 = t64(x) + W["wo"] @ att
    x2n = rms64(x2)
    h1 = W["w1"] @ x2n
    gate = torch.relu(h1) ** 2
    ref = x2 + W["w2"] @ gate
    close(out, ref, 2e-6)
    for name, r in (("x_norm", xn), ("q", q), ("k", k), ("v", v), ("att_out", att), ("x2", x2), ("x2_norm", x2n),
                    ("h1", h1), ("gate", gate)):
        close(taps[name], r, 2e-6)
    # the taps the reference derives on the host from others, exactly
    assert np.array_equal(taps["gate"], np.where(taps["h1"] <= 0, 0, taps["h1"] * taps["h1"]).astype(np.float32))
    assert np.array_equal(taps["x2_norm"], oracle.rmsnorm_noweight_cf(taps["x2"]))


def test_attention_backward_is_the_gradient_of_the_attention_block():
    rng = np.random.default_rng(2)
    w = weights(rng)
    q, k, v = (rng.standard_normal((D, S)).astype(np.float32) for _ in range(3))
    dx2 = rng.standard_normal((D, S)).astype(np.float32)
    dxn, dq, dk, dv = oracle.seam_attention_backward(w, NH, q, k, v, dx2)
    W = {n: t64(a) for n, a in w.items()}
    Q, K, Vv = (t64(a).requires_grad_() for a in (q, k, v))
    # x2 = x + Wo attention(q, k, v): the block's output gradient dx2 reaches q, k, v through Wo
    (t64(dx2) * (W["wo"] @ attention64(Q, K, Vv))).sum().backward()
    close(dq, Q.grad, 5e-6)
    close(dk, K.grad, 5e-6)
    close(dv, Vv.grad, 5e-6)
    # dx_norm: q, k, v = W xn, so xn collects Wq^T dq + Wk^T dk + Wv^T dv
    xn = torch.zeros(D, S, dtype=torch.float64, requires_grad=True)
    ((t64(dq) * (W["wq"] @ xn)).sum() + (t64(dk) * (W["wk"] @ xn)).sum() + (t64(dv) * (W["wv"] @ xn)).sum()).backward()
    close(dxn, xn.grad, 2e-6)


def test_ffn_backward_is_the_gradient_of_the_ffn_block():
    rng = np.random.default_rng(3)
    w = weights(rng)
    h1 = rng.standard_normal((H, S)).astype(np.float32)
    dffn = rng.standard_normal((D, S)).astype(np.float32)
    dxn, dh1 = oracle.seam_ffn_backward(w, dffn, h1)
    W = {n: t64(a) for n, a in w.items()}
    Hh = t64(h1).requires_grad_()
    (t64(dffn) * (W["w2"] @ torch.relu(Hh) ** 2)).sum().backward()
    close(dh1, Hh.grad, 2e-6)
    xn = torch.zeros(D, S, dtype=torch.float64, requires_grad=True)
    (t64(dh1) * (W["w1"] @ xn)).sum().backward()
    close(dxn, xn.grad, 2e-6)


def test_offload_functions_match_float64():
    rng = np.random.default_rng(4)
    embed = (rng.standard_normal((V, D)) * 0.5).astype(np.float32)
    xn = rng.standard_normal((D, S)).astype(np.float32)
    logits = oracle.matmul_vocab_seq(embed, xn)
    close(logits, t64(embed) @ t64(xn), 2e-6)
    probs = oracle.seam_softmax_vocab(logits)
    close(probs, torch.softmax(t64(logits), dim=0), 2e-6)
    np.testing.assert_allclose(probs.sum(axis=0), 1.0, rtol=1e-5)
    dl = rng.standard_normal((V, S)).astype(np.float32)
    close(oracle.matmul_embed_t(embed, dl), t64(embed).T @ t64(dl), 2e-6)
    x = rng.standard_normal((D, S)).astype(np.float32) * 3
    dy = rng.standard_normal((D, S)).astype(np.float32)
    X = t64(x).requires_grad_()
    (t64(dy) * rms64(X)).sum().backward()
    close(oracle.rmsnorm_noweight_bwd_cf(dy, x), X.grad, 2e-6)
    close(oracle.rmsnorm_noweight_cf(x), rms64(t64(x)), 2e-6)


@pytest.mark.parametrize("planted", ["scale_one", "transposed_wo"])
def test_pins_catch_planted_mistakes(planted):
    """The autograd pin rejects an attention backward at score scale 1 (the
    CPU path's own backward, ane/train_full.go:268-269) and one that skips
    the Wo transpose."""
    rng = np.random.default_rng(5)
    w = weights(rng)
    q, k, v = (rng.standard_normal((D, S)).astype(np.float32) for _ in range(3))
    dx2 = rng.standard_normal((D, S)).astype(np.float32)
    W = {n: t64(a) for n, a in w.items()}
    Q, K, Vv = (t64(a).requires_grad_() for a in (q, k, v))
    (t64(dx2) * (W["wo"] @ attention64(Q, K, Vv))).sum().backward()
    if planted == "scale_one":
        da = oracle.linear_cf(np.ascontiguousarray(w["wo"].T), dx2)
        import ctypes as C
        dq, dk, dv = (np.zeros_like(q) for _ in range(3))
        f = oracle._f
        oracle.lib().orc_causal_attention_bwd_cf(f(dq), f(dk), f(dv), f(da), f(q), f(k), f(v), NH, HD, S,
                                                 C.c_float(1.0))
    else:
        w2 = dict(w, wo=np.ascontiguousarray(w["wo"].T))
        _, dq, dk, dv = oracle.seam_attention_backward(w2, NH, q, k, v, dx2)
    err = np.abs(dq - Q.grad.numpy()).max() / np.abs(Q.grad.numpy()).max()
    assert err > 1e-2
