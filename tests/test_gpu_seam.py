"""The per-object seam (include/ane_objects.h through ane.objects) against the
seam oracle (oracle/refseam.c) at the reference's shapes: stories dim 768,
hidden 2048, 12 heads, seq 256, vocab 32000 (ane/stories/config.go:4-10),
and a shorter sequence.  Bounds are the contract's: weight-gradient-like
outputs (the backward objects' dx, dq, dk, dv, dh1 and the classifier's dy)
at relative L2 <= 1e-2, logits at max-abs <= 2e-2, activations and taps at
relative L2 <= 5e-3 (fp16 operands, fp32 accumulation)."""
import numpy as np
import pytest

import oracle
from ane import objects

pytestmark = pytest.mark.gpu

D, H, NH, V = 768, 2048, 12, 32000


def layer_weights(rng, dim=D, hidden=H):
    def m(o, i):
        return (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)
    return {"wq": m(dim, dim), "wk": m(dim, dim), "wv": m(dim, dim), "wo": m(dim, dim), "w1": m(hidden, dim),
            "w2": m(dim, hidden)}


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def check(name, got, ref, tol):
    err = rel_l2(got, ref)
    print(f"{name}: rel L2 {err:.2e}", flush=True)
    assert err <= tol, (name, err)


@pytest.mark.parametrize("seq", [256, 128])
def test_layer_forward_and_taps_match_oracle(seq):
    print(f"seam layer forward seq={seq}", flush=True)
    rng = np.random.default_rng(10 + seq)
    w = layer_weights(rng)
    x = rng.standard_normal((D, seq)).astype(np.float32)
    ref_out, ref_taps = oracle.seam_layer_forward(w, NH, x)
    lf = objects.compile_stories_layer_forward(w, seq, heads=NH)
    out = np.full(D * seq, np.nan, np.float32)
    cache = objects.LayerCache(D, H, seq)
    lf.run_with_taps(out, x.ravel(), cache)
    assert cache.att_taps_ready and cache.ffn_taps_ready
    check("out", out, ref_out, 5e-3)
    for n in ("x_norm", "q", "k", "v", "att_out", "x2", "x2_norm", "h1", "gate"):
        check(n, getattr(cache, n), ref_taps[n], 5e-3)
    # the reference squares the h1 tap on the host: gate is exactly relu(h1)^2 of it
    h1 = cache.h1
    assert np.array_equal(cache.gate, np.where(h1 <= 0, 0, h1 * h1).astype(np.float32))
    # run (no taps) computes the same output, bit for bit
    out2 = np.full(D * seq, np.nan, np.float32)
    lf.run(out2, x.ravel())
    assert np.array_equal(out, out2)
    lf.close()


@pytest.mark.parametrize("seq", [256, 128])
def test_layer_backward_matches_oracle(seq):
    print(f"seam layer backward seq={seq}", flush=True)
    rng = np.random.default_rng(20 + seq)
    w = layer_weights(rng)
    x = rng.standard_normal((D, seq)).astype(np.float32)
    _, taps = oracle.seam_layer_forward(w, NH, x)  # realistic q, k, v, h1
    dx2 = rng.standard_normal((D, seq)).astype(np.float32)
    dffn = rng.standard_normal((D, seq)).astype(np.float32)
    lb = objects.compile_stories_layer_backward(w, seq, heads=NH)
    outs = [np.full(D * seq, np.nan, np.float32) for _ in range(4)]
    lb.run_attention(*outs, taps["q"].ravel(), taps["k"].ravel(), taps["v"].ravel(), dx2.ravel())
    ref = oracle.seam_attention_backward(w, NH, taps["q"], taps["k"], taps["v"], dx2)
    for n, got, r in zip(("dx_norm", "dq", "dk", "dv"), outs, ref):
        check(n, got, r, 1e-2)
    dxn = np.full(D * seq, np.nan, np.float32)
    dh1 = np.full(H * seq, np.nan, np.float32)
    lb.run_ffn(dxn, dh1, dffn.ravel(), taps["h1"].ravel())
    ref_dx, ref_dh1 = oracle.seam_ffn_backward(w, dffn, taps["h1"])
    check("ffn dx_norm", dxn, ref_dx, 1e-2)
    check("dh1", dh1, ref_dh1, 1e-2)
    lb.close()


def test_offload_matches_oracle():
    print("seam offload vocab=32000 seq=256", flush=True)
    seq = 256
    rng = np.random.default_rng(30)
    embed = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    xn = oracle.rmsnorm_noweight_cf(rng.standard_normal((D, seq)).astype(np.float32) * 2)
    off = objects.new_offload(embed, seq)
    for has in (off.has_rms_forward, off.has_classifier_forward, off.has_softmax, off.has_classifier_backward,
                off.has_rms_backward):
        assert has()
    logits = np.full(V * seq, np.nan, np.float32)
    off.run_classifier_forward(logits, xn.ravel())
    ref_logits = oracle.matmul_vocab_seq(embed, xn)
    err = np.abs(logits - ref_logits.ravel()).max()
    print(f"logits max-abs {err:.2e}", flush=True)
    assert err <= 2e-2
    check("logits", logits, ref_logits, 5e-3)
    # softmax over the vocabulary, in place, of the logits the caller holds
    probs = ref_logits.ravel().copy()
    off.run_softmax(probs)
    ref_probs = oracle.seam_softmax_vocab(ref_logits)
    assert np.abs(probs - ref_probs.ravel()).max() <= 1e-6
    np.testing.assert_allclose(probs.reshape(V, seq).sum(0), 1.0, rtol=1e-4)
    # classifier + softmax in one call
    probs2 = np.full(V * seq, np.nan, np.float32)
    off.run_classifier_softmax(probs2, xn.ravel())
    check("classifier softmax", probs2, oracle.seam_softmax_vocab(ref_logits), 5e-3)
    # dy = Embed^T dlogits (the head's softmax - onehot gradients)
    dl = (ref_probs - (rng.random((V, seq)) < 1.0 / V)).astype(np.float32) / seq
    dy = np.full(D * seq, np.nan, np.float32)
    off.run_classifier_backward(dy, dl.ravel())
    check("dy", dy, oracle.matmul_embed_t(embed, dl), 1e-2)
    # parameterless RMSNorm, forward and backward
    x = (rng.standard_normal((D, seq)) * 3).astype(np.float32)
    g = rng.standard_normal((D, seq)).astype(np.float32)
    r = np.full(D * seq, np.nan, np.float32)
    off.run_rms_forward(r, x.ravel())
    check("rms forward", r, oracle.rmsnorm_noweight_cf(x), 1e-5)
    off.run_rms_backward(r, g.ravel(), x.ravel())
    check("rms backward", r, oracle.rmsnorm_noweight_bwd_cf(g, x), 1e-5)
    off.close()


def test_refresh_close_and_disable():
    print("seam refresh / close / disable", flush=True)
    seq, dim, hidden, heads, vocab = 128, 256, 512, 4, 1024
    rng = np.random.default_rng(40)
    w0, w1 = layer_weights(rng, dim, hidden), layer_weights(rng, dim, hidden)
    x = rng.standard_normal((dim, seq)).astype(np.float32)
    lf = objects.compile_stories_layer_forward(w0, seq, heads=heads)
    out = np.zeros(dim * seq, np.float32)
    lf.refresh_weights(w1)  # refreshWeights restages: results follow the new weights
    lf.run(out, x.ravel())
    check("refreshed forward", out, oracle.seam_layer_forward(w1, heads, x)[0], 5e-3)
    lf.close()
    with pytest.raises(objects.SeamError, match="run layer forward: layer is closed"):
        lf.run(out, x.ravel())
    lb = objects.compile_stories_layer_backward(w0, seq, heads=heads)
    lb.refresh_weights(w1)
    dffn = rng.standard_normal((dim, seq)).astype(np.float32)
    h1 = rng.standard_normal((hidden, seq)).astype(np.float32)
    dxn, dh1 = np.zeros(dim * seq, np.float32), np.zeros(hidden * seq, np.float32)
    lb.run_ffn(dxn, dh1, dffn.ravel(), h1.ravel())
    check("refreshed ffn backward", dxn, oracle.seam_ffn_backward(w1, dffn, h1)[0], 1e-2)
    lb.close()
    with pytest.raises(objects.SeamError, match="run layer backward ffn: layer is closed"):
        lb.run_ffn(dxn, dh1, dffn.ravel(), h1.ravel())
    e0 = (rng.standard_normal((vocab, dim)) * 0.05).astype(np.float32)
    e1 = (rng.standard_normal((vocab, dim)) * 0.05).astype(np.float32)
    off = objects.new_offload(e0, seq)
    off.refresh_weights(e1)
    xn = rng.standard_normal((dim, seq)).astype(np.float32)
    lg = np.zeros(vocab * seq, np.float32)
    off.run_classifier_forward(lg, xn.ravel())
    check("refreshed classifier", lg, oracle.matmul_vocab_seq(e1, xn), 5e-3)
    off.disable_softmax()
    assert not off.has_softmax() and off.has_classifier_forward()
    with pytest.raises(objects.SeamError, match="softmax kernel is unavailable"):
        off.run_softmax(lg)
    off = objects.refresh_offload(off, e1, seq, cpu_classifier_head=True)
    assert off.has_rms_forward() and off.has_rms_backward()
    assert not (off.has_classifier_forward() or off.has_softmax() or off.has_classifier_backward())
    with pytest.raises(objects.SeamError, match="classifier forward kernel is unavailable"):
        off.run_classifier_forward(lg, xn.ravel())
    off.close()
    assert not off.has_rms_forward()


@pytest.mark.parametrize("seq", [64, 512])
def test_layer_forward_edge_sequence_lengths(seq):
    """The shortest sequence the objects take and the longest a forward
    object takes (ane/layer_darwin.go compiles per sequence length), at a
    small width: every tap against the seam oracle."""
    print(f"seam layer forward edge seq={seq}", flush=True)
    dim, hidden, heads = 256, 512, 4
    rng = np.random.default_rng(50 + seq)
    w = layer_weights(rng, dim, hidden)
    x = rng.standard_normal((dim, seq)).astype(np.float32)
    ref_out, ref_taps = oracle.seam_layer_forward(w, heads, x)
    lf = objects.compile_stories_layer_forward(w, seq, heads=heads)
    out = np.full(dim * seq, np.nan, np.float32)
    cache = objects.LayerCache(dim, hidden, seq)
    lf.run_with_taps(out, x.ravel(), cache)
    check("out", out, ref_out, 5e-3)
    for n in ("x_norm", "q", "k", "v", "att_out", "x2", "x2_norm", "h1", "gate"):
        check(n, getattr(cache, n), ref_taps[n], 5e-3)
    lf.close()


@pytest.mark.parametrize("seq", [64, 256])
def test_layer_backward_edge_sequence_lengths(seq):
    """The backward object at the shortest and the longest sequence it
    takes, at a small width, against the seam oracle."""
    print(f"seam layer backward edge seq={seq}", flush=True)
    dim, hidden, heads = 256, 512, 4
    rng = np.random.default_rng(60 + seq)
    w = layer_weights(rng, dim, hidden)
    x = rng.standard_normal((dim, seq)).astype(np.float32)
    _, taps = oracle.seam_layer_forward(w, heads, x)
    dx2 = rng.standard_normal((dim, seq)).astype(np.float32)
    dffn = rng.standard_normal((dim, seq)).astype(np.float32)
    lb = objects.compile_stories_layer_backward(w, seq, heads=heads)
    outs = [np.full(dim * seq, np.nan, np.float32) for _ in range(4)]
    lb.run_attention(*outs, taps["q"].ravel(), taps["k"].ravel(), taps["v"].ravel(), dx2.ravel())
    ref = oracle.seam_attention_backward(w, heads, taps["q"], taps["k"], taps["v"], dx2)
    for n, got, r in zip(("dx_norm", "dq", "dk", "dv"), outs, ref):
        check(n, got, r, 1e-2)
    dxn = np.full(dim * seq, np.nan, np.float32)
    dh1 = np.full(hidden * seq, np.nan, np.float32)
    lb.run_ffn(dxn, dh1, dffn.ravel(), taps["h1"].ravel())
    ref_dx, ref_dh1 = oracle.seam_ffn_backward(w, dffn, taps["h1"])
    check("ffn dx_norm", dxn, ref_dx, 1e-2)
    check("dh1", dh1, ref_dh1, 1e-2)
    lb.close()
