"""The oracle reproduces the committed golden fixtures (tests/golden, written
by tests/golden/make_golden.py): a regression pin on the oracle itself.
Integer data (tokens, expert ids, drand48 draws) must match exactly; floats
to 1e-5 relative (same code, possibly another libm)."""
import numpy as np
import pytest

import ane
import oracle
from ane.moe import MoeConfig, init_moe_params
from golden_io import load, manifest


def test_manifest_files_exist():
    m = manifest()
    assert len(m) >= 20
    for name in m:
        arr, tol = load(name)
        assert arr.size > 0


@pytest.mark.parametrize("arch", ["llama2", "nanochat"])
def test_forward_fixture(arch):
    cfg = ane.tiny(arch)
    p = ane.init_params(cfg, seed=0, std=0.08)
    tok, _ = load(f"forward_{arch}_tokens")
    want_tok, _ = ane.make_tokens(cfg, 1, seed=1)
    np.testing.assert_array_equal(tok, want_tok)
    _, tgt = ane.make_tokens(cfg, 1, seed=1)
    mean, _, lg = oracle.forward_loss(cfg, p, tok, tgt, want_logits=True)
    np.testing.assert_allclose(lg[0], load(f"forward_{arch}_logits")[0], rtol=1e-5, atol=1e-6)
    assert abs(mean - float(load(f"forward_{arch}_loss")[0][0])) < 1e-5


@pytest.mark.parametrize("arch,mode", [("llama2", "true"), ("nanochat", "compat")])
def test_grad_fixture(arch, mode):
    cfg = ane.tiny(arch, grad_mode=mode)
    p = ane.init_params(cfg, seed=21, std=0.08)
    tok, tgt = ane.make_tokens(cfg, 2, seed=22)
    loss, g = oracle.grads(cfg, p, tok, tgt)
    norms, heads = [], []
    for name, off, shape in ane.param_layout(cfg):
        seg = g[off:off + int(np.prod(shape))]
        norms.append(np.linalg.norm(seg.astype(np.float64)))
        h = np.zeros(32, np.float32)
        h[:min(32, seg.size)] = seg[:32]
        heads.append(h)
    np.testing.assert_allclose(norms, load(f"grads_{arch}_{mode}_norms")[0], rtol=1e-5)
    np.testing.assert_allclose(np.stack(heads), load(f"grads_{arch}_{mode}_heads")[0], rtol=1e-4, atol=1e-7)


def test_drand48_fixture():
    np.testing.assert_array_equal(oracle.drand48_stream(42, 16), load("drand48_seed42")[0])


def test_decode_fixture():
    cfg = ane.tiny_decode()
    p = ane.init_params(cfg, seed=61, std=0.05)
    prefix, _ = load("decode_gqa_prefix")
    forced, _ = load("decode_gqa_forced")
    toks, lg = oracle.decode(cfg, p, prefix, 2, forced=forced, want_logits=True, threads=1)
    np.testing.assert_array_equal(toks, load("decode_gqa_tokens")[0])
    np.testing.assert_allclose(lg, load("decode_gqa_logits")[0], rtol=1e-5, atol=1e-6)


def test_moe_fixture():
    cfg = MoeConfig(dim=64, hidden=128, experts=8)
    p = init_moe_params(cfg, seed=71, std=0.1)
    x, _ = load("moe_small_x")
    out, idx, w = oracle.moe_forward(p, x, cfg.hidden, cfg.experts, threads=1)
    np.testing.assert_array_equal(idx, load("moe_small_experts")[0])
    np.testing.assert_allclose(w, load("moe_small_weights")[0], rtol=1e-6)
    np.testing.assert_allclose(out, load("moe_small_out")[0], rtol=1e-5, atol=1e-6)
