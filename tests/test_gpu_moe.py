"""Mixture-of-experts FFN layer on the GPU against the CPU oracle
(oracle/refmoe.c, pinned in tests/test_oracle_moe.py).

Expert assignment is compared bit-exactly (fp32 router in the oracle's
operation order, ties to the lower expert).  Outputs use fp16 expert weights
and activations with fp32 accumulation: relative L2 error <= 5e-3 and
max-abs error <= 2e-2 of the output's RMS.
"""
import ctypes as C

import numpy as np
import pytest

import ane
import oracle
from ane import _lib
from ane.moe import MoeConfig, MoeLayer, init_moe_params, make_moe_input

pytestmark = pytest.mark.gpu


def _check_out(got, ref):
    rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
    rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    mx = float(np.abs(got - ref).max())
    print(f"moe out rel L2 {rel:.2e}, max-abs {mx:.2e} (rms {rms:.3e})")
    assert rel <= 5e-3 and mx <= 2e-2 * rms


def test_small_layer_matches_oracle():
    cfg = MoeConfig(dim=128, hidden=256, experts=8)
    p = init_moe_params(cfg, seed=11, std=0.05)
    x = make_moe_input(cfg, 300, seed=12)
    layer = MoeLayer(cfg, p, max_tokens=512)
    try:
        out, idx, w = layer.Forward(x)
        out2, idx2, w2 = layer.Forward(x)
    finally:
        layer.Close()
    ref, ridx, rw = oracle.moe_forward(p, x, cfg.hidden, cfg.experts)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=1e-7)
    _check_out(out, ref)
    np.testing.assert_array_equal(out, out2)  # deterministic


@pytest.mark.parametrize("experts,tokens", [(2, 513), (4, 1000), (16, 777), (16, 4096), (8, 1), (8, 256)])
def test_expert_counts_and_ragged_token_counts(experts, tokens):
    """Every supported expert count, token counts that leave a partial
    256-token permutation block, (16 x 4096) several full blocks and tile
    groups per expert, and one token or exactly one block (a single
    permutation block forms every group's offsets and the tile table)."""
    cfg = MoeConfig(dim=128, hidden=192, experts=experts)
    p = init_moe_params(cfg, seed=31 + experts, std=0.05)
    x = make_moe_input(cfg, tokens, seed=32 + tokens)
    layer = MoeLayer(cfg, p, max_tokens=tokens)
    try:
        out, idx, w = layer.Forward(x)
    finally:
        layer.Close()
    ref, ridx, rw = oracle.moe_forward(p, x, cfg.hidden, cfg.experts)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=1e-7)
    _check_out(out, ref)


def test_full_size_routing_bit_exact_and_sampled_outputs():
    """dim 768, 8 experts of SwiGLU 2048, 8192 tokens,
    router and experts N(0, 0.02), activations N(0, 1), seed 5."""
    cfg = MoeConfig()
    p = init_moe_params(cfg, seed=5, std=0.02)
    x = make_moe_input(cfg, 8192, seed=5)
    layer = MoeLayer(cfg, p, max_tokens=8192)
    try:
        out, idx, w = layer.Forward(x)
    finally:
        layer.Close()
    ridx, rw = oracle.moe_route(p, x, cfg.hidden, cfg.experts)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=1e-7)
    counts = np.bincount(idx.reshape(-1), minlength=cfg.experts)
    print("tokens per expert", counts.tolist())
    sample = np.random.default_rng(7).choice(8192, 96, replace=False)
    ref, _, _ = oracle.moe_forward(p, x[sample], cfg.hidden, cfg.experts)
    _check_out(out[sample], ref)


def test_ties_go_to_lower_expert():
    cfg = MoeConfig(dim=64, hidden=64, experts=4)
    p = init_moe_params(cfg, seed=21, std=0.05)
    router = p[:cfg.experts * cfg.dim].reshape(cfg.experts, cfg.dim)
    router[...] = 0.0
    for e in range(cfg.experts):
        router[e, e] = 1.0
    x = np.zeros((4, cfg.dim), np.float32)
    x[0, :4] = [0.5, 0.5, 0.5, 0.5]
    x[1, :4] = [0.0, 0.7, 0.7, 0.1]
    x[2, :4] = [0.2, 0.1, 0.2, 0.2]
    x[3, :4] = [-1.0, -1.0, -3.0, -1.0]
    layer = MoeLayer(cfg, p, max_tokens=64)
    try:
        _, idx, _ = layer.Forward(x)
    finally:
        layer.Close()
    assert idx.tolist() == [[0, 1], [1, 2], [0, 2], [0, 1]]
    ridx, _ = oracle.moe_route(p, x, cfg.hidden, cfg.experts)
    np.testing.assert_array_equal(idx, ridx)


def test_router_products_and_sums_separately_rounded():
    """linearCF rounds every product and every partial sum.  With row 1 =
    (1, a) and x = (1, x1): fl(a * x1) is exactly 2^-24 while the exact
    product is a little larger, so 1 + fl(a * x1) is a tie that rounds to
    even (1.0, equal to row 0's logit: the lower expert comes first), whereas
    a fused multiply-add would round up to 1 + 2^-23 and put expert 1 first."""
    cfg = MoeConfig(dim=64, hidden=64, experts=4)
    p = init_moe_params(cfg, seed=22, std=0.05)
    router = p[:cfg.experts * cfg.dim].reshape(cfg.experts, cfg.dim)
    router[...] = 0.0
    a = np.float32(1 + 2049 * 2.0 ** -23)
    x1 = np.float32(2.0 ** -24 * (1 - 2048 * 2.0 ** -23))
    assert a * x1 == np.float32(2.0 ** -24)                    # product rounds down onto 2^-24
    assert np.float32(1) + a * x1 == np.float32(1)             # and the sum ties to even
    router[0, 0] = 1.0
    router[1, 0], router[1, 1] = 1.0, a
    x = np.zeros((2, cfg.dim), np.float32)
    x[0, 0], x[0, 1] = 1.0, x1
    x[1, 0], x[1, 1] = 1.0, np.float32(2.0 ** -22)  # a clear win for expert 1
    layer = MoeLayer(cfg, p, max_tokens=64)
    try:
        _, idx, _ = layer.Forward(x)
    finally:
        layer.Close()
    assert idx.tolist() == [[0, 1], [1, 0]]
    ridx, _ = oracle.moe_route(p, x, cfg.hidden, cfg.experts)
    np.testing.assert_array_equal(idx, ridx)


def test_moe_errors():
    lib = _lib.load()
    for bad in (_lib.MoeCfg(768, 2048, 8, 3, 16, 0), _lib.MoeCfg(768, 2048, 6, 2, 16, 0),
                _lib.MoeCfg(100, 2048, 8, 2, 16, 0), _lib.MoeCfg(768, 2048, 8, 2, 0, 0)):
        h = C.c_void_p()
        rc = lib.ane_moe_open(C.byref(bad), C.byref(h))
        assert rc == _lib.ANE_ERR_ARG, lib.ane_moe_last_error(h)
        lib.ane_moe_destroy(h)
    cfg = MoeConfig(dim=64, hidden=64, experts=2)
    layer = MoeLayer(cfg, init_moe_params(cfg, 1), max_tokens=8)
    try:
        with pytest.raises(ane.EngineError) as ei:
            layer.Run()
        assert ei.value.code == _lib.ANE_ERR_STATE
        with pytest.raises(ane.EngineError) as ei:
            layer.Load(np.zeros((9, 64), np.float32))
        assert ei.value.code == _lib.ANE_ERR_ARG
        with pytest.raises(ane.EngineError):
            layer.SetParams(np.zeros(5, np.float32))
    finally:
        layer.Close()
