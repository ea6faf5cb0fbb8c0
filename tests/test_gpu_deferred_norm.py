"""The deferred RMSNorm of the llama2 eval forward.

The reference normalises before each projection (RMSNorm with gain,
ane/stories/cpu.go; y = x / rms(x) * g, then linearCF).  The eval forward
here runs no norm kernel: the residual GEMM's epilogue leaves fp16(x * g)
and per-row partial sums of x^2 (one per column block), and the projection
that consumes them scales its output rows by 1 / rms(x), which the product
commutes with.  Each epilogue is checked against float64 on every tile the
dispatcher offers it; the whole forward (EvalLoss, the default; and with
ANE_FUSED_NORM=0, the norm launches) is checked against the oracle and the
two paths against each other.
"""
import ctypes as C

import numpy as np
import pytest

import ane
import oracle
from ane import _lib

pytestmark = pytest.mark.gpu

EPI_RESID_NORM, EPI_STORE_H_RR, EPI_SWIGLU_RR = 13, 14, 15
M, N, K = 512, 768, 192


def _u16(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def _fp(a):
    return None if a is None else a.ctypes.data_as(C.POINTER(C.c_float))


def run(epi, A, B, Cout, X=None, gain=None, ssq=None, part=None, rr_dim=0, tile=(0, 0, 4)):
    lib = _lib.load()
    bm, bn, nw = tile
    m, k = A.shape
    n = B.shape[0]
    nparts = 0 if part is None else part.shape[0]
    rc = lib.ane_debug_gemm_norm(epi, m, n, k, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)), _fp(X),
                                 _u16(Cout.view(np.uint16)), _fp(gain), _fp(ssq), _fp(part), nparts, rr_dim, bm, bn,
                                 nw)
    assert rc == 0, lib.ane_debug_last_error()


def operands(seed, n=N):
    r = np.random.default_rng(seed)
    A = (r.standard_normal((M, K)) * 0.5).astype(np.float16)
    B = (r.standard_normal((n, K)) * 0.5).astype(np.float16)
    return r, A, B, A.astype(np.float64) @ B.astype(np.float64).T


def rr_of(part, dim):
    return 1.0 / np.sqrt(part.astype(np.float64).sum(0) / dim + 1e-5)


@pytest.mark.parametrize("tile", [(128, 64, 4), (64, 64, 4), (128, 128, 4), (256, 64, 4), (128, 192, 4),
                                  (256, 192, 4)])
def test_residual_with_norm_inputs(tile):
    r, A, B, acc = operands(11)
    X = r.standard_normal((M, N)).astype(np.float32)
    gain = (1.0 + 0.3 * r.standard_normal(N)).astype(np.float32)
    bn = tile[1]
    ssq = np.zeros((N // bn, M), np.float32)
    xg = np.zeros((M, N), np.float16)
    ref = X.astype(np.float64) + acc
    run(EPI_RESID_NORM, A, B, xg, X=X, gain=gain, ssq=ssq, tile=tile)
    np.testing.assert_allclose(X, ref, rtol=1e-5, atol=5e-4)
    # fp16(x * g) of the stored x: the exact product rounded to fp16 (the
    # device may round it once, or through fp32 first: at most 1 fp16 ulp)
    ref_xg = (X.astype(np.float64) * gain.astype(np.float64)).astype(np.float16)
    ulp = np.abs(np.spacing(ref_xg).astype(np.float64))
    assert np.all(np.abs(xg.astype(np.float64) - ref_xg.astype(np.float64)) <= ulp)
    assert np.mean(xg == ref_xg) > 0.999
    ref_ssq = (X.astype(np.float64) ** 2).reshape(M, N // bn, bn).sum(-1).T
    np.testing.assert_allclose(ssq, ref_ssq, rtol=2e-5)
    # the partials make up the whole row: the rms the consumers form
    np.testing.assert_allclose(ssq.astype(np.float64).sum(0), (X.astype(np.float64) ** 2).sum(1), rtol=2e-5)


@pytest.mark.parametrize("nparts", [1, 12, 16])
@pytest.mark.parametrize("tile", [(128, 192, 4), (128, 128, 4), (64, 64, 4), (256, 256, 8), (128, 64, 4)])
def test_store_scaled_by_row_rms(tile, nparts):
    r, A, B, acc = operands(12 + nparts)
    part = (r.random((nparts, M)) * 40.0 + 1e-3).astype(np.float32)
    h = np.zeros((M, N), np.float16)
    run(EPI_STORE_H_RR, A, B, h, part=part, rr_dim=N, tile=tile)
    ref = acc * rr_of(part, N)[:, None]
    np.testing.assert_allclose(h.astype(np.float64), ref, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("tile", [(256, 256, 8), (128, 128, 4), (64, 128, 4), (256, 256, 4)])
def test_swiglu_scaled_by_row_rms(tile):
    r, A, B, acc = operands(21, n=1024)
    part = (r.random((12, M)) * 40.0 + 1e-3).astype(np.float32)
    gate = np.zeros((M, 512), np.float16)
    run(EPI_SWIGLU_RR, A, B, gate, part=part, rr_dim=768, tile=tile)
    a = acc * rr_of(part, 768)[:, None]
    blk = a.reshape(M, 1024 // 64, 2, 32)
    h1, h3 = blk[:, :, 0, :], blk[:, :, 1, :]
    ref = (h1 / (1.0 + np.exp(-h1)) * h3).reshape(M, 512)
    np.testing.assert_allclose(gate.astype(np.float64), ref, rtol=2e-3, atol=2e-3)


def test_forward_with_and_without_norm_launches(monkeypatch):
    """stories110M-llama2 at B2: the deferred-norm forward and the one with
    RMSNorm launches give per-sequence losses within 5e-4 of each other and
    within 1e-3 of the oracle."""
    cfg = ane.stories110m("llama2")
    p = ane.init_params(cfg, seed=0)
    tok, tgt = ane.make_tokens(cfg, 2, seed=31)
    _, per_ref, _ = oracle.forward_loss(cfg, p, tok, tgt)
    per = {}
    for fused in ("1", "0"):
        monkeypatch.setenv("ANE_FUSED_NORM", fused)
        eng = ane.Open(ane.Options(Config=cfg, Params=p, MaxBatch=2))
        try:
            per[fused] = eng.EvalLoss(tok, tgt)[1]
        finally:
            eng.Destroy()
    print("per-sequence loss deferred", per["1"], "launches", per["0"], "oracle", per_ref)
    np.testing.assert_allclose(per["1"], per["0"], atol=5e-4)
    np.testing.assert_allclose(per["1"], per_ref, atol=1e-3)
