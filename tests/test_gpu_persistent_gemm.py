"""The persistent form of the 8-wave 256x256 GEMM (ANE_GEMM_PERSIST=1).

With more 256x256 tiles than CUs (the classifier, and W1|W3 at B32), one
block per CU walks its tiles, requesting each next tile's first k-tiles
(and its rr partials and target ids) before the current tile's epilogue.
Measured no faster than one block per tile on the B32 forward, so it is
opt-in; each epilogue that takes the form is checked here, with the form
switched on, on a shape of 17 x 16 tiles (more than the 256 CUs, so some
blocks take two) against float64: fp16 store, SwiGLU, the deferred-norm
forms scaled by 1 / rms, and the classifier's cross-entropy partials and
target logits.
"""
import ctypes as C

import numpy as np
import pytest

from ane import _lib

pytestmark = pytest.mark.gpu

MB, NB = 17, 16          # tile grid: 272 tiles of 256 x 256
M, N, K = 256 * MB, 256 * NB, 128
TILE = (256, 256, 8)


@pytest.fixture(autouse=True)
def persistent(monkeypatch):
    monkeypatch.setenv("ANE_GEMM_PERSIST", "1")


def _u16(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def _fp(a):
    return None if a is None else a.ctypes.data_as(C.POINTER(C.c_float))


def _vp(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def operands(seed, m=M, n=N, k=K, sa=0.5):
    r = np.random.default_rng(seed)
    A = (r.standard_normal((m, k)) * sa).astype(np.float16)
    B = (r.standard_normal((n, k)) * 0.5).astype(np.float16)
    return r, A, B, A.astype(np.float64) @ B.astype(np.float64).T


def swiglu_ref(a):
    blk = a.reshape(a.shape[0], a.shape[1] // 64, 2, 32)
    h1, h3 = blk[:, :, 0, :], blk[:, :, 1, :]
    return (h1 / (1.0 + np.exp(-h1)) * h3).reshape(a.shape[0], a.shape[1] // 2)


def test_store_half():
    lib = _lib.load()
    _, A, B, acc = operands(1)
    out = np.zeros((M, N), np.float16)
    rc = lib.ane_debug_gemm(0, 0, 0, M, N, K, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)), _vp(out), *TILE, 0, 1)
    assert rc == 0, lib.ane_debug_last_error()
    np.testing.assert_allclose(out.astype(np.float64), acc, rtol=2e-3, atol=2e-3)


def test_swiglu():
    lib = _lib.load()
    _, A, B, acc = operands(2)
    gate = np.zeros((M, N // 2), np.float16)
    h13 = np.zeros((M, N), np.float16)
    rc = lib.ane_debug_gemm_epi(4, M, N, K, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)), _vp(gate), _vp(h13),
                                None, None, 1.0, 0.0, 0, *TILE)
    assert rc == 0, lib.ane_debug_last_error()
    np.testing.assert_allclose(gate.astype(np.float64), swiglu_ref(acc), rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(h13.astype(np.float64), acc, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("epi", [14, 15])
def test_deferred_norm_forms(epi):
    """rr = 1 / rms from 12 partials per row, staged by LDS DMA per tile."""
    lib = _lib.load()
    r, A, B, acc = operands(3 + epi)
    part = (r.random((12, M)) * 40.0 + 1e-3).astype(np.float32)
    rr = 1.0 / np.sqrt(part.astype(np.float64).sum(0) / 768 + 1e-5)
    out = np.zeros((M, N if epi == 14 else N // 2), np.float16)
    rc = lib.ane_debug_gemm_norm(epi, M, N, K, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)), None,
                                 _u16(out.view(np.uint16)), None, None, _fp(part), 12, 768, *TILE)
    assert rc == 0, lib.ane_debug_last_error()
    a = acc * rr[:, None]
    ref = a if epi == 14 else swiglu_ref(a)
    np.testing.assert_allclose(out.astype(np.float64), ref, rtol=2e-3, atol=2e-3)


def test_classifier_partials_and_targets():
    lib = _lib.load()
    r, A, B, acc = operands(9, sa=0.35)
    tg = r.integers(0, M, N).astype(np.uint16)
    tg[::37] = 65535
    pm = np.zeros((MB, N), np.float32)
    ps = np.zeros((MB, N), np.float32)
    tl = np.zeros(N, np.float32)
    rc = lib.ane_debug_classifier(M, N, K, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)), _u16(tg), 0, M,
                                  *TILE, _fp(pm), _fp(ps), _fp(tl), None, None, None, None)
    assert rc == 0, lib.ane_debug_last_error()
    for b in range(MB):
        blk = acc[b * 256:(b + 1) * 256]
        np.testing.assert_allclose(pm[b], blk.max(axis=0), rtol=1e-5, atol=5e-4)
        np.testing.assert_allclose(ps[b], np.exp(blk - pm[b].astype(np.float64)).sum(axis=0), rtol=2e-4)
    ok = tg < M
    np.testing.assert_allclose(tl[ok], acc[tg[ok].astype(np.int64), np.nonzero(ok)[0]], rtol=1e-5, atol=5e-4)
    assert np.isnan(tl[~ok]).all()
