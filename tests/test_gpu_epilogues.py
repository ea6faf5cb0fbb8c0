"""Fused GEMM epilogues of the forward pass, one GEMM each, against a float64
reference of the same formula: fp16 / fp32 stores, logits (plain and
softcapped), the residual add (alpha R + acc + beta X0, with its copy), the
SwiGLU over 32-column interleaved W1|W3 (gate and the saved h1|h3), relu^2
(and the saved pre-activation) and the smear gate (per-sequence first rows
have no predecessor).  Every block tile the dispatcher offers for the
epilogue, including the hand-ordered 4-wave 256x256 kernel."""
import ctypes as C

import numpy as np
import pytest

from ane import _lib

pytestmark = pytest.mark.gpu

EPI_STORE_H, EPI_STORE_F, EPI_LOGITS, EPI_RESID, EPI_SWIGLU, EPI_RELU2, EPI_SMEAR = 0, 1, 2, 3, 4, 5, 6
TILES = [(256, 256, 4), (256, 256, 8), (128, 128, 4), (64, 128, 4), (128, 64, 4), (64, 64, 4)]
M, N, K = 512, 512, 192


def _u16(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def _fp(a):
    return None if a is None else a.ctypes.data_as(C.POINTER(C.c_float))


def _vp(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def run(epi, A, B, C_out, C2=None, X0=None, R=None, alpha=1.0, beta=0.0, seq=0, tile=(0, 0, 0)):
    lib = _lib.load()
    bm, bn, nw = tile
    m, k = A.shape
    n = B.shape[0]
    rc = lib.ane_debug_gemm_epi(epi, m, n, k, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)), _vp(C_out), _vp(C2),
                                _fp(X0), _fp(R), alpha, beta, seq, bm, bn, nw)
    assert rc == 0, lib.ane_debug_last_error()


def operands(seed):
    r = np.random.default_rng(seed)
    A = (r.standard_normal((M, K)) * 0.5).astype(np.float16)
    B = (r.standard_normal((N, K)) * 0.5).astype(np.float16)
    return r, A, B, A.astype(np.float64) @ B.astype(np.float64).T


def close16(got, ref):
    np.testing.assert_allclose(got.astype(np.float64), ref, rtol=2e-3, atol=2e-3)


def close32(got, ref):
    np.testing.assert_allclose(got.astype(np.float64), ref, rtol=1e-5, atol=5e-4)


@pytest.mark.parametrize("tile", TILES)
def test_store_and_logits(tile):
    _, A, B, acc = operands(1)
    h = np.zeros((M, N), np.float16)
    run(EPI_STORE_H, A, B, h, tile=tile)
    close16(h, acc)
    f = np.zeros((M, N), np.float32)
    run(EPI_STORE_F, A, B, f, tile=tile)
    close32(f, acc)
    run(EPI_LOGITS, A, B, f, seq=-1, tile=tile)
    close32(f, 15.0 * np.tanh(acc / 15.0))


@pytest.mark.parametrize("tile", TILES)
def test_residual(tile):
    r, A, B, acc = operands(2)
    R = r.standard_normal((M, N)).astype(np.float32)
    X0 = r.standard_normal((M, N)).astype(np.float32)
    out = np.zeros((M, N), np.float32)
    copy = np.zeros((M, N), np.float32)
    run(EPI_RESID, A, B, out, C2=copy, X0=X0, R=R, alpha=0.75, beta=-0.5, tile=tile)
    ref = 0.75 * R.astype(np.float64) + acc - 0.5 * X0.astype(np.float64)
    close32(out, ref)
    np.testing.assert_array_equal(copy, out)
    run(EPI_RESID, A, B, out, R=R, tile=tile)  # plain residual, no X0 / copy
    close32(out, R.astype(np.float64) + acc)


@pytest.mark.parametrize("tile", [t for t in TILES if t[1] >= 128])
def test_swiglu(tile):
    _, A, B, acc = operands(3)
    gate = np.zeros((M, N // 2), np.float16)
    h13 = np.zeros((M, N), np.float16)
    run(EPI_SWIGLU, A, B, gate, C2=h13, tile=tile)
    blk = acc.reshape(M, N // 64, 2, 32)          # [m, pair, W1|W3, 32]
    h1, h3 = blk[:, :, 0, :], blk[:, :, 1, :]
    ref = (h1 / (1.0 + np.exp(-h1)) * h3).reshape(M, N // 2)
    close16(gate, ref)
    close16(h13, acc)


@pytest.mark.parametrize("tile", TILES)
def test_relu2(tile):
    _, A, B, acc = operands(4)
    out = np.zeros((M, N), np.float16)
    pre = np.zeros((M, N), np.float16)
    run(EPI_RELU2, A, B, out, C2=pre, tile=tile)
    close16(out, np.maximum(acc, 0.0) ** 2)
    close16(pre, acc)


@pytest.mark.parametrize("tile", TILES)
def test_smear(tile):
    r, A, B, acc = operands(5)
    seq = 128
    X0 = r.standard_normal((M, N)).astype(np.float32)
    out = np.zeros((M, N), np.float32)
    gate = np.zeros((M, N), np.float32)
    run(EPI_SMEAR, A, B, out, C2=gate, X0=X0, alpha=0.3, seq=seq, tile=tile)
    g = 1.0 / (1.0 + np.exp(-acc))
    prev = np.zeros_like(X0, dtype=np.float64)
    prev[1:] = X0[:-1]
    prev[::seq] = 0.0
    close32(gate, g)
    close32(out, X0.astype(np.float64) + 0.3 * g * prev)


@pytest.mark.parametrize("tile", [(128, 192, 4), (256, 192, 4)])
def test_192_wide_tiles(tile):
    """The 192-wide tiles (three 32-column MFMA tiles per wave) with the
    epilogues they serve: fp16 / fp32 store (QKV) and the residual add."""
    r = np.random.default_rng(7)
    m, n, k = 512, 384, 320
    A = (r.standard_normal((m, k)) * 0.5).astype(np.float16)
    B = (r.standard_normal((n, k)) * 0.5).astype(np.float16)
    acc = A.astype(np.float64) @ B.astype(np.float64).T
    h = np.zeros((m, n), np.float16)
    run(EPI_STORE_H, A, B, h, tile=tile)
    close16(h, acc)
    f = np.zeros((m, n), np.float32)
    run(EPI_STORE_F, A, B, f, tile=tile)
    close32(f, acc)
    R = r.standard_normal((m, n)).astype(np.float32)
    X0 = r.standard_normal((m, n)).astype(np.float32)
    out = np.zeros((m, n), np.float32)
    run(EPI_RESID, A, B, out, X0=X0, R=R, alpha=0.75, beta=-0.5, tile=tile)
    close32(out, 0.75 * R.astype(np.float64) + acc - 0.5 * X0.astype(np.float64))


CE_TILES = [(256, 256, 8), (256, 256, 4), (256, 128, 4), (128, 256, 4), (128, 128, 4), (64, 128, 4),
            (128, 64, 4), (64, 64, 4)]


@pytest.mark.parametrize("softcap", [0, 1])
@pytest.mark.parametrize("tile", CE_TILES)
def test_classifier_ce_and_dlogits(tile, softcap):
    """The classifier's cross-entropy epilogue (per-block (max, sum exp)
    partials and the target logit) and the dlogits epilogue, on every tile
    the dispatcher offers for them, including the 8-wave 256x256 tile the
    engine picks at B32 x 256 (rows = vocabulary, columns = tokens), against
    float64 log-sum-exp and softmax of the same fp16 operands."""
    lib = _lib.load()
    bm, bn, nw = tile
    Mv, Nt, Kd = 1024, 512, 192
    r = np.random.default_rng(70 + bm + bn + nw + softcap)
    A = (r.standard_normal((Mv, Kd)) * (1.0 if softcap else 0.35)).astype(np.float16)
    B = (r.standard_normal((Nt, Kd)) * 0.5).astype(np.float16)
    tg = r.integers(0, Mv, Nt).astype(np.uint16)
    tg[::37] = 65535                       # excluded targets: no lane claims them
    tg[1], tg[2], tg[3] = 0, Mv - 1, bm    # first, last row, first row of the second block row
    acc = A.astype(np.float64) @ B.astype(np.float64).T   # [Mv, Nt]
    v = 15.0 * np.tanh(acc / 15.0) if softcap else acc
    nb = Mv // bm
    pm = np.zeros((nb, Nt), np.float32)
    ps = np.zeros((nb, Nt), np.float32)
    tl = np.zeros(Nt, np.float32)
    rc = lib.ane_debug_classifier(Mv, Nt, Kd, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)), _u16(tg), softcap,
                                  Mv, bm, bn, nw, _fp(pm), _fp(ps), _fp(tl), None, None, None, None)
    assert rc == 0, lib.ane_debug_last_error()
    # each block row's partial against its own rows
    for b in range(nb):
        blk = v[b * bm:(b + 1) * bm]
        mx = blk.max(axis=0)
        np.testing.assert_allclose(pm[b], mx, rtol=1e-5, atol=5e-4)
        np.testing.assert_allclose(ps[b], np.exp(blk - pm[b].astype(np.float64)).sum(axis=0), rtol=2e-4)
    M_ = pm.astype(np.float64).max(axis=0)
    lse = M_ + np.log((ps.astype(np.float64) * np.exp(pm.astype(np.float64) - M_)).sum(axis=0))
    mref = v.max(axis=0)
    lse_ref = mref + np.log(np.exp(v - mref).sum(axis=0))
    np.testing.assert_allclose(lse, lse_ref, rtol=0, atol=2e-4)
    ok = tg < Mv
    np.testing.assert_allclose(tl[ok], v[tg[ok].astype(np.int64), np.nonzero(ok)[0]], rtol=1e-5, atol=5e-4)
    assert np.isnan(tl[~ok]).all()
    # dlogits with a vocabulary end short of the padded rows
    vocab = Mv - 40
    cs = (r.random(Nt) * 64.0).astype(np.float32)
    lse32 = lse_ref.astype(np.float32)
    dl = np.zeros((Mv, Nt), np.float16)
    dlt = np.zeros((Nt, Mv), np.float16)
    rc = lib.ane_debug_classifier(Mv, Nt, Kd, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)), _u16(tg), softcap,
                                  vocab, bm, bn, nw, _fp(pm), _fp(ps), _fp(tl), _fp(lse32), _fp(cs),
                                  _u16(dl.view(np.uint16)), _u16(dlt.view(np.uint16)))
    assert rc == 0, lib.ane_debug_last_error()
    p = np.exp(v - lse32.astype(np.float64))
    onehot = np.zeros_like(p)
    onehot[tg[ok].astype(np.int64), np.nonzero(ok)[0]] = 1.0
    ref = (p - onehot) * cs.astype(np.float64)
    if softcap:
        ref *= 1.0 - np.tanh(acc / 15.0) ** 2
    ref[vocab:] = 0.0
    np.testing.assert_allclose(dl.astype(np.float64), ref, rtol=3e-3, atol=2e-3)
    assert (dl[vocab:] == 0).all()
    np.testing.assert_array_equal(dlt, dl.T)
