"""Single-kernel parity on the GPU (through the C-ABI debug entry points).

GEMM: every operand layout and block tile against a float64 matmul of the
same fp16-rounded operands (fp32 accumulation: ~1e-6 relative).
Attention: the fused causal kernel (RoPE, optional QK-norm) against a
float64 numpy restatement of causalAttentionCF (ane/common.go:61-89) with
RoPE (ane/train_util.go:204-224) and QK-norm (ane/common.go:199-227).
"""
import ctypes as C

import numpy as np
import pytest

from ane import _lib

pytestmark = pytest.mark.gpu


def _u16(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def run_gemm(A, B, a_t, b_t, bm=0, bn=0, out_f16=False, nw=0, ns=0, splits=1):
    """A: (M,K) logical, B: (N,K) logical, both float16 arrays."""
    lib = _lib.load()
    M, K = A.shape
    N = B.shape[0]
    As = np.ascontiguousarray(A.T if a_t else A).view(np.uint16)
    Bs = np.ascontiguousarray(B.T if b_t else B).view(np.uint16)
    out = np.zeros((M, N), np.float16 if out_f16 else np.float32)
    rc = lib.ane_debug_gemm(int(a_t), int(b_t), 0 if out_f16 else 1, M, N, K, _u16(As), _u16(Bs),
                            out.ctypes.data_as(C.c_void_p), bm, bn, nw, ns, splits)
    assert rc == 0, lib.ane_debug_last_error()
    return out


TILES = [(256, 256, 4), (256, 256, 8), (256, 128, 4), (128, 256, 4), (128, 128, 4), (64, 128, 4),
         (128, 64, 4), (256, 64, 4), (64, 64, 4)]
TILES_3STAGE = [(256, 128), (128, 128), (64, 128), (128, 64), (64, 64)]


@pytest.mark.parametrize("a_t,b_t", [(False, False), (False, True), (True, True)])
@pytest.mark.parametrize("bm,bn,nw", TILES)
def test_gemm_layouts_and_tiles(a_t, b_t, bm, bn, nw):
    r = np.random.default_rng(bm * 7 + bn + 3 * a_t + b_t + nw)
    M, N, K = 512, 256, 320
    A = r.standard_normal((M, K)).astype(np.float16)
    B = r.standard_normal((N, K)).astype(np.float16)
    got = run_gemm(A, B, a_t, b_t, bm, bn, nw=nw)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-4)


@pytest.mark.parametrize("bm,bn,nw", [(256, 256, 4), (256, 256, 8), (128, 128, 4)])
@pytest.mark.parametrize("K", [64, 128, 192, 256, 832])
def test_gemm_every_k_tile_count(bm, bn, nw, K):
    """Prefetch schedules (loads of tile kt+2 issued around tile kt's
    barrier): 1, 2, 3, 4 and 13 k-tiles; the 4-wave 256x256 tile is the
    hand-ordered kernel."""
    r = np.random.default_rng(bm + nw + K)
    M, N = 512, 512
    A = r.standard_normal((M, K)).astype(np.float16)
    B = r.standard_normal((N, K)).astype(np.float16)
    got = run_gemm(A, B, False, False, bm, bn, nw=nw)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-4)


@pytest.mark.parametrize("bm,bn", TILES_3STAGE)
@pytest.mark.parametrize("K", [64, 128, 192, 640])
def test_gemm_three_stage_pipeline(bm, bn, K):
    """3-stage LDS pipeline: every k-tile count from 1 (prologue only) up."""
    r = np.random.default_rng(bm + bn + K)
    M, N = 512, 256
    A = r.standard_normal((M, K)).astype(np.float16)
    B = r.standard_normal((N, K)).astype(np.float16)
    got = run_gemm(A, B, False, False, bm, bn, ns=3)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-4)


def test_gemm_three_stage_rejects_unsupported():
    lib = _lib.load()
    A = np.zeros((256, 64), np.float16)
    B = np.zeros((256, 64), np.float16)
    out = np.zeros((256, 256), np.float32)
    for (bm, bn, nw, at) in [(256, 256, 4, 0), (128, 128, 4, 1), (256, 256, 8, 0)]:
        rc = lib.ane_debug_gemm(at, 0, 1, 256, 256, 64, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)),
                                out.ctypes.data_as(C.c_void_p), bm, bn, nw, 3, 1)
        assert rc != 0


@pytest.mark.parametrize("bm,bn,nw", [(256, 256, 8), (128, 128, 4), (128, 64, 4), (64, 128, 4), (64, 64, 4)])
@pytest.mark.parametrize("splits", [2, 3, 4, 8])
@pytest.mark.parametrize("out_f16", [False, True])
def test_gemm_split_k(bm, bn, nw, splits, out_f16):
    """Split-K: fp32 partials per K range, summed in split order, then the
    epilogue; 1, 2 and 3 k-tiles per split."""
    r = np.random.default_rng(bm + bn + splits + out_f16)
    M, N = 512, 256
    for kps in (1, 2, 3):
        K = 64 * kps * splits
        A = r.standard_normal((M, K)).astype(np.float16)
        B = r.standard_normal((N, K)).astype(np.float16)
        got = run_gemm(A, B, False, False, bm, bn, out_f16=out_f16, nw=nw, splits=splits)
        ref = A.astype(np.float64) @ B.astype(np.float64).T
        if out_f16:
            np.testing.assert_allclose(got.astype(np.float64), ref, rtol=2e-3, atol=2e-2)
        else:
            np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-4)


@pytest.mark.parametrize("a_t,b_t", [(False, True), (True, True)])
@pytest.mark.parametrize("bm,bn,nw", [(256, 256, 8), (128, 128, 4), (128, 64, 4), (64, 64, 4)])
@pytest.mark.parametrize("splits", [2, 5])
def test_gemm_split_k_m_major(a_t, b_t, bm, bn, nw, splits):
    """Split-K over M-major operands (the weight gradients dW = dY^T X with
    dY and X token-major, read through transposing LDS loads): each split's
    K range is a range of rows of the stored operands."""
    r = np.random.default_rng(bm + bn + splits + 11 * a_t + 13 * b_t)
    M, N = 512, 256
    for kps in (1, 3):
        K = 64 * kps * splits
        A = r.standard_normal((M, K)).astype(np.float16)
        B = r.standard_normal((N, K)).astype(np.float16)
        got = run_gemm(A, B, a_t, b_t, bm, bn, nw=nw, splits=splits)
        ref = A.astype(np.float64) @ B.astype(np.float64).T
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-4)


def test_gemm_split_k_rejects_unsupported():
    lib = _lib.load()
    A = np.zeros((256, 256), np.float16)
    B = np.zeros((256, 256), np.float16)
    out = np.zeros((256, 256), np.float32)
    # transposed operand; K not divisible into 64-wide splits
    for (at, K, sp) in [(1, 256, 2), (0, 192, 2), (0, 256, 8)]:
        rc = lib.ane_debug_gemm(at, 0, 1, 256, 256, K, _u16(A.view(np.uint16)), _u16(B.view(np.uint16)),
                                out.ctypes.data_as(C.c_void_p), 128, 128, 0, 0, sp)
        assert rc != 0


def test_gemm_real_shapes_auto_tile():
    r = np.random.default_rng(5)
    for (M, N, K) in [(1024, 2304, 768), (512, 768, 2048), (1024, 4096, 768)]:
        A = (r.standard_normal((M, K)) * 0.5).astype(np.float16)
        B = (r.standard_normal((N, K)) * 0.02).astype(np.float16)
        got = run_gemm(A, B, False, False)
        ref = A.astype(np.float64) @ B.astype(np.float64).T
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
    got16 = run_gemm(A, B, False, False, out_f16=True)
    np.testing.assert_allclose(got16.astype(np.float64), ref, rtol=2e-3, atol=1e-3)


def attn_ref(qkv, nseq, S, NH, qknorm, theta, scale=0.125):
    x = qkv.astype(np.float64).reshape(nseq, S, 3, NH, 64)
    q, k, v = x[:, :, 0], x[:, :, 1], x[:, :, 2]
    ang = np.arange(S)[:, None] / theta ** (2 * np.arange(32)[None, :] / 64)
    c, s = np.cos(ang)[None, :, None, :], np.sin(ang)[None, :, None, :]

    def rope(z):
        e, o = z[..., 0::2], z[..., 1::2]
        out = np.empty_like(z)
        out[..., 0::2] = e * c - o * s
        out[..., 1::2] = o * c + e * s
        return out

    q, k = rope(q), rope(k)
    if qknorm:
        q = 1.2 * q / np.sqrt((q * q).mean(-1, keepdims=True) + 1e-5)
        k = 1.2 * k / np.sqrt((k * k).mean(-1, keepdims=True) + 1e-5)
    sc = np.einsum("bshd,bthd->bhst", q, k) * scale
    sc = np.where(np.tril(np.ones((S, S), bool))[None, None], sc, -np.inf)
    mx = sc.max(-1, keepdims=True)
    p = np.exp(sc - mx)
    lse = (mx[..., 0] + np.log(p.sum(-1)))
    p /= p.sum(-1, keepdims=True)
    out = np.einsum("bhst,bthd->bshd", p, v).reshape(nseq * S, NH * 64)
    return out, lse.transpose(0, 2, 1).reshape(nseq * S, NH)


@pytest.mark.parametrize("S,NH,nseq,qknorm", [(256, 12, 2, True), (256, 4, 3, False), (64, 2, 1, True),
                                             (128, 3, 2, False), (512, 2, 1, True),
                                             (256, 12, 25, False),  # 300 heads: 1.5 heads per block on 88 blocks
                                             (256, 12, 32, True), (256, 12, 32, False)])  # 384: every block 1.5
def test_attention_matches_f64(S, NH, nseq, qknorm):
    lib = _lib.load()
    r = np.random.default_rng(S + NH + nseq)
    D = 64 * NH
    qkv = r.standard_normal((nseq * S, 3 * D)).astype(np.float16)
    out = np.zeros((nseq * S, D), np.float16)
    lse = np.zeros((nseq * S, NH), np.float32)
    theta = 100000.0 if qknorm else 10000.0
    rc = lib.ane_debug_attention(nseq, S, NH, int(qknorm), theta, 0.125, 0, _u16(qkv.view(np.uint16)),
                                 _u16(out.view(np.uint16)), lse.ctypes.data_as(C.POINTER(C.c_float)))
    assert rc == 0, lib.ane_debug_last_error()
    ref, ref_lse = attn_ref(qkv, nseq, S, NH, qknorm, theta)
    tol = 2e-2 if qknorm else 6e-3
    np.testing.assert_allclose(out.astype(np.float64), ref, atol=tol)
    np.testing.assert_allclose(lse, ref_lse, atol=tol * 2)
    # row 0 of every sequence attends only to itself: out = v[0]
    v0 = qkv.reshape(nseq, S, 3, D)[:, 0, 2].astype(np.float64)
    np.testing.assert_allclose(out.reshape(nseq, S, D)[:, 0].astype(np.float64), v0, atol=2e-3)


def test_attention_split_scores_at_scale_1():
    """The scale-1 recompute (the reference's backward probabilities) with
    QK-norm: split hi+lo operands bring the log-sum-exp to ~fp32 accuracy,
    plain fp16 operands do not."""
    lib = _lib.load()
    nseq, S, NH = 2, 256, 4
    D = 64 * NH
    qkv = np.random.default_rng(77).standard_normal((nseq * S, 3 * D)).astype(np.float16)
    ref, ref_lse = attn_ref(qkv, nseq, S, NH, True, 100000.0, scale=1.0)
    errs = {}
    for hilo in (0, 1):
        out = np.zeros((nseq * S, D), np.float16)
        lse = np.zeros((nseq * S, NH), np.float32)
        rc = lib.ane_debug_attention(nseq, S, NH, 1, 100000.0, 1.0, hilo, _u16(qkv.view(np.uint16)),
                                     _u16(out.view(np.uint16)), lse.ctypes.data_as(C.POINTER(C.c_float)))
        assert rc == 0, lib.ane_debug_last_error()
        errs[hilo] = (np.abs(lse - ref_lse).max(), np.abs(out.astype(np.float64) - ref).max())
    print("scale-1 (lse err, out err): fp16", errs[0], "split", errs[1])
    assert errs[1][0] < 1e-3 and errs[1][1] < 4e-3
    assert errs[1][0] < errs[0][0] / 5


@pytest.mark.parametrize("ra,ca,rb,cb", [(64, 64, 0, 0), (4096, 768, 4096, 4096), (256, 2304, 128, 64),
                                         (192, 64, 64, 320)])
def test_transpose_pairs_bit_exact(ra, ca, rb, cb):
    """The training step's transpose (8x8 register blocks, two jobs per
    launch) against numpy, bit for bit, on random fp16 bit patterns."""
    lib = _lib.load()
    rng = np.random.default_rng(ra + ca + rb + cb)
    a = rng.integers(0, 1 << 16, (ra, ca), dtype=np.uint16)
    oa = np.zeros((ca, ra), np.uint16)
    b = rng.integers(0, 1 << 16, (rb, cb), dtype=np.uint16) if rb else None
    ob = np.zeros((cb, rb), np.uint16) if rb else None
    u16 = lambda x: x.ctypes.data_as(C.POINTER(C.c_uint16)) if x is not None else None
    rc = lib.ane_debug_transpose2(ra, ca, u16(a), u16(oa), rb, cb, u16(b), u16(ob))
    assert rc == 0, lib.ane_debug_last_error()
    np.testing.assert_array_equal(oa, a.T)
    if rb:
        np.testing.assert_array_equal(ob, b.T)
    assert lib.ane_debug_transpose2(100, 64, u16(a), u16(oa), 0, 0, None, None) != 0  # rows not a multiple of 64


@pytest.mark.parametrize("T,D,add,half", [(4096, 768, True, True), (4096, 768, False, True), (100, 64, True, False),
                                          (37, 1024, True, True), (8, 192, False, False)])
def test_norm_bwd_gain_form(T, D, add, half):
    """The training step's RMSNorm backward, gain form (stories.RMSNormBackward,
    ane/stories/cpu.go:191-210, gain on both terms as there): the gain-form
    kernel the llama2 step runs and the general kernel, each against a
    float64 restatement, and the fp16 copy as the rounded fp32 output.  Row
    counts that leave a partial last block (100, 37) and D below one float4
    per lane (64, 192) included."""
    lib = _lib.load()
    rng = np.random.default_rng(T * 7 + D)
    dy = rng.standard_normal((T, D)).astype(np.float32)
    x = rng.standard_normal((T, D)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    ad = rng.standard_normal((T, D)).astype(np.float32) if add else None
    alpha = 0.75
    nb = (T + 7) // 8
    f32 = lambda a: a.ctypes.data_as(C.POINTER(C.c_float)) if a is not None else None
    x64, dy64, g64 = x.astype(np.float64), dy.astype(np.float64), g.astype(np.float64)
    rr = 1.0 / np.sqrt((x64 * x64).mean(1, keepdims=True) + 1e-5)
    c = (dy64 * x64 * g64).sum(1, keepdims=True) * rr * rr / D
    ref = (dy64 - x64 * c) * rr * g64 + (alpha * ad.astype(np.float64) if add else 0.0)
    dg = dy64 * x64 * rr
    dg_ref = np.stack([dg[8 * b:8 * b + 8].sum(0) for b in range(nb)])
    outs = []
    for general in (0, 1):
        out = np.zeros((T, D), np.float32)
        oh = np.zeros((T, D), np.float16) if half else None
        part = np.zeros((nb, D), np.float32)
        rc = lib.ane_debug_norm_bwd(T, D, f32(dy), f32(x), f32(g), f32(ad), alpha, f32(out),
                                    _u16(oh) if half else None, f32(part), general)
        assert rc == 0, lib.ane_debug_last_error()
        scale = np.abs(ref).max()
        assert np.abs(out - ref).max() <= 2e-6 * scale, (general, np.abs(out - ref).max(), scale)
        assert np.abs(part - dg_ref).max() <= 2e-6 * np.abs(dg_ref).max() * 8, general
        if half:
            np.testing.assert_array_equal(oh, out.astype(np.float16))
        outs.append(out)
    # the two kernels: the same function, fp32 rounding apart
    assert np.abs(outs[0] - outs[1]).max() <= 2e-6 * np.abs(ref).max()
    assert lib.ane_debug_norm_bwd(T, 96, f32(dy), f32(x), f32(g), None, 1.0, f32(outs[0]), None, f32(part), 0) != 0
