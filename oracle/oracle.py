"""ctypes front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module, and only as the checker.  The product never imports it.

The oracle itself is oracle/refcpu.c, a plain-C restatement of the
reference's CPU path; see that file for the per-function citations.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librefcpu.so")

ARCH = {"nanochat": 0, "llama2": 1}
GRAD = {"compat": 0, "true": 1}


class OrcCfg(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden", C.c_int32), ("heads", C.c_int32),
                ("layers", C.c_int32), ("vocab", C.c_int32), ("seq", C.c_int32),
                ("arch", C.c_int32), ("grad_mode", C.c_int32), ("rope_theta", C.c_double)]


class OrcDecCfg(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden", C.c_int32), ("heads", C.c_int32), ("kv_heads", C.c_int32),
                ("layers", C.c_int32), ("vocab", C.c_int32), ("rope_theta", C.c_double)]


class OrcMoeCfg(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden", C.c_int32), ("experts", C.c_int32)]


class OrcSeamLayer(C.Structure):
    _fields_ = [(n, C.POINTER(C.c_float)) for n in ("wq", "wk", "wv", "wo", "w1", "w2")]


SEAM_TAPS = ("x_norm", "q", "k", "v", "att_out", "x2", "x2_norm", "h1", "gate")


class OrcSeamTaps(C.Structure):
    _fields_ = [(n, C.POINTER(C.c_float)) for n in SEAM_TAPS]


class OrcAdam(C.Structure):
    _fields_ = [(n, C.c_float) for n in (
        "lr", "beta1", "beta2", "eps", "weight_decay", "grad_clip", "embed_lr_mult",
        "scalar_lr_mult", "lambda_lr_mult", "lambda_beta1", "lambda_beta2")]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        fp = C.POINTER(C.c_float)
        u16 = C.POINTER(C.c_uint16)
        L.orc_param_count.restype = C.c_size_t
        L.orc_param_count.argtypes = [C.POINTER(OrcCfg)]
        L.orc_param_segments.restype = C.c_int
        L.orc_param_segments.argtypes = [C.POINTER(OrcCfg), C.POINTER(C.c_int64),
                                         C.POINTER(C.c_int64), C.c_int]
        L.orc_forward_loss.restype = C.c_float
        L.orc_forward_loss.argtypes = [C.POINTER(OrcCfg), fp, u16, u16, C.c_int, fp, fp]
        L.orc_grads.restype = C.c_float
        L.orc_grads.argtypes = [C.POINTER(OrcCfg), fp, u16, u16, C.c_int, C.c_float, fp]
        L.orc_adam_update.restype = None
        L.orc_adam_update.argtypes = [C.POINTER(OrcCfg), fp, fp, fp, fp, C.c_int, C.POINTER(OrcAdam)]
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_set_parallel_linear.argtypes = [C.c_int]
        L.orc_linear_cf.argtypes = [fp, fp, fp, C.c_int, C.c_int, C.c_int]
        L.orc_rmsnorm_noweight_cf.argtypes = [fp, fp, C.c_int, C.c_int]
        L.orc_rmsnorm_cf.argtypes = [fp, fp, fp, C.c_int, C.c_int]
        L.orc_causal_attention_cf.argtypes = [fp, fp, fp, fp, C.c_int, C.c_int, C.c_int]
        L.orc_build_rope.argtypes = [fp, fp, C.c_int, C.c_int, C.c_double]
        L.orc_apply_rope_cf.argtypes = [fp, C.c_int, C.c_int, C.c_int, fp, fp]
        L.orc_qknorm_cf.argtypes = [fp, fp, C.c_int, C.c_int, C.c_int]
        L.orc_cross_entropy.restype = C.c_float
        L.orc_cross_entropy.argtypes = [fp, fp, u16, C.c_int, C.c_int]
        L.orc_softcap.argtypes = [fp, C.c_size_t]
        L.orc_drand48_seed.restype = C.c_uint64
        L.orc_drand48_seed.argtypes = [C.c_int64]
        L.orc_drand48_next.restype = C.c_double
        L.orc_drand48_next.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_dec_param_count.restype = C.c_size_t
        L.orc_dec_param_count.argtypes = [C.POINTER(OrcDecCfg)]
        L.orc_decode.restype = None
        L.orc_decode.argtypes = [C.POINTER(OrcDecCfg), fp, u16, C.c_int, C.c_int, u16, C.c_int, C.c_int, u16, fp]
        i32 = C.POINTER(C.c_int32)
        L.orc_moe_param_count.restype = C.c_size_t
        L.orc_moe_param_count.argtypes = [C.POINTER(OrcMoeCfg)]
        L.orc_moe_route.restype = None
        L.orc_moe_route.argtypes = [C.POINTER(OrcMoeCfg), fp, fp, C.c_int, i32, fp]
        L.orc_moe_forward.restype = None
        L.orc_moe_forward.argtypes = [C.POINTER(OrcMoeCfg), fp, fp, C.c_int, C.c_int, fp, i32, fp]
        L.orc_linear_bwd_dx_cf.argtypes = [fp, fp, fp, C.c_int, C.c_int, C.c_int]
        L.orc_rmsnorm_noweight_bwd_cf.argtypes = [fp, fp, fp, C.c_int, C.c_int]
        L.orc_causal_attention_bwd_cf.argtypes = [fp, fp, fp, fp, fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_float]
        L.orc_matmul_vocab_seq.argtypes = [fp, fp, fp, C.c_int, C.c_int, C.c_int]
        L.orc_matmul_embedT.argtypes = [fp, fp, fp, C.c_int, C.c_int, C.c_int]
        L.orc_softmax_row.argtypes = [fp, fp, C.c_int]
        L.orc_seam_layer_forward.argtypes = [C.POINTER(OrcSeamLayer), C.c_int, C.c_int, C.c_int, C.c_int, fp, fp,
                                             C.POINTER(OrcSeamTaps)]
        L.orc_seam_attention_backward.argtypes = [C.POINTER(OrcSeamLayer), C.c_int, C.c_int, C.c_int, fp, fp, fp,
                                                  fp, fp, fp, fp, fp]
        L.orc_seam_ffn_backward.argtypes = [C.POINTER(OrcSeamLayer), C.c_int, C.c_int, C.c_int, fp, fp, fp, fp]
        L.orc_seam_softmax_vocab.argtypes = [fp, C.c_int, C.c_int]
        ncpu = os.cpu_count() or 1
        L.orc_set_threads(min(ncpu, 64))
        L.orc_set_parallel_linear(1)
        _lib = L
    return _lib


def set_threads(n: int, parallel_linear: bool = True):
    lib().orc_set_threads(int(n))
    lib().orc_set_parallel_linear(1 if parallel_linear else 0)


def _f(a):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _u16(a):
    assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def cfg_struct(cfg) -> OrcCfg:
    """cfg: any object with dim/hidden/heads/layers/vocab/seq/arch/grad_mode/rope_theta."""
    return OrcCfg(cfg.dim, cfg.hidden, cfg.heads, cfg.layers, cfg.vocab, cfg.seq,
                  ARCH[cfg.arch], GRAD[cfg.grad_mode], float(cfg.rope_theta))


def param_count(cfg) -> int:
    return int(lib().orc_param_count(C.byref(cfg_struct(cfg))))


def param_segments(cfg):
    c = cfg_struct(cfg)
    n = lib().orc_param_segments(C.byref(c), None, None, 0)
    off = (C.c_int64 * n)()
    sz = (C.c_int64 * n)()
    lib().orc_param_segments(C.byref(c), off, sz, n)
    return [(int(off[i]), int(sz[i])) for i in range(n)]


def forward_loss(cfg, params, tokens, targets, want_logits=False):
    """tokens/targets: uint16 [nseq, seq]. Returns (mean, per_seq, logits|None);
    logits are [nseq, V, seq] vocab-major, as EvalLogits returns them."""
    tokens = np.ascontiguousarray(tokens, dtype=np.uint16).reshape(-1, cfg.seq)
    targets = np.ascontiguousarray(targets, dtype=np.uint16).reshape(-1, cfg.seq)
    n = tokens.shape[0]
    per = np.zeros(n, np.float32)
    lg = np.zeros((n, cfg.vocab, cfg.seq), np.float32) if want_logits else None
    m = lib().orc_forward_loss(C.byref(cfg_struct(cfg)), _f(params), _u16(tokens), _u16(targets), n,
                               _f(lg) if lg is not None else None, _f(per))
    return float(m), per, lg


def grads(cfg, params, tokens, targets, loss_scale=256.0):
    tokens = np.ascontiguousarray(tokens, dtype=np.uint16).reshape(-1, cfg.seq)
    targets = np.ascontiguousarray(targets, dtype=np.uint16).reshape(-1, cfg.seq)
    g = np.zeros(param_count(cfg), np.float32)
    loss = lib().orc_grads(C.byref(cfg_struct(cfg)), _f(params), _u16(tokens), _u16(targets),
                           tokens.shape[0], float(loss_scale), _f(g))
    return float(loss), g


def adam_update(cfg, params, g, m, v, step, hp: dict):
    h = OrcAdam(**{k: float(hp[k]) for k in (
        "lr", "beta1", "beta2", "eps", "weight_decay", "grad_clip", "embed_lr_mult",
        "scalar_lr_mult", "lambda_lr_mult", "lambda_beta1", "lambda_beta2")})
    lib().orc_adam_update(C.byref(cfg_struct(cfg)), _f(params), _f(g), _f(m), _f(v), int(step), C.byref(h))


# --- single ops (channel-first, reference signatures) ---------------------
def linear_cf(w, x):
    oc, ic = w.shape
    seq = x.shape[1]
    out = np.zeros((oc, seq), np.float32)
    lib().orc_linear_cf(_f(out), _f(w), _f(x), oc, ic, seq)
    return out


def rmsnorm_noweight_cf(x):
    out = np.zeros_like(x)
    lib().orc_rmsnorm_noweight_cf(_f(out), _f(x), x.shape[0], x.shape[1])
    return out


def rmsnorm_cf(x, w):
    out = np.zeros_like(x)
    lib().orc_rmsnorm_cf(_f(out), _f(x), _f(w), x.shape[0], x.shape[1])
    return out


def causal_attention_cf(q, k, v, heads):
    out = np.zeros_like(q)
    dim, seq = q.shape
    lib().orc_causal_attention_cf(_f(out), _f(q), _f(k), _f(v), heads, dim // heads, seq)
    return out


def rope_tables(seq, head_dim, theta):
    c = np.zeros((seq, head_dim // 2), np.float32)
    s = np.zeros((seq, head_dim // 2), np.float32)
    lib().orc_build_rope(_f(c), _f(s), seq, head_dim, float(theta))
    return c, s


def apply_rope_cf(x, heads, cos_t, sin_t):
    x = np.ascontiguousarray(x.copy())
    dim, seq = x.shape
    lib().orc_apply_rope_cf(_f(x), heads, dim // heads, seq, _f(cos_t), _f(sin_t))
    return x


def qknorm_cf(q, k, heads):
    q = np.ascontiguousarray(q.copy())
    k = np.ascontiguousarray(k.copy())
    lib().orc_qknorm_cf(_f(q), _f(k), q.shape[0], heads, q.shape[1])
    return q, k


def cross_entropy(logits, targets):
    v, s = logits.shape
    dl = np.zeros_like(logits)
    t = np.ascontiguousarray(targets, dtype=np.uint16)
    loss = lib().orc_cross_entropy(_f(dl), _f(np.ascontiguousarray(logits)), _u16(t), v, s)
    return float(loss), dl


def softcap(x):
    x = np.ascontiguousarray(x.copy(), dtype=np.float32)
    lib().orc_softcap(_f(x), x.size)
    return x


def dec_cfg_struct(cfg) -> OrcDecCfg:
    return OrcDecCfg(cfg.dim, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.layers, cfg.vocab, float(cfg.rope_theta))


def dec_param_count(cfg) -> int:
    return int(lib().orc_dec_param_count(C.byref(dec_cfg_struct(cfg))))


def decode(cfg, params, prefix, nsteps, forced=None, want_logits=False, threads=None):
    """Greedy KV-cache decoding (oracle/refdecode.c).  prefix: uint16
    [nseq, plen].  Returns (tokens [nseq, nsteps+1], logits [nseq, nsteps+1, V]
    or None); tokens[:, 0] follows the prefix, tokens[:, i+1] decode step i,
    whose input is forced[:, i] if given, else tokens[:, i]."""
    prefix = np.ascontiguousarray(prefix, dtype=np.uint16)
    nseq, plen = prefix.shape
    if forced is not None:
        forced = np.ascontiguousarray(forced, dtype=np.uint16).reshape(nseq, nsteps)
    toks = np.zeros((nseq, nsteps + 1), np.uint16)
    lg = np.zeros((nseq, nsteps + 1, cfg.vocab), np.float32) if want_logits else None
    th = threads or min(nseq, os.cpu_count() or 1)
    lib().orc_decode(C.byref(dec_cfg_struct(cfg)), _f(params), _u16(prefix), nseq, plen,
                     _u16(forced) if forced is not None else None, int(nsteps), int(th), _u16(toks),
                     _f(lg) if lg is not None else None)
    return toks, lg


def _moe_cfg(dim, hidden, experts):
    return OrcMoeCfg(int(dim), int(hidden), int(experts))


def moe_param_count(dim, hidden, experts) -> int:
    return int(lib().orc_moe_param_count(C.byref(_moe_cfg(dim, hidden, experts))))


def moe_route(params, x, hidden, experts):
    """x fp32 [T, D] -> (expert ids int32 [T, 2], weights fp32 [T, 2])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, D = x.shape
    idx = np.zeros((T, 2), np.int32)
    w = np.zeros((T, 2), np.float32)
    lib().orc_moe_route(C.byref(_moe_cfg(D, hidden, experts)), _f(params), _f(x), T,
                        idx.ctypes.data_as(C.POINTER(C.c_int32)), _f(w))
    return idx, w


def moe_forward(params, x, hidden, experts, threads=None):
    """Mixture-of-experts FFN (oracle/refmoe.c): returns (out [T, D], idx, w)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, D = x.shape
    out = np.zeros((T, D), np.float32)
    idx = np.zeros((T, 2), np.int32)
    w = np.zeros((T, 2), np.float32)
    lib().orc_moe_forward(C.byref(_moe_cfg(D, hidden, experts)), _f(params), _f(x), T,
                          int(threads or os.cpu_count() or 1), _f(out),
                          idx.ctypes.data_as(C.POINTER(C.c_int32)), _f(w))
    return out, idx, w


def drand48_stream(seed, n):
    st = C.c_uint64(lib().orc_drand48_seed(int(seed)))
    return np.array([lib().orc_drand48_next(C.byref(st)) for _ in range(n)])


# --- the per-object accelerator seam (refseam.c) --------------------------
def _seam_layer(w):
    """w: dict of fp32 arrays wq, wk, wv, wo [D, D], w1 [H, D], w2 [D, H]."""
    keep = {n: np.ascontiguousarray(w[n], dtype=np.float32) for n in ("wq", "wk", "wv", "wo", "w1", "w2")}
    return OrcSeamLayer(*[_f(keep[n]) for n in ("wq", "wk", "wv", "wo", "w1", "w2")]), keep


def seam_layer_forward(w, heads, x):
    """The layer forward the accelerator programs compute; x [D, seq].
    Returns (out, taps) with the runWithTaps taps as a dict."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    dim, seq = x.shape
    hidden = w["w1"].shape[0]
    lw, keep = _seam_layer(w)
    out = np.zeros_like(x)
    taps = {n: np.zeros((hidden if n in ("h1", "gate") else dim, seq), np.float32) for n in SEAM_TAPS}
    t = OrcSeamTaps(*[_f(taps[n]) for n in SEAM_TAPS])
    lib().orc_seam_layer_forward(C.byref(lw), dim, hidden, heads, seq, _f(x), _f(out), C.byref(t))
    return out, taps


def seam_attention_backward(w, heads, q, k, v, dx2):
    """Returns (dx_norm, dq, dk, dv), each [D, seq]."""
    q, k, v, dx2 = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, dx2))
    dim, seq = q.shape
    lw, keep = _seam_layer(w)
    outs = [np.zeros_like(q) for _ in range(4)]
    lib().orc_seam_attention_backward(C.byref(lw), dim, heads, seq, _f(q), _f(k), _f(v), _f(dx2),
                                      *[_f(o) for o in outs])
    return tuple(outs)


def seam_ffn_backward(w, dffn, h1):
    """Returns (dx_norm [D, seq], dh1 [H, seq])."""
    dffn = np.ascontiguousarray(dffn, dtype=np.float32)
    h1 = np.ascontiguousarray(h1, dtype=np.float32)
    dim, seq = dffn.shape
    hidden = h1.shape[0]
    lw, keep = _seam_layer(w)
    dx = np.zeros_like(dffn)
    dh1 = np.zeros_like(h1)
    lib().orc_seam_ffn_backward(C.byref(lw), dim, hidden, seq, _f(dffn), _f(h1), _f(dx), _f(dh1))
    return dx, dh1


def seam_softmax_vocab(logits):
    p = np.ascontiguousarray(logits, dtype=np.float32).copy()
    lib().orc_seam_softmax_vocab(_f(p), p.shape[0], p.shape[1])
    return p


def rmsnorm_noweight_bwd_cf(dy, x):
    dy = np.ascontiguousarray(dy, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    dx = np.zeros_like(x)
    lib().orc_rmsnorm_noweight_bwd_cf(_f(dx), _f(dy), _f(x), x.shape[0], x.shape[1])
    return dx


def matmul_vocab_seq(embed, x):
    """logits [V, seq] = Embed [V, D] x [D, seq]."""
    embed = np.ascontiguousarray(embed, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros((embed.shape[0], x.shape[1]), np.float32)
    lib().orc_matmul_vocab_seq(_f(out), _f(embed), _f(x), embed.shape[0], embed.shape[1], x.shape[1])
    return out


def matmul_embed_t(embed, dlogits):
    """dy [D, seq] = Embed^T dlogits."""
    embed = np.ascontiguousarray(embed, dtype=np.float32)
    dlogits = np.ascontiguousarray(dlogits, dtype=np.float32)
    out = np.zeros((embed.shape[1], dlogits.shape[1]), np.float32)
    lib().orc_matmul_embedT(_f(out), _f(embed), _f(dlogits), embed.shape[0], embed.shape[1], dlogits.shape[1])
    return out
