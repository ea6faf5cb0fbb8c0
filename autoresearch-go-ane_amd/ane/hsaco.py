"""The llama2 eval forward + loss driven over the gfx950 code objects alone.

This is the boundary a pure-Go host would use through purego (the
reference's engine reaches its accelerator that way, with no CGo): dlopen
libamdhip64, hipModuleLoad the `.hsaco` files the build writes next to
libane_hip.so (`include/ane_kernels.h`), look the kernels up by their C
names and launch them with hipModuleLaunchKernel.  Nothing of libane_hip.so
runs here except `ane_kernel_abi`, which reports the argument structs'
layout this module checks its ctypes mirrors against.

`eval_loss` runs the same kernels with the same arguments as the library's
EvalLoss for a llama2 model (the deferred-norm forward: the residual GEMMs
leave fp16(x * gain) and per-row partial sums of squares, the consumers
scale by 1 / rms) and returns the per-sequence mean losses
(ane/engine.go:464-482; the forward of ane/stories/cpu.go and the
cross-entropy of ane/stories/cpu.go:212-292).  No fallback: a missing code
object or a HIP error raises.
"""
import ctypes as C
import math
import os

import numpy as np

from . import _lib
from .config import Config, param_layout

HERE = os.path.dirname(os.path.abspath(__file__))
MODULES = {"gemm": "ane_gemm.hsaco", "attention": "ane_attention.hsaco", "rowops": "ane_rowops.hsaco"}


class AneGemmArgs(C.Structure):
    _fields_ = [("A", C.c_void_p), ("B", C.c_void_p), ("lda", C.c_int32), ("ldb", C.c_int32), ("M", C.c_int32),
                ("N", C.c_int32), ("K", C.c_int32), ("a_t", C.c_uint8), ("b_t", C.c_uint8), ("grp", C.c_void_p),
                ("b_group_stride", C.c_size_t), ("splits", C.c_int32), ("ws", C.c_void_p), ("pf", C.c_void_p),
                ("pf_bytes", C.c_size_t)]


class AneEpiParams(C.Structure):
    _fields_ = [("C", C.c_void_p), ("ldc", C.c_int32), ("C2", C.c_void_p), ("ldc2", C.c_int32), ("R", C.c_void_p),
                ("X0", C.c_void_p), ("alpha", C.c_float), ("beta", C.c_float), ("scale", C.c_float),
                ("alpha_ptr", C.c_void_p), ("beta_ptr", C.c_void_p), ("accumulate", C.c_int32), ("seq", C.c_int32),
                ("targets", C.c_void_p), ("partial", C.c_void_p), ("tgt_logit", C.c_void_p), ("lse", C.c_void_p),
                ("colscale", C.c_void_p), ("softcap", C.c_int32), ("cap", C.c_float), ("vocab", C.c_int32),
                ("C3", C.c_void_p), ("rowscale", C.c_void_p), ("gain", C.c_void_p), ("ssq_part", C.c_void_p),
                ("ssq_ld", C.c_int32), ("rr_part", C.c_void_p), ("rr_ld", C.c_int32), ("rr_nparts", C.c_int32),
                ("rr_dim", C.c_int32)]


class AneAttnArgs(C.Structure):
    _fields_ = [("qkv", C.c_void_p), ("out", C.c_void_p), ("lse", C.c_void_p), ("rope_cos", C.c_void_p),
                ("rope_sin", C.c_void_p), ("nseq", C.c_int32), ("S", C.c_int32), ("NH", C.c_int32),
                ("qknorm", C.c_int32), ("scale", C.c_float), ("ve_x", C.c_void_p), ("ve_gate", C.c_void_p),
                ("ve_embed", C.c_void_p), ("tokens", C.c_void_p), ("vocab", C.c_int32), ("qkvt", C.c_void_p),
                ("qkvt_lo", C.c_void_p), ("hilo", C.c_int32), ("pf", C.c_void_p), ("pf_bytes", C.c_size_t),
                ("split_from", C.c_int32)]


STRUCTS = {"AneGemmArgs": AneGemmArgs, "AneEpiParams": AneEpiParams, "AneAttnArgs": AneAttnArgs}


def check_abi(lib=None):
    """The ctypes mirrors against the layout the kernels were compiled with."""
    lib = lib or _lib.load()
    for name, st in STRUCTS.items():
        size = C.c_int64()
        offs = (C.c_int64 * 64)()
        n = lib.ane_kernel_abi(name.encode(), C.byref(size), offs, 64)
        mine = [getattr(st, f).offset for f, _ in st._fields_]
        if n != len(mine) or size.value != C.sizeof(st) or list(offs[:n]) != mine:
            raise RuntimeError(f"{name}: kernel layout {size.value} B {list(offs[:n])}, mirror {C.sizeof(st)} B {mine}")


class Hip:
    """The few libamdhip64 entry points the driver needs (its C API)."""

    def __init__(self):
        # the process's HIP runtime if one is loaded (same SONAME), else the installed one
        self.lib = C.CDLL("libamdhip64.so.7", mode=C.RTLD_GLOBAL)
        L = self.lib
        L.hipModuleLoad.argtypes = [C.POINTER(C.c_void_p), C.c_char_p]
        L.hipModuleGetFunction.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_char_p]
        L.hipModuleLaunchKernel.argtypes = [C.c_void_p] + [C.c_uint] * 7 + [C.c_void_p, C.POINTER(C.c_void_p),
                                                                          C.POINTER(C.c_void_p)]
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.hipFree.argtypes = [C.c_void_p]
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipDeviceSynchronize.argtypes = []
        L.hipModuleUnload.argtypes = [C.c_void_p]
        L.hipGetErrorString.restype = C.c_char_p
        L.hipGetErrorString.argtypes = [C.c_int]

    def check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"storiesane hsaco: {what}: {self.lib.hipGetErrorString(rc).decode()}")

    def malloc(self, nbytes):
        p = C.c_void_p()
        self.check(self.lib.hipMalloc(C.byref(p), max(int(nbytes), 16)), "hipMalloc")
        return p.value

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.malloc(arr.nbytes)
        self.check(self.lib.hipMemcpy(p, arr.ctypes.data, arr.nbytes, 1), "hipMemcpy HtoD")
        return p

    def download(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        self.check(self.lib.hipMemcpy(out.ctypes.data, p, out.nbytes, 2), "hipMemcpy DtoH")
        return out


class CodeObjects:
    """The three modules and a launch helper (kernelParams: one pointer per argument)."""

    def __init__(self, hip, directory=HERE):
        self.hip = hip
        self.mods, self.fns = {}, {}
        for key, fname in MODULES.items():
            path = os.path.join(directory, fname)
            if not os.path.exists(path):
                raise RuntimeError(f"storiesane hsaco: {path} not built; run __graft_entry__.build()")
            m = C.c_void_p()
            hip.check(hip.lib.hipModuleLoad(C.byref(m), path.encode()), f"hipModuleLoad {fname}")
            self.mods[key] = m.value

    def fn(self, module, name):
        if name not in self.fns:
            f = C.c_void_p()
            self.hip.check(self.hip.lib.hipModuleGetFunction(C.byref(f), self.mods[module], name.encode()),
                           f"hipModuleGetFunction {name}")
            self.fns[name] = f.value
        return self.fns[name]

    def launch(self, module, name, grid, block, *args):
        arr = (C.c_void_p * len(args))(*[C.cast(C.pointer(a), C.c_void_p) for a in args])
        g = tuple(grid) + (1,) * (3 - len(grid))
        self.hip.check(self.hip.lib.hipModuleLaunchKernel(self.fn(module, name), g[0], g[1], g[2], block, 1, 1, 0,
                                                           None, arr, None), f"launch {name}")

    def close(self):
        for m in self.mods.values():
            self.hip.lib.hipModuleUnload(m)
        self.mods, self.fns = {}, {}


def rope_tables(S, theta):
    """buildRoPETables (ane/train_util.go:183-202): [S][32] cos and sin, float32."""
    pos = np.arange(S, dtype=np.float64)[:, None]
    i = np.arange(32, dtype=np.float64)[None, :]
    freq = pos / np.power(theta, 2.0 * i / 64.0)
    return np.cos(freq).astype(np.float32), np.sin(freq).astype(np.float32)


def _gemm(M, N, K, A, lda, B, ldb):
    return AneGemmArgs(A=A, B=B, lda=lda, ldb=ldb, M=M, N=N, K=K, a_t=0, b_t=0, grp=None, b_group_stride=0, splits=1,
                       ws=None, pf=None, pf_bytes=0)


def eval_loss(cfg: Config, params: np.ndarray, tokens: np.ndarray, targets: np.ndarray) -> np.ndarray:
    """Per-sequence mean cross-entropy of a llama2 model over [nseq, seq]
    token / target windows, by the code objects' kernels only."""
    if cfg.arch != "llama2":
        raise ValueError("storiesane hsaco: the exported forward is the llama2 one")
    tokens = np.ascontiguousarray(tokens, np.uint16)
    targets = np.ascontiguousarray(targets, np.uint16)
    nseq, S = tokens.shape
    D, H, V, NH, L = cfg.dim, cfg.hidden, cfg.vocab, cfg.heads, cfg.layers
    T = nseq * S
    # the exported kernels' tiles: 128x192 (Wq|Wk|Wv), 128x64 (Wo, W2), 256x256 (W1|W3, classifier); S = 256
    if (S != cfg.seq or S != 256 or T % 256 or (3 * D) % 192 or D % 64 or D > 64 * 16 or (2 * H) % 256 or
            V % 256 or D != 64 * NH):
        raise ValueError("storiesane hsaco: shapes outside the exported kernels' tiles")
    lay = {name: (off, shape) for name, off, shape in param_layout(cfg)}
    p = np.ascontiguousarray(params, np.float32)

    def w(name):
        off, shape = lay[name]
        return p[off:off + int(np.prod(shape))].reshape(shape)

    hip = Hip()
    check_abi()
    co = CodeObjects(hip)
    bufs = []

    def dev(arr):
        bufs.append(hip.upload(arr))
        return bufs[-1]

    def zeros(nbytes):
        return dev(np.zeros(int(nbytes), np.uint8))

    try:
        P = dev(p)
        f32 = 4
        # fp16 weights as the library's shadows hold them: Wq|Wk|Wv stacked,
        # W1 / W3 rows interleaved by 32, W2 and the embedding as they are
        layers = []
        for l in range(L):
            pre = f"layers.{l}."
            wqkv = np.concatenate([w(pre + "wq"), w(pre + "wk"), w(pre + "wv")]).astype(np.float16)
            w1, w3 = w(pre + "w1").reshape(H // 32, 32, D), w(pre + "w3").reshape(H // 32, 32, D)
            w13 = np.stack([w1, w3], axis=1).reshape(2 * H, D).astype(np.float16)
            layers.append(dict(wqkv=dev(wqkv), wo=dev(w(pre + "wo").astype(np.float16)), w13=dev(w13),
                               w2=dev(w(pre + "w2").astype(np.float16)),
                               g_att=P + lay[pre + "g_att"][0] * f32, g_ffn=P + lay[pre + "g_ffn"][0] * f32))
        embed_h = dev(w("embed").astype(np.float16))
        cs, sn = rope_tables(S, cfg.rope_theta)
        rope_cos, rope_sin = dev(cs), dev(sn)
        tok, tgt = dev(tokens.reshape(-1)), dev(targets.reshape(-1))
        x = zeros(T * D * 4)
        xh = zeros(T * D * 2)
        ssq = zeros(16 * T * 4)
        qkv = zeros(T * 3 * D * 2)
        att = zeros(T * D * 2)
        gate = zeros(T * H * 2)
        npart = V // 256
        partial = zeros(npart * T * 8)
        tgt_logit = zeros(T * 4)
        lse = zeros(T * 4)
        tok_loss = zeros(T * 4)
        loss_seq = zeros(nseq * 4)

        def ip(v):
            return C.c_void_p(v)

        i32, u64 = C.c_int32, C.c_size_t
        # embedding + the first norm's inputs (one partial per row)
        co.launch("rowops", "ane_k_embed_xg", ((T + 3) // 4,), 256, ip(x), ip(xh), ip(ssq),
                  ip(P + lay["embed"][0] * f32), ip(tok), ip(layers[0]["g_att"]), i32(T), i32(D), i32(V), ip(None),
                  u64(0))
        nparts = 1
        heads = nseq * NH
        # the library's dispatch: 1.5 heads per block for 256 < heads <= 384
        # (unless ANE_ATT_15=0), else whole heads with the heads past 256 as
        # two half blocks each
        by15 = S == 256 and 256 < heads <= 384 and os.environ.get("ANE_ATT_15", "1") != "0"
        split = 256 if 256 < heads < 512 and not by15 else 0
        for l, lw in enumerate(layers):
            g = _gemm(T, 3 * D, D, xh, D, lw["wqkv"], D)
            e = AneEpiParams(C=qkv, ldc=3 * D, scale=1.0, alpha=1.0, cap=15.0, rr_part=ssq, rr_ld=T, rr_nparts=nparts,
                             rr_dim=D)
            co.launch("gemm", "ane_k_gemm_qkv_rr", ((T // 128) * (3 * D // 192),), 256, g, e)
            a = AneAttnArgs(qkv=qkv, out=att, rope_cos=rope_cos, rope_sin=rope_sin, nseq=nseq, S=S, NH=NH, qknorm=0,
                            scale=0.125, split_from=split)
            if by15:
                co.launch("attention", "ane_k_attn_fwd15", (256,), 768, a)
            else:
                grid = (256 + 2 * (heads - 256),) if split else (1, NH, nseq)
                co.launch("attention", "ane_k_attn_fwd", grid, 512, a)
            g = _gemm(T, D, D, att, D, lw["wo"], D)
            e = AneEpiParams(C=x, ldc=D, R=x, C2=xh, ldc2=D, gain=lw["g_ffn"], ssq_part=ssq, ssq_ld=T, scale=1.0,
                             alpha=1.0, cap=15.0)
            co.launch("gemm", "ane_k_gemm_resid_norm", ((T // 128) * (D // 64),), 256, g, e)
            nparts = D // 64
            g = _gemm(T, 2 * H, D, xh, D, lw["w13"], D)
            e = AneEpiParams(C=gate, ldc=H, scale=1.0, alpha=1.0, cap=15.0, rr_part=ssq, rr_ld=T, rr_nparts=nparts,
                             rr_dim=D)
            co.launch("gemm", "ane_k_gemm_swiglu_rr", ((T // 256) * (2 * H // 256),), 512, g, e)
            g = _gemm(T, D, H, gate, H, lw["w2"], H)
            gain = layers[l + 1]["g_att"] if l + 1 < L else P + lay["g_final"][0] * f32
            e = AneEpiParams(C=x, ldc=D, R=x, C2=xh, ldc2=D, gain=gain, ssq_part=ssq, ssq_ld=T, scale=1.0, alpha=1.0,
                             cap=15.0)
            co.launch("gemm", "ane_k_gemm_resid_norm", ((T // 128) * (D // 64),), 256, g, e)
        # classifier (rows = vocabulary) with the final norm's 1 / rms on its token columns
        g = _gemm(V, T, D, embed_h, D, xh, D)
        e = AneEpiParams(targets=tgt, partial=partial, tgt_logit=tgt_logit, softcap=0, cap=15.0, vocab=V, scale=1.0,
                         alpha=1.0, rr_part=ssq, rr_ld=T, rr_nparts=nparts, rr_dim=D)
        co.launch("gemm", "ane_k_gemm_ce_rr", ((V // 256) * (T // 256),), 512, g, e)
        co.launch("rowops", "ane_k_ce_token", ((T + 31) // 32,), 256, ip(lse), ip(tok_loss), ip(partial),
                  i32(npart), ip(tgt_logit), ip(tgt), i32(V), i32(T))
        co.launch("rowops", "ane_k_ce_reduce", (nseq,), 256, ip(loss_seq), ip(None), C.c_float(0.0), ip(tok_loss),
                  ip(tgt), i32(V), i32(S))
        hip.check(hip.lib.hipDeviceSynchronize(), "hipDeviceSynchronize")
        return hip.download(loss_seq, (nseq,), np.float32)
    finally:
        for b in bufs:
            hip.lib.hipFree(C.c_void_p(b))
        co.close()
