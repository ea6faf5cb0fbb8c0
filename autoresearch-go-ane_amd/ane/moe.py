"""Mixture-of-experts FFN layer over the HIP C-ABI (``ane_moe_*``).

No counterpart in the reference (its FFN is dense); this serves the MoE
benchmark configuration: dim 768, 8 SwiGLU experts of hidden 2048, top-2
softmax router.  Routing is computed in fp32 in the reference's linearCF
summation order so the expert assignment is bit-exact with the CPU path;
the expert FFNs run as grouped fp16 MFMA GEMMs with fp32 accumulation.
Parameters (flat fp32): router [E][D], then per expert W1 [H][D], W3 [H][D],
W2 [D][H].
"""
from __future__ import annotations

import ctypes as C
import dataclasses

import numpy as np

from . import _lib
from .engine import EngineError


@dataclasses.dataclass
class MoeConfig:
    dim: int = 768
    hidden: int = 2048
    experts: int = 8
    top_k: int = 2


def moe_param_layout(cfg: MoeConfig):
    D, H, E = cfg.dim, cfg.hidden, cfg.experts
    out, off = [("router", 0, (E, D))], E * D
    for e in range(E):
        for name, shape in ((f"experts.{e}.w1", (H, D)), (f"experts.{e}.w3", (H, D)),
                            (f"experts.{e}.w2", (D, H))):
            out.append((name, off, shape))
            off += int(np.prod(shape))
    return out


def moe_param_count(cfg: MoeConfig) -> int:
    return cfg.experts * cfg.dim + cfg.experts * 3 * cfg.hidden * cfg.dim


def init_moe_params(cfg: MoeConfig, seed: int = 5, std: float = 0.02) -> np.ndarray:
    """Every weight ~ N(0, std) from numpy's PCG64 stream of ``seed``."""
    rng = np.random.default_rng(seed)
    flat = rng.standard_normal(moe_param_count(cfg), dtype=np.float32)
    flat *= np.float32(std)
    return flat


def make_moe_input(cfg: MoeConfig, tokens: int, seed: int = 5) -> np.ndarray:
    """Activations ~ N(0, 1), [tokens, dim] fp32."""
    return np.random.default_rng(seed + 1_000_003).standard_normal((tokens, cfg.dim), dtype=np.float32)


def _f(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


class MoeLayer:
    """Open(cfg, params, max_tokens) -> Forward(x) / Load + Run + Read."""

    def __init__(self, cfg: MoeConfig, params, max_tokens: int = 8192, device: int = 0):
        self._lib = _lib.load()
        self.cfg = cfg
        self._c = _lib.MoeCfg(cfg.dim, cfg.hidden, cfg.experts, cfg.top_k, int(max_tokens), int(device))
        h = C.c_void_p()
        rc = self._lib.ane_moe_open(C.byref(self._c), C.byref(h))
        if rc != _lib.ANE_OK:
            msg = self._lib.ane_moe_last_error(h) if h.value else b"storiesane moe open: failed"
            if h.value:
                self._lib.ane_moe_destroy(h)
            raise EngineError(rc, msg.decode())
        self._h = h
        self.tokens = 0
        try:
            self.SetParams(params)
        except Exception:
            self.Close()
            raise

    def _check(self, rc):
        if rc != _lib.ANE_OK:
            raise EngineError(rc, self._lib.ane_moe_last_error(self._h).decode())

    def _live(self):
        if self._h is None:
            raise EngineError(_lib.ANE_ERR_CLOSED, "storiesane moe: layer is closed")

    def SetParams(self, params):
        self._live()
        p = np.ascontiguousarray(params, dtype=np.float32)
        self._check(self._lib.ane_moe_set_params(self._h, _f(p), p.size))

    def Load(self, x):
        """Copies x [T, D] fp32 into device memory (inputs resident for Run)."""
        self._live()
        x = np.ascontiguousarray(x, dtype=np.float32)
        self._check(self._lib.ane_moe_load_input(self._h, _f(x), x.shape[0]))
        self.tokens = x.shape[0]

    def Run(self):
        """Routing, grouping, expert GEMMs and combine on the resident input."""
        self._live()
        self._check(self._lib.ane_moe_run(self._h))

    def Read(self):
        """-> (out [T, D] fp32, expert ids int32 [T, 2], weights fp32 [T, 2])."""
        self._live()
        T, D = self.tokens, self.cfg.dim
        out = np.zeros((T, D), np.float32)
        idx = np.zeros((T, 2), np.int32)
        w = np.zeros((T, 2), np.float32)
        self._check(self._lib.ane_moe_read_output(self._h, _f(out), idx.ctypes.data_as(C.POINTER(C.c_int32)),
                                                  _f(w)))
        return out, idx, w

    def Forward(self, x):
        self.Load(x)
        self.Run()
        return self.Read()

    def LastMs(self) -> float:
        self._live()
        return float(self._lib.ane_moe_last_ms(self._h))

    def Close(self):
        if getattr(self, "_h", None) is not None:
            self._lib.ane_moe_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.Close()
        except Exception:
            pass
