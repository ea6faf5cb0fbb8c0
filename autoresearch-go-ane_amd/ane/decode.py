"""Greedy KV-cache decoder over the HIP C-ABI (``ane_decode_*``).

The reference has no decode path; this serves the decode benchmark's
Llama2-style model with grouped-query attention (``Config.kv_heads`` key /
value heads), built from the same primitives as the engine.  Errors follow
the engine's convention: a negative status raises ``EngineError`` with the
library's message; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .config import Config, param_count
from .engine import EngineError


def _u16(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def _f(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


class Decoder:
    """Open(cfg, params, max_batch, max_ctx) -> Prefill -> Step / Generate."""

    def __init__(self, cfg: Config, params, max_batch: int = 64, max_ctx: int = 1152, device: int = 0):
        if cfg.arch != "llama2":
            raise EngineError(_lib.ANE_ERR_ARG, "storiesane decode open: arch must be llama2")
        self._lib = _lib.load()
        self.cfg = cfg
        self._c = _lib.DecodeCfg(cfg.dim, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.layers, cfg.vocab,
                                 int(max_batch), int(max_ctx), float(cfg.rope_theta), int(device))
        h = C.c_void_p()
        rc = self._lib.ane_decode_open(C.byref(self._c), C.byref(h))
        if rc != _lib.ANE_OK:
            msg = self._lib.ane_decode_last_error(h) if h.value else b"storiesane decode open: failed"
            if h.value:
                self._lib.ane_decode_destroy(h)
            raise EngineError(rc, msg.decode())
        self._h = h
        self.nseq = 0
        try:
            self.SetParams(params)
        except Exception:
            self.Close()
            raise

    def _check(self, rc):
        if rc != _lib.ANE_OK:
            raise EngineError(rc, self._lib.ane_decode_last_error(self._h).decode())

    def _live(self):
        if self._h is None:
            raise EngineError(_lib.ANE_ERR_CLOSED, "storiesane decode: decoder is closed")

    def SetParams(self, params):
        self._live()
        p = np.ascontiguousarray(params, dtype=np.float32)
        n = int(self._lib.ane_decode_param_count(C.byref(self._c)))
        if p.size != n or n != param_count(self.cfg):
            raise EngineError(_lib.ANE_ERR_ARG, f"storiesane decode set params: len={p.size} want={n}")
        self._check(self._lib.ane_decode_set_params(self._h, _f(p), p.size))

    def Prefill(self, prefix, want_logits=False):
        """prefix uint16 [nseq, plen] -> (next tokens [nseq], logits [nseq, V] | None)."""
        self._live()
        pre = np.ascontiguousarray(prefix, dtype=np.uint16)
        nseq, plen = pre.shape
        nxt = np.zeros(nseq, np.uint16)
        lg = np.zeros((nseq, self.cfg.vocab), np.float32) if want_logits else None
        self._check(self._lib.ane_decode_prefill(self._h, _u16(pre), nseq, plen, _u16(nxt),
                                                 _f(lg) if lg is not None else None))
        self.nseq = nseq
        return nxt, lg

    def Step(self, tokens=None, want_logits=False):
        """One step; tokens [nseq] (None: the previous greedy tokens)."""
        self._live()
        t = None if tokens is None else np.ascontiguousarray(tokens, dtype=np.uint16).reshape(self.nseq)
        nxt = np.zeros(self.nseq, np.uint16)
        lg = np.zeros((self.nseq, self.cfg.vocab), np.float32) if want_logits else None
        self._check(self._lib.ane_decode_step(self._h, _u16(t) if t is not None else None, _u16(nxt),
                                              _f(lg) if lg is not None else None))
        return nxt, lg

    def Generate(self, nsteps: int):
        """nsteps greedy steps on the device; returns tokens [nseq, nsteps]."""
        self._live()
        out = np.zeros((nsteps, max(self.nseq, 1)), np.uint16)
        self._check(self._lib.ane_decode_generate(self._h, int(nsteps), _u16(out)))
        return np.ascontiguousarray(out[:, :self.nseq].T)

    def Position(self) -> int:
        self._live()
        return int(self._lib.ane_decode_position(self._h))

    def FusedChain(self) -> int:
        """1: steps run the fused per-layer chain; 0: one launch per GEMM;
        2: one launch per GEMM since a chain wait timed out (the call was
        redone that way and the decoder stays on it)."""
        self._live()
        return int(self._lib.ane_decode_fused_chain(self._h))

    def DebugFillCache(self, byte: int = 0xFF):
        """Test-only: every byte of the KV cache set to `byte` (0xFF: NaN)."""
        self._live()
        self._check(self._lib.ane_decode_debug_fill_cache(self._h, int(byte)))

    def LastMs(self) -> float:
        self._live()
        return float(self._lib.ane_decode_last_ms(self._h))

    def Close(self):
        if getattr(self, "_h", None) is not None:
            self._lib.ane_decode_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.Close()
        except Exception:
            pass
