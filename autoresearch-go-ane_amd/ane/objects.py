"""The reference's per-object accelerator seam, on the GPU.

The reference's Engine calls three accelerator objects -- layerForward,
layerBackward and offload -- and falls back to its CPU functions, for good,
when one fails (ane/engine.go:887-894; ane/train_full.go:373-380,488-493).
The non-darwin build stubs all three as unavailable
(ane/engine_other.go:15-89).  This module is the host side of the HIP
objects that replace them (include/ane_objects.h), with the reference's
constructor and method names:

  compile_stories_layer_forward  compileStoriesLayerForward  ane/layer_darwin.go:50-62
    .run / .run_with_taps / .refresh_weights / .close        ane/layer_darwin.go:175-324
  compile_stories_layer_backward compileStoriesLayerBackward ane/backward_darwin.go:40-180
    .run_ffn / .run_attention / .refresh_weights / .close     ane/backward_darwin.go:182-328
  new_offload / refresh_offload  newOffload / refreshOffload ane/offload_darwin.go:55-79
    .has_* / .disable_* / .run_* / .refresh_weights / .close  ane/offload_darwin.go:236-560

Buffers are the reference's channel-first fp32 slices ([channels, seq],
flat or 2-D, C-contiguous float32); outputs are written in place, as the
Go methods write their slices.  Errors raise SeamError with the message
the library reports ("run layer forward: layer is closed", ...), the
error value the Go methods return.  The CPU fallback belongs to the caller
(the reference's Engine keeps its own); nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

STORIES_HEADS = 12  # stories.Heads


class SeamError(RuntimeError):
    pass


def _check(rc: int):
    if rc != _lib.ANE_OK:
        raise SeamError(_lib.load().ane_seam_last_error().decode())


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _buf(op: str, name: str, a, want: int, writable: bool = False):
    """checkLen (ane/backward_darwin.go:397-402) plus the layout the C-ABI reads."""
    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags["C_CONTIGUOUS"]:
        raise SeamError(f"{op}: {name} must be a C-contiguous float32 array")
    if writable and not a.flags["WRITEABLE"]:
        raise SeamError(f"{op}: {name} is read-only")
    if a.size != want:
        raise SeamError(f"{op}: {name} len={a.size} want={want}")
    return _fp(a)


class _Weights:
    """stories.LayerWeights as ane_layer_weights; keeps the arrays alive for the call."""

    def __init__(self, op: str, layer, dim: int, hidden: int):
        shapes = {"wq": dim * dim, "wk": dim * dim, "wv": dim * dim, "wo": dim * dim, "w1": hidden * dim,
                  "w2": dim * hidden}
        self.keep = {}
        for n, size in shapes.items():
            a = np.ascontiguousarray(_get(layer, n), dtype=np.float32)
            if a.size != size:
                raise SeamError(f"{op}: {n} len={a.size} want={size}")
            self.keep[n] = a
        self.c = _lib.LayerWeights(*[_fp(self.keep[n]) for n in shapes])


def _get(layer, name: str):
    """A weight by the Go field name (Wq ...) or the lower-case one (wq ...)."""
    if isinstance(layer, dict):
        return layer[name] if name in layer else layer[name[0].upper() + name[1:]]
    return getattr(layer, name, None) if hasattr(layer, name) else getattr(layer, name[0].upper() + name[1:])


def _dims(layer, heads: int):
    wq = np.asarray(_get(layer, "wq"))
    w1 = np.asarray(_get(layer, "w1"))
    dim = wq.shape[0] if wq.ndim == 2 else int(round(np.sqrt(wq.size)))
    hidden = w1.size // dim
    return dim, hidden, heads


class LayerCache:
    """The taps of layerCache (ane/train_full.go:12-37) that runWithTaps fills."""

    def __init__(self, dim: int, hidden: int, seq: int):
        for n in _lib.LAYER_TAPS:
            setattr(self, n, np.zeros((hidden if n in ("h1", "gate") else dim) * seq, np.float32))
        self.att_taps_ready = False
        self.ffn_taps_ready = False


class LayerForward:
    """layerForward (ane/layer_darwin.go:22-46) for one layer."""

    def __init__(self, handle, dim, hidden, heads, seq):
        self._h = handle
        self.dim, self.hidden, self.heads, self.seq = dim, hidden, heads, seq

    def run(self, out, x):
        """run (ane/layer_darwin.go:195-197)."""
        self.run_with_taps(out, x, None)

    def run_with_taps(self, out, x, cache: LayerCache | None):
        """runWithTaps (ane/layer_darwin.go:199-313)."""
        op = "run layer forward"
        want = self.dim * self.seq
        px = _buf(op, "input", x, want)
        po = _buf(op, "output", out, want, writable=True)
        if cache is None:
            _check(_lib.load().ane_layer_forward_run(self._h, po, px))
            return
        hs = self.hidden * self.seq
        taps = [_buf(op, n, getattr(cache, n), hs if n in ("h1", "gate") else want, writable=True)
                for n in _lib.LAYER_TAPS]
        c = _lib.LayerCache(*taps, 0, 0)
        cache.att_taps_ready = cache.ffn_taps_ready = False
        _check(_lib.load().ane_layer_forward_run_taps(self._h, po, px, C.byref(c)))
        cache.att_taps_ready = bool(c.att_taps_ready)
        cache.ffn_taps_ready = bool(c.ffn_taps_ready)

    def refresh_weights(self, w):
        """refreshWeights (ane/layer_darwin.go:315-324)."""
        if self._h is None:
            raise SeamError("refresh layer forward: layer is nil")
        cw = _Weights("refresh layer forward", w, self.dim, self.hidden)
        _check(_lib.load().ane_layer_forward_refresh(self._h, C.byref(cw.c)))

    def close(self):
        """close (ane/layer_darwin.go:175-193): later calls report "layer is closed"."""
        if self._h is not None:
            _lib.load().ane_layer_forward_close(self._h)

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h is not None and _lib._lib is not None:
            _lib._lib.ane_layer_forward_destroy(h)


def compile_stories_layer_forward(layer, seq: int, heads: int = STORIES_HEADS) -> LayerForward:
    """compileStoriesLayerForward (ane/layer_darwin.go:50-62)."""
    dim, hidden, heads = _dims(layer, heads)
    cw = _Weights("compile layer forward", layer, dim, hidden)
    h = C.c_void_p()
    _check(_lib.load().ane_layer_forward_open(dim, hidden, heads, seq, C.byref(cw.c), C.byref(h)))
    return LayerForward(h, dim, hidden, heads, seq)


class LayerBackward:
    """layerBackward (ane/backward_darwin.go:13-36) for one layer."""

    def __init__(self, handle, dim, hidden, heads, seq):
        self._h = handle
        self.dim, self.hidden, self.heads, self.seq = dim, hidden, heads, seq

    def run_ffn(self, dx_norm, dh1, dffn, h1):
        """runFFN (ane/backward_darwin.go:207-242)."""
        op = "run layer backward ffn"
        dn, hn = self.dim * self.seq, self.hidden * self.seq
        args = (_buf(op, "dffn", dffn, dn), _buf(op, "h1", h1, hn))
        outs = (_buf(op, "dx", dx_norm, dn, True), _buf(op, "dh1", dh1, hn, True))
        _check(_lib.load().ane_layer_backward_run_ffn(self._h, outs[0], outs[1], *args))

    def run_attention(self, dx_norm, dq, dk, dv, q, k, v, dx2):
        """runAttention (ane/backward_darwin.go:244-318)."""
        op = "run layer backward attention"
        n = self.dim * self.seq
        ins = [_buf(op, nm, a, n) for nm, a in (("q", q), ("k", k), ("v", v), ("dx2", dx2))]
        outs = [_buf(op, nm, a, n, True) for nm, a in (("dx", dx_norm), ("dq", dq), ("dk", dk), ("dv", dv))]
        _check(_lib.load().ane_layer_backward_run_attention(self._h, *outs, *ins))

    def refresh_weights(self, layer):
        """refreshWeights (ane/backward_darwin.go:320-328)."""
        if self._h is None:
            raise SeamError("refresh layer backward: layer is nil")
        cw = _Weights("refresh layer backward", layer, self.dim, self.hidden)
        _check(_lib.load().ane_layer_backward_refresh(self._h, C.byref(cw.c)))

    def close(self):
        if self._h is not None:
            _lib.load().ane_layer_backward_close(self._h)

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h is not None and _lib._lib is not None:
            _lib._lib.ane_layer_backward_destroy(h)


def compile_stories_layer_backward(layer, seq: int, heads: int = STORIES_HEADS) -> LayerBackward:
    """compileStoriesLayerBackward (ane/backward_darwin.go:40-180)."""
    dim, hidden, heads = _dims(layer, heads)
    cw = _Weights("compile layer backward", layer, dim, hidden)
    h = C.c_void_p()
    _check(_lib.load().ane_layer_backward_open(dim, hidden, heads, seq, C.byref(cw.c), C.byref(h)))
    return LayerBackward(h, dim, hidden, heads, seq)


RMS_FORWARD, CLASSIFIER_FORWARD, SOFTMAX, CLASSIFIER_BACKWARD, RMS_BACKWARD = 1, 2, 4, 8, 16


class Offload:
    """offload (ane/offload_darwin.go:34-53): the final head's pieces."""

    def __init__(self, handle, vocab, dim, seq):
        self._h = handle
        self.vocab, self.dim, self.seq = vocab, dim, seq

    def _has(self, piece):
        return self._h is not None and bool(_lib.load().ane_offload_has(self._h, piece))

    def _disable(self, piece):
        if self._h is not None:
            _lib.load().ane_offload_disable(self._h, piece)

    # has* / disable* (ane/offload_darwin.go:283-337)
    def has_rms_forward(self): return self._has(RMS_FORWARD)
    def has_classifier_forward(self): return self._has(CLASSIFIER_FORWARD)
    def has_softmax(self): return self._has(SOFTMAX)
    def has_classifier_backward(self): return self._has(CLASSIFIER_BACKWARD)
    def has_rms_backward(self): return self._has(RMS_BACKWARD)
    def disable_rms_forward(self): self._disable(RMS_FORWARD)
    def disable_classifier_forward(self): self._disable(CLASSIFIER_FORWARD)
    def disable_softmax(self): self._disable(SOFTMAX)
    def disable_classifier_backward(self): self._disable(CLASSIFIER_BACKWARD)
    def disable_rms_backward(self): self._disable(RMS_BACKWARD)

    def run_rms_forward(self, out, x):
        """runRMSForward (ane/offload_darwin.go:339-350)."""
        n = self.dim * self.seq
        _check(_lib.load().ane_offload_run_rms_forward(self._h, _buf("run rms forward", "out", out, n, True),
                                                       _buf("run rms forward", "x", x, n)))

    def run_classifier_forward(self, logits, x_norm):
        """runClassifierForward (ane/offload_darwin.go:352-399): logits vocab-major [vocab * seq]."""
        op = "run classifier forward"
        _check(_lib.load().ane_offload_run_classifier_forward(
            self._h, _buf(op, "logits", logits, self.vocab * self.seq, True), _buf(op, "xNorm", x_norm,
                                                                                    self.dim * self.seq)))

    def run_classifier_softmax(self, probs, x_norm):
        """runClassifierSoftmax (ane/offload_darwin.go:401-454)."""
        op = "run classifier softmax"
        _check(_lib.load().ane_offload_run_classifier_softmax(
            self._h, _buf(op, "probs", probs, self.vocab * self.seq, True), _buf(op, "xNorm", x_norm,
                                                                                  self.dim * self.seq)))

    def run_softmax(self, probs):
        """runSoftmax (ane/offload_darwin.go:456-464), in place."""
        _check(_lib.load().ane_offload_run_softmax(self._h, _buf("run softmax", "probs", probs,
                                                                  self.vocab * self.seq, True)))

    def run_classifier_backward(self, dy, dlogits):
        """runClassifierBackward (ane/offload_darwin.go:466-525)."""
        op = "run classifier backward"
        _check(_lib.load().ane_offload_run_classifier_backward(
            self._h, _buf(op, "dy", dy, self.dim * self.seq, True), _buf(op, "dLogits", dlogits,
                                                                          self.vocab * self.seq)))

    def run_rms_backward(self, dx, dy, x):
        """runRMSBackward (ane/offload_darwin.go:527-547)."""
        op = "run rms backward"
        n = self.dim * self.seq
        _check(_lib.load().ane_offload_run_rms_backward(self._h, _buf(op, "dx", dx, n, True), _buf(op, "dy", dy, n),
                                                        _buf(op, "x", x, n)))

    def refresh_weights(self, embed):
        """refreshWeights (ane/offload_darwin.go:549-573): restages the tied embedding."""
        if self._h is None:
            raise SeamError("refresh offload weights: offload is nil")
        e = np.ascontiguousarray(embed, dtype=np.float32)
        if e.size != self.vocab * self.dim:
            raise SeamError(f"refresh offload weights: embed len={e.size} want={self.vocab * self.dim}")
        _check(_lib.load().ane_offload_refresh(self._h, _fp(e)))

    def close(self):
        if self._h is not None:
            _lib.load().ane_offload_close(self._h)

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h is not None and _lib._lib is not None:
            _lib._lib.ane_offload_destroy(h)


def new_offload(embed, seq: int, use_ane: bool = True, cpu_classifier_head: bool = False,
                vocab: int | None = None, dim: int | None = None) -> Offload | None:
    """newOffload (ane/offload_darwin.go:55-57): None when the accelerator is
    off (the Engine then takes its CPU head).  embed: [vocab, dim]."""
    if not use_ane or seq <= 0:
        return None
    e = np.ascontiguousarray(embed, dtype=np.float32)
    if vocab is None or dim is None:
        vocab, dim = e.shape
    if e.size != vocab * dim:
        raise SeamError(f"new offload: embed len={e.size} want={vocab * dim}")
    h = C.c_void_p()
    _check(_lib.load().ane_offload_open(vocab, dim, seq, _fp(e), 1 if cpu_classifier_head else 0, C.byref(h)))
    return Offload(h, vocab, dim, seq)


def refresh_offload(prev: Offload | None, embed, seq: int, use_ane: bool = True,
                    cpu_classifier_head: bool = False) -> Offload | None:
    """refreshOffload (ane/offload_darwin.go:59-79): the previous object is
    closed and a new one staged from the current weights."""
    if prev is not None:
        prev.close()
    return new_offload(embed, seq, use_ane, cpu_classifier_head)
