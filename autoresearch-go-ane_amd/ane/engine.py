"""Host-side mirror of the reference's ``ane.Engine`` over libane_hip.so.

Names, argument meaning and error wording follow ane/engine.go:
``Open(Options)`` (ane/engine.go:184), ``Engine.EvalLogits`` (:449),
``Engine.Step`` (:381), ``Flush`` (:484), ``LR``/``SetLR`` (:358,366),
``State``/``LoadState`` (:498,506), ``Close`` (:567).  Errors raise
``EngineError`` carrying the library's message ("storiesane <op>: ...")
where the Go API returns ``error``.

Additions of this engine (no reference counterpart): ``Options.Config``
(model shape; the reference hard-codes stories110M), ``Options.Params``
(flat fp32 weights in the canonical layout, in place of a model file),
``Options.MaxBatch`` (sequences per device call), ``EvalLoss`` /
``EvalLossWindows`` (batched forward + loss), and ``Profile*``.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from typing import Optional

import numpy as np

from . import _lib
from .config import Config, param_count


class EngineError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


@dataclasses.dataclass
class Options:
    """ane/engine.go:14-40 (zero values take the defaults of Open)."""
    ModelPath: str = ""
    Tokens: Optional[np.ndarray] = None
    Seq: int = 0
    AccumSteps: int = 0
    LR: float = 0.0
    Seed: int = 0
    AdamBeta1: float = 0.0
    AdamBeta2: float = 0.0
    AdamEps: float = 0.0
    WeightDecay: float = 0.0
    GradClip: float = 0.0
    LossScale: float = 0.0
    CPUClassifierHead: bool = False
    GradTaskLimit: int = 0
    UseANE: bool = False
    HybridBackward: bool = False
    EmbedLRMult: float = 0.0
    ScalarLRMult: float = 0.0
    LambdaLRMult: float = 0.0
    LambdaBeta1: float = 0.0
    LambdaBeta2: float = 0.0
    # additions of this engine
    Config: Optional[Config] = None
    Params: Optional[np.ndarray] = None
    MaxBatch: int = 1
    Device: int = 0


def _check(lib, eng, rc):
    if rc != _lib.ANE_OK:
        msg = lib.ane_last_error(eng)
        raise EngineError(rc, msg.decode() if msg else f"storiesane: error {rc}")


def _f32(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _u16(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def _load_model(path: str, cfg: Config, training: bool):
    """Open's weight load (ane/engine.go:240-248): a llama2.c file
    (LoadPretrained), else a training checkpoint of any version
    (stories.LoadCheckpoint into fresh weights; its Adam moments too when the
    engine trains, i.e. Options.Tokens is set).  -> (params, moments|None)."""
    from .checkpoint import load_pretrained, read_checkpoint
    try:
        params, _ = load_pretrained(path, cfg)
        return params, None
    except (OSError, ValueError) as err:
        if cfg.arch == "nanochat":
            try:
                _, params, m, v, _ = read_checkpoint(path, cfg)
                return params, ((m, v) if training else None)
            except (OSError, ValueError):
                pass
        raise EngineError(_lib.ANE_ERR_ARG, f"storiesane open: load model: {err}") from None


def Open(opts: Options) -> "Engine":
    """ane/engine.go:184-355.  Weights come from ``opts.Params`` or, as in the
    reference, from the file at ``opts.ModelPath``: llama2.c weights or a
    V2-V5 training checkpoint (see ane.checkpoint); the model shape is
    ``opts.Config`` (stories110M by default), which the file must match."""
    lib = _lib.load()
    if opts.Params is None and not opts.ModelPath:
        raise EngineError(_lib.ANE_ERR_ARG, "storiesane open: model path is empty")
    cfg = opts.Config or Config()
    if cfg.kv_heads != cfg.heads:
        raise EngineError(_lib.ANE_ERR_ARG, "storiesane open: grouped-query attention (kv_heads != heads) "
                                            "is served by ane.decode.Decoder only")
    if opts.Seq and opts.Seq != cfg.seq:
        cfg = dataclasses.replace(cfg, seq=opts.Seq)
    params, moments = opts.Params, None
    if params is None:
        params, moments = _load_model(opts.ModelPath, cfg, opts.Tokens is not None and len(opts.Tokens) > 0)
    tokens = None
    if opts.Tokens is not None and len(opts.Tokens) > 0:
        tokens = np.ascontiguousarray(opts.Tokens, dtype=np.uint16)
        if len(tokens) < cfg.seq + 1:
            raise EngineError(_lib.ANE_ERR_ARG, f"storiesane open: not enough tokens for seq={cfg.seq}")
    o = _lib.Options(opts.AccumSteps, opts.LR, opts.Seed, opts.AdamBeta1, opts.AdamBeta2, opts.AdamEps,
                     opts.WeightDecay, opts.GradClip, opts.LossScale, opts.EmbedLRMult, opts.ScalarLRMult,
                     opts.LambdaLRMult, opts.LambdaBeta1, opts.LambdaBeta2, max(1, opts.MaxBatch), opts.Device)
    mc = _lib.model_cfg(cfg)
    h = C.c_void_p()
    rc = lib.ane_open(C.byref(mc), C.byref(o), C.byref(h))
    if rc != _lib.ANE_OK:
        msg = lib.ane_last_error(h) if h.value else b"storiesane open: failed"
        if h.value:
            lib.ane_destroy(h)
        raise EngineError(rc, msg.decode())
    eng = Engine(lib, h, cfg, o)
    try:
        eng.SetParams(params)
        if moments is not None:
            eng.SetOptState(*moments)
        if tokens is not None:
            _check(lib, h, lib.ane_set_tokens(h, _u16(tokens), len(tokens)))
            eng._ntokens = len(tokens)
    except Exception:
        eng.Destroy()
        raise
    return eng


class Engine:
    def __init__(self, lib, handle, cfg: Config, opts):
        self._lib = lib
        self._h = handle
        self.cfg = cfg
        self.max_batch = opts.max_batch
        self.seed = opts.seed or 42  # Open's default (ane/engine.go:201-203)
        self._ntokens = 0

    # -- weights ---------------------------------------------------------
    def SetParams(self, flat: np.ndarray):
        flat = np.ascontiguousarray(flat, dtype=np.float32).reshape(-1)
        if flat.size != param_count(self.cfg):
            raise EngineError(_lib.ANE_ERR_ARG, f"storiesane set params: len={flat.size} "
                                                f"want={param_count(self.cfg)}")
        _check(self._lib, self._h, self._lib.ane_set_params(self._h, _f32(flat), flat.size))

    def Params(self) -> np.ndarray:
        out = np.empty(param_count(self.cfg), np.float32)
        _check(self._lib, self._h, self._lib.ane_get_params(self._h, _f32(out), out.size))
        return out

    # -- forward ---------------------------------------------------------
    def EvalLogits(self, tokens) -> np.ndarray:
        """ane/engine.go:449-462: a fresh [vocab*seq] vocab-major fp32 slice."""
        tok = np.ascontiguousarray(tokens, dtype=np.uint16).reshape(-1)
        out = np.empty(self.cfg.vocab * self.cfg.seq, np.float32)
        _check(self._lib, self._h, self._lib.ane_eval_logits(self._h, _u16(tok), tok.size, _f32(out)))
        return out

    def EvalLoss(self, tokens, targets):
        """Batched forward + loss.  tokens/targets [nseq, seq] -> (mean, per_seq)."""
        tok = np.ascontiguousarray(tokens, dtype=np.uint16).reshape(-1, self.cfg.seq)
        tgt = np.ascontiguousarray(targets, dtype=np.uint16).reshape(-1, self.cfg.seq)
        if tok.shape != tgt.shape:
            raise EngineError(_lib.ANE_ERR_ARG, "storiesane eval loss: tokens/targets shape mismatch")
        n = tok.shape[0]
        per = np.zeros(n, np.float32)
        mean = C.c_float()
        _check(self._lib, self._h, self._lib.ane_eval_loss(self._h, _u16(tok), _u16(tgt), n, _f32(per),
                                                           C.byref(mean)))
        return float(mean.value), per

    def EvalLossWindows(self, positions):
        pos = np.ascontiguousarray(positions, dtype=np.uint64).reshape(-1)
        per = np.zeros(pos.size, np.float32)
        mean = C.c_float()
        _check(self._lib, self._h, self._lib.ane_eval_loss_windows(
            self._h, pos.ctypes.data_as(C.POINTER(C.c_uint64)), pos.size, _f32(per), C.byref(mean)))
        return float(mean.value), per

    # -- training --------------------------------------------------------
    def Step(self) -> "_lib.StepResult":
        """ane/engine.go:381-442: one drand48-sampled window, AdamW every AccumSteps."""
        r = _lib.StepResult()
        _check(self._lib, self._h, self._lib.ane_step(self._h, C.byref(r)))
        return r

    def TrainBatch(self, nseq: int) -> "_lib.StepResult":
        """nseq consecutive Steps fused into one batched forward/backward."""
        r = _lib.StepResult()
        _check(self._lib, self._h, self._lib.ane_train_batch(self._h, int(nseq), C.byref(r)))
        return r

    def Flush(self) -> int:
        """ane/engine.go:484-496: applies pending gradients; returns the
        weight-refresh duration in nanoseconds (0 when nothing was pending)."""
        ns = C.c_int64()
        _check(self._lib, self._h, self._lib.ane_flush(self._h, C.byref(ns)))
        return int(ns.value)

    def LR(self) -> float:
        return float(self._lib.ane_lr(self._h)) if self._h else 0.0

    def SetLR(self, lr: float):
        _check(self._lib, self._h, self._lib.ane_set_lr(self._h, float(lr)))

    def State(self) -> "_lib.State":
        s = _lib.State()
        self._lib.ane_get_state(self._h, C.byref(s))
        return s

    def LoadState(self, s: "_lib.State"):
        _check(self._lib, self._h, self._lib.ane_load_state(self._h, C.byref(s)))

    def Grads(self, tokens, targets):
        """Gradient of the mean loss over explicit sequences (flushed scale)."""
        tok = np.ascontiguousarray(tokens, dtype=np.uint16).reshape(-1, self.cfg.seq)
        tgt = np.ascontiguousarray(targets, dtype=np.uint16).reshape(-1, self.cfg.seq)
        g = np.zeros(param_count(self.cfg), np.float32)
        mean = C.c_float()
        _check(self._lib, self._h, self._lib.ane_grads(self._h, _u16(tok), _u16(tgt), tok.shape[0], _f32(g),
                                                       C.byref(mean)))
        return float(mean.value), g

    def SetGrads(self, grads: np.ndarray, pending: int):
        g = np.ascontiguousarray(grads, dtype=np.float32).reshape(-1)
        _check(self._lib, self._h, self._lib.ane_set_grads(self._h, _f32(g), g.size, int(pending)))

    def OptState(self):
        n = param_count(self.cfg)
        m = np.zeros(n, np.float32)
        v = np.zeros(n, np.float32)
        _check(self._lib, self._h, self._lib.ane_get_opt_state(self._h, _f32(m), _f32(v), n))
        return m, v

    def SetOptState(self, m, v):
        n = param_count(self.cfg)
        m = np.ascontiguousarray(m, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
        _check(self._lib, self._h, self._lib.ane_set_opt_state(self._h, _f32(m), _f32(v), n))

    def AccumGrads(self) -> np.ndarray:
        """The pending loss-scaled gradient sum (what the checkpoint trailer stores)."""
        g = np.zeros(param_count(self.cfg), np.float32)
        _check(self._lib, self._h, self._lib.ane_get_accum_grads(self._h, _f32(g), g.size))
        return g

    # -- checkpoints (ane/engine.go:515-564) -------------------------------
    def SaveCheckpoint(self, path: str, meta=None):
        """V5 file + SANE trailer; meta's LR / loss / counters come from the engine."""
        from .checkpoint import TrainMeta, write_checkpoint
        if not self._h:
            raise EngineError(_lib.ANE_ERR_CLOSED, "storiesane save checkpoint: engine is closed")
        meta = dataclasses.replace(meta) if meta is not None else TrainMeta()
        st = self.State()
        meta.LR = self.LR()
        meta.Loss = st.last_loss
        meta.CumTrain = st.cum_train_ms
        meta.CumWall = st.cum_wall_ms
        meta.CumSteps = int(st.cum_steps)
        meta.CumBatches = int(st.cum_batches)
        meta.AdamT = int(st.adam_t)
        m, v = self.OptState()
        write_checkpoint(path, self.cfg, meta, self.Params(), m, v, token_pos=int(st.token_pos),
                         pending=int(st.pending_steps), accum=self.AccumGrads())

    def LoadCheckpoint(self, path: str):
        """Restores weights, moments, LR, counters and the pending gradients;
        re-seeds the window sampler with Options.Seed + meta.Step."""
        from .checkpoint import read_checkpoint
        if not self._h:
            raise EngineError(_lib.ANE_ERR_CLOSED, "storiesane load checkpoint: engine is closed")
        # tensors an older version lacks keep the engine's current values
        meta, params, m, v, trailer = read_checkpoint(path, self.cfg, base=self.Params())
        self.SetParams(params)
        self.SetOptState(m, v)
        self.SetLR(meta.LR)
        pending, token_pos, accum = 0, 0, None
        if trailer is not None:
            pending, token_pos, accum = trailer["pending"], trailer["token_pos"], trailer["accum"]
        self.SetGrads(accum if accum is not None else np.zeros(param_count(self.cfg), np.float32),
                      pending if accum is not None else 0)
        st = _lib.State(token_pos, meta.Loss, meta.CumTrain, meta.CumWall, meta.CumSteps, meta.CumBatches,
                        meta.AdamT, pending if accum is not None else 0)
        self.LoadState(st)
        _check(self._lib, self._h, self._lib.ane_seed_sampler(self._h, int(self.seed) + int(meta.Step)))
        return meta

    def Prepare(self):
        """ane/runtime.go:10: nothing to compile ahead of time on this engine."""

    # -- diagnostics -----------------------------------------------------
    def ProfileEnable(self, on: bool = True):
        _check(self._lib, self._h, self._lib.ane_profile_enable(self._h, 1 if on else 0))

    def ProfileRead(self, reset: bool = True) -> dict:
        arr = (_lib.ProfEntry * 8)()
        _check(self._lib, self._h, self._lib.ane_profile_read(self._h, arr, 8, 1 if reset else 0))
        return {name: dict(launches=int(arr[i].launches), ms=float(arr[i].ms), flops=float(arr[i].flops),
                           bytes=float(arr[i].bytes)) for i, name in enumerate(_lib.PROF_CLASSES)}

    def Sync(self):
        _check(self._lib, self._h, self._lib.ane_sync(self._h))

    # -- lifecycle -------------------------------------------------------
    def Close(self):
        """ane/engine.go:567: frees device memory; later calls fail with 'engine is closed'."""
        if self._h:
            self._lib.ane_close(self._h)

    def Destroy(self):
        if self._h:
            self._lib.ane_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.Destroy()
        except Exception:
            pass
