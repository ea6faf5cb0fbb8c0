"""Model files of the reference: llama2.c weights, V2-V5 training
checkpoints and the "SANE" engine trailer.

llama2.c ``.bin`` (LoadPretrained, ane/stories/weights.go:73-153; header
ane/stories/config.go:20-28): int32 dim, hidden_dim, n_layers, n_heads,
n_kv_heads, vocab_size (negative: the file has its own classifier), seq_len;
then fp32 token embedding [vocab][dim], rms_att [L][dim], wq, wk, wv, wo
[L][dim][dim], rms_ffn [L][dim], w1 [L][hidden][dim], w2 [L][dim][hidden],
w3 [L][hidden][dim], rms_final [dim] (anything after it is not read).

Training checkpoints, byte layout of the reference's files
(ane/stories/ckpt.go:77-269 writer, :271-712 reader; trailer
ane/engine.go:684-767), so checkpoints move between the reference and this
engine in both directions.  V5 is written; V2-V5 are read:

  header, 96 bytes little-endian: int32 magic 0x424C5A54, int32 version 5,
    int32 step, total_steps, n_layers, vocab, dim, hidden, heads, seq;
    float32 lr, loss; float64 cum_compile, cum_train, cum_wall;
    int32 cum_steps, cum_batches, adam_t; 3 x int32 reserved (0)
  per layer, weights: Wq Wk Wv Wo W1 W2 [VEEmbed VEGate on VE layers]
  per layer, Adam moments: M then V of each of those tensors
  model level, each as weights, M, V: Embed, ResidLambdas, X0Lambdas,
    SmearGate, SmearLambda, BackoutLambda
  trailer: "SANE", uint32 version (2), uint64 token_pos, uint32
    pending_steps, the pending loss-scaled gradient sum in writeModelGrad
    order (ane/engine.go:811-840)

Older versions (read only; ane/stories/ckpt.go:427-712):
  V4  per layer Wq Wk Wv Wo W1 W2, a W3 [hidden][dim] (skipped), VEEmbed on
      VE layers, a dim-sized VEGate on VE layers (skipped: VEGate keeps its
      value); per-layer moments likewise (W3 and the old VEGate moments
      skipped); model level as V5
  V3  per layer Wq Wk Wv Wo W1 W2, W3, RMSAtt [dim], RMSFFN [dim] (the last
      three skipped; no value embeddings); per-layer moments of the six
      matrices, then W3 and RMS moments (skipped); RMSFinal weight + moments
      (skipped); Embed weight + moments; no lambdas, no smear gate
  V2  as V3 with every per-layer moment skipped
  V2 and V3 then take the default lambdas of initLambdasDefault
  (ane/stories/weights.go:155-162): ResidLambdas 1, SmearLambda 0,
  BackoutLambda 0; tensors a version lacks keep their prior values.

V5 has no slots for the Llama2 variant's W3 and RMSNorm gains, so only the
reference's own model (arch nanochat) is saved in this format.
"""
from __future__ import annotations

import dataclasses
import os
import struct

import numpy as np

from .config import Config, param_layout

CKPT_MAGIC = 0x424C5A54
CKPT_V2, CKPT_V3, CKPT_V4, CKPT_V5 = 2, 3, 4, 5
LLAMA2_HEADER = struct.Struct("<7i")
TRAILER_MAGIC = b"SANE"
TRAILER_V1, TRAILER_V2 = 1, 2
HEADER = struct.Struct("<10i2f3d3i3i")
assert HEADER.size == 96


@dataclasses.dataclass
class TrainMeta:
    """stories.TrainMeta (ane/stories/ckpt.go:26-37)."""
    Step: int = 0
    TotalSteps: int = 0
    LR: float = 0.0
    Loss: float = 0.0
    CumCompile: float = 0.0
    CumTrain: float = 0.0
    CumWall: float = 0.0
    CumSteps: int = 0
    CumBatches: int = 0
    AdamT: int = 0


def _check_arch(cfg: Config, op: str):
    if cfg.arch != "nanochat":
        raise ValueError(f"storiesane {op}: the V5 checkpoint format holds the nanochat model only "
                         f"(arch={cfg.arch})")


def _segments(cfg: Config):
    """(layer_segments, model_segments) as lists of (offset, size)."""
    lay, model = [], []
    for name, off, shape in param_layout(cfg):
        (lay if name.startswith("layers.") else model).append((off, int(np.prod(shape))))
    return lay, model


def checkpoint_size(cfg: Config) -> int:
    """storiesCheckpointSize (ane/engine.go:769-791): header + weights and
    both moments of every tensor, 4 bytes each."""
    _check_arch(cfg, "checkpoint size")
    lay, model = _segments(cfg)
    return HEADER.size + 4 * (3 * sum(n for _, n in lay) + 3 * sum(n for _, n in model))


def write_checkpoint(path: str, cfg: Config, meta: TrainMeta, params, m, v, token_pos: int = 0,
                     pending: int = 0, accum=None):
    """Writes path atomically (temporary file + rename, as the reference)."""
    _check_arch(cfg, "save checkpoint")
    params, m, v = (np.ascontiguousarray(a, dtype="<f4").reshape(-1) for a in (params, m, v))
    lay, model = _segments(cfg)
    d = os.path.dirname(os.path.abspath(path))
    os.makedirs(d, exist_ok=True)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(HEADER.pack(CKPT_MAGIC, CKPT_V5, int(meta.Step), int(meta.TotalSteps), cfg.layers, cfg.vocab,
                            cfg.dim, cfg.hidden, cfg.heads, cfg.seq, float(meta.LR), float(meta.Loss),
                            float(meta.CumCompile), float(meta.CumTrain), float(meta.CumWall), int(meta.CumSteps),
                            int(meta.CumBatches), int(meta.AdamT), 0, 0, 0))
        end = lay[-1][0] + lay[-1][1]
        f.write(params[:end].tobytes())                      # per-layer weights, layer order
        for off, n in lay:                                    # per-layer moments
            f.write(m[off:off + n].tobytes())
            f.write(v[off:off + n].tobytes())
        for off, n in model:                                  # model level: w, m, v
            for a in (params, m, v):
                f.write(a[off:off + n].tobytes())
        f.write(TRAILER_MAGIC)
        f.write(struct.pack("<IQI", TRAILER_V2, int(token_pos), int(pending)))
        g = np.zeros_like(params) if accum is None else np.ascontiguousarray(accum, dtype="<f4").reshape(-1)
        f.write(g.tobytes())
        f.flush()
        os.fsync(f.fileno())
    os.replace(tmp, path)


def _tensors(cfg: Config) -> dict:
    return {name: (off, int(np.prod(shape))) for name, off, shape in param_layout(cfg)}


class _Reader:
    def __init__(self, f, op="load checkpoint"):
        self.f, self.op = f, op

    def f32(self, n):
        b = self.f.read(4 * n)
        if len(b) != 4 * n:
            raise ValueError(f"storiesane {self.op}: truncated file")
        return np.frombuffer(b, dtype="<f4").astype(np.float32)

    def into(self, dst, off, n):
        dst[off:off + n] = self.f32(n)

    def skip(self, n):
        self.f.seek(4 * n, os.SEEK_CUR)


def _read_v5(r, cfg, params, m, v):
    lay, model = _segments(cfg)
    end = lay[-1][0] + lay[-1][1]
    r.into(params, 0, end)                       # per-layer weights, layer order
    for off, n in lay:                           # per-layer moments
        r.into(m, off, n)
        r.into(v, off, n)
    for off, n in model:                         # model level: w, m, v
        for a in (params, m, v):
            r.into(a, off, n)


def _read_v4(r, cfg, params, m, v):
    """loadCheckpointV4V5 with isV5 = false (ane/stories/ckpt.go:427-600)."""
    t = _tensors(cfg)
    D, H, L = cfg.dim, cfg.hidden, cfg.layers
    mats = ("wq", "wk", "wv", "wo", "w1", "w2")
    for l in range(L):
        for nm in mats:
            r.into(params, *t[f"layers.{l}.{nm}"])
        r.skip(H * D)                                   # W3
        if f"layers.{l}.ve_embed" in t:
            r.into(params, *t[f"layers.{l}.ve_embed"])
            r.skip(D)                                   # the old dim-sized VEGate
    for l in range(L):
        for nm in mats:
            off, n = t[f"layers.{l}.{nm}"]
            r.into(m, off, n)
            r.into(v, off, n)
        r.skip(2 * H * D)                               # W3 moments
        if f"layers.{l}.ve_embed" in t:
            off, n = t[f"layers.{l}.ve_embed"]
            r.into(m, off, n)
            r.into(v, off, n)
            r.skip(2 * D)                               # old VEGate moments
    for nm in ("embed", "resid_lambdas", "x0_lambdas", "smear_gate", "smear_lambda", "backout_lambda"):
        off, n = t[nm]
        for a in (params, m, v):
            r.into(a, off, n)


def _read_v3(r, cfg, params, m, v, ver):
    """loadCheckpointV3 (ane/stories/ckpt.go:633-712), V2 and V3."""
    t = _tensors(cfg)
    D, H, L = cfg.dim, cfg.hidden, cfg.layers
    mats = ("wq", "wk", "wv", "wo", "w1", "w2")
    for l in range(L):
        for nm in mats:
            r.into(params, *t[f"layers.{l}.{nm}"])
        r.skip(H * D + 2 * D)                           # W3, RMSAtt, RMSFFN
    per_layer_moments = sum(2 * t[f"layers.0.{nm}"][1] for nm in mats) + 2 * H * D + 4 * D
    for l in range(L):
        if ver == CKPT_V3:
            for nm in mats:
                off, n = t[f"layers.{l}.{nm}"]
                r.into(m, off, n)
                r.into(v, off, n)
            r.skip(2 * H * D + 4 * D)                   # W3 and RMS moments
        else:
            r.skip(per_layer_moments)
    r.skip(3 * D)                                       # RMSFinal weight and moments
    off, n = t["embed"]
    for a in (params, m, v):
        r.into(a, off, n)
    # initLambdasDefault (ane/stories/weights.go:155-162)
    o, n = t["resid_lambdas"]
    params[o:o + n] = 1.0
    params[t["smear_lambda"][0]] = 0.0
    params[t["backout_lambda"][0]] = 0.0


def read_checkpoint(path: str, cfg: Config, base=None):
    """LoadCheckpoint (ane/stories/ckpt.go:271-406 and the engine's trailer,
    ane/engine.go:534-564, 714-766) -> (meta, params, m, v, trailer) with
    trailer None or a dict with token_pos, pending and accum (None for a V1
    trailer).  Versions 2-5.  base: parameter values for the tensors an
    older version does not hold (the engine's current weights; default
    zeros).  The moments start from zero (zeroOptimState).  The trailer is
    looked for where a V5 body ends, as the reference does."""
    _check_arch(cfg, "load checkpoint")
    lay, model = _segments(cfg)
    total = sum(n for _, n in lay) + sum(n for _, n in model)
    with open(path, "rb") as f:
        raw = f.read(HEADER.size)
        if len(raw) < HEADER.size:
            raise ValueError("storiesane load checkpoint: short header")
        h = HEADER.unpack(raw)
        magic, ver = h[0], h[1]
        if magic != CKPT_MAGIC or ver not in (CKPT_V2, CKPT_V3, CKPT_V4, CKPT_V5):
            raise ValueError(f"bad checkpoint header magic={magic:x} version={ver}")
        if (h[4], h[5], h[6], h[7], h[8]) != (cfg.layers, cfg.vocab, cfg.dim, cfg.hidden, cfg.heads):
            raise ValueError("checkpoint config mismatch")
        meta = TrainMeta(Step=h[2], TotalSteps=h[3], LR=h[10], Loss=h[11], CumCompile=h[12], CumTrain=h[13],
                         CumWall=h[14], CumSteps=h[15], CumBatches=h[16], AdamT=h[17])
        params = np.zeros(total, np.float32) if base is None else np.array(base, dtype=np.float32).reshape(-1)
        if params.size != total:
            raise ValueError(f"storiesane load checkpoint: base len={params.size} want={total}")
        m = np.zeros(total, np.float32)
        v = np.zeros(total, np.float32)
        r = _Reader(f)
        if ver == CKPT_V5:
            _read_v5(r, cfg, params, m, v)
        elif ver == CKPT_V4:
            _read_v4(r, cfg, params, m, v)
        else:
            _read_v3(r, cfg, params, m, v, ver)
        trailer = None
        f.seek(checkpoint_size(cfg))
        tm = f.read(4)
        if tm == TRAILER_MAGIC:
            tv, token_pos, pending = struct.unpack("<IQI", f.read(16))
            if tv == TRAILER_V1:      # accumGRMS [dim] and accumGEmbed [vocab*dim], no longer used
                f.seek(4 * (cfg.dim + cfg.vocab * cfg.dim), os.SEEK_CUR)
                accum = None
            elif tv == TRAILER_V2:
                accum = _Reader(f, "load trailer").f32(total)
            else:
                raise ValueError(f"storiesane load trailer: unsupported version {tv}")
            trailer = {"token_pos": token_pos, "pending": pending, "accum": accum}
    return meta, params, m, v, trailer


@dataclasses.dataclass
class Llama2Header:
    """stories.Llama2Config (ane/stories/config.go:20-28)."""
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab_size: int
    seq_len: int

    @property
    def shared_classifier(self) -> bool:
        return self.vocab_size > 0


def read_llama2_header(path: str) -> Llama2Header:
    with open(path, "rb") as f:
        raw = f.read(LLAMA2_HEADER.size)
    if len(raw) < LLAMA2_HEADER.size:
        raise ValueError("read config: unexpected EOF")
    return Llama2Header(*LLAMA2_HEADER.unpack(raw))


def load_pretrained(path: str, cfg: Config):
    """LoadPretrained (ane/stories/weights.go:73-153) -> (params, header).

    The header's dim, hidden_dim and n_layers must equal cfg's ("config
    mismatch: got dim=.. hidden=.. layers=..") and |vocab_size| must equal
    cfg.vocab.  arch nanochat follows the reference: the RMSNorm gains and
    W3 are skipped and the weights run through the reference's model, with
    initLambdasDefault (ResidLambdas 1, X0Lambdas 0, SmearLambda 0,
    BackoutLambda 0) and zero value embeddings, VE gates and smear gate.
    arch llama2 (this engine's Llama2 variant) keeps W3 and the gains."""
    hdr = read_llama2_header(path)
    if (hdr.dim, hdr.hidden_dim, hdr.n_layers) != (cfg.dim, cfg.hidden, cfg.layers):
        raise ValueError(f"config mismatch: got dim={hdr.dim} hidden={hdr.hidden_dim} layers={hdr.n_layers}")
    if abs(hdr.vocab_size) != cfg.vocab:
        raise ValueError(f"config mismatch: vocab={abs(hdr.vocab_size)} want={cfg.vocab}")
    if hdr.n_heads != cfg.heads:
        raise ValueError(f"config mismatch: heads={hdr.n_heads} want={cfg.heads}")
    t = _tensors(cfg)
    D, H, L, V = cfg.dim, cfg.hidden, cfg.layers, cfg.vocab
    params = np.zeros(param_count_of(cfg), np.float32)
    llama = cfg.arch == "llama2"
    with open(path, "rb") as f:
        f.seek(LLAMA2_HEADER.size)
        r = _Reader(f, "load pretrained")

        def group(name, n_each):
            for l in range(L):
                key = f"layers.{l}.{name}"
                if name and key in t:
                    r.into(params, *t[key])
                else:
                    r.skip(n_each)

        r.into(params, *t["embed"])
        group("g_att" if llama else "", D)          # rms_att
        for nm in ("wq", "wk", "wv", "wo"):
            group(nm, D * D)
        group("g_ffn" if llama else "", D)          # rms_ffn
        group("w1", H * D)
        group("w2", D * H)
        group("w3" if llama else "", H * D)
        if llama:
            r.into(params, *t["g_final"])
        else:
            r.skip(D)                               # rms_final
    if not llama:
        o, n = t["resid_lambdas"]
        params[o:o + n] = 1.0
    return params, hdr


def param_count_of(cfg: Config) -> int:
    lay, model = _segments(cfg)
    return sum(n for _, n in lay) + sum(n for _, n in model)
