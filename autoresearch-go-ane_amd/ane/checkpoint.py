"""V5 training checkpoints with the "SANE" engine trailer.

Byte layout of the reference's files (ane/stories/ckpt.go:77-269 writer,
:280-406 reader; trailer ane/engine.go:684-767), so checkpoints move between
the reference and this engine in both directions:

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
CKPT_V5 = 5
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


def read_checkpoint(path: str, cfg: Config):
    """-> (meta, params, m, v, trailer) with trailer None or a dict with
    token_pos, pending and accum (None for a V1 trailer)."""
    _check_arch(cfg, "load checkpoint")
    lay, model = _segments(cfg)
    total = sum(n for _, n in lay) + sum(n for _, n in model)
    with open(path, "rb") as f:
        raw = f.read(HEADER.size)
        if len(raw) < HEADER.size:
            raise ValueError("storiesane load checkpoint: short header")
        h = HEADER.unpack(raw)
        magic, ver = h[0], h[1]
        if magic != CKPT_MAGIC or ver != CKPT_V5:
            raise ValueError(f"bad checkpoint header magic={magic:x} version={ver}")
        if (h[4], h[5], h[6], h[7], h[8]) != (cfg.layers, cfg.vocab, cfg.dim, cfg.hidden, cfg.heads):
            raise ValueError("checkpoint config mismatch")
        meta = TrainMeta(Step=h[2], TotalSteps=h[3], LR=h[10], Loss=h[11], CumCompile=h[12], CumTrain=h[13],
                         CumWall=h[14], CumSteps=h[15], CumBatches=h[16], AdamT=h[17])

        def read_f32(n):
            b = f.read(4 * n)
            if len(b) != 4 * n:
                raise ValueError("storiesane load checkpoint: truncated file")
            return np.frombuffer(b, dtype="<f4").astype(np.float32)

        params = np.zeros(total, np.float32)
        m = np.zeros(total, np.float32)
        v = np.zeros(total, np.float32)
        end = lay[-1][0] + lay[-1][1]
        params[:end] = read_f32(end)
        for off, n in lay:
            m[off:off + n] = read_f32(n)
            v[off:off + n] = read_f32(n)
        for off, n in model:
            for a in (params, m, v):
                a[off:off + n] = read_f32(n)
        trailer = None
        tm = f.read(4)
        if tm == TRAILER_MAGIC:
            tv, token_pos, pending = struct.unpack("<IQI", f.read(16))
            if tv == TRAILER_V1:      # accumGRMS [dim] and accumGEmbed [vocab*dim], no longer used
                f.seek(4 * (cfg.dim + cfg.vocab * cfg.dim), os.SEEK_CUR)
                accum = None
            elif tv == TRAILER_V2:
                accum = read_f32(total)
            else:
                raise ValueError(f"storiesane load trailer: unsupported version {tv}")
            trailer = {"token_pos": token_pos, "pending": pending, "accum": accum}
    return meta, params, m, v, trailer
