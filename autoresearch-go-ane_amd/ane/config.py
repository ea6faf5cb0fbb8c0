"""Model configuration, canonical parameter layout and seeded init.

The model constants follow ane/stories/config.go:3-18 (Dim 768, Hidden 2048,
Heads 12, Layers 12, Vocab 32000, SeqDefault 256).  Two architectures share
the kernels:

* ``nanochat`` -- the reference's CPU-path model (ane/engine.go:954-1038):
  ReLU^2 FFN, parameterless RMSNorm, QK-norm x1.2, RoPE theta 1e5, tied
  classifier with 15*tanh softcap, value embeddings on odd layers, smear,
  backout and per-layer residual / x0 lambdas.
* ``llama2`` -- the Llama2-style stories110M the benchmark configs name:
  SwiGLU FFN (W1, W3, W2), RMSNorm gains, RoPE theta 1e4, tied classifier,
  no softcap.

The flat parameter vector order is the interchange format of the C-ABI
(``ane_set_params`` / ``ane_get_params`` / ``ane_get_grads``); for nanochat
it is the order of the reference's writeModelGrad (ane/engine.go:811-840).
"""
from __future__ import annotations

import dataclasses

import numpy as np

VE_GATE_CHANNELS = 12  # ane/stories/weights.go:28


@dataclasses.dataclass
class Config:
    dim: int = 768
    hidden: int = 2048
    heads: int = 12
    layers: int = 12
    vocab: int = 32000
    seq: int = 256
    arch: str = "llama2"          # "llama2" | "nanochat"
    grad_mode: str = "compat"     # nanochat backward: "compat" (reference) | "true"
    rope_theta: float = 0.0       # 0 -> arch default
    kv_heads: int = 0             # key/value heads (llama2 only; 0 -> heads, i.e. no grouping)

    def __post_init__(self):
        if self.arch not in ("llama2", "nanochat"):
            raise ValueError(f"unknown arch {self.arch!r}")
        if self.grad_mode not in ("compat", "true"):
            raise ValueError(f"unknown grad_mode {self.grad_mode!r}")
        if not self.rope_theta:
            self.rope_theta = 10000.0 if self.arch == "llama2" else 100000.0
        if not self.kv_heads:
            self.kv_heads = self.heads
        if self.heads % self.kv_heads or (self.arch != "llama2" and self.kv_heads != self.heads):
            raise ValueError(f"kv_heads={self.kv_heads} must divide heads={self.heads} (llama2 only)")

    @property
    def head_dim(self) -> int:
        return self.dim // self.heads


def stories110m(arch: str = "llama2", seq: int = 256, **kw) -> Config:
    return Config(arch=arch, seq=seq, **kw)


def tiny(arch: str = "llama2", **kw) -> Config:
    """A small model that keeps every kernel's tiling constraints."""
    base = dict(dim=128, hidden=256, heads=2, layers=2, vocab=512, seq=64, arch=arch)
    base.update(kw)
    return Config(**base)


def decode_gqa(**kw) -> Config:
    """The decode benchmark's model: 12 layers, dim 768, 12 query / 4 key-value
    heads of 64, vocab 32000, SwiGLU hidden 2048, tied classifier, RoPE 1e4
    (Llama2 blocks with grouped-query attention; no reference counterpart)."""
    base = dict(dim=768, hidden=2048, heads=12, kv_heads=4, layers=12, vocab=32000, seq=1024, arch="llama2")
    base.update(kw)
    return Config(**base)


def tiny_decode(**kw) -> Config:
    """A small grouped-query model (4 query heads over 2 key-value heads)."""
    base = dict(dim=256, hidden=512, heads=4, kv_heads=2, layers=2, vocab=1024, seq=128, arch="llama2")
    base.update(kw)
    return Config(**base)


def is_ve_layer(cfg: Config, l: int) -> bool:
    """ane/stories/weights.go:22 (nanochat only)."""
    return cfg.arch == "nanochat" and (l % 2) == ((cfg.layers - 1) % 2)


def param_layout(cfg: Config):
    """Ordered list of (name, offset, shape) for the flat parameter vector."""
    D, H, V, NH, L = cfg.dim, cfg.hidden, cfg.vocab, cfg.heads, cfg.layers
    KVD = cfg.kv_heads * cfg.head_dim
    out = []
    off = 0

    def seg(name, shape):
        nonlocal off
        n = int(np.prod(shape))
        out.append((name, off, tuple(shape)))
        off += n

    for l in range(L):
        seg(f"layers.{l}.wq", (D, D))
        seg(f"layers.{l}.wk", (KVD, D))
        seg(f"layers.{l}.wv", (KVD, D))
        seg(f"layers.{l}.wo", (D, D))
        seg(f"layers.{l}.w1", (H, D))
        seg(f"layers.{l}.w2", (D, H))
        if cfg.arch == "llama2":
            seg(f"layers.{l}.w3", (H, D))
            seg(f"layers.{l}.g_att", (D,))
            seg(f"layers.{l}.g_ffn", (D,))
        elif is_ve_layer(cfg, l):
            seg(f"layers.{l}.ve_embed", (V, D))
            seg(f"layers.{l}.ve_gate", (NH * VE_GATE_CHANNELS,))
    seg("embed", (V, D))
    if cfg.arch == "llama2":
        seg("g_final", (D,))
    else:
        seg("resid_lambdas", (L,))
        seg("x0_lambdas", (L,))
        seg("smear_gate", (D, D))
        seg("smear_lambda", (1,))
        seg("backout_lambda", (1,))
    return out


def param_count(cfg: Config) -> int:
    name, off, shape = param_layout(cfg)[-1]
    return off + int(np.prod(shape))


def views(cfg: Config, flat: np.ndarray) -> dict:
    return {name: flat[off:off + int(np.prod(shape))].reshape(shape)
            for name, off, shape in param_layout(cfg)}


def init_params(cfg: Config, seed: int = 0, std: float = 0.02) -> np.ndarray:
    """Seeded init used identically for the oracle and the device engine.

    Every matrix ~ N(0, std) from numpy's PCG64 stream of ``seed`` in layout
    order; norm gains = 1; nanochat scalars as ane/stories/weights.go:190-202
    (resid 1.0, x0 0.1, smear 0.01, backout 0.01).
    """
    n = param_count(cfg)
    rng = np.random.default_rng(seed)
    flat = rng.standard_normal(n, dtype=np.float32)
    flat *= np.float32(std)
    v = views(cfg, flat)
    for name, arr in v.items():
        if name.endswith(("g_att", "g_ffn", "g_final")):
            arr[...] = 1.0
    if cfg.arch == "nanochat":
        v["resid_lambdas"][...] = 1.0
        v["x0_lambdas"][...] = 0.1
        v["smear_lambda"][...] = 0.01
        v["backout_lambda"][...] = 0.01
    return flat


def make_tokens(cfg: Config, batch: int, seed: int):
    """Token ids uniform in [0, vocab) from ``seed``; targets = ids shifted by one.

    Draws batch*(seq+1) ids as one stream and slices overlapping windows per
    sequence, like the reference's window sampler (ane/engine.go:403-404).
    """
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, cfg.vocab, size=(batch, cfg.seq + 1), dtype=np.int64).astype(np.uint16)
    return np.ascontiguousarray(ids[:, :-1]), np.ascontiguousarray(ids[:, 1:])
