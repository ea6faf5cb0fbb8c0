"""Writes the golden fixtures of tests/golden (run in this container; the
output is committed).  The reference ships no vectors for this path, so the
fixtures are produced by the pinned C oracle (oracle/refcpu.c,
refdecode.c, refmoe.c) on small seeded cases and stored as little-endian
.bin files with a JSON manifest (name, dtype, shape, seed, tolerance):

  forward_{llama2,nanochat}   tiny model, one 64-token sequence: logits
                              [V, seq] vocab-major + loss
  grads_{llama2_true,nanochat_compat}
                              tiny model, two sequences: per-segment L2 norm
                              and the first 32 values of every gradient segment
  drand48_seed42              the first 16 drand48 draws of seed 42
  decode_gqa                  tiny grouped-query model: greedy tokens and the
                              logits of the prefix and two forced steps
  moe_small                   16 tokens of a dim-64 MoE layer: expert ids,
                              weights, outputs

Usage:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "autoresearch-go-ane_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, p)

import ane  # noqa: E402
import oracle  # noqa: E402
from ane.moe import MoeConfig, init_moe_params, make_moe_input  # noqa: E402


def main():
    manifest = []

    def put(name, arr, seed, tol, note):
        arr = np.ascontiguousarray(arr)
        fn = f"{name}.bin"
        arr.astype(arr.dtype.newbyteorder("<")).tofile(os.path.join(HERE, fn))
        manifest.append({"name": name, "file": fn, "dtype": str(arr.dtype), "shape": list(arr.shape),
                         "seed": seed, "tolerance": tol, "note": note})

    oracle.set_threads(1, parallel_linear=False)
    for arch in ("llama2", "nanochat"):
        cfg = ane.tiny(arch)
        p = ane.init_params(cfg, seed=0, std=0.08)
        tok, tgt = ane.make_tokens(cfg, 1, seed=1)
        mean, _, lg = oracle.forward_loss(cfg, p, tok, tgt, want_logits=True)
        put(f"forward_{arch}_tokens", tok, 1, 0, f"ane.tiny('{arch}') make_tokens(batch 1, seed 1)")
        put(f"forward_{arch}_logits", lg[0], 0, 2e-2, "params init_params(seed 0, std 0.08); logits [V, seq]")
        put(f"forward_{arch}_loss", np.array([mean], np.float32), 0, 1e-3, "mean cross-entropy")
    for arch, mode in (("llama2", "true"), ("nanochat", "compat")):
        cfg = ane.tiny(arch, grad_mode=mode)
        p = ane.init_params(cfg, seed=21, std=0.08)
        tok, tgt = ane.make_tokens(cfg, 2, seed=22)
        loss, g = oracle.grads(cfg, p, tok, tgt)
        norms, heads = [], []
        for name, off, shape in ane.param_layout(cfg):
            n = int(np.prod(shape))
            seg = g[off:off + n]
            norms.append(np.linalg.norm(seg.astype(np.float64)))
            head = np.zeros(32, np.float32)
            head[:min(32, n)] = seg[:32]
            heads.append(head)
        put(f"grads_{arch}_{mode}_norms", np.array(norms, np.float64), 21, 1e-2,
             "per-segment L2 norm of the mean gradient (tiny, 2 seqs, tokens seed 22)")
        put(f"grads_{arch}_{mode}_heads", np.stack(heads), 21, 1e-2, "first 32 values of every segment")
        put(f"grads_{arch}_{mode}_loss", np.array([loss], np.float32), 21, 1e-3, "mean loss")
    put("drand48_seed42", oracle.drand48_stream(42, 16), 42, 0, "ane/engine.go:873-880 (libc drand48)")

    dcfg = ane.tiny_decode()
    dp = ane.init_params(dcfg, seed=61, std=0.05)
    r = np.random.default_rng(62)
    prefix = r.integers(0, dcfg.vocab, (2, 64)).astype(np.uint16)
    forced = r.integers(0, dcfg.vocab, (2, 2)).astype(np.uint16)
    toks, dlg = oracle.decode(dcfg, dp, prefix, 2, forced=forced, want_logits=True, threads=1)
    put("decode_gqa_prefix", prefix, 62, 0, "ane.tiny_decode(); params init_params(seed 61, std 0.05)")
    put("decode_gqa_forced", forced, 62, 0, "inputs of the two decode steps")
    put("decode_gqa_tokens", toks.astype(np.uint16), 61, 0, "greedy tokens after the prefix and each step")
    put("decode_gqa_logits", dlg, 61, 2e-2, "[seq, step, vocab] logits")

    mcfg = MoeConfig(dim=64, hidden=128, experts=8)
    mp = init_moe_params(mcfg, seed=71, std=0.1)
    mx = make_moe_input(mcfg, 16, seed=72)
    out, idx, w = oracle.moe_forward(mp, mx, mcfg.hidden, mcfg.experts, threads=1)
    put("moe_small_x", mx, 72, 0, "MoeConfig(dim 64, hidden 128, experts 8); params init_moe_params(seed 71, std 0.1)")
    put("moe_small_experts", idx, 71, 0, "chosen experts (bit-exact)")
    put("moe_small_weights", w, 71, 1e-6, "router weights")
    put("moe_small_out", out, 71, 5e-3, "layer output (relative L2 on a GPU)")

    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    total = sum(os.path.getsize(os.path.join(HERE, m["file"])) for m in manifest)
    print(f"wrote {len(manifest)} fixtures, {total / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
