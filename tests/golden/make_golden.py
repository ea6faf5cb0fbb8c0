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

Benchmark-shape fixtures (--bench; several minutes of oracle time), the
exact inputs bench.py measures:

  bench_fwd_b32_llama2        stories110M-llama2, weights seed 0, 32 x 256
                              tokens seed 2: the oracle's 32 per-sequence
                              losses
  bench_grads_b16_{llama2_true,nanochat_compat}
                              stories110M, weights seed 0, 16 x 256 tokens
                              seed 3: per-segment L2 norms of the mean
                              gradient and a few sampled rows of every
                              segment (the token embedding: 16 of the
                              batch's token rows and 16 other rows; the
                              value embeddings: token rows)
  bench_decode_b64            the decode model (weights seed 4), 64
                              sequences of 1024 prefix ids seed 4: for 4
                              sampled sequences the oracle's greedy tokens
                              after the prefix and 3 steps and the fp16
                              logits of those 4 positions

  bench_grads_b16_nanochat_compat_repeat
                              nanochat compat, weights seed 0, 16 windows
                              that each repeat one id (seed 5): the scalar
                              gradients (the smear lambda's sum over
                              positions does not cancel on such windows)

Usage:  python tests/golden/make_golden.py [--bench | --bench-grads | --bench-smear | --all]
        (--bench-grads / --bench-smear: only those fixtures, the others kept)
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "autoresearch-go-ane_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, p)

sys.path.insert(0, os.path.dirname(HERE))
import ane  # noqa: E402
import oracle  # noqa: E402
from golden_io import repeated_windows, sampled_rows  # noqa: E402
from ane.moe import MoeConfig, init_moe_params, make_moe_input  # noqa: E402


BENCH_DECODE_SEQS = (0, 21, 42, 63)


def grad_fingerprint(cfg, g, tokens, seed=90):
    """(norms [segments] f64, rows: concatenated sampled rows f32)."""
    norms, rows = [], []
    for i, (name, off, shape) in enumerate(ane.param_layout(cfg)):
        seg = g[off:off + int(np.prod(shape))]
        norms.append(np.linalg.norm(seg.astype(np.float64)))
        idx = sampled_rows(cfg, name.split(".")[-1], shape, tokens, seed + i)
        rows.append(seg if idx is None else seg.reshape(shape)[idx].reshape(-1))
    return np.array(norms, np.float64), np.concatenate(rows).astype(np.float32)


def bench_fixtures(put, only=None):
    import time
    oracle.set_threads(os.cpu_count() or 1, parallel_linear=True)
    t0 = time.time()
    if only == "grads":
        return bench_grads(put)
    if only == "smear":
        return bench_smear(put)
    cfg = ane.stories110m("llama2")
    p = ane.init_params(cfg, seed=0, std=0.02)
    tok, tgt = ane.make_tokens(cfg, 32, seed=2)
    mean, per, _ = oracle.forward_loss(cfg, p, tok, tgt)
    put("bench_fwd_b32_llama2_loss_per_seq", per, 2, 1e-3,
        "stories110m('llama2'), init_params(seed 0, std 0.02), make_tokens(batch 32, seed 2): oracle loss per sequence")
    print(f"forward B32: mean {mean:.6f} ({time.time() - t0:.0f} s)", flush=True)
    bench_grads(put)
    bench_smear(put)
    bench_decode(put)


def bench_grads(put):
    import time
    for arch, mode in (("llama2", "true"), ("nanochat", "compat")):
        t0 = time.time()
        cfg = ane.stories110m(arch, grad_mode=mode)
        p = ane.init_params(cfg, seed=0, std=0.02)
        tok, tgt = ane.make_tokens(cfg, 16, seed=3)
        loss, g = oracle.grads(cfg, p, tok, tgt)
        norms, rows = grad_fingerprint(cfg, g, tok)
        put(f"bench_grads_b16_{arch}_{mode}_norms", norms, 3, 1e-2,
            f"stories110m('{arch}', grad_mode '{mode}'), init_params(seed 0), make_tokens(batch 16, seed 3): "
            "per-segment L2 norm of the mean gradient")
        put(f"bench_grads_b16_{arch}_{mode}_rows", rows, 3, 1e-2,
            "sampled rows of every segment, concatenated in layout order (tests/golden/make_golden.py "
            "sampled_rows)")
        put(f"bench_grads_b16_{arch}_{mode}_loss", np.array([loss], np.float32), 3, 1e-3, "mean loss")
        print(f"grads B16 {arch}/{mode}: loss {loss:.6f} ({time.time() - t0:.0f} s)", flush=True)


def bench_smear(put):
    """nanochat compat at B16 on repeated-token windows: the scalar gradients
    (smear, residual, x0, backout lambdas) and the loss.  On random windows
    the smear lambda's gradient is a sum of ~3M terms that nearly cancels
    (rounding only the parameters to fp16 moves it by ~17%); here it moves
    by 3e-4."""
    import time
    t0 = time.time()
    cfg = ane.stories110m("nanochat", grad_mode="compat")
    p = ane.init_params(cfg, seed=0, std=0.02)
    tok, tgt = repeated_windows(cfg, 16, 5)
    loss, g = oracle.grads(cfg, p, tok, tgt)
    vals = []
    for name, off, shape in ane.param_layout(cfg):
        if name in ("resid_lambdas", "x0_lambdas", "smear_lambda", "backout_lambda"):
            vals.append(g[off:off + int(np.prod(shape))])
    put("bench_grads_b16_nanochat_compat_repeat_scalars", np.concatenate(vals).astype(np.float32), 5, 1e-2,
        "stories110m('nanochat', grad_mode 'compat'), init_params(seed 0), 16 windows each one repeated id "
        "(rng(5).integers(0, 32000, 16)), targets the same ids: gradients of resid_lambdas, x0_lambdas, "
        "smear_lambda, backout_lambda in layout order")
    put("bench_grads_b16_nanochat_compat_repeat_loss", np.array([loss], np.float32), 5, 1e-3, "mean loss")
    print(f"smear B16 repeated: loss {loss:.6f} ({time.time() - t0:.0f} s)", flush=True)


def bench_decode(put):
    import time
    t0 = time.time()
    dcfg = ane.decode_gqa()
    dp = ane.init_params(dcfg, seed=4, std=0.02)
    prefix = np.random.default_rng(4).integers(0, dcfg.vocab, (64, 1024)).astype(np.uint16)
    sel = np.array(BENCH_DECODE_SEQS, np.int64)
    toks, lg = oracle.decode(dcfg, dp, prefix[sel], 3, want_logits=True, threads=len(sel))
    put("bench_decode_b64_seqs", sel.astype(np.int32), 4, 0, "sampled sequences of the 64")
    put("bench_decode_b64_tokens", toks.astype(np.uint16), 4, 0,
        "decode_gqa(), init_params(seed 4, std 0.02), prefix rng(4).integers(0, 32000, (64, 1024)): oracle "
        "greedy tokens after the prefix and after each of 3 steps")
    put("bench_decode_b64_logits", lg.astype(np.float16), 4, 2e-2, "[seq, position, vocab] logits (fp16)")
    print(f"decode B64: ({time.time() - t0:.0f} s)", flush=True)


def main():
    only = "grads" if "--bench-grads" in sys.argv else "smear" if "--bench-smear" in sys.argv else None
    bench = "--bench" in sys.argv or "--all" in sys.argv or only is not None
    small = "--bench" not in sys.argv and only is None
    path = os.path.join(HERE, "manifest.json")
    old = json.load(open(path)) if os.path.exists(path) else []
    manifest = []

    def put(name, arr, seed, tol, note):
        arr = np.ascontiguousarray(arr)
        fn = f"{name}.bin"
        arr.astype(arr.dtype.newbyteorder("<")).tofile(os.path.join(HERE, fn))
        manifest.append({"name": name, "file": fn, "dtype": str(arr.dtype), "shape": list(arr.shape),
                         "seed": seed, "tolerance": tol, "note": note})

    if bench:
        bench_fixtures(put, only)
        if only:  # keep the other benchmark-shape fixtures
            written = {m["name"] for m in manifest}
            manifest.extend(m for m in old if m["name"].startswith("bench_") and m["name"] not in written)
    if not small:
        # keep the small fixtures written earlier
        manifest.extend(m for m in old if not m["name"].startswith("bench_"))
        return finish(manifest, path)
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

    if not bench:
        # keep the benchmark-shape fixtures written earlier
        manifest.extend(m for m in old if m["name"].startswith("bench_"))
    finish(manifest, path)


def finish(manifest, path):
    with open(path, "w") as f:
        json.dump(manifest, f, indent=1)
    total = sum(os.path.getsize(os.path.join(HERE, m["file"])) for m in manifest)
    print(f"manifest: {len(manifest)} fixtures, {total / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
