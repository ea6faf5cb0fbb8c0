"""Reader of the golden fixtures in tests/golden (manifest.json + .bin)."""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def manifest():
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        return {m["name"]: m for m in json.load(f)}


def load(name):
    m = manifest()[name]
    arr = np.fromfile(os.path.join(GOLDEN, m["file"]), dtype=np.dtype(m["dtype"]).newbyteorder("<"))
    return arr.reshape(m["shape"]).astype(np.dtype(m["dtype"])), m["tolerance"]


BENCH_GRAD_ROWS = 2
BENCH_EMBED_ROWS = 16


def embed_row_split(shape, tokens):
    """(token rows, other rows) of the token embedding: the rows of the ids
    that occur in the batch, whose gradient also holds the back-propagated
    lookup gradient, and the rest, which hold only the classifier part."""
    tok_rows = np.unique(np.asarray(tokens).reshape(-1).astype(np.int64))
    tok_rows = tok_rows[tok_rows < shape[0]]
    return tok_rows, np.setdiff1d(np.arange(shape[0], dtype=np.int64), tok_rows)


def sampled_rows(cfg, name, shape, tokens, seed):
    """Row indices of a gradient segment that the benchmark-shape gradient
    fixtures keep: for the value-embedding tables the rows of the first
    tokens of the batch (the only rows their gradient touches); for the
    token embedding BENCH_EMBED_ROWS rows drawn from `seed` among the
    batch's token rows, then as many among the other rows (a stratified
    sample, so that the whole tensor's relative error can be estimated);
    else rows drawn from `seed`; 1-D segments are kept whole (None)."""
    if len(shape) == 1:
        return None
    r = np.random.default_rng(seed)
    if name == "embed":
        tok_rows, other = embed_row_split(shape, tokens)
        a = np.sort(r.choice(tok_rows, BENCH_EMBED_ROWS, replace=False))
        b = np.sort(r.choice(other, BENCH_EMBED_ROWS, replace=False))
        return np.concatenate([a, b]).astype(np.int64)
    if name.endswith("ve_embed"):
        seen = []
        for t in tokens.reshape(-1):
            if int(t) not in seen:
                seen.append(int(t))
            if len(seen) == BENCH_GRAD_ROWS:
                break
        return np.array(seen, np.int64)
    return np.sort(r.choice(shape[0], BENCH_GRAD_ROWS, replace=False)).astype(np.int64)


def stratified_rel_l2(got, want, n_strata, sizes):
    """Relative L2 error of a whole tensor estimated from equal-sized row
    samples of its strata (rows concatenated stratum by stratum): each
    stratum's squared error and squared norm are scaled by its row count
    over the sampled count."""
    got = np.asarray(got, np.float64).reshape(n_strata, -1)
    want = np.asarray(want, np.float64).reshape(n_strata, -1)
    err = sum(w * np.sum((g - t) ** 2) for g, t, w in zip(got, want, sizes))
    ref = sum(w * np.sum(t ** 2) for t, w in zip(want, sizes))
    return float(np.sqrt(err / max(ref, 1e-300)))


def repeated_windows(cfg, batch, seed):
    """batch windows that each repeat one token id (ids uniform in
    [0, vocab) from `seed`), targets the same ids: nanochat's smear-lambda
    gradient, a sum over positions and channels, then adds up over the
    positions instead of nearly cancelling as it does on random windows."""
    ids = np.random.default_rng(seed).integers(0, cfg.vocab, batch)
    tok = np.repeat(ids[:, None], cfg.seq, 1).astype(np.uint16)
    return tok, tok.copy()
