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


def sampled_rows(cfg, name, shape, tokens, seed):
    """Row indices of a gradient segment that the benchmark-shape gradient
    fixtures keep: for the value-embedding tables the rows of the first
    tokens of the batch (the only rows their gradient touches); for the
    token embedding those token rows followed by as many rows drawn from
    `seed` (its classifier part reaches every row); else rows drawn from
    `seed`; 1-D segments are kept whole (None)."""
    if len(shape) == 1:
        return None
    r = np.random.default_rng(seed)
    if name == "embed" or name.endswith("ve_embed"):
        seen = []
        for t in tokens.reshape(-1):
            if int(t) not in seen:
                seen.append(int(t))
            if len(seen) == BENCH_GRAD_ROWS:
                break
        if name == "embed":
            others = [int(i) for i in r.permutation(shape[0]) if int(i) not in seen][:BENCH_GRAD_ROWS]
            seen += sorted(others)
        return np.array(seen, np.int64)
    return np.sort(r.choice(shape[0], BENCH_GRAD_ROWS, replace=False)).astype(np.int64)
