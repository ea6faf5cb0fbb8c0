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
