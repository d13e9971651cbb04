"""The chosen-token log-probability's recorded cases and bounds, read the way dash-conformance
reads them (crates/dash-conformance/src/logprob.rs:1-140), shared by the oracle tests and the GPU
tests. Pure numpy."""
from __future__ import annotations

import json
import os

import numpy as np

from fixtures import GOLDEN, File

CASES = ["basic", "peaked", "wide"]
# chunks small enough that every case crosses several, the last partial, and uneven row blocks
# (logprob.rs:34-39 SMALL_CHUNKS)
SMALL_CHUNKS = dict(vocab_chunk=128, row_chunk=10)
PARTS = ["logprob", "entropy", "grad_hidden"]


def bounds(dtype: str):
    """[logprob, entropy, grad_hidden] relative to max|want| (logprob.rs:126-140)."""
    return {"f32": [2e-7, 2e-6, 1e-6], "bf16": [2e-7, 2e-6, 4e-3]}[dtype]


class Case:
    def __init__(self, name: str):
        f = File("logprob/cases.safetensors")
        meta = json.load(open(os.path.join(GOLDEN, "logprob", "meta.json")))[name]
        self.name, self.n, self.v, self.d = name, meta["n"], meta["v"], meta["d"]
        self.masked = list(meta["masked"])
        self.hidden, self.weight = f[f"{name}.hidden"], f[f"{name}.weight"]
        self.targets, self.upstream = f[f"{name}.targets"], f[f"{name}.upstream"]
        self.masked_reference = [f[f"{name}.{p}"] for p in PARTS]
        self.unmasked_reference = [f[f"{name}.{p}_unmasked"] for p in PARTS]


def rel_error(got, want) -> float:
    """max|got - want| / max|want| over the finite entries; -inf must match -inf exactly
    (logprob.rs:10-12)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    ninf = np.isneginf(want)
    assert np.array_equal(np.isneginf(got), ninf), "-inf where the reference has it"
    g, w = got[~ninf], want[~ninf]
    if w.size == 0:
        return 0.0
    scale = np.max(np.abs(w))
    return float(np.max(np.abs(g - w)) / (scale if scale > 0 else 1.0))
