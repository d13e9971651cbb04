"""The fused linear cross-entropy's recorded cases (crates/dash-ops/tests/loss.rs:1-300), shared by
the oracle tests and the GPU tests. Pure numpy."""
from __future__ import annotations

import json
import os

import numpy as np

from fixtures import GOLDEN, File, round_bf16

CASES = ["basic", "peaked", "wide"]
# chunks of 64 tokens (the last partial in every case) and row blocks of 10 or fewer
# (loss.rs:56-62 SMALL_CHUNKS)
SMALL_CHUNKS = dict(vocab_chunk=64, row_chunk=10)
PARTS = ["loss", "logprob", "entropy", "grad_hidden", "grad_weight"]
# [loss, logprob, entropy, grad_hidden, grad_weight] relative to max|want| (loss.rs:463-470,
# :983-992): the reference path in f32, the kernel path from bf16 inputs (the logits' gradient
# rounded to bf16 for the products)
BOUNDS = {"f32": [2e-7, 2e-7, 1e-6, 4e-6, 4e-6], "bf16": [2e-7, 2e-7, 3e-7, 5e-3, 5e-3]}


class Case:
    def __init__(self, name: str):
        self.f = File("loss/cases.safetensors")
        self.meta = json.load(open(os.path.join(GOLDEN, "loss", "meta.json")))[name]
        self.name, self.n, self.v, self.d = name, self.meta["n"], self.meta["v"], self.meta["d"]
        self.hidden, self.weight = self.f[f"{name}.hidden"], self.f[f"{name}.weight"]
        self.targets = self.f[f"{name}.targets"]
        self.g_loss, self.g_lp, self.g_ent = (self.f[f"{name}.{k}"]
                                              for k in ("g_loss", "g_lp", "g_ent"))
        self.variants = list(self.meta["variants"])

    def inputs(self, precision):
        if precision == "bf16":
            return round_bf16(self.hidden), round_bf16(self.weight)
        return self.hidden, self.weight

    def options(self, variant):
        m = self.meta["variants"][variant]
        return dict(reduction=m["reduction"], ignore_index=m["ignore_index"], eps=m["eps"],
                    lam=m["lam"], masked=list(m["masked"]), entropy=True)

    def want(self, precision, variant, term=None):
        key = lambda k: self.f[f"{self.name}.{precision}.{variant}.{k}"]  # noqa: E731
        grad = (lambda k: key(f"{term}_only.{k}")) if term else key
        return [key("loss"), key("logprob"), key("entropy"), grad("grad_hidden"),
                grad("grad_weight")]

    def upstream(self, reduction, counted, term=None):
        """[3, n]: the objective's gradients of the loss, logprob and entropy rows (loss.rs:
        350-365): the mean's 1 / (counted rows), the sum's 1, or g_loss unreduced."""
        n = self.n
        if reduction == "mean":
            gl = np.full(n, 1.0 / max(float(counted.sum()), 1.0), np.float32)
        elif reduction == "sum":
            gl = np.ones(n, np.float32)
        else:
            gl = self.g_loss.astype(np.float32)
        gp, ge = self.g_lp.astype(np.float32), self.g_ent.astype(np.float32)
        if term == "loss":
            gp, ge = gp * 0, ge * 0
        elif term == "lp":
            gl, ge = gl * 0, ge * 0
        elif term == "ent":
            gl, gp = gl * 0, gp * 0
        return np.stack([gl, gp, ge]).astype(np.float32)


def reduce(rows, reduction):
    """The loss as linear_cross_entropy reduces the rows (loss.rs:872-877)."""
    if reduction == "none":
        return rows[0]
    total = np.sum(rows[0].astype(np.float64))
    if reduction == "sum":
        return np.array([total], np.float32)
    return np.array([total / np.sum(rows[6])], np.float32)


def rel_error(got, want) -> float:
    """max|got - want| / max|want| over the finite entries; an infinity must match."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf) and np.array_equal(got[inf], want[inf]), \
        "infinities where the reference has them"
    g, w = got[~inf], want[~inf]
    if w.size == 0:
        return 0.0
    scale = np.max(np.abs(w))
    return float(np.max(np.abs(g - w)) / (scale if scale > 0 else 1.0))
