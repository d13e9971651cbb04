"""The causal conv1d's recorded cases and bounds, read the way dash-conformance reads them
(crates/dash-conformance/src/conv1d.rs:23-229, conv1d_state.rs:36-245), shared by the oracle
tests and the GPU tests. Pure numpy."""
from __future__ import annotations

import json

import numpy as np

from fixtures import File, round_bf16, round_f16

GENERAL = "conv1d/general.safetensors"
TRANSFORMERS = "conv1d/conv1d.safetensors"
STATES = "conv1d_state/cases.safetensors"


def bound(dtype: str, part: str) -> float:
    """conv1d.rs:210-229, the CUDA / Flex column (not `other`)."""
    table = {
        ("f32", "out"): 1.4e-7, ("f32", "step"): 1.8e-7, ("f32", "grad_x"): 2.6e-7,
        ("f32", "grad_weight"): 6.1e-7, ("f32", "grad_bias"): 4.1e-7,
        ("bf16", "out"): 3.7e-3, ("bf16", "step"): 3.7e-3, ("bf16", "grad_x"): 3.2e-3,
        ("bf16", "grad_weight"): 3.4e-3, ("bf16", "grad_bias"): 3.4e-3,
        ("f16", "out"): 2.7e-4, ("f16", "step"): 3.2e-4, ("f16", "grad_x"): 3.2e-4,
        ("f16", "grad_weight"): 3.4e-4, ("f16", "grad_bias"): 2.7e-4,
    }
    return table[(dtype, part)]


def state_bound(dtype: str, part: str) -> float:
    """conv1d_state.rs:230-245."""
    if part == "final_state":
        return 0.0
    table = {
        ("f32", "out"): 1.8e-7, ("f32", "grad_x"): 1.7e-7, ("f32", "grad_weight"): 4.1e-7,
        ("f32", "grad_bias"): 4.5e-7, ("f32", "grad_initial_state"): 1.2e-7,
        ("bf16", "out"): 2.7e-3, ("bf16", "grad_x"): 2.6e-3, ("bf16", "grad_weight"): 2.5e-3,
        ("bf16", "grad_bias"): 2.1e-3, ("bf16", "grad_initial_state"): 1.5e-7,
    }
    return table[(dtype, part)]


def to_dtype(x, dtype: str):
    """An f32 result rounded once to the dtype, as the operation returns it."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return round_f16(x)
    return np.asarray(x, np.float32)


class Case:
    """One recorded case of conv1d/{general,conv1d}.safetensors (conv1d.rs:66-167)."""

    def __init__(self, f: File, name: str, meta: dict):
        self.f, self.name, self.meta = f, name, meta
        if "dtype" in meta:
            self.dtype = meta["dtype"]
        else:
            self.dtype = "bf16" if meta.get("bf16") else "f32"
        self.step = meta["kind"] == "step"
        self.silu = bool(meta["silu"])
        self.has_bias = bool(meta.get("bias", False))
        # transformers' decoding state is [B, C, W] in the inputs' dtype
        self.transposed_state = "dtype" not in meta

    def __getitem__(self, part):
        return self.f[f"{self.name}.{part}"]

    def has(self, part):
        return f"{self.name}.{part}" in self.f

    @property
    def bias(self):
        return self["bias"] if self.has_bias else None

    @property
    def state(self):
        s = self["state"]
        return np.ascontiguousarray(np.swapaxes(s, 1, 2)) if self.transposed_state else s

    def recorded_layout(self, state):
        return np.ascontiguousarray(np.swapaxes(state, 1, 2)) if self.transposed_state else state


def cases():
    out = []
    for path in (GENERAL, TRANSFORMERS):
        f = File(path)
        for name, meta in sorted(json.loads(f.meta("cases")).items()):
            out.append(Case(f, name, meta))
    return out


class StateCase:
    """One case of conv1d_state/cases.safetensors (conv1d_state.rs:44-180)."""

    def __init__(self, f: File, name: str, meta: dict):
        self.f, self.name, self.meta = f, name, meta
        self.dtype = meta["dtype"]
        self.silu = bool(meta["silu"])
        self.has_bias = bool(meta["bias"])
        self.w = meta.get("W")
        self.w_out = meta.get("W_out")
        self.k = meta["K"]
        self.cu = self["cu_seqlens"] if meta["kind"] == "packed" else None

    def __getitem__(self, part):
        return self.f[f"{self.name}.{part}"]

    @property
    def bias(self):
        return self["bias"] if self.has_bias else None

    @property
    def h0(self):
        return self["initial_state"] if self.w is not None else None

    @property
    def grad_final(self):
        return self["grad_final_state"] if self.w_out is not None else None


def state_cases():
    f = File(STATES)
    return [StateCase(f, n, m) for n, m in sorted(json.loads(f.meta("cases")).items())]
