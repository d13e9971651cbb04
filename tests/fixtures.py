"""Reads the reference's recorded fixtures (``tests/golden/``, copied unchanged from
``crates/dash-ops/tests/fixtures/``) the way ``crates/dash-conformance/src/fixtures.rs:36-153``
does: safetensors with f32, bf16, i64 and u8-as-bool tensors plus string metadata. Pure numpy;
nothing in a file is executed."""
from __future__ import annotations

import json
import os
import struct

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


class File:
    def __init__(self, relative: str):
        self.name = relative
        with open(os.path.join(GOLDEN, relative), "rb") as f:
            raw = f.read()
        n = struct.unpack("<Q", raw[:8])[0]
        header = json.loads(raw[8:8 + n])
        self.metadata = header.pop("__metadata__", None) or {}
        body = raw[8 + n:]
        self.tensors = {}
        for key, info in header.items():
            a, b = info["data_offsets"]
            buf = body[a:b]
            shape = tuple(info["shape"])
            dt = info["dtype"]
            if dt == "F32":
                x = np.frombuffer(buf, "<f4").reshape(shape).copy()
            elif dt == "BF16":
                u = np.frombuffer(buf, "<u2").astype(np.uint32) << 16
                x = u.view(np.float32).reshape(shape).copy()
            elif dt == "I64":
                x = np.frombuffer(buf, "<i8").reshape(shape).copy()
            elif dt == "U8":
                x = (np.frombuffer(buf, "u1") != 0).reshape(shape).copy()
            else:
                raise ValueError(f"{relative}: {key} has dtype {dt}")
            self.tensors[key] = x
        self.dtypes = {k: v["dtype"] for k, v in header.items()}

    def __getitem__(self, key):
        return self.tensors[key]

    def __contains__(self, key):
        return key in self.tensors

    def meta(self, key, default=None):
        return self.metadata.get(key, default)


def errors(actual, expected):
    """dash-conformance's error measure (attention.rs:206-228, lib.rs:707-718): the largest
    absolute difference and that over the largest reference magnitude, over the entries where
    the reference is finite. A -inf reference must be matched exactly."""
    a = np.asarray(actual, np.float32).ravel()
    e = np.asarray(expected, np.float32).ravel()
    assert a.shape == e.shape, (a.shape, e.shape)
    neg = e == -np.inf
    assert np.all(a[neg] == -np.inf), "an entry is not -inf where -inf is expected"
    a, e = a[~neg], e[~neg]
    assert np.all(np.isfinite(a)), "non-finite value"
    if a.size == 0:
        return 0.0, 0.0
    m = float(np.max(np.abs(a - e)))
    scale = float(np.max(np.abs(e)))
    return m, m / max(scale, np.finfo(np.float32).tiny)


def swap_1_2(x):
    """[B, H, T, ...] <-> [B, T, H, ...] (dash-conformance attention.rs:192-211)."""
    return np.ascontiguousarray(np.swapaxes(x, 1, 2))


def round_bf16(x):
    """Round-to-nearest-even to bf16, returned as f32 values."""
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def round_f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
