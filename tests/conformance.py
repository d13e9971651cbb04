"""The conformance bodies of the hot path, restated from ``crates/dash-conformance/src``
(``lib.rs:125-567``, ``attention.rs``, ``gated_delta_chunk.rs``, ``gated_delta_packed.rs``,
``gated_delta_recurrent.rs``): the recorded cases, their bounds, and test bodies written once and
driven through an adapter, so that the CPU oracle and the HIP library are held to the same
records with the same measure.

An adapter has the methods of dash-conformance's ``trait Adapter`` (lib.rs:176-215) for this path:
``describe()``, ``has(dtype)``, ``attention(call)``, ``attention_decode(call)``,
``chunk_gated_delta_rule(call)`` and ``gated_delta_step(call)``; a call it does not run raises
``Unsupported``. Host tensors are :class:`HostTensor`: values as f32 numpy arrays plus the dtype
they are given in (lib.rs:125-168).
"""
from __future__ import annotations

import dataclasses
import math
from typing import List, Optional

import numpy as np

from dashmag_amd.contract import (AttentionMask, AttentionOptions, ChunkGatedDeltaOptions,
                                  GatedDeltaStepOptions, UNBOUNDED, Unsupported)
from fixtures import File, errors, round_bf16, round_f16, swap_1_2


@dataclasses.dataclass
class HostTensor:
    dtype: str  # "f32" | "bf16" | "f16"
    values: np.ndarray  # f32 values, exactly the dtype's

    @property
    def shape(self):
        return self.values.shape

    def with_dtype(self, dtype):
        return HostTensor(dtype, self.values)


def as_dtype(values, dtype) -> HostTensor:
    """Values rounded to ``dtype`` (what the adapter receives is exactly the dtype's)."""
    v = np.asarray(values, np.float32)
    if dtype == "bf16":
        v = round_bf16(v)
    elif dtype == "f16":
        v = round_f16(v)
    return HostTensor(dtype, np.ascontiguousarray(v))


# ------------------------------------------------------------------------------------------
# Calls and results (lib.rs:294-506)
# ------------------------------------------------------------------------------------------

@dataclasses.dataclass
class Attention:
    q: HostTensor
    k: HostTensor
    v: HostTensor
    mask: AttentionMask
    options: AttentionOptions
    grad: Optional[HostTensor] = None


@dataclasses.dataclass
class AttentionOut:
    out: HostTensor
    lse: HostTensor
    grads: Optional[tuple] = None  # (dq, dk, dv) HostTensors


@dataclasses.dataclass
class AttentionDecode:
    q: HostTensor
    k: HostTensor
    v: HostTensor
    lengths: Optional[np.ndarray]
    options: AttentionOptions


@dataclasses.dataclass
class ChunkGatedDelta:
    q: HostTensor
    k: HostTensor
    v: HostTensor
    g: HostTensor
    beta: HostTensor
    initial_state: Optional[HostTensor]
    cu_seqlens: Optional[np.ndarray]
    options: ChunkGatedDeltaOptions
    grad: Optional[tuple] = None  # (d_out HostTensor, d_final HostTensor | None)


@dataclasses.dataclass
class ChunkGatedDeltaOut:
    out: HostTensor
    final_state: Optional[HostTensor]
    grads: Optional[dict] = None  # q, k, v, g, beta, initial_state


@dataclasses.dataclass
class GatedDeltaStep:
    q: HostTensor
    k: HostTensor
    v: HostTensor
    g: HostTensor
    beta: HostTensor
    state: HostTensor
    cu_seqlens: Optional[np.ndarray]
    options: GatedDeltaStepOptions
    grad: Optional[tuple] = None  # (d_out HostTensor, d_state HostTensor), lib.rs:378-385


@dataclasses.dataclass
class GatedDeltaStepOut:
    out: HostTensor
    state: HostTensor
    grads: Optional[dict] = None  # q, k, v, g, beta, state (lib.rs:398-413)


def ran(label, thunk):
    """Runs a call; ``None`` (and a printed skip) if the adapter refuses it (lib.rs:640-681)."""
    try:
        return thunk()
    except Unsupported as e:
        print(f"skipped: {label}: {e}")
        return None


# ------------------------------------------------------------------------------------------
# Attention (crates/dash-conformance/src/attention.rs)
# ------------------------------------------------------------------------------------------

CAUSAL = ["gqa8x2_d256_t40", "gqa6x2_d64_tq24_tk56"]
MASKS = [
    "none_b2_gqa2x1_d64_tq19_tk33",
    "causal_b2_gqa4x2_d64_tq17_tk41",
    "causal_window9_gqa3x1_d64_t40",
    "window6x4_b2_gqa2x1_d64_tq24_tk37",
    "padding_b3_gqa2x1_d64_t29",
    "padding_causal_b2_gqa2x1_d64_t26",
    "packed_causal_gqa2x1_d64",
    "packed_cross_causal_window5_gqa2x1_d64",
]
PARTS = ["o", "lse", "dq", "dk", "dv"]


@dataclasses.dataclass(frozen=True)
class Bounds:
    causal: tuple
    masks: tuple


# attention.rs:70-108
FLEX_F32 = Bounds((3e-7, 1.1e-7, 5e-7, 3.5e-7, 3.5e-7), (3.2e-7, 1.2e-7, 3.2e-7, 4.1e-7, 3.5e-7))
CUBE_F32 = Bounds((3.2e-7, 1.1e-7, 8.5e-7, 4.6e-7, 4.1e-7), (5.5e-7, 1.4e-7, 5.3e-7, 4.3e-7, 3.4e-7))
AUTOTUNE_F32 = Bounds((1e-6, 2e-7, 1e-6, 1e-6, 1e-6), (1e-6, 2e-7, 1e-6, 1e-6, 1e-6))
BF16 = Bounds((3.4e-3, 2.5e-7, 4.7e-3, 4e-3, 4.2e-3), (3.2e-3, 1.2e-7, 4.3e-3, 4.4e-3, 3.6e-3))
F16 = Bounds((4.6e-4, 1.7e-7, 4.7e-4, 3.6e-4, 4e-4), (3.9e-4, 1.2e-7, 7.4e-4, 6.9e-4, 6.4e-4))


class AttentionRecord:
    """One record (attention.rs:133-185), swapped to the contract's [B, T, H, D]."""

    def __init__(self, name):
        f = File(f"attention/{name}.safetensors")
        self.name = name
        self.causal_set = name in CAUSAL
        read = lambda part: swap_1_2(f[part].astype(np.float32))  # noqa: E731
        self.q = read("q")
        scale = float(f.meta("scale"))
        d = self.q.shape[3]
        causal = f.meta("causal") in (None, "true")
        opts = AttentionOptions().with_causal(causal)
        if np.float32(scale) != np.float32(1.0 / math.sqrt(d)):
            opts = opts.with_scale(scale)
        left = int(f.meta("window_left", "-1"))
        right = int(f.meta("window_right", "-1"))
        if left >= 0 or right >= 0:
            side = lambda r: UNBOUNDED if r < 0 else r  # noqa: E731
            opts = opts.with_window(side(left), side(right))
        kind = f.meta("kind")
        if kind in (None, "none"):
            self.mask = AttentionMask.none()
        elif kind == "padding":
            self.mask = AttentionMask.key_padding(f["key_padding"])
        elif kind == "packed":
            self.mask = AttentionMask.packed(f["cu_seqlens_q"], f["cu_seqlens_k"])
        else:
            raise ValueError(kind)
        self.options = opts
        self.k, self.v, self.grad = read("k"), read("v"), read("do")
        self.expected = [read(p) for p in PARTS]

    def call(self, dtype, deterministic=True, grad=True) -> Attention:
        return Attention(
            q=HostTensor(dtype, self.q), k=HostTensor(dtype, self.k), v=HostTensor(dtype, self.v),
            mask=self.mask, options=self.options.with_deterministic(deterministic),
            grad=HostTensor(dtype, self.grad) if grad else None)


def attention_records():
    return [AttentionRecord(n) for n in CAUSAL + MASKS]


def check_empty_rows(label, o, dq, expected_lse):
    d = o.shape[3]
    o2 = o.reshape(-1, d)
    dq2 = None if dq is None else dq.reshape(-1, d)
    empty = 0
    for row, l in enumerate(expected_lse.ravel()):
        if l != -np.inf:
            continue
        empty += 1
        assert np.all(o2[row] == 0), f"{label}: query {row} sees no key, its output is not zero"
        if dq2 is not None:
            assert np.all(dq2[row] == 0), f"{label}: query {row} sees no key, dq is not zero"
    return empty


def check_attention(label, actual, expected, bounds):
    empty = check_empty_rows(label, actual[0], actual[2], expected[1])
    worst = []
    for name, a, e, bound in zip(PARTS, actual, expected, bounds):
        ab, rel = errors(a, e)
        print(f"{label} {name}: max abs {ab:.3e}, relative {rel:.3e} (tolerance {bound:.1e})")
        assert rel <= bound, f"{label} {name}: relative error {rel:.3e} > {bound:.1e}"
        worst.append(rel)
    return worst, empty


def matches_torch(adapter, label, dtype, deterministic, bounds: Bounds):
    """attention.rs:330-383: every record in one dtype, with gradients, against torch."""
    if not adapter.has(dtype):
        print(f"skipped: {adapter.describe()} has no {dtype}")
        return None
    worst = [[0.0] * 5, [0.0] * 5]
    empty = compared = 0
    for rec in attention_records():
        lab = f"{label} {rec.name}"
        call = rec.call(dtype, deterministic, True)
        out = ran(lab, lambda: adapter.attention(call))
        if out is None:
            continue
        assert out.out.dtype == dtype and out.lse.dtype == "f32"
        dq, dk, dv = out.grads
        actual = [out.out.values, out.lse.values, dq.values, dk.values, dv.values]
        st = 0 if rec.causal_set else 1
        w, e = check_attention(lab, actual, rec.expected,
                               bounds.causal if rec.causal_set else bounds.masks)
        worst[st] = [max(a, b) for a, b in zip(worst[st], w)]
        empty += e
        compared += 1
    assert compared == 0 or empty > 0, "no record has a query that sees no key"
    return worst, compared


def without_gradients(adapter, label, bounds: Bounds):
    """attention.rs:385-429."""
    for name in ["padding_causal_b2_gqa2x1_d64_t26", "packed_causal_gqa2x1_d64"]:
        rec = AttentionRecord(name)
        call = rec.call("f32", True, False)
        out = ran(name, lambda: adapter.attention(call))
        if out is None:
            continue
        assert out.grads is None
        check_empty_rows(name, out.out.values, None, rec.expected[1])
        for i, actual in enumerate([out.out.values, out.lse.values]):
            ab, rel = errors(actual, rec.expected[i])
            print(f"{label} no gradient {name} {PARTS[i]}: abs {ab:.3e} rel {rel:.3e}")
            assert rel <= bounds.masks[i]


def seeded(shape, seed):
    """attention.rs:433-452: xorshift values in about [-2, 2], rounded to bf16."""
    state = (seed * 0x9E3779B97F4A7C15 & (2**64 - 1)) | 1
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    m = 2**64 - 1
    for i in range(n):
        state ^= (state << 13) & m
        state ^= state >> 7
        state ^= (state << 17) & m
        u = np.float32(state >> 40) / np.float32(1 << 24)
        out[i] = (u - np.float32(0.5)) * np.float32(4.0)
    return round_bf16(out).reshape(shape)


def decoding_is_attention_with_one_query(adapter, label, bounds):
    """attention.rs:484-565."""
    b, s, hq, hkv, d = 3, 50, 4, 2, 64
    q = seeded([b, 1, hq, d], 400)
    k = seeded([b, s, hkv, d], 401)
    v = seeded([b, s, hkv, d], 402)
    step_q = q.reshape(b, hq, d)
    for options in [AttentionOptions(), AttentionOptions().with_window(7, 0)]:
        dec = AttentionDecode(HostTensor("f32", step_q), HostTensor("f32", k),
                              HostTensor("f32", v), None, options)
        step = ran(label, lambda: adapter.attention_decode(dec))
        if step is None:
            continue
        assert step.values.shape == (b, hq, d)
        call = Attention(HostTensor("f32", q), HostTensor("f32", k), HostTensor("f32", v),
                         AttentionMask.none(), options.with_causal(True))
        full = ran(label, lambda: adapter.attention(call))
        diff = float(np.max(np.abs(step.values.ravel() - full.out.values.ravel())))
        print(f"{label} decode {options}: max abs {diff:.3e}")
        assert diff <= bounds[0]
    lengths = [50, 17, 1]
    options = AttentionOptions().with_window(9, 0)
    dec = AttentionDecode(HostTensor("f32", step_q), HostTensor("f32", k), HostTensor("f32", v),
                          np.array(lengths, np.int64), options)
    step = ran(label, lambda: adapter.attention_decode(dec))
    if step is not None:
        for bi, ln in enumerate(lengths):
            call = Attention(HostTensor("f32", q[bi:bi + 1]), HostTensor("f32", k[bi:bi + 1, :ln]),
                             HostTensor("f32", v[bi:bi + 1, :ln]), AttentionMask.none(), options)
            full = adapter.attention(call)
            diff = float(np.max(np.abs(step.values[bi].ravel() - full.out.values.ravel())))
            print(f"{label} decode lengths: sequence {bi} of {ln} keys, max abs {diff:.3e}")
            assert diff <= bounds[1]


# ------------------------------------------------------------------------------------------
# Gated delta rule (gated_delta_chunk.rs, gated_delta_packed.rs, gated_delta_recurrent.rs)
# ------------------------------------------------------------------------------------------

# gated_delta_chunk.rs:141-158
CHUNK_F32_TOL = 2e-6
CHUNK_BF16_TOL = 3e-3
CHUNK_BF16_TC_TOL = 6.5e-3
CHUNK_F32_CASES = ["f32_l2norm_state", "f32_plain", "f32_short"]
# gated_delta_packed.rs:43-63
F32_VS_F64 = 1.5e-6
F32_VS_FLA = 2.5e-6
BF16_VS_F64 = 3e-3
BF16_TC_VS_F64 = 6e-3
STEP_VS_REF = 3e-7
PACKED_VS_SEQUENCES = 0.0
CHUNK_PACKED_F32 = ["chunk_f32", "chunk_f32_scale", "chunk_wide_k", "chunk_wide_v"]
STEPS = ["step_f32", "step_f32_scale"]
# gated_delta_recurrent.rs:34-45
STEP_F32_OUT = 8e-7
STEP_F32_STATE = 4e-7
# gated_delta_recurrent.rs:44: the step's gradients against torch autograd
STEP_GRAD_VS_TORCH = 2e-6
# gated_delta_packed.rs:57-59: the packed step's gradients against float64
STEP_GRAD = 4e-7
STEP_BF16_VS_TORCH_BF16 = (8e-3, 4e-3)
STEP_BF16_VS_UPCAST = (4e-3, 4e-7)


def check_results(name, label, res, case, suffix, tol):
    """gated_delta_chunk.rs:118-139 / gated_delta_packed.rs:148-177."""
    failed = []
    keys = sorted(k for k in res if f"{k}{suffix}" in case)
    assert keys, f"{name}: nothing to compare with {suffix}"
    for key in keys:
        ab, rel = errors(res[key], case[f"{key}{suffix}"])
        print(f"{name:20} {label:12} {key:6} vs {suffix or 'torch'}: max abs {ab:.3e} rel {rel:.3e}")
        if rel > tol:
            failed.append(f"{key} {rel:.3e}")
    assert not failed, f"{name} {label}: relative errors above {tol:.1e} against {suffix}: {failed}"


def _flag(f, key):
    import json
    return bool(json.loads(f.meta(key)))


def run_chunk_case(adapter, f: File, dtype, packed: bool, g_f32=False, name=""):
    """gated_delta_chunk.rs:69-116 / gated_delta_packed.rs:189-231."""
    import json
    inp = lambda k: as_dtype(f[k], dtype)  # noqa: E731
    state_grad = _flag(f, "final_state_grad")
    scale = json.loads(f.meta("scale", "null"))
    options = ChunkGatedDeltaOptions(qk_l2norm=_flag(f, "l2norm"),
                                     scale=None if scale is None else float(scale),
                                     output_final_state=True if packed else state_grad)
    call = ChunkGatedDelta(
        q=inp("q"), k=inp("k"), v=inp("v"),
        g=HostTensor("f32", f["g"]) if g_f32 else inp("g"), beta=inp("beta"),
        initial_state=HostTensor("f32", f["h0"]) if _flag(f, "initial_state") else None,
        cu_seqlens=f["cu_seqlens"] if packed else None, options=options,
        grad=(HostTensor("f32", f["d_out"]),
              HostTensor("f32", f["d_state"]) if state_grad else None))
    r = ran(name, lambda: adapter.chunk_gated_delta_rule(call))
    if r is None:
        return None
    assert r.out.dtype == dtype
    res = {"out": r.out.values}
    if r.final_state is not None:
        assert r.final_state.dtype == "f32"
        res["state"] = r.final_state.values
    gr = r.grads
    for k in ["q", "k", "v", "g", "beta"]:
        res[f"d{k}"] = gr[k].values
    if gr.get("initial_state") is not None:
        res["dh0"] = gr["initial_state"].values
    return res


def check_chunk_f32_cases(adapter, label):
    for name in CHUNK_F32_CASES:
        f = File(f"gated_delta_chunk/{name}.safetensors")
        res = run_chunk_case(adapter, f, "f32", False, name=name)
        if res is None:
            continue
        check_results(name, label, res, f, "", CHUNK_F32_TOL)
        check_results(name, label, res, f, "_f64", CHUNK_F32_TOL)


def check_chunk_bf16_case(adapter, label, tol):
    f = File("gated_delta_chunk/bf16_l2norm_state.safetensors")
    res = run_chunk_case(adapter, f, "bf16", False, name="bf16_l2norm_state")
    if res is not None:
        check_results("bf16_l2norm_state", label, res, f, "_f64", tol)


def check_chunk_packed_f32(adapter, label, tol_f64=F32_VS_F64, tol_fla=F32_VS_FLA):
    for name in CHUNK_PACKED_F32:
        f = File(f"gated_delta_packed/{name}.safetensors")
        res = run_chunk_case(adapter, f, "f32", True, g_f32=True, name=name)
        if res is None:
            continue
        check_results(name, label, res, f, "_f64", tol_f64)
        if _flag(f, "fla"):
            check_results(name, label, res, f, "_fla", tol_fla)


def check_chunk_packed_bf16(adapter, label, tol):
    f = File("gated_delta_packed/chunk_bf16.safetensors")
    res = run_chunk_case(adapter, f, "bf16", True, g_f32=True, name="chunk_bf16")
    if res is not None:
        check_results("chunk_bf16", label, res, f, "_f64", tol)


def packed_against_sequences(adapter, name, label):
    """gated_delta_packed.rs:233-336: packed equals per-sequence calls, to the bit."""
    import json
    f = File(f"gated_delta_packed/{name}.safetensors")
    packed = run_chunk_case(adapter, f, "f32", True, g_f32=True, name=name)
    if packed is None:
        return None
    cu = f["cu_seqlens"]
    scale = json.loads(f.meta("scale", "null"))
    options = ChunkGatedDeltaOptions(qk_l2norm=_flag(f, "l2norm"),
                                     scale=None if scale is None else float(scale),
                                     output_final_state=True)
    parts = {}
    state_len = int(np.prod(f["h0"].shape[1:])) if "h0" in f else None
    for s in range(len(cu) - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        h0 = HostTensor("f32", f["h0"][s:s + 1]) if _flag(f, "initial_state") else None
        dst = f["d_state"][s:s + 1] if _flag(f, "final_state_grad") else None
        if a == b:
            shape_state = (1,) + f["state_f64"].shape[1:]
            parts.setdefault("state", []).append(
                h0.values if h0 is not None else np.zeros(shape_state, np.float32))
            if h0 is not None:
                parts.setdefault("dh0", []).append(
                    dst if dst is not None else np.zeros(shape_state, np.float32))
            continue
        sl = lambda k: HostTensor("f32", f[k][:, a:b])  # noqa: E731
        call = ChunkGatedDelta(q=sl("q"), k=sl("k"), v=sl("v"), g=sl("g"), beta=sl("beta"),
                               initial_state=h0, cu_seqlens=None, options=options,
                               grad=(sl("d_out"), None if dst is None else HostTensor("f32", dst)))
        r = adapter.chunk_gated_delta_rule(call)
        parts.setdefault("out", []).append(r.out.values)
        parts.setdefault("state", []).append(r.final_state.values)
        for k in ["q", "k", "v", "g", "beta"]:
            parts.setdefault(f"d{k}", []).append(r.grads[k].values)
        if r.grads.get("initial_state") is not None:
            parts.setdefault("dh0", []).append(r.grads["initial_state"].values)
    worst = 0.0
    for key in sorted(packed):
        axis = 0 if key in ("state", "dh0") else 1
        apart = np.concatenate(parts[key], axis=axis)
        ab, rel = errors(packed[key], apart)
        print(f"{name:16} {label:12} {key:6} packed vs per sequence max abs {ab:.3e} rel {rel:.3e}")
        worst = max(worst, rel)
    return worst


def run_step_case(adapter, f: File, packed_rows=None):
    import json
    scale = json.loads(f.meta("scale", "null"))
    opts = GatedDeltaStepOptions(_flag(f, "l2norm"), None if scale is None else float(scale))
    call = GatedDeltaStep(*(HostTensor("f32", f[k]) for k in ["q", "k", "v", "g", "beta", "h0"]),
                          cu_seqlens=f["cu_seqlens"], options=opts)
    r = ran(f.name, lambda: adapter.gated_delta_step(call))
    return None if r is None else {"out": r.out.values, "state": r.state.values}


def check_steps(adapter, label):
    """gated_delta_packed.rs:459-502: packed step against f64 and fla, and against itself token by
    token (to the bit)."""
    import json
    for name in STEPS:
        f = File(f"gated_delta_packed/{name}.safetensors")
        res = run_step_case(adapter, f)
        if res is None:
            continue
        check_results(name, label, res, f, "_f64", STEP_VS_REF)
        check_results(name, label, res, f, "_fla", STEP_VS_REF)
        scale = json.loads(f.meta("scale", "null"))
        opts = GatedDeltaStepOptions(_flag(f, "l2norm"), None if scale is None else float(scale))
        cu = f["cu_seqlens"]
        outs, states = [], []
        for s in range(len(cu) - 1):
            st = HostTensor("f32", f["h0"][s:s + 1])
            for t in range(int(cu[s]), int(cu[s + 1])):
                row = lambda k: HostTensor("f32", f[k][t:t + 1])  # noqa: E731
                r = adapter.gated_delta_step(GatedDeltaStep(row("q"), row("k"), row("v"), row("g"),
                                                            row("beta"), st, None, opts))
                outs.append(r.out.values)
                st = r.state
            states.append(st.values)
        for key, apart in [("out", np.concatenate(outs, 0)), ("state", np.concatenate(states, 0))]:
            ab, rel = errors(res[key], apart)
            print(f"{name:16} {label:12} {key:6} packed vs token by token abs {ab:.3e} rel {rel:.3e}")
            assert rel <= PACKED_VS_SEQUENCES, (name, key, rel)


def check_f32_steps(adapter, label):
    """gated_delta_recurrent.rs:107-137."""
    f = File("gated_delta_recurrent/steps_f32.safetensors")
    for case, l2 in [("step_small", False), ("step_small_l2", True), ("step_head128", True)]:
        call = GatedDeltaStep(*(HostTensor("f32", f[f"{case}.{k}"])
                                for k in ["q", "k", "v", "g", "beta", "state"]),
                              cu_seqlens=None, options=GatedDeltaStepOptions(qk_l2norm=l2))
        r = ran(case, lambda: adapter.gated_delta_step(call))
        if r is None:
            continue
        for what, act, exp, tol in [("out", r.out.values, f[f"{case}.out"], STEP_F32_OUT),
                                    ("new_state", r.state.values, f[f"{case}.new_state"],
                                     STEP_F32_STATE)]:
            ab, rel = errors(act, exp)
            print(f"{label} {case}.{what}: max abs {ab:.3e}, relative {rel:.3e} (tol {tol:.0e})")
            assert rel <= tol


def check_prefill_then_decode(adapter, label):
    """gated_delta_recurrent.rs:155-205."""
    f = File("gated_delta_recurrent/prefill_decode.safetensors")
    n = lambda k: f[f"prefill_decode.{k}"]  # noqa: E731
    q, k, v, g, beta = (n(x) for x in ["q", "k", "v", "g", "beta"])
    b, tokens, h, _ = q.shape
    state = HostTensor("f32", n("prefill_state"))
    outs = []
    for t in range(tokens):
        call = GatedDeltaStep(HostTensor("f32", q[:, t]), HostTensor("f32", k[:, t]),
                              HostTensor("f32", v[:, t]), HostTensor("f32", g[:, t]),
                              HostTensor("f32", beta[:, t]), state, None,
                              GatedDeltaStepOptions(qk_l2norm=True))
        r = ran("prefill_decode", lambda: adapter.gated_delta_step(call))
        if r is None:
            return
        outs.append(r.out.values)
        state = r.state
    out = np.stack(outs, 1)
    for what, act, exp, tol in [("out", out, n("out"), STEP_F32_OUT),
                                ("final_state", state.values, n("final_state"), STEP_F32_STATE)]:
        ab, rel = errors(act, exp)
        print(f"{label} prefill_decode.{what}: abs {ab:.3e} rel {rel:.3e}")
        assert rel <= tol


def check_bf16_step(adapter, label):
    """gated_delta_recurrent.rs:207-241."""
    f = File("gated_delta_recurrent/step_bf16.safetensors")
    n = lambda k: f[f"step_bf16.{k}"]  # noqa: E731
    call = GatedDeltaStep(HostTensor("bf16", n("q")), HostTensor("bf16", n("k")),
                          HostTensor("bf16", n("v")), HostTensor("f32", n("g")),
                          HostTensor("bf16", n("beta")), HostTensor("f32", n("state")), None,
                          GatedDeltaStepOptions(qk_l2norm=True))
    r = ran("step_bf16", lambda: adapter.gated_delta_step(call))
    if r is None:
        return
    assert r.out.dtype == "bf16" and r.state.dtype == "f32"
    for what, data, tol in [("out_torch_bf16", r.out.values, STEP_BF16_VS_TORCH_BF16[0]),
                            ("new_state_torch_bf16", r.state.values, STEP_BF16_VS_TORCH_BF16[1]),
                            ("out_f32_upcast", r.out.values, STEP_BF16_VS_UPCAST[0]),
                            ("new_state_f32_upcast", r.state.values, STEP_BF16_VS_UPCAST[1])]:
        ab, rel = errors(data, n(what))
        print(f"{label} step_bf16 against {what}: abs {ab:.3e} rel {rel:.3e} (tol {tol:.0e})")
        assert rel <= tol, (what, rel)


def check_gradients(adapter, label):
    """gated_delta_recurrent.rs:229-269: one step's output, new state and the gradients of every
    input against torch autograd through the same step."""
    f = File("gated_delta_recurrent/step_grad.safetensors")
    n = lambda k: f[f"step_grad.{k}"]  # noqa: E731
    call = GatedDeltaStep(*(HostTensor("f32", n(k)) for k in ["q", "k", "v", "g", "beta", "state"]),
                          cu_seqlens=None, options=GatedDeltaStepOptions(qk_l2norm=True),
                          grad=(HostTensor("f32", n("w_out")), HostTensor("f32", n("w_state"))))
    r = ran("step_grad", lambda: adapter.gated_delta_step(call))
    if r is None:
        return False
    checks = [("out", r.out.values, n("out"), STEP_F32_OUT),
              ("new_state", r.state.values, n("new_state"), STEP_F32_STATE)]
    assert r.grads is not None, "step_grad: the gradients asked for"
    for name in ["q", "k", "v", "g", "beta", "state"]:
        checks.append((f"grad_{name}", r.grads[name].values, n(f"grad_{name}"),
                       STEP_GRAD_VS_TORCH))
    for what, act, exp, tol in checks:
        ab, rel = errors(act, exp)
        print(f"{label} step_grad {what}: max abs {ab:.3e}, relative {rel:.3e} (tol {tol:.0e})")
        assert rel <= tol, (what, rel)
    return True


def check_step_gradients(adapter, label):
    """gated_delta_packed.rs:419-443, :504-517: the packed step's gradients (cotangents of the
    output and of the final states) against transformers in float64, sequences of 1, 3, 0 and 2
    tokens (an empty one passes the state's gradient through) and of 2, 1 and 4."""
    import json
    ran_cases = 0
    for name in STEPS:
        f = File(f"gated_delta_packed/{name}.safetensors")
        scale = json.loads(f.meta("scale", "null"))
        opts = GatedDeltaStepOptions(_flag(f, "l2norm"), None if scale is None else float(scale))
        call = GatedDeltaStep(*(HostTensor("f32", f[k]) for k in ["q", "k", "v", "g", "beta",
                                                                   "h0"]),
                              cu_seqlens=f["cu_seqlens"], options=opts,
                              grad=(HostTensor("f32", f["d_out"]), HostTensor("f32", f["d_state"])))
        r = ran(name, lambda: adapter.gated_delta_step(call))
        if r is None:
            continue
        assert r.grads is not None, f"{name}: the gradients asked for"
        res = {"dq": r.grads["q"].values, "dk": r.grads["k"].values, "dv": r.grads["v"].values,
               "dg": r.grads["g"].values, "dbeta": r.grads["beta"].values,
               "dh0": r.grads["state"].values}
        check_results(name, label, res, f, "_f64", STEP_GRAD)
        ran_cases += 1
    return ran_cases


def the_default_scale_is_one_over_the_root_of_dk(adapter, label):
    """gated_delta_packed.rs:519-548: giving the scale 1 / sqrt(Dk) explicitly changes nothing,
    to the bit (chunk_f32, normalised queries and keys, final states)."""
    f = File("gated_delta_packed/chunk_f32.safetensors")
    dk = f["q"].shape[3]

    def run(scale):
        options = ChunkGatedDeltaOptions(qk_l2norm=True, scale=scale, output_final_state=True)
        call = ChunkGatedDelta(
            q=HostTensor("f32", f["q"]), k=HostTensor("f32", f["k"]), v=HostTensor("f32", f["v"]),
            g=HostTensor("f32", f["g"]), beta=HostTensor("f32", f["beta"]),
            initial_state=HostTensor("f32", f["h0"]), cu_seqlens=f["cu_seqlens"], options=options)
        r = ran("chunk_f32", lambda: adapter.chunk_gated_delta_rule(call))
        return None if r is None else (r.out.values, r.final_state.values)

    by_default = run(None)
    # the scale as the contract computes it in f32: 1 / sqrt(Dk) (dash-contract lib.rs query_scale)
    given = run(float(np.float32(1.0) / np.sqrt(np.float32(dk))))
    if by_default is None or given is None:
        return False
    for a, b in zip(by_default, given):
        assert np.array_equal(a, b), f"{label}: an explicit 1/sqrt(Dk) changed the result"
    print(f"{label} default scale: out and final states identical to the bit")
    return True
