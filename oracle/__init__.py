"""CPU oracle for the attention and gated-delta-rule hot path (TEST INFRASTRUCTURE ONLY).

A ctypes front end over ``oracle/liboracle.so``, the plain-C restatement of dash-ops' reference
implementations (``crates/dash-ops/src/attention/reference.rs``,
``crates/dash-ops/src/gated_delta/chunk/reference.rs``,
``crates/dash-ops/src/gated_delta/recurrent.rs:309-404``, ``crates/dash-ops/src/conv1d/reference.rs``). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this module: as the
checker of the HIP path, and as the timed CPU baseline. The product package ``dashmag_amd`` never
imports it.

Every function takes and returns numpy float32 arrays in the contract's layouts
(``[B, T, H, D]``, states ``[S, H, Dk, Dv]``); ``precision`` picks the C body compiled in f32 (the
reference's precision) or in f64.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compiles the oracle with the committed Makefile; returns the library's path."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)
    return _LIB_PATH


class _Attention(ctypes.Structure):
    _fields_ = [
        ("b", ctypes.c_int64), ("tq", ctypes.c_int64), ("tk", ctypes.c_int64),
        ("hq", ctypes.c_int64), ("hkv", ctypes.c_int64), ("d", ctypes.c_int64),
        ("causal", ctypes.c_int32), ("scale", ctypes.c_float),
        ("left", ctypes.c_int64), ("right", ctypes.c_int64),
        ("mask_kind", ctypes.c_int32),
        ("padding", ctypes.c_void_p), ("cu_q", ctypes.c_void_p), ("cu_k", ctypes.c_void_p),
        ("nseq", ctypes.c_int64),
    ]


class _Gdr(ctypes.Structure):
    _fields_ = [
        ("b", ctypes.c_int64), ("t", ctypes.c_int64), ("h", ctypes.c_int64),
        ("dk", ctypes.c_int64), ("dv", ctypes.c_int64),
        ("cu", ctypes.c_void_p), ("nseq", ctypes.c_int64),
        ("qk_l2norm", ctypes.c_int32), ("scale", ctypes.c_float),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.dmo_attention_visible.restype = ctypes.c_int
        _lib.dmo_attention_visible.argtypes = [ctypes.POINTER(_Attention), ctypes.c_int64,
                                               ctypes.c_int64, ctypes.c_int64]
    return _lib


def set_threads(n: int) -> None:
    lib().dmo_set_threads(int(n))


def threads() -> int:
    return int(lib().dmo_threads())


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _i64(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int64))


def _p(x):
    return None if x is None else x.ctypes.data_as(ctypes.c_void_p)


def _side(x):
    return -1 if x is None else int(x)


class AttentionCall:
    """The arguments of one attention call, as the C oracle takes them.

    ``mask`` is ``None``, ``("padding", bool[B, Tk])`` or ``("packed", cu_q, cu_k)``;
    ``left``/``right`` are window sides (``None`` unbounded).
    """

    def __init__(self, q, k, v, mask=None, causal=False, scale=None, left=None, right=None):
        self.q, self.k, self.v = _f32(q), _f32(k), _f32(v)
        b, tq, hq, d = self.q.shape
        _, tk, hkv, _ = self.k.shape
        self.keep = []
        s = _Attention(b=b, tq=tq, tk=tk, hq=hq, hkv=hkv, d=d, causal=int(bool(causal)),
                       scale=float(np.float32(1.0 / math.sqrt(d)) if scale is None else scale),
                       left=_side(left), right=_side(right), mask_kind=0)
        if mask is not None and mask[0] == "padding":
            pad = np.ascontiguousarray(np.asarray(mask[1], dtype=np.uint8))
            self.keep.append(pad)
            s.mask_kind, s.padding = 1, pad.ctypes.data
        elif mask is not None and mask[0] == "packed":
            cq, ck = _i64(mask[1]), _i64(mask[2])
            self.keep += [cq, ck]
            s.mask_kind, s.cu_q, s.cu_k, s.nseq = 2, cq.ctypes.data, ck.ctypes.data, len(cq) - 1
        self.s = s

    def visible(self, b, i, j) -> bool:
        return bool(lib().dmo_attention_visible(ctypes.byref(self.s), b, i, j))

    def visible_matrix(self, b=0) -> np.ndarray:
        tq, tk = self.s.tq, self.s.tk
        return np.array([[self.visible(b, i, j) for j in range(tk)] for i in range(tq)], bool)


def attention_fwd(call: AttentionCall, precision="f32"):
    """Output ``[B, Tq, Hq, D]`` and natural log-sum-exp ``[B, Tq, Hq]`` (reference.rs:305-348)."""
    s = call.s
    o = np.zeros((s.b, s.tq, s.hq, s.d), np.float32)
    lse = np.zeros((s.b, s.tq, s.hq), np.float32)
    getattr(lib(), f"dmo_attention_fwd_{precision}")(
        ctypes.byref(s), _p(call.q), _p(call.k), _p(call.v), _p(o), _p(lse))
    return o, lse


def attention_bwd(call: AttentionCall, o, lse, d_o, precision="f32"):
    """Gradients ``(dq, dk, dv)`` from the forward's output and lse (reference.rs:352-431)."""
    s = call.s
    o, lse, d_o = _f32(o), _f32(lse), _f32(d_o)
    dq = np.zeros_like(call.q)
    dk = np.zeros_like(call.k)
    dv = np.zeros_like(call.v)
    getattr(lib(), f"dmo_attention_bwd_{precision}")(
        ctypes.byref(s), _p(call.q), _p(call.k), _p(call.v), _p(o), _p(lse), _p(d_o),
        _p(dq), _p(dk), _p(dv))
    return dq, dk, dv


def attention_decode(q, k, v, lengths=None, left=None, scale=None, precision="f32"):
    """One query per sequence ``[B, Hq, D]`` against ``[B, S, Hkv, D]`` (reference.rs:433-467)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, hq, d = q.shape
    _, s, hkv, _ = k.shape
    ln = None if lengths is None else _i64(lengths)
    sc = float(np.float32(1.0 / math.sqrt(d)) if scale is None else scale)
    o = np.zeros_like(q)
    f = getattr(lib(), f"dmo_attention_decode_{precision}")
    f.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_float,
                                                                  ctypes.c_void_p]
    f(b, s, hq, hkv, d, _p(q), _p(k), _p(v), _p(ln), _side(left), sc, _p(o))
    return o


def _gdr(q, v, cu, l2norm, scale):
    b, t, h, dk = q.shape[0], q.shape[1], q.shape[2], q.shape[3]
    dv = v.shape[3]
    cu = None if cu is None else _i64(cu)
    sc = float(np.float32(1.0 / math.sqrt(dk)) if scale is None else scale)
    s = _Gdr(b=b, t=t, h=h, dk=dk, dv=dv, cu=None if cu is None else cu.ctypes.data,
             nseq=0 if cu is None else len(cu) - 1, qk_l2norm=int(bool(l2norm)), scale=sc)
    return s, cu


def gdr_chunk_fwd(q, k, v, g, beta, h0=None, cu=None, l2norm=False, scale=None,
                  precision="f32"):
    """Chunked gated delta rule forward (chunk/reference.rs:481-509, packed :697-735): output
    ``[B, T, H, Dv]`` and final states ``[S, H, Dk, Dv]``."""
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    s, cu = _gdr(q, v, cu, l2norm, scale)
    nseq = s.nseq if cu is not None else s.b
    h0 = None if h0 is None else _f32(h0)
    out = np.zeros(q.shape[:3] + (s.dv,), np.float32)
    fin = np.zeros((nseq, s.h, s.dk, s.dv), np.float32)
    rc = getattr(lib(), f"dmo_gdr_chunk_fwd_{precision}")(
        ctypes.byref(s), _p(q), _p(k), _p(v), _p(g), _p(beta), _p(h0), _p(out), _p(fin))
    assert rc == 0
    return out, fin


def gdr_chunk_bwd(q, k, v, g, beta, h0, d_out, d_final, cu=None, l2norm=False, scale=None,
                  precision="f32"):
    """Chunked gated delta rule backward (chunk/reference.rs:519-695, packed :737-780):
    ``(dq, dk, dv, dg, dbeta, dh0)``."""
    q, k, v, g, beta, d_out = map(_f32, (q, k, v, g, beta, d_out))
    s, cu = _gdr(q, v, cu, l2norm, scale)
    nseq = s.nseq if cu is not None else s.b
    h0 = None if h0 is None else _f32(h0)
    d_final = None if d_final is None else _f32(d_final)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    dg, db = np.zeros_like(g), np.zeros_like(beta)
    dh0 = np.zeros((nseq, s.h, s.dk, s.dv), np.float32)
    rc = getattr(lib(), f"dmo_gdr_chunk_bwd_{precision}")(
        ctypes.byref(s), _p(q), _p(k), _p(v), _p(g), _p(beta), _p(h0), _p(d_out), _p(d_final),
        _p(dq), _p(dk), _p(dv), _p(dg), _p(db), _p(dh0))
    assert rc == 0
    return dq, dk, dv, dg, db, dh0


def gdr_step(q, k, v, g, beta, state, cu=None, l2norm=False, scale=None, precision="f32"):
    """The recurrent step (recurrent.rs:309-404): ``q``, ``k`` ``[B, H, Dk]`` (packed: ``[T, H,
    Dk]``), state ``[S, H, Dk, Dv]``; returns ``(out, new_state)``."""
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    st = _f32(state).copy()
    # the step's rows as a batch of one of T tokens
    s, cu = _gdr(q[None], v[None], cu, l2norm, scale)
    s.b = q.shape[0]
    out = np.zeros(v.shape, np.float32)
    rc = getattr(lib(), f"dmo_gdr_step_{precision}")(
        ctypes.byref(s), _p(q), _p(k), _p(v), _p(g), _p(beta), _p(st), _p(out))
    assert rc == 0
    return out, st


def gdr_step_bwd(q, k, v, g, beta, state, d_out, d_state, cu=None, l2norm=False, scale=None,
                 precision="f32"):
    """The step's gradients (reverse-mode through recurrent.rs:362-404, as the reference's
    tracked step gets them, :89-130): ``(dq, dk, dv, dg, dbeta, d_state_in)``; ``d_out`` or
    ``d_state`` may be ``None`` (zeros)."""
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    st = _f32(state)
    s, cu = _gdr(q[None], v[None], cu, l2norm, scale)
    s.b = q.shape[0]
    d_out = None if d_out is None else _f32(d_out)
    d_state = None if d_state is None else _f32(d_state)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    dg, db = np.zeros_like(g), np.zeros_like(beta)
    dst = np.zeros_like(st)
    rc = getattr(lib(), f"dmo_gdr_step_bwd_{precision}")(
        ctypes.byref(s), _p(q), _p(k), _p(v), _p(g), _p(beta), _p(st), _p(d_out), _p(d_state),
        _p(dq), _p(dk), _p(dv), _p(dg), _p(db), _p(dst))
    assert rc == 0
    return dq, dk, dv, dg, db, dst


class _Conv1d(ctypes.Structure):
    _fields_ = [
        ("b", ctypes.c_int64), ("t", ctypes.c_int64), ("c", ctypes.c_int64), ("k", ctypes.c_int64),
        ("cu", ctypes.c_void_p), ("nseq", ctypes.c_int64),
        ("has_bias", ctypes.c_int32), ("silu", ctypes.c_int32),
        ("has_h0", ctypes.c_int32), ("w", ctypes.c_int64),
        ("has_final", ctypes.c_int32), ("w_out", ctypes.c_int64),
    ]


def _conv1d(x, weight, bias, h0, cu, silu, w_out):
    b, t, c = x.shape
    k = weight.shape[1]
    cu = None if cu is None else _i64(cu)
    s = _Conv1d(b=b, t=t, c=c, k=k, cu=None if cu is None else cu.ctypes.data,
                nseq=0 if cu is None else len(cu) - 1, has_bias=int(bias is not None),
                silu=int(bool(silu)), has_h0=int(h0 is not None),
                w=0 if h0 is None else h0.shape[1], has_final=int(w_out is not None),
                w_out=0 if w_out is None else int(w_out))
    return s, cu, (len(cu) - 1 if cu is not None else b)


def conv1d_fwd(x, weight, bias=None, h0=None, cu=None, silu=False, w_out=None,
               precision="f32"):
    """The causal depthwise conv1d (conv1d/reference.rs:223-268): ``x`` ``[B, T, C]``,
    ``weight`` ``[C, K]``, ``bias`` ``[C]``, initial states ``h0`` ``[S, W, C]``; returns the
    output ``[B, T, C]`` and, with ``w_out``, the final states ``[S, w_out, C]``."""
    x, weight = _f32(x), _f32(weight)
    bias = None if bias is None else _f32(bias)
    h0 = None if h0 is None else _f32(h0)
    s, cu, nseq = _conv1d(x, weight, bias, h0, cu, silu, w_out)
    out = np.zeros_like(x)
    fin = np.zeros((nseq, s.w_out, s.c), np.float32) if w_out is not None else None
    rc = getattr(lib(), f"dmo_conv1d_fwd_{precision}")(
        ctypes.byref(s), _p(x), _p(weight), _p(bias), _p(h0), _p(out), _p(fin))
    assert rc == 0
    return out, fin


def conv1d_bwd(x, weight, bias, h0, grad_out, grad_final=None, cu=None, silu=False,
               precision="f32"):
    """The conv1d's gradients (conv1d/reference.rs:270-482): ``(grad_x, grad_weight, grad_bias,
    grad_h0)``, ``grad_bias`` None without a bias, ``grad_h0`` None without initial states; the
    final states' gradient ``grad_final`` ``[S, W', C]`` is optional."""
    x, weight, grad_out = _f32(x), _f32(weight), _f32(grad_out)
    bias = None if bias is None else _f32(bias)
    h0 = None if h0 is None else _f32(h0)
    grad_final = None if grad_final is None else _f32(grad_final)
    s, cu, nseq = _conv1d(x, weight, bias, h0, cu, silu,
                          None if grad_final is None else grad_final.shape[1])
    gx, gw = np.zeros_like(x), np.zeros_like(weight)
    gb = np.zeros(x.shape[2], np.float32) if bias is not None else None
    gh = np.zeros_like(h0) if h0 is not None else None
    rc = getattr(lib(), f"dmo_conv1d_bwd_{precision}")(
        ctypes.byref(s), _p(x), _p(weight), _p(bias), _p(h0), _p(grad_out), _p(grad_final),
        _p(gx), _p(gw), _p(gb), _p(gh))
    assert rc == 0
    return gx, gw, gb, gh


def conv1d_update(x, weight, bias, state, silu=False, precision="f32"):
    """One decoding step (conv1d/reference.rs:484-520): ``x`` ``[B, C]``, ``state`` ``[B, W, C]``;
    returns ``(out [B, C], next_state [B, W, C])``."""
    x, weight, state = _f32(x), _f32(weight), _f32(state)
    bias = None if bias is None else _f32(bias)
    b, c = x.shape
    k, w = weight.shape[1], state.shape[1]
    out, nxt = np.zeros_like(x), np.zeros_like(state)
    f = getattr(lib(), f"dmo_conv1d_update_{precision}")
    f.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int32] * 2 + [ctypes.c_void_p] * 6
    rc = f(b, c, k, w, int(bias is not None), int(bool(silu)), _p(x), _p(weight), _p(bias),
           _p(state), _p(out), _p(nxt))
    assert rc == 0
    return out, nxt


class _Logprob(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int64), ("v", ctypes.c_int64), ("d", ctypes.c_int64),
        ("targets", ctypes.c_void_p), ("masked", ctypes.c_void_p), ("n_masked", ctypes.c_int64),
        ("vocab_chunk", ctypes.c_int64), ("row_chunk", ctypes.c_int64),
    ]


def chosen_logprob(hidden, weight, targets, masked=(), vocab_chunk=0, row_chunk=3072,
                   with_grad=True, precision="f32"):
    """The chosen-token log-probability and entropy (logprob/reference.rs:64-287): ``hidden``
    ``[n, D]``, ``weight`` ``[V, D]``, ``targets`` ``[n]``, ``masked`` token ids (any order,
    each ``< V``); returns ``(logprob [n], entropy [n], grad [n, D] or None)``, ``grad`` the
    gradient of each ``logprob[i]`` with respect to ``hidden[i]``."""
    hidden, weight = _f32(hidden), _f32(weight)
    targets = _i64(targets)
    n, d = hidden.shape
    v = weight.shape[0]
    ids = np.unique(np.asarray(masked, np.int64)).astype(np.uint32)
    assert np.all(ids < v), "masked ids lie below V"
    assert row_chunk >= 1
    s = _Logprob(n=n, v=v, d=d, targets=targets.ctypes.data, masked=ids.ctypes.data if ids.size
                 else None, n_masked=ids.size, vocab_chunk=int(vocab_chunk),
                 row_chunk=int(row_chunk))
    lp, ent = np.zeros(n, np.float32), np.zeros(n, np.float32)
    grad = np.zeros((n, d), np.float32) if with_grad else None
    rc = getattr(lib(), f"dmo_logprob_{precision}")(ctypes.byref(s), _p(hidden), _p(weight),
                                                   _p(lp), _p(ent), _p(grad))
    assert rc == 0
    return lp, ent, grad


class _Lce(ctypes.Structure):
    _fields_ = [("lp", _Logprob), ("ignore_index", ctypes.c_int64), ("eps", ctypes.c_float),
                ("lam", ctypes.c_float), ("entropy", ctypes.c_int32)]


def _lce(hidden, weight, targets, masked, vocab_chunk, row_chunk, ignore_index, eps, lam,
         entropy):
    hidden, weight = _f32(hidden), _f32(weight)
    targets = _i64(targets)
    ids = np.unique(np.asarray(masked, np.int64)).astype(np.uint32)
    assert np.all(ids < weight.shape[0])
    lp = _Logprob(n=hidden.shape[0], v=weight.shape[0], d=hidden.shape[1],
                  targets=targets.ctypes.data, masked=ids.ctypes.data if ids.size else None,
                  n_masked=ids.size, vocab_chunk=int(vocab_chunk), row_chunk=int(row_chunk))
    s = _Lce(lp=lp, ignore_index=int(ignore_index), eps=float(eps), lam=float(lam),
             entropy=int(bool(entropy)))
    return s, hidden, weight, (targets, ids)


def linear_cross_entropy_fwd(hidden, weight, targets, masked=(), vocab_chunk=0, row_chunk=3072,
                             ignore_index=-100, eps=0.0, lam=0.0, entropy=False,
                             precision="f32"):
    """The fused linear cross-entropy's per-row outputs (loss.rs:411-525): ``rows`` ``[8, n]``
    f32 = loss, logprob, entropy, lse, q (1 - p(target)), s, counted, found."""
    s, hidden, weight, keep = _lce(hidden, weight, targets, masked, vocab_chunk, row_chunk,
                                   ignore_index, eps, lam, entropy)
    rows = np.zeros((8, hidden.shape[0]), np.float32)
    rc = getattr(lib(), f"dmo_lce_fwd_{precision}")(ctypes.byref(s), _p(hidden), _p(weight),
                                                   _p(rows))
    assert rc == 0
    return rows


def linear_cross_entropy_bwd(hidden, weight, targets, rows, upstream, masked=(), vocab_chunk=0,
                             row_chunk=3072, ignore_index=-100, eps=0.0, lam=0.0, entropy=False,
                             precision="f32"):
    """Its gradients (loss.rs:527-668 and logprob/reference.rs:289-380) from ``rows`` and the
    upstream gradients ``[3, n]`` of the loss, logprob and entropy rows: ``(grad_hidden [n, D],
    grad_weight [V, D])`` f32."""
    s, hidden, weight, keep = _lce(hidden, weight, targets, masked, vocab_chunk, row_chunk,
                                   ignore_index, eps, lam, entropy)
    rows, upstream = _f32(rows), _f32(upstream)
    gh, gw = np.zeros_like(hidden), np.zeros_like(weight)
    rc = getattr(lib(), f"dmo_lce_bwd_{precision}")(ctypes.byref(s), _p(hidden), _p(weight),
                                                   _p(rows), _p(upstream), _p(gh), _p(gw))
    assert rc == 0
    return gh, gw
