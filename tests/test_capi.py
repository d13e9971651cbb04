"""The C ABI without a GPU: the library loads, exports every symbol include/dashmi.h declares,
and its host-side visibility intervals equal the oracle's element-wise mask, to the bit."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from dashmag_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "dashmi.h")).read()
    return sorted(set(re.findall(r"\b(dm_[a-z0-9_]+)\s*\(", text)))


def test_header_and_bindings_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lb = _lib.lib()
    for name in declared_symbols():
        assert hasattr(lb, name), name


def _desc(tq, tk, causal, left, right, kind, cu_q=None, cu_k=None):
    d = _lib.AttentionDesc(b=1, tq=tq, tk=tk, hq=1, hkv=1, d=8, dtype=_lib.DM_F32,
                           mask_kind=kind)
    d.options.causal = int(causal)
    if left is not None or right is not None:
        d.options.has_window = 1
        d.options.window_left = _lib.DM_UNBOUNDED if left is None else left
        d.options.window_right = _lib.DM_UNBOUNDED if right is None else right
    keep = []
    if kind == _lib.DM_MASK_PACKED:
        cq = np.ascontiguousarray(cu_q, np.int32)
        ck = np.ascontiguousarray(cu_k, np.int32)
        keep = [cq, ck]
        d.cu_seqlens_q, d.cu_seqlens_k = cq.ctypes.data, ck.ctypes.data
        d.nseq = len(cq) - 1
    return d, keep


@pytest.mark.parametrize("case", range(60))
def test_row_bounds_equal_the_oracle_mask(case):
    rng = np.random.default_rng(1000 + case)
    tq, tk = int(rng.integers(1, 24)), int(rng.integers(1, 24))
    causal = bool(rng.integers(0, 2))
    left = None if rng.random() < 0.4 else int(rng.integers(0, 9))
    right = None if rng.random() < 0.4 else int(rng.integers(0, 9))
    packed = case % 2 == 1
    cu_q = cu_k = None
    if packed:
        s = int(rng.integers(1, 5))
        cu_q = np.concatenate([[0], np.sort(rng.integers(0, tq + 1, s))])
        cu_k = np.concatenate([[0], np.sort(rng.integers(0, tk + 1, s))])
    d, keep = _desc(tq, tk, causal, left, right,
                    _lib.DM_MASK_PACKED if packed else _lib.DM_MASK_NONE, cu_q, cu_k)
    q = np.zeros((1, tq, 1, 8), np.float32)
    k = np.zeros((1, tk, 1, 8), np.float32)
    call = oracle.AttentionCall(q, k, k, ("packed", cu_q, cu_k) if packed else None, causal,
                                None, left, right)
    want = call.visible_matrix(0)
    lo, hi = ctypes.c_int64(), ctypes.c_int64()
    for i in range(tq):
        assert _lib.lib().dm_attention_row_bounds(ctypes.byref(d), 0, i, ctypes.byref(lo),
                                                  ctypes.byref(hi)) == 0
        got = np.zeros(tk, bool)
        got[lo.value:hi.value] = True
        assert np.array_equal(got, want[i]), (i, lo.value, hi.value, want[i])


def test_refusal_names_the_operation():
    d, _ = _desc(4, 4, False, None, None, _lib.DM_MASK_NONE)
    d.hq, d.hkv = 3, 2
    rc = _lib.lib().dm_attention_fwd(ctypes.byref(d), None, None, None, None, None, None, 0, None)
    assert rc == _lib.DM_ERR_REFUSED
    assert _lib.last_error().startswith("attention: the query heads (3)")


def test_paged_decode_refusals():
    """The paged decode refuses before any launch: capacity and page size disagree, a packed
    offset array instead of a block table, a missing block table."""
    lb = _lib.lib()
    d, _ = _desc(1, 64, False, None, None, _lib.DM_MASK_NONE)
    d.dtype = _lib.DM_BF16
    call = lambda ps, bt, mp: lb.dm_attention_decode_paged(  # noqa: E731
        ctypes.byref(d), None, None, None, 4, ps, bt, mp, None, None, None, 0, None)
    assert call(16, None, 3) == _lib.DM_ERR_REFUSED
    assert _lib.last_error().startswith("attention_decode_paged: desc->tk (64)")
    assert call(0, None, 4) == _lib.DM_ERR_REFUSED
    assert "page_size must be positive" in _lib.last_error()
    assert call(16, None, 4) == _lib.DM_ERR_REFUSED
    assert "block table" in _lib.last_error()
    ck = np.zeros(2, np.int32)
    d.cu_seqlens_k = ck.ctypes.data
    assert call(16, None, 4) == _lib.DM_ERR_REFUSED
    assert "not cu_seqlens_k" in _lib.last_error()


def test_packed_decode_refuses_a_wrong_sequence_count():
    d, _ = _desc(1, 8, False, None, None, _lib.DM_MASK_NONE)
    ck = np.zeros(3, np.int32)
    d.cu_seqlens_k, d.nseq = ck.ctypes.data, 2
    rc = _lib.lib().dm_attention_decode(ctypes.byref(d), None, None, None, None, None, None, 0,
                                        None)
    assert rc == _lib.DM_ERR_REFUSED
    assert _lib.last_error().startswith("attention_decode: a packed cache")


def test_logprob_refusals():
    """The log-probability refuses before any launch: a masked id outside the vocabulary, every
    token masked, an f16 operand, a zero row_chunk."""
    lb = _lib.lib()
    d = _lib.LogprobDesc(n=4, v=5, d=8, hidden_dtype=_lib.DM_BF16, weight_dtype=_lib.DM_BF16,
                         vocab_chunk=0, row_chunk=3072)

    def call(ids):
        arr = (ctypes.c_uint32 * max(len(ids), 1))(*ids)
        return lb.dm_chosen_logprob(ctypes.byref(d), None, None, None,
                                    ctypes.cast(arr, ctypes.c_void_p), len(ids), None, None,
                                    None, None, 0, None)

    assert call([7]) == _lib.DM_ERR_REFUSED
    assert _lib.last_error() == ("chosen_logprob: masked token id 7 is not below the "
                                 "vocabulary size 5")
    assert call([4, 3, 2, 1, 0, 0]) == _lib.DM_ERR_REFUSED
    assert _lib.last_error() == "chosen_logprob: at least one token must stay unmasked"
    assert call([1, 1]) == _lib.DM_ERR_REFUSED  # passes the ids, stops at the workspace
    assert "workspace" in _lib.last_error()
    d.hidden_dtype = _lib.DM_F16
    assert call([]) == _lib.DM_ERR_REFUSED
    assert _lib.last_error() == "chosen_logprob: the log-probability takes bf16 or f32"
    d.hidden_dtype, d.row_chunk = _lib.DM_BF16, 0
    assert call([]) == _lib.DM_ERR_REFUSED
    assert _lib.last_error() == "chosen_logprob: row_chunk must be at least 1"


def test_noalloc_decode_refuses_calls_beyond_its_scratch():
    """The no-allocation decode refuses, before touching the device, a call whose partials would
    not fit its 16 MiB scratch (here 1024 x 64 rows of 256 f32 partials, 64 MiB)."""
    d = _lib.AttentionDesc(b=1024, tq=1, tk=100_000, hq=64, hkv=8, d=256, dtype=_lib.DM_BF16,
                           mask_kind=_lib.DM_MASK_NONE)
    lb = _lib.lib()
    assert lb.dm_attention_decode_workspace(ctypes.byref(d)) > (16 << 20)
    rc = lb.dm_attention_decode_noalloc(ctypes.byref(d), None, None, None, None, None, None)
    assert rc == _lib.DM_ERR_REFUSED
    assert _lib.last_error().startswith("attention_decode: the call needs")
