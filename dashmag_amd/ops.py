"""The hot path's operations on device tensors, mirroring dash-ops' public functions (same names,
argument meaning and refusals): ``attention``, ``attention_with_lse``, ``attention_backward``,
``attention_decode`` (crates/dash-ops/src/attention.rs:648-806), ``chunk_gated_delta_rule``
(gated_delta/chunk.rs:856-981) with its explicit backward ``chunk_gated_delta_rule_backward``,
and ``gated_delta_step`` (gated_delta/recurrent.rs:158).

Tensors are torch tensors on the GPU (PyTorch is the device-memory and stream plumbing); every
computation runs in ``libdashmi.so`` through its C ABI, on torch's current stream. A call
outside the contract raises :class:`~dashmag_amd.contract.Unsupported` whose message starts
``"<operation>: "``, as a ``Result``-returning implementation reports it (dash-mlx's convention).
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib
from .contract import (Activation, AttentionMask, AttentionOptions, CausalConv1dOptions,
                       CausalConv1dStepOptions, ChunkGatedDeltaOptions, GatedDeltaStepOptions,
                       CrossEntropyOptions, LogprobOptions, Reduction, UNBOUNDED, Unsupported)

_DT = {torch.float32: _lib.DM_F32, torch.bfloat16: _lib.DM_BF16, torch.float16: _lib.DM_F16}


def _dtype(op, t):
    if t.dtype not in _DT:
        raise Unsupported(f"{op}: dtype {t.dtype} is not f32, bf16 or f16")
    return _DT[t.dtype]


def _device(op, *ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise Unsupported(f"{op}: the tensors must be on the GPU (got {t.device})")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(op, rc):
    if rc == _lib.DM_OK:
        return
    msg = _lib.last_error()
    if rc == _lib.DM_ERR_REFUSED:
        raise Unsupported(msg if msg.startswith(op) else f"{op}: {msg}")
    raise RuntimeError(msg)


def _readable(t):
    """``t`` as the kernels read it in place: a view whose last dimension is contiguous, and for
    16-bit dtypes strides that are multiples of 8 elements on a 16-byte aligned base (what the
    MFMA and split kernels' vector loads take); otherwise a contiguous copy, as dash-ops copies
    what its kernels cannot read in place (crates/dash-ops/src/attention.rs:85-93)."""
    if t.dim() == 0 or t.numel() == 0:
        return t.contiguous()
    st = t.stride()
    if st[-1] != 1 and t.shape[-1] > 1:
        return t.contiguous()
    if t.element_size() == 2 and (any(x % 8 for x in st[:-1]) or t.data_ptr() % 16):
        c = t.contiguous()
        # a contiguous view at an offset is its own contiguous(): copy it to a fresh allocation
        return c.clone() if c.data_ptr() % 16 else c
    return t


def _gdr_view(t, rows_b, fast):
    """A gated-delta-rule input as the kernels read it in place: ``_readable`` for q, k, v and
    d_out (``fast``), any view for g and beta; and, for a batch of more than one, rows that
    follow one another (b stride = T x t stride), else a contiguous copy."""
    t = _readable(t) if fast else t
    if rows_b and t.dim() >= 2 and t.shape[0] > 1 and t.stride(0) != t.shape[1] * t.stride(1):
        t = t.contiguous()
    return t


def _gdr_strides(desc, step, **tensors):
    desc.strided = 1
    dims = (0, None, 1) if step else (0, 1, 2)
    for name, t in tensors.items():
        _set_strides(getattr(desc, name), t, dims)


def _set_strides(field, t, dims):
    """Fills a ``dm_strides`` from ``t``'s strides along ``dims`` (``b``, ``t``, ``h`` in that
    order; None for an axis the tensor lacks)."""
    st = t.stride()
    field.b, field.t, field.h = (0 if i is None else st[i] for i in dims)


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


_I32_MAX = (1 << 31) - 1


def _offsets(t, device, op=None, what="offsets"):
    """Offsets of any int dtype as the int32 device array the kernels read; with ``op``, values
    outside int32 are refused rather than wrapped by the cast."""
    t = torch.as_tensor(t)
    if op is not None and t.numel() and t.dtype not in (torch.int32, torch.int16, torch.uint8,
                                                       torch.int8):
        lo, hi = int(t.min()), int(t.max())
        if lo < -_I32_MAX - 1 or hi > _I32_MAX:
            raise Unsupported(f"{op}: {what} must fit in int32, got values in [{lo}, {hi}]")
    return t.to(device=device, dtype=torch.int32).contiguous()


def _cu_seqlens(op, t, device, tokens, exact=True, what="cu_seqlens"):
    """Sequence offsets, checked on the host as dash-ops' ``read_cu_seqlens`` checks them
    (crates/dash-ops/src/sequences.rs:49-67): they start at 0 and do not decrease, and they end
    at ``tokens`` (``exact``) or, for attention's packed mask, at most there (positions past the
    last offset belong to no sequence, crates/dash-contract/src/attention.rs:49-54). Offsets the
    kernels would index rows with are never passed on unchecked. Returns the int32 device
    array."""
    host = torch.as_tensor(t).detach().to("cpu", torch.int64)
    cu = host.tolist()
    ok = (len(cu) >= 1 and cu[0] == 0 and all(a <= b for a, b in zip(cu, cu[1:]))
          and (cu[-1] == tokens if exact else cu[-1] <= tokens))
    if not ok:
        end = f"T = {tokens}" if exact else f"at most T = {tokens}"
        raise Unsupported(f"{op}: {what} must go from 0 to {end} without decreasing, got {cu}")
    return _offsets(host, device, op, what)


# ------------------------------------------------------------------------------------------
# Attention
# ------------------------------------------------------------------------------------------

def _attention_desc(op, q, k, v, mask: AttentionMask, options: AttentionOptions, keep):
    if q.dim() != 4:
        raise Unsupported(f"{op}: query is [B, Tq, Hq, D]")
    if k.dim() != 4:
        raise Unsupported(f"{op}: key is [B, Tk, Hkv, D]")
    b, tq, hq, d = q.shape
    bk, tk, hkv, dk = k.shape
    if tuple(k.shape) != tuple(v.shape):
        raise Unsupported(f"{op}: key and value must have one shape")
    if b != bk:
        raise Unsupported(f"{op}: query and key must have one batch size")
    if d != dk:
        raise Unsupported(f"{op}: query and key must have one head dimension")
    if hkv == 0 or hq % hkv != 0:
        raise Unsupported(f"{op}: the query heads ({hq}) must be a multiple of the key-value "
                          f"heads ({hkv})")
    if not (q.dtype == k.dtype == v.dtype):
        raise Unsupported(f"{op}: query, key and value must share one dtype")
    desc = _lib.AttentionDesc(b=b, tq=tq, tk=tk, hq=hq, hkv=hkv, d=d, dtype=_dtype(op, q),
                              mask_kind=_lib.DM_MASK_NONE)
    if mask.kind == AttentionMask.KEY_PADDING:
        pad = torch.as_tensor(mask.padding)
        if tuple(pad.shape) != (b, tk):
            raise Unsupported(f"{op}: the key padding mask is [B, Tk] = [{b}, {tk}]")
        pad = pad.to(device=q.device, dtype=torch.uint8).contiguous()
        keep.append(pad)
        desc.mask_kind, desc.key_padding = _lib.DM_MASK_KEY_PADDING, pad.data_ptr()
    elif mask.kind == AttentionMask.PACKED:
        cq, ck = torch.as_tensor(mask.cu_seqlens_q), torch.as_tensor(mask.cu_seqlens_k)
        if b != 1:
            raise Unsupported(f"{op}: packed sequences lie along the time, B = 1")
        if cq.dim() != 1 or ck.dim() != 1 or cq.shape != ck.shape or cq.shape[0] < 1:
            raise Unsupported(f"{op}: cu_seqlens_q and cu_seqlens_k are [S + 1], one S, got "
                              f"{list(cq.shape)}, {list(ck.shape)}")
        cq = _cu_seqlens(op, cq, q.device, tq, exact=False, what="cu_seqlens_q")
        ck = _cu_seqlens(op, ck, q.device, tk, exact=False, what="cu_seqlens_k")
        keep += [cq, ck]
        desc.mask_kind = _lib.DM_MASK_PACKED
        desc.cu_seqlens_q, desc.cu_seqlens_k = cq.data_ptr(), ck.data_ptr()
        desc.nseq = cq.shape[0] - 1
    o = desc.options
    o.causal = int(bool(options.causal))
    o.has_scale = int(options.scale is not None)
    o.scale = float(options.scale) if options.scale is not None else 0.0
    o.has_window = int(options.window is not None)
    if options.window is not None:
        o.window_left = min(int(options.window.left), UNBOUNDED)
        o.window_right = min(int(options.window.right), UNBOUNDED)
    o.deterministic = int(bool(options.deterministic))
    return desc


def attention_with_lse(query, key, value, mask: Optional[AttentionMask] = None,
                       options: Optional[AttentionOptions] = None):
    """``(output [B, Tq, Hq, D] in the queries' dtype, lse [B, Tq, Hq] f32)``
    (crates/dash-ops/src/attention.rs:660)."""
    op = "attention"
    mask = mask or AttentionMask.none()
    options = options or AttentionOptions()
    _device(op, query, key, value)
    keep = []
    desc = _attention_desc(op, query, key, value, mask, options, keep)
    q, k, v = _readable(query), _readable(key), _readable(value)
    desc.strided = 1
    for f, t in ((desc.sq, q), (desc.sk, k), (desc.sv, v)):
        _set_strides(f, t, (0, 1, 2))
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    nbytes = _lib.lib().dm_attention_fwd_workspace(ctypes.byref(desc))
    ws = _workspace(nbytes, q.device)
    _check(op, _lib.lib().dm_attention_fwd(ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v),
                                           _ptr(out), _ptr(lse), _ptr(ws), nbytes, _stream()))
    return out, lse


def attention(query, key, value, mask=None, options=None):
    """The output alone (attention.rs:648)."""
    return attention_with_lse(query, key, value, mask, options)[0]


def attention_backward(query, key, value, output, lse, grad_output, mask=None, options=None):
    """``(dq, dk, dv)`` in their inputs' dtype and shape, from the forward's output and lse
    (attention.rs:689). The output's gradient is read in the output's dtype."""
    op = "attention_backward"
    mask = mask or AttentionMask.none()
    options = options or AttentionOptions()
    _device(op, query, key, value, output, lse, grad_output)
    keep = []
    desc = _attention_desc(op, query, key, value, mask, options, keep)
    if tuple(output.shape) != tuple(query.shape) or tuple(grad_output.shape) != tuple(query.shape):
        raise Unsupported(f"{op}: the output and its gradient are [B, Tq, Hq, D]")
    if tuple(lse.shape) != tuple(query.shape[:3]):
        raise Unsupported(f"{op}: the log-sum-exp is [B, Tq, Hq]")
    q, k, v = _readable(query), _readable(key), _readable(value)
    o = _readable(output.to(q.dtype))
    g = _readable(grad_output.to(q.dtype))
    ls = lse.to(torch.float32).contiguous()
    desc.strided = 1
    for f, t in ((desc.sq, q), (desc.sk, k), (desc.sv, v), (desc.so, o), (desc.sdo, g)):
        _set_strides(f, t, (0, 1, 2))
    dq, dk, dv = (torch.empty(x.shape, dtype=x.dtype, device=x.device) for x in (q, k, v))
    nbytes = _lib.lib().dm_attention_bwd_workspace(ctypes.byref(desc))
    ws = _workspace(nbytes, q.device)
    _check(op, _lib.lib().dm_attention_bwd(ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v),
                                           _ptr(o), _ptr(ls), _ptr(g), _ptr(dq), _ptr(dk),
                                           _ptr(dv), _ptr(ws), nbytes, _stream()))
    return dq, dk, dv


def attention_decode(query, key, value, lengths=None, options=None):
    """One query per sequence ``[B, Hq, D]`` against the cache ``[B, S, Hkv, D]``, sequence ``b``
    holding its first ``lengths[b]`` keys (attention.rs:732); ``[B, Hq, D]`` in the queries'
    dtype."""
    op = "attention_decode"
    options = options or AttentionOptions()
    _device(op, query, key, value)
    if query.dim() != 3:
        raise Unsupported(f"{op}: query is [B, Hq, D]")
    if key.dim() != 4:
        raise Unsupported(f"{op}: key is [B, S, Hkv, D]")
    b, hq, d = query.shape
    keep = []
    desc = _attention_desc(op, query.unsqueeze(1), key, value, AttentionMask.none(), options,
                           keep)
    ln = None
    if lengths is not None:
        lt = torch.as_tensor(lengths)
        if tuple(lt.shape) != (b,):
            raise Unsupported(f"{op}: the cache lengths are [B] = [{b}]")
        ln = _cache_lengths(op, lt, b, query.device)
    q, k, v = _readable(query), _readable(key), _readable(value)
    _decode_strides(desc, q, k, v, (0, 1, 2))
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    nbytes = _lib.lib().dm_attention_decode_workspace(ctypes.byref(desc))
    ws = _workspace(nbytes, q.device)
    _check(op, _lib.lib().dm_attention_decode(ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v),
                                              _ptr(ln), _ptr(out), _ptr(ws), nbytes, _stream()))
    return out


def _decode_desc(op, query, key, value, tk, options):
    """The descriptor of a decode over a cache whose rows are ``key.shape[-2:] = [Hkv, D]``."""
    if query.dim() != 3:
        raise Unsupported(f"{op}: query is [B, Hq, D]")
    if tuple(key.shape) != tuple(value.shape):
        raise Unsupported(f"{op}: key and value must have one shape")
    b, hq, d = query.shape
    hkv, dk = key.shape[-2], key.shape[-1]
    if d != dk:
        raise Unsupported(f"{op}: query and key must have one head dimension")
    if hkv == 0 or hq % hkv != 0:
        raise Unsupported(f"{op}: the query heads ({hq}) must be a multiple of the key-value "
                          f"heads ({hkv})")
    if not (query.dtype == key.dtype == value.dtype):
        raise Unsupported(f"{op}: query, key and value must share one dtype")
    desc = _lib.AttentionDesc(b=b, tq=1, tk=tk, hq=hq, hkv=hkv, d=d, dtype=_dtype(op, query),
                              mask_kind=_lib.DM_MASK_NONE)
    o = desc.options
    o.has_scale = int(options.scale is not None)
    o.scale = float(options.scale) if options.scale is not None else 0.0
    o.has_window = int(options.window is not None)
    if options.window is not None:
        o.window_left = min(int(options.window.left), UNBOUNDED)
        o.window_right = min(int(options.window.right), UNBOUNDED)
    return desc


def _decode_strides(desc, q, k, v, cache_dims):
    desc.strided = 1
    _set_strides(desc.sq, q, (0, None, 1))
    _set_strides(desc.sk, k, cache_dims)
    _set_strides(desc.sv, v, cache_dims)


def _cache_lengths(op, lengths, b, device):
    if lengths is None:
        return None
    lt = torch.as_tensor(lengths)
    if tuple(lt.shape) != (b,):
        raise Unsupported(f"{op}: the cache lengths are [B] = [{b}]")
    if lt.numel() and int(lt.min()) < 0:
        raise Unsupported(f"{op}: the cache lengths are not negative")
    return _offsets(lt, device, op, "the cache lengths")


def attention_decode_packed(query, key, value, cu_seqlens_k, lengths=None, options=None,
                            max_len=None):
    """Decoding against a packed cache ``key, value [N, Hkv, D]``: sequence ``b``'s keys are rows
    ``cu_seqlens_k[b] .. cu_seqlens_k[b + 1] - 1``, the first ``lengths[b]`` of them (all
    without lengths). The same operation as ``attention_decode`` (attention.rs:732) over a
    cache that keeps each sequence at an offset; ``max_len`` bounds every sequence's span (by
    default the longest span of ``cu_seqlens_k``)."""
    op = "attention_decode"
    options = options or AttentionOptions()
    _device(op, query, key, value)
    if key.dim() != 3:
        raise Unsupported(f"{op}: a packed key cache is [N, Hkv, D]")
    b = query.shape[0] if query.dim() == 3 else -1
    cu = torch.as_tensor(cu_seqlens_k)
    if cu.dim() != 1 or cu.shape[0] != b + 1:
        raise Unsupported(f"{op}: cu_seqlens_k is [B + 1] = [{b + 1}]")
    host = cu.detach().to("cpu", torch.int64)
    if b > 0 and (int(host.min()) < 0 or int(host.max()) > key.shape[0]
                  or bool((host[1:] < host[:-1]).any())):
        raise Unsupported(f"{op}: cu_seqlens_k must lie within the cache's {key.shape[0]} "
                          "rows without decreasing")
    if max_len is None:
        max_len = int((host[1:] - host[:-1]).max()) if b > 0 else 0
    desc = _decode_desc(op, query, key, value, max(int(max_len), 0), options)
    cu = _offsets(cu, query.device, op, "cu_seqlens_k")
    desc.cu_seqlens_k, desc.nseq = cu.data_ptr(), b
    ln = _cache_lengths(op, lengths, b, query.device)
    q, k, v = _readable(query), _readable(key), _readable(value)
    _decode_strides(desc, q, k, v, (None, 0, 1))
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    nbytes = _lib.lib().dm_attention_decode_workspace(ctypes.byref(desc))
    ws = _workspace(nbytes, q.device)
    _check(op, _lib.lib().dm_attention_decode(ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v),
                                              _ptr(ln), _ptr(out), _ptr(ws), nbytes, _stream()))
    return out


def attention_decode_paged(query, key_pages, value_pages, block_table, lengths=None,
                           options=None):
    """Decoding against a paged cache ``key_pages, value_pages [P, page_size, Hkv, D]``: key
    ``j`` of sequence ``b`` is row ``j % page_size`` of page ``block_table[b, j // page_size]``
    (``block_table [B, max_pages]`` int). The same operation as ``attention_decode``
    (attention.rs:732) over the dense cache this table describes; sequence ``b`` holds its
    first ``lengths[b]`` keys (all ``max_pages * page_size`` without lengths)."""
    op = "attention_decode_paged"
    options = options or AttentionOptions()
    _device(op, query, key_pages, value_pages)
    if key_pages.dim() != 4:
        raise Unsupported(f"{op}: the key pages are [P, page_size, Hkv, D]")
    b = query.shape[0] if query.dim() == 3 else -1
    bt = torch.as_tensor(block_table)
    if bt.dim() != 2 or bt.shape[0] != b:
        raise Unsupported(f"{op}: the block table is [B, max_pages] with B = {b}")
    npages, page_size = key_pages.shape[0], key_pages.shape[1]
    if page_size < 1:
        raise Unsupported(f"{op}: pages hold at least one key")
    max_pages = bt.shape[1]
    desc = _decode_desc(op, query, key_pages, value_pages, max_pages * page_size, options)
    bt = _offsets(bt, query.device, op, "the block table")
    ln = _cache_lengths(op, lengths, b, query.device)
    q, k, v = _readable(query), _readable(key_pages), _readable(value_pages)
    _decode_strides(desc, q, k, v, (0, 1, 2))
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    nbytes = _lib.lib().dm_attention_decode_paged_workspace(ctypes.byref(desc), page_size)
    ws = _workspace(nbytes, q.device)
    _check(op, _lib.lib().dm_attention_decode_paged(
        ctypes.byref(desc), _ptr(q), _ptr(k), _ptr(v), npages, page_size, _ptr(bt), max_pages,
        _ptr(ln), _ptr(out), _ptr(ws), nbytes, _stream()))
    return out


# ------------------------------------------------------------------------------------------
# Gated delta rule
# ------------------------------------------------------------------------------------------

def _gdr_desc(op, q, k, v, g, beta, cu_seqlens, qk_l2norm, scale, step, keep):
    if step:
        if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
            raise Unsupported(f"{op}: q, k and v are [B, H, D], got {list(q.shape)}, "
                              f"{list(k.shape)}, {list(v.shape)}")
        b, h, dk = q.shape
        t = 1
        dv = v.shape[2]
        if tuple(k.shape) != (b, h, dk):
            raise Unsupported(f"{op}: k must match q [B, H, Dk]")
        if tuple(v.shape[:2]) != (b, h):
            raise Unsupported(f"{op}: v must be [B, H, Dv] with q's B, H")
        if tuple(g.shape) != (b, h):
            raise Unsupported(f"{op}: g must be [B, H]")
        if tuple(beta.shape) != (b, h):
            raise Unsupported(f"{op}: beta must be [B, H]")
    else:
        if q.dim() != 4:
            raise Unsupported(f"{op}: queries are [B, T, H, Dk]")
        b, t, h, dk = q.shape
        dv = v.shape[3]
        if tuple(k.shape) != (b, t, h, dk):
            raise Unsupported(f"{op}: keys must have the queries' shape [B, T, H, Dk]")
        if tuple(v.shape) != (b, t, h, dv):
            raise Unsupported(f"{op}: values must be [B, T, H, Dv] with the queries' B, T, H")
        if tuple(g.shape) != (b, t, h):
            raise Unsupported(f"{op}: g must be [B, T, H]")
        if tuple(beta.shape) != (b, t, h):
            raise Unsupported(f"{op}: beta must be [B, T, H]")
        if t == 0:
            raise Unsupported(f"{op}: the sequence must not be empty")
    if not (q.dtype == k.dtype == v.dtype):
        raise Unsupported(f"{op}: queries, keys and values must share one dtype, got "
                          f"{q.dtype}, {k.dtype}, {v.dtype}")
    dt = _dtype(op, q)
    for name, x in (("g", g), ("beta", beta)):
        if x.dtype not in (torch.float32, q.dtype):
            raise Unsupported(f"{op}: {name} must be f32 or the queries' dtype")
    desc = _lib.GdrDesc(b=b, t=t, h=h, dk=dk, dv=dv, dtype=dt, g_dtype=_DT[g.dtype],
                        beta_dtype=_DT[beta.dtype], qk_l2norm=int(bool(qk_l2norm)),
                        has_scale=int(scale is not None),
                        scale=float(scale) if scale is not None else 0.0)
    nseq = b
    if cu_seqlens is not None:
        cu = torch.as_tensor(cu_seqlens)
        if not step and b != 1:
            raise Unsupported(f"{op}: packed sequences lie along T of a batch of one, got B = {b}")
        if cu.dim() != 1 or cu.shape[0] < 2:
            raise Unsupported(f"{op}: cu_seqlens must hold S + 1 >= 2 offsets, got "
                              f"{cu.shape[0] if cu.dim() == 1 else list(cu.shape)}")
        cu = _cu_seqlens(op, cu, q.device, t if not step else b)
        keep.append(cu)
        desc.cu_seqlens, desc.nseq = cu.data_ptr(), cu.shape[0] - 1
        nseq = cu.shape[0] - 1
    return desc, nseq, (b, t, h, dk, dv)


def chunk_gated_delta_rule(q, k, v, g, beta, initial_state=None, cu_seqlens=None,
                           options: Optional[ChunkGatedDeltaOptions] = None):
    """The chunked gated delta rule (gated_delta/chunk.rs:856): ``(out [B, T, H, Dv] in the
    queries' dtype, final states [S, H, Dk, Dv] f32 if asked else None)``."""
    op = "chunk_gated_delta_rule"
    options = options or ChunkGatedDeltaOptions()
    _device(op, q, k, v, g, beta, initial_state)
    keep = []
    desc, nseq, (b, t, h, dk, dv) = _gdr_desc(op, q, k, v, g, beta, cu_seqlens,
                                              options.qk_l2norm, options.scale, False, keep)
    if initial_state is not None and tuple(initial_state.shape) != (nseq, h, dk, dv):
        raise Unsupported(f"{op}: the initial state must be [S, H, Dk, Dv], one per sequence")
    qc, kc, vc = (_gdr_view(x, True, True) for x in (q, k, v))
    gc, bc = (_gdr_view(x, True, False) for x in (g, beta))
    _gdr_strides(desc, False, sq=qc, sk=kc, sv=vc, sg=gc, sbeta=bc)
    h0 = None if initial_state is None else initial_state.to(torch.float32).contiguous()
    out = torch.empty((b, t, h, dv), dtype=q.dtype, device=q.device)
    fin = torch.empty((nseq, h, dk, dv), dtype=torch.float32, device=q.device) \
        if options.output_final_state else None
    nbytes = _lib.lib().dm_gdr_chunk_fwd_workspace(ctypes.byref(desc))
    ws = _workspace(nbytes, q.device)
    _check(op, _lib.lib().dm_gdr_chunk_fwd(ctypes.byref(desc), _ptr(qc), _ptr(kc), _ptr(vc),
                                           _ptr(gc), _ptr(bc), _ptr(h0), _ptr(out), _ptr(fin),
                                           _ptr(ws), nbytes, _stream()))
    return out, fin


def chunk_gated_delta_rule_backward(q, k, v, g, beta, initial_state, cu_seqlens, d_out,
                                    d_final_state=None,
                                    options: Optional[ChunkGatedDeltaOptions] = None):
    """The written-out backward of :func:`chunk_gated_delta_rule` (gated_delta/chunk.rs:542-767,
    chunk/reference.rs:519-695): ``(dq, dk, dv, dg, dbeta, dh0)``, each in its input's dtype,
    ``dh0`` f32 (``None`` without an initial state)."""
    op = "chunk_gated_delta_rule_backward"
    options = options or ChunkGatedDeltaOptions()
    _device(op, q, k, v, g, beta, initial_state, d_out, d_final_state)
    keep = []
    desc, nseq, (b, t, h, dk, dv) = _gdr_desc(op, q, k, v, g, beta, cu_seqlens,
                                              options.qk_l2norm, options.scale, False, keep)
    if tuple(d_out.shape) != (b, t, h, dv):
        raise Unsupported(f"{op}: the output's gradient is [B, T, H, Dv]")
    if d_final_state is not None and tuple(d_final_state.shape) != (nseq, h, dk, dv):
        raise Unsupported(f"{op}: the final state's gradient is [S, H, Dk, Dv]")
    qc, kc, vc = (_gdr_view(x, True, True) for x in (q, k, v))
    gc, bc = (_gdr_view(x, True, False) for x in (g, beta))
    do = _gdr_view(d_out.to(q.dtype), True, True)
    _gdr_strides(desc, False, sq=qc, sk=kc, sv=vc, sg=gc, sbeta=bc, sdo=do)
    h0 = None if initial_state is None else initial_state.to(torch.float32).contiguous()
    dfin = None if d_final_state is None else d_final_state.to(torch.float32).contiguous()
    dq, dk_, dv_ = (torch.empty(x.shape, dtype=x.dtype, device=x.device) for x in (qc, kc, vc))
    dg, db = (torch.empty(x.shape, dtype=x.dtype, device=x.device) for x in (gc, bc))
    dh0 = torch.empty((nseq, h, dk, dv), dtype=torch.float32, device=q.device) \
        if initial_state is not None else None
    nbytes = _lib.lib().dm_gdr_chunk_bwd_workspace(ctypes.byref(desc))
    ws = _workspace(nbytes, q.device)
    _check(op, _lib.lib().dm_gdr_chunk_bwd(
        ctypes.byref(desc), _ptr(qc), _ptr(kc), _ptr(vc), _ptr(gc), _ptr(bc), _ptr(h0),
        _ptr(do), _ptr(dfin), _ptr(dq), _ptr(dk_), _ptr(dv_), _ptr(dg), _ptr(db), _ptr(dh0),
        _ptr(ws), nbytes, _stream()))
    return dq, dk_, dv_, dg, db, dh0


def gated_delta_step(q, k, v, g, beta, state, cu_seqlens=None,
                     options: Optional[GatedDeltaStepOptions] = None, in_place: bool = False):
    """A step of the recurrent gated delta rule (gated_delta/recurrent.rs:158): ``(out [B, H,
    Dv] in q's dtype, new states shaped as ``state`` in f32)``. With ``in_place`` the new states
    are written over ``state`` (which must then be contiguous f32), as the kernel path does when
    it owns the state (recurrent/kernel.rs:355-377)."""
    op = "gated_delta_step"
    options = options or GatedDeltaStepOptions()
    _device(op, q, k, v, g, beta, state)
    keep = []
    desc, nseq, (b, _, h, dk, dv) = _gdr_desc(op, q, k, v, g, beta, cu_seqlens,
                                              options.qk_l2norm, options.scale, True, keep)
    if tuple(state.shape) != (nseq, h, dk, dv):
        raise Unsupported(f"{op}: state must be [S, H, Dk, Dv], one per sequence")
    if state.dtype != torch.float32:
        raise Unsupported(f"{op}: the state is f32")
    qc, kc, vc = (_gdr_view(x, False, True) for x in (q, k, v))
    _gdr_strides(desc, True, sq=qc, sk=kc, sv=vc, sg=g, sbeta=beta)
    gc, bc = g, beta
    if in_place:
        if not state.is_contiguous():
            raise Unsupported(f"{op}: an in-place state must be contiguous")
        st_in = st_out = state
    else:
        st_in = state.contiguous()
        st_out = torch.empty_like(st_in)
    out = torch.empty((b, h, dv), dtype=q.dtype, device=q.device)
    _check(op, _lib.lib().dm_gdr_step(ctypes.byref(desc), _ptr(qc), _ptr(kc), _ptr(vc),
                                      _ptr(gc), _ptr(bc), _ptr(st_in), _ptr(st_out), _ptr(out),
                                      _stream()))
    return out, st_out


def gated_delta_step_backward(q, k, v, g, beta, state, cu_seqlens, d_out, d_state=None,
                              options: Optional[GatedDeltaStepOptions] = None):
    """The gradients of :func:`gated_delta_step` (what the reference's tracked step gets from
    autodiff over its reference, gated_delta/recurrent.rs:89-130): from the output's gradient
    ``d_out`` ``[B, H, Dv]`` (``None``: zeros; rounded to q's dtype, as the output is) and the new
    states' ``d_state`` (``None``: zeros), ``(dq, dk, dv, dg, dbeta, d_state_in)``, each in its
    input's dtype, ``d_state_in`` f32."""
    op = "gated_delta_step_backward"
    options = options or GatedDeltaStepOptions()
    _device(op, q, k, v, g, beta, state, d_out, d_state)
    keep = []
    desc, nseq, (b, _, h, dk, dv) = _gdr_desc(op, q, k, v, g, beta, cu_seqlens,
                                              options.qk_l2norm, options.scale, True, keep)
    if tuple(state.shape) != (nseq, h, dk, dv):
        raise Unsupported(f"{op}: state must be [S, H, Dk, Dv], one per sequence")
    if state.dtype != torch.float32:
        raise Unsupported(f"{op}: the state is f32")
    if d_out is not None and tuple(d_out.shape) != (b, h, dv):
        raise Unsupported(f"{op}: the output's gradient is [B, H, Dv]")
    if d_state is not None and tuple(d_state.shape) != (nseq, h, dk, dv):
        raise Unsupported(f"{op}: the new states' gradient is [S, H, Dk, Dv]")
    qc, kc, vc = (_gdr_view(x, False, True) for x in (q, k, v))
    do = None if d_out is None else _gdr_view(d_out.to(q.dtype), False, True)
    views = dict(sq=qc, sk=kc, sv=vc, sg=g, sbeta=beta)
    if do is not None:
        views["sdo"] = do
    _gdr_strides(desc, True, **views)
    st_in = state.contiguous()
    dst = None if d_state is None else d_state.to(torch.float32).contiguous()
    dq = torch.empty((b, h, dk), dtype=q.dtype, device=q.device)
    dk_ = torch.empty((b, h, dk), dtype=q.dtype, device=q.device)
    dv_ = torch.empty((b, h, dv), dtype=q.dtype, device=q.device)
    dg = torch.empty((b, h), dtype=g.dtype, device=q.device)
    db = torch.empty((b, h), dtype=beta.dtype, device=q.device)
    dst_in = torch.empty_like(st_in)
    nbytes = _lib.lib().dm_gdr_step_bwd_workspace(ctypes.byref(desc))
    ws = _workspace(nbytes, q.device)
    _check(op, _lib.lib().dm_gdr_step_bwd(
        ctypes.byref(desc), _ptr(qc), _ptr(kc), _ptr(vc), _ptr(g), _ptr(beta), _ptr(st_in),
        _ptr(do), _ptr(dst), _ptr(dq), _ptr(dk_), _ptr(dv_), _ptr(dg), _ptr(db), _ptr(dst_in),
        _ptr(ws), nbytes, _stream()))
    return dq, dk_, dv_, dg, db, dst_in


# ------------------------------------------------------------------------------------------
# Causal conv1d
# ------------------------------------------------------------------------------------------

def _conv1d_desc(op, x, weight, bias, states, cu_seqlens, activation, keep):
    """The descriptor of a call, after dash-ops' checks (conv1d.rs:774-820): ``x`` ``[B, T, C]``
    (or ``[B, C]`` for the step), ``weight`` ``[C, K]``, ``bias`` ``[C]``, states ``[S, W, C]``
    f32; the refusals raise :class:`Unsupported` with dash-ops' messages."""
    if x.dim() not in (2, 3):
        raise Unsupported(f"{op}: x must be [B, T, C] (or [B, C] for a step)")
    c = x.shape[-1]
    if weight.dim() != 2:
        raise Unsupported(f"{op}: weight must be [C, K]")
    wc, k = weight.shape
    if k < 1:
        raise Unsupported(f"{op}: the kernel width must be at least 1")
    if wc != c:
        raise Unsupported(f"{op}: x has {c} channels, weight [C, K] has {wc}")
    if weight.dtype != x.dtype:
        raise Unsupported(f"{op}: x and weight must share one dtype")
    if bias is not None:
        if tuple(bias.shape) != (c,):
            raise Unsupported(f"{op}: x has {c} channels, bias [C] has {tuple(bias.shape)}")
        if bias.dtype != x.dtype:
            raise Unsupported(f"{op}: x and bias must share one dtype")
    if activation not in (Activation.NONE, Activation.SILU):
        raise Unsupported(f"{op}: activation {activation} is not implemented")
    desc = _lib.Conv1dDesc()
    desc.dtype = _dtype(op, x)
    desc.c, desc.k = c, k
    desc.has_bias = int(bias is not None)
    desc.activation = _lib.DM_ACT_SILU if activation == Activation.SILU else _lib.DM_ACT_NONE
    if x.dim() == 3:
        desc.b, desc.t = x.shape[0], x.shape[1]
    else:
        desc.b, desc.t = x.shape[0], 1
    nseq = desc.b
    if cu_seqlens is not None:
        if x.shape[0] != 1:
            raise Unsupported(f"{op}: packed sequences lie along T of a batch of one, "
                              f"got B = {x.shape[0]}")
        n_off = torch.as_tensor(cu_seqlens).numel()
        if n_off < 2:
            raise Unsupported(f"{op}: cu_seqlens must hold N + 1 >= 2 offsets, got {n_off}")
        cu = _cu_seqlens(op, cu_seqlens, x.device, desc.t)
        keep.append(cu)
        desc.cu_seqlens = cu.data_ptr()
        desc.nseq = nseq = cu.numel() - 1
    for what, st in states:
        if st is None:
            continue
        if st.dim() != 3 or st.shape[0] != nseq or st.shape[2] != c:
            raise Unsupported(f"{op}: the {what} {list(st.shape)} must be [S, W, C] with "
                              f"S = {nseq} sequences and C = {c} channels")
        if st.shape[1] + 1 < k:
            raise Unsupported(f"{op}: a {what} of {st.shape[1]} steps cannot feed a kernel of "
                              f"width {k}; it needs at least {k - 1}")
        if st.dtype != torch.float32:
            raise Unsupported(f"{op}: the {what} is f32")
    return desc, nseq


def causal_conv1d(x, weight, bias=None, initial_state=None, cu_seqlens=None,
                  options: Optional[CausalConv1dOptions] = None):
    """The causal depthwise conv1d (dash-ops conv1d.rs:690, contract conv1d.rs:1-79): ``x``
    ``[B, T, C]``, ``weight`` ``[C, K]``, ``bias`` ``[C]``, ``initial_state`` ``[S, W, C]`` f32;
    returns ``(out [B, T, C] in x's dtype, final states [S, W', C] f32 or None)``."""
    op = "causal_conv1d"
    options = options or CausalConv1dOptions()
    _device(op, x, weight, bias, initial_state)
    keep = []
    desc, nseq = _conv1d_desc(op, x, weight, bias, [("initial state", initial_state)],
                              cu_seqlens, options.activation, keep)
    if initial_state is not None:
        desc.has_initial, desc.w = 1, initial_state.shape[1]
    fin = None
    if options.output_final_state:
        if options.final_state_len is not None:
            w_out = options.final_state_len
        else:
            w_out = initial_state.shape[1] if initial_state is not None else desc.k - 1
        desc.has_final, desc.w_out = 1, int(w_out)
        fin = torch.empty((nseq, int(w_out), desc.c), dtype=torch.float32, device=x.device)
    xc, wc = x.contiguous(), weight.contiguous()
    bc = None if bias is None else bias.contiguous()
    h0 = None if initial_state is None else initial_state.contiguous()
    out = torch.empty_like(xc)
    _check(op, _lib.lib().dm_causal_conv1d_fwd(ctypes.byref(desc), _ptr(xc), _ptr(wc), _ptr(bc),
                                               _ptr(h0), _ptr(out), _ptr(fin), _stream()))
    return out, fin


def causal_conv1d_backward(x, weight, bias, initial_state, cu_seqlens, grad_out,
                           grad_final_state=None, options: Optional[CausalConv1dOptions] = None):
    """The conv1d's gradients (CausalConv1dBackend::causal_conv1d_backward, conv1d.rs:300-329),
    from the output's (``grad_out``, f32 or x's dtype) and the final states' (``[S, W', C]`` f32,
    or None): ``(grad_x, grad_weight, grad_bias or None, grad_initial_state or None)``."""
    op = "causal_conv1d_backward"
    options = options or CausalConv1dOptions()
    _device(op, x, weight, bias, initial_state, grad_out, grad_final_state)
    keep = []
    desc, nseq = _conv1d_desc(op, x, weight, bias, [("initial state", initial_state)],
                              cu_seqlens, options.activation, keep)
    if tuple(grad_out.shape) != tuple(x.shape):
        raise Unsupported(f"{op}: the output's gradient must be shaped as x")
    if grad_out.dtype not in (torch.float32, x.dtype):
        raise Unsupported(f"{op}: the output's gradient is f32 or x's dtype")
    if initial_state is not None:
        desc.has_initial, desc.w = 1, initial_state.shape[1]
    if grad_final_state is not None:
        if (grad_final_state.dim() != 3 or grad_final_state.shape[0] != nseq
                or grad_final_state.shape[2] != desc.c
                or grad_final_state.dtype != torch.float32):
            raise Unsupported(f"{op}: the final states' gradient must be [S, W', C] f32")
        desc.has_final, desc.w_out = 1, grad_final_state.shape[1]
    xc, wc, gc = x.contiguous(), weight.contiguous(), grad_out.contiguous()
    bc = None if bias is None else bias.contiguous()
    h0 = None if initial_state is None else initial_state.contiguous()
    gf = None if grad_final_state is None else grad_final_state.contiguous()
    gx, gw = torch.empty_like(xc), torch.empty_like(wc)
    gb = None if bias is None else torch.empty_like(bc)
    gh = None if initial_state is None else torch.empty_like(h0)
    ws = _workspace(_lib.lib().dm_causal_conv1d_bwd_workspace(ctypes.byref(desc)), x.device)
    _check(op, _lib.lib().dm_causal_conv1d_bwd(
        ctypes.byref(desc), _ptr(xc), _ptr(wc), _ptr(bc), _ptr(h0), _ptr(gc),
        _DT[grad_out.dtype], _ptr(gf), _ptr(gx), _ptr(gw), _ptr(gb), _ptr(gh), _ptr(ws),
        ws.numel(), _stream()))
    return gx, gw, gb, gh


def causal_conv1d_update(x, weight, bias, state,
                         options: Optional[CausalConv1dStepOptions] = None,
                         in_place: bool = False):
    """One decoding step (conv1d.rs:750): ``x`` ``[B, C]``, ``state`` ``[B, W, C]`` f32 to
    ``(out [B, C] in x's dtype, next state [B, W, C] f32)``; with ``in_place`` the next state is
    written over ``state`` (which must be contiguous)."""
    op = "causal_conv1d_update"
    options = options or CausalConv1dStepOptions()
    _device(op, x, weight, bias, state)
    keep = []
    if x.dim() != 2:
        raise Unsupported(f"{op}: x must be [B, C]")
    desc, _ = _conv1d_desc(op, x, weight, bias, [("state", state)], None, options.activation,
                           keep)
    desc.w = state.shape[1]
    xc, wc = x.contiguous(), weight.contiguous()
    bc = None if bias is None else bias.contiguous()
    if in_place:
        if not state.is_contiguous():
            raise Unsupported(f"{op}: an in-place state must be contiguous")
        st_in = st_out = state
    else:
        st_in = state.contiguous()
        st_out = torch.empty_like(st_in)
    out = torch.empty_like(xc)
    _check(op, _lib.lib().dm_causal_conv1d_update(ctypes.byref(desc), _ptr(xc), _ptr(wc),
                                                  _ptr(bc), _ptr(st_in), _ptr(out), _ptr(st_out),
                                                  _stream()))
    return out, st_out


# ------------------------------------------------------------------------------------------
# Chosen-token log-probability
# ------------------------------------------------------------------------------------------

def _masked_ids(op, masked, v):
    """The masked token ids as a list, each checked against the vocabulary here, before the
    uint32 array the C ABI takes is built (a larger id would wrap in that cast)."""
    ids = [int(i) for i in masked]
    if any(i < 0 for i in ids):
        raise Unsupported(f"{op}: masked token ids are not negative")
    for i in ids:
        if i >= v:
            raise Unsupported(f"{op}: masked token id {i} is not below the vocabulary size {v}")
    return ids


def _logprob(hidden, weight, targets, masked, options, with_grad):
    op = "chosen_logprob"
    options = options or LogprobOptions()
    _device(op, hidden, weight)
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise Unsupported(f"{op}: hidden [n, D] and weight [V, D] must share D, got "
                          f"{list(hidden.shape)}, {list(weight.shape)}")
    for t in (hidden, weight):
        if t.dtype not in (torch.bfloat16, torch.float32):
            raise Unsupported(f"{op}: the log-probability takes bf16 or f32")
    n, d = hidden.shape
    v = weight.shape[0]
    tg = torch.as_tensor(targets)
    if tuple(tg.shape) != (n,):
        raise Unsupported(f"{op}: targets must be [n] = [{n}]")
    tg = tg.to(device=hidden.device, dtype=torch.int64).contiguous()
    ids = _masked_ids(op, masked, v)
    ids_c = (ctypes.c_uint32 * max(len(ids), 1))(*ids)
    desc = _lib.LogprobDesc(n=n, v=v, d=d, hidden_dtype=_dtype(op, hidden),
                            weight_dtype=_dtype(op, weight),
                            vocab_chunk=int(options.vocab_chunk), row_chunk=int(options.row_chunk))
    h, w = hidden.contiguous(), weight.contiguous()
    lp = torch.empty(n, dtype=torch.float32, device=h.device)
    ent = torch.empty(n, dtype=torch.float32, device=h.device)
    grad = torch.empty(n, d, dtype=torch.float32, device=h.device) if with_grad else None
    nbytes = _lib.lib().dm_chosen_logprob_workspace(ctypes.byref(desc), int(with_grad))
    ws = _workspace(nbytes, h.device)
    _check(op, _lib.lib().dm_chosen_logprob(ctypes.byref(desc), _ptr(h), _ptr(w), _ptr(tg),
                                            ctypes.cast(ids_c, ctypes.c_void_p), len(ids),
                                            _ptr(lp), _ptr(ent), _ptr(grad), _ptr(ws), nbytes,
                                            _stream()))
    return lp, ent, grad


def chosen_logprob(hidden, weight, targets, masked=(), options=None):
    """``(logprob [n], entropy [n])`` f32 of ``targets`` under ``softmax(hidden weightᵀ)`` without
    the ``masked`` token ids (crates/dash-ops/src/logprob.rs:127-138; the contract's definition,
    crates/dash-contract/src/logprob.rs:4-15): ``hidden`` ``[n, D]``, ``weight`` ``[V, D]``, bf16
    or f32; a masked or out-of-range target gives ``-inf``."""
    lp, ent, _ = _logprob(hidden, weight, targets, masked, options, False)
    return lp, ent


def chosen_logprob_with_grad(hidden, weight, targets, masked=(), options=None):
    """``(logprob, entropy, grad [n, D] f32)``, ``grad[i]`` the gradient of ``logprob[i]`` with
    respect to ``hidden[i]`` (logprob.rs:140-160); the backward of the log-probability is
    ``upstream[:, None] * grad``, cast to ``hidden``'s dtype (logprob.rs:160-190)."""
    return _logprob(hidden, weight, targets, masked, options, True)


# ------------------------------------------------------------------------------------------
# Fused linear cross-entropy
# ------------------------------------------------------------------------------------------

_LCE_ROWS = ("loss", "logprob", "entropy", "lse", "q", "s", "counted", "found")


def _lce_desc(op, hidden, weight, targets, options):
    _device(op, hidden, weight)
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise Unsupported(f"{op}: hidden [n, D] and weight [V, D] must share D, got "
                          f"{list(hidden.shape)}, {list(weight.shape)}")
    if hidden.dtype != weight.dtype:
        raise Unsupported(f"{op}: hidden and weight share one dtype")
    n, d = hidden.shape
    tg = torch.as_tensor(targets)
    if tuple(tg.shape) != (n,):
        raise Unsupported(f"{op}: targets must be [n] = [{n}]")
    tg = tg.to(device=hidden.device, dtype=torch.int64).contiguous()
    ids = _masked_ids(op, options.masked, weight.shape[0])
    ids_c = (ctypes.c_uint32 * max(len(ids), 1))(*ids)
    dt = _dtype(op, hidden)
    lp = _lib.LogprobDesc(n=n, v=weight.shape[0], d=d, hidden_dtype=dt, weight_dtype=dt,
                          vocab_chunk=int(options.chunks.vocab_chunk),
                          row_chunk=int(options.chunks.row_chunk))
    desc = _lib.LceDesc(lp=lp, ignore_index=int(options.ignore_index),
                        label_smoothing=float(options.label_smoothing),
                        z_loss=float(options.z_loss), entropy=int(bool(options.entropy)))
    return desc, tg, ids_c, len(ids)


def linear_cross_entropy(hidden, weight, targets, options=None):
    """torch's ``F.cross_entropy(F.linear(hidden, weight), targets)`` with label smoothing, a
    z-loss and masked ids, without the n x V logits (crates/dash-ops/src/loss.rs:820-895;
    crates/dash-contract/src/loss.rs): ``(loss, logprob [n], entropy [n] or None, rows)``, the
    loss ``[1]`` (mean, sum) or ``[n]`` (none), all f32; ``rows`` ``[8, n]`` (loss, logprob,
    entropy, lse, q, s, counted, found) is what ``linear_cross_entropy_backward`` takes."""
    op = "linear_cross_entropy"
    options = options or CrossEntropyOptions()
    desc, tg, ids_c, nid = _lce_desc(op, hidden, weight, targets, options)
    h, w = hidden.contiguous(), weight.contiguous()
    n = h.shape[0]
    rows = torch.zeros(len(_LCE_ROWS), n, dtype=torch.float32, device=h.device)
    nbytes = _lib.lib().dm_linear_cross_entropy_workspace(ctypes.byref(desc), 0)
    ws = _workspace(nbytes, h.device)
    _check(op, _lib.lib().dm_linear_cross_entropy_fwd(
        ctypes.byref(desc), _ptr(h), _ptr(w), _ptr(tg), ctypes.cast(ids_c, ctypes.c_void_p), nid,
        _ptr(rows), _ptr(ws), nbytes, _stream()))
    if options.reduction == Reduction.NONE:
        loss = rows[0]
    elif options.reduction == Reduction.SUM:
        loss = rows[0].sum().reshape(1)
    else:  # the mean over the counted rows (NaN when every row is ignored, as torch)
        loss = (rows[0].sum() / rows[6].sum()).reshape(1)
    return loss, rows[1], (rows[2] if options.entropy else None), rows


def linear_cross_entropy_backward(hidden, weight, targets, rows, upstream, options=None,
                                  grad_hidden=True, grad_weight=True):
    """The gradients for ``hidden`` and ``weight`` (crates/dash-ops/src/loss.rs:157-200,
    :527-668): ``upstream`` ``[3, n]`` f32 holds the gradients of the loss, logprob and entropy
    rows (for a reduced loss: the mean's 1 / counted or the sum's 1 on each row). Returns
    ``(grad_hidden, grad_weight)`` in the inputs' dtype, each None when not asked for."""
    op = "linear_cross_entropy"
    options = options or CrossEntropyOptions()
    desc, tg, ids_c, nid = _lce_desc(op, hidden, weight, targets, options)
    h, w = hidden.contiguous(), weight.contiguous()
    up = torch.as_tensor(upstream, dtype=torch.float32).to(h.device).contiguous()
    if tuple(up.shape) != (3, h.shape[0]):
        raise Unsupported(f"{op}: upstream is [3, n]")
    gh = torch.empty_like(h) if grad_hidden else None
    gw = torch.empty_like(w) if grad_weight else None
    nbytes = _lib.lib().dm_linear_cross_entropy_workspace(ctypes.byref(desc),
                                                          1 if grad_weight else 2)
    ws = _workspace(nbytes, h.device)
    _check(op, _lib.lib().dm_linear_cross_entropy_bwd(
        ctypes.byref(desc), _ptr(h), _ptr(w), _ptr(tg), ctypes.cast(ids_c, ctypes.c_void_p), nid,
        _ptr(rows.contiguous()), _ptr(up), _ptr(gh), _ptr(gw), _ptr(ws), nbytes, _stream()))
    return gh, gw
