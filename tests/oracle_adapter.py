"""The CPU oracle (``oracle/``) behind the conformance adapter interface: what dash-ops'
reference on Flex is to dash-conformance (crates/dash-ops/tests/common/adapter.rs:306), the
oracle is to these tests. Outputs are rounded to the inputs' dtype, as the reference rounds them
(reference.rs:345-347)."""
from __future__ import annotations

import numpy as np

import oracle
from conformance import (AttentionOut, ChunkGatedDeltaOut, GatedDeltaStepOut, HostTensor, as_dtype)
from dashmag_amd.contract import AttentionMask, UNBOUNDED, query_scale


def _side(x):
    return None if x is None or x >= UNBOUNDED else int(x)


class OracleAdapter:
    def __init__(self, precision="f32"):
        self.precision = precision

    def describe(self):
        return f"CPU oracle ({self.precision})"

    def has(self, dtype):
        return True

    def _call(self, call):
        m = call.mask
        mask = None
        if m.kind == AttentionMask.KEY_PADDING:
            mask = ("padding", m.padding)
        elif m.kind == AttentionMask.PACKED:
            mask = ("packed", m.cu_seqlens_q, m.cu_seqlens_k)
        o = call.options
        left, right = (None, None) if o.window is None else (_side(o.window.left),
                                                             _side(o.window.right))
        return oracle.AttentionCall(call.q.values, call.k.values, call.v.values, mask, o.causal,
                                    o.scale_for(call.q.shape[3]), left, right)

    def attention(self, call):
        dt = call.q.dtype
        c = self._call(call)
        o, lse = oracle.attention_fwd(c, self.precision)
        o_r = as_dtype(o, dt)
        grads = None
        if call.grad is not None:
            # the cotangent is rounded to the output's dtype (lib.rs:466-468); the backward
            # reads the forward's output as returned
            g = as_dtype(call.grad.values, dt).values
            dq, dk, dv = oracle.attention_bwd(c, o_r.values, lse, g, self.precision)
            grads = (as_dtype(dq, dt), as_dtype(dk, dt), as_dtype(dv, dt))
        return AttentionOut(o_r, HostTensor("f32", lse), grads)

    def attention_decode(self, call):
        o = call.options
        left = None if o.window is None else _side(o.window.left)
        out = oracle.attention_decode(call.q.values, call.k.values, call.v.values, call.lengths,
                                      left, o.scale_for(call.q.shape[2]), self.precision)
        return as_dtype(out, call.q.dtype)

    def chunk_gated_delta_rule(self, call):
        dt = call.q.dtype
        o = call.options
        dk = call.q.shape[3]
        scale = query_scale(o.scale, dk)
        h0 = None if call.initial_state is None else call.initial_state.values
        args = [call.q.values, call.k.values, call.v.values, call.g.values, call.beta.values]
        out, fin = oracle.gdr_chunk_fwd(*args, h0=h0, cu=call.cu_seqlens, l2norm=o.qk_l2norm,
                                        scale=scale, precision=self.precision)
        grads = None
        if call.grad is not None:
            d_out, d_fin = call.grad
            r = oracle.gdr_chunk_bwd(*args, h0, d_out.values,
                                     None if d_fin is None else d_fin.values, cu=call.cu_seqlens,
                                     l2norm=o.qk_l2norm, scale=scale, precision=self.precision)
            grads = {"q": as_dtype(r[0], dt), "k": as_dtype(r[1], call.k.dtype),
                     "v": as_dtype(r[2], call.v.dtype), "g": as_dtype(r[3], call.g.dtype),
                     "beta": as_dtype(r[4], call.beta.dtype),
                     "initial_state": None if h0 is None else HostTensor("f32", r[5])}
        return ChunkGatedDeltaOut(as_dtype(out, dt),
                                  HostTensor("f32", fin) if o.output_final_state else None, grads)

    def gated_delta_step(self, call):
        o = call.options
        scale = query_scale(o.scale, call.q.shape[2])
        args = [call.q.values, call.k.values, call.v.values, call.g.values, call.beta.values,
                call.state.values]
        out, st = oracle.gdr_step(*args, cu=call.cu_seqlens, l2norm=o.qk_l2norm, scale=scale,
                                  precision=self.precision)
        grads = None
        if call.grad is not None:
            # the output's cotangent meets the output in its dtype (the reference's cast back)
            d_out = as_dtype(call.grad[0].values, call.q.dtype).values
            r = oracle.gdr_step_bwd(*args, d_out, call.grad[1].values, cu=call.cu_seqlens,
                                    l2norm=o.qk_l2norm, scale=scale, precision=self.precision)
            grads = {"q": as_dtype(r[0], call.q.dtype), "k": as_dtype(r[1], call.k.dtype),
                     "v": as_dtype(r[2], call.v.dtype), "g": as_dtype(r[3], call.g.dtype),
                     "beta": as_dtype(r[4], call.beta.dtype), "state": HostTensor("f32", r[5])}
        return GatedDeltaStepOut(as_dtype(out, call.q.dtype), HostTensor("f32", st), grads)
