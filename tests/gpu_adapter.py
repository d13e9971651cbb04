"""The HIP library behind the conformance adapter interface: host tensors go to the GPU in
their dtype, through ``dashmag_amd``'s operations (and so through ``libdashmi.so``'s C ABI),
and back as f32 values; gradients come from the explicit backward entry points, composed as
the adapter of crates/dash-ops/tests/common/adapter.rs:594-677 composes autodiff (the loss
``sum(out * d_out) + sum(final * d_final)``)."""
from __future__ import annotations

import numpy as np
import torch

import dashmag_amd as dm
from conformance import AttentionOut, ChunkGatedDeltaOut, GatedDeltaStepOut, HostTensor
from dashmag_amd.contract import AttentionMask, Unsupported

TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
NAME = {v: k for k, v in TORCH.items()}


def dev(t: HostTensor):
    return torch.from_numpy(np.ascontiguousarray(t.values)).to("cuda").to(TORCH[t.dtype])


def host(x) -> HostTensor:
    return HostTensor(NAME[x.dtype], x.detach().float().cpu().numpy())


class GpuAdapter:
    def describe(self):
        from dashmag_amd import _lib
        return _lib.describe()

    def has(self, dtype):
        return True

    def _mask(self, m):
        if m.kind == AttentionMask.KEY_PADDING:
            return AttentionMask.key_padding(torch.as_tensor(np.asarray(m.padding)).cuda())
        if m.kind == AttentionMask.PACKED:
            return AttentionMask.packed(torch.as_tensor(np.asarray(m.cu_seqlens_q)).cuda(),
                                        torch.as_tensor(np.asarray(m.cu_seqlens_k)).cuda())
        return m

    def attention(self, call):
        q, k, v = dev(call.q), dev(call.k), dev(call.v)
        mask = self._mask(call.mask)
        out, lse = dm.attention_with_lse(q, k, v, mask, call.options)
        grads = None
        if call.grad is not None:
            g = dev(call.grad)
            dq, dk, dv = dm.attention_backward(q, k, v, out, lse, g, mask, call.options)
            grads = (host(dq), host(dk), host(dv))
        return AttentionOut(host(out), host(lse), grads)

    def attention_decode(self, call):
        lengths = None if call.lengths is None else torch.as_tensor(call.lengths).cuda()
        out = dm.attention_decode(dev(call.q), dev(call.k), dev(call.v), lengths, call.options)
        return host(out)

    def chunk_gated_delta_rule(self, call):
        q, k, v, g, beta = (dev(x) for x in (call.q, call.k, call.v, call.g, call.beta))
        h0 = None if call.initial_state is None else dev(call.initial_state)
        cu = None if call.cu_seqlens is None else torch.as_tensor(call.cu_seqlens).cuda()
        out, fin = dm.chunk_gated_delta_rule(q, k, v, g, beta, h0, cu, call.options)
        grads = None
        if call.grad is not None:
            d_out, d_fin = call.grad
            r = dm.chunk_gated_delta_rule_backward(
                q, k, v, g, beta, h0, cu, dev(d_out).to(q.dtype),
                None if d_fin is None else dev(d_fin), call.options)
            grads = {"q": host(r[0]), "k": host(r[1]), "v": host(r[2]), "g": host(r[3]),
                     "beta": host(r[4]), "initial_state": None if r[5] is None else host(r[5])}
        return ChunkGatedDeltaOut(host(out), None if fin is None else host(fin), grads)

    def gated_delta_step(self, call):
        q, k, v, g, beta, st = (dev(x) for x in (call.q, call.k, call.v, call.g, call.beta,
                                                 call.state))
        cu = None if call.cu_seqlens is None else torch.as_tensor(call.cu_seqlens).cuda()
        out, ns = dm.gated_delta_step(q, k, v, g, beta, st, cu, call.options)
        grads = None
        if call.grad is not None:
            d_out, d_state = call.grad
            r = dm.gated_delta_step_backward(q, k, v, g, beta, st, cu, dev(d_out).to(q.dtype),
                                             dev(d_state), call.options)
            grads = {"q": host(r[0]), "k": host(r[1]), "v": host(r[2]), "g": host(r[3]),
                     "beta": host(r[4]), "state": host(r[5])}
        return GatedDeltaStepOut(host(out), host(ns), grads)
