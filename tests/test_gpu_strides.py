"""Strided inputs read in place (crates/dash-ops/src/attention.rs:85-93, attention/cube.rs:428-461):
q, k and v as slices of one fused projection [B, T, (Hq + 2 Hkv) D], and as [B, H, T, D] tensors
seen through a permutation; the output's gradient as a view; decode caches as views. The kernels
run the same arithmetic in the same order on the same values, so every strided call must equal
the contiguous call to the bit, and the launch probes show that the fast kernels ran (no copy to
a contiguous layout is made: the views' strides are multiples of 16 bytes)."""
import pytest
import torch

import dashmag_amd as dm
from dashmag_amd import _lib, synthetic as syn

pytestmark = pytest.mark.gpu


def _fused(b, t, hq, hkv, d, seed, dtype):
    qkv = syn.normal(seed, (b, t, (hq + 2 * hkv) * d), "cuda").to(dtype)
    q = qkv[..., :hq * d].unflatten(-1, (hq, d))
    k = qkv[..., hq * d:(hq + hkv) * d].unflatten(-1, (hkv, d))
    v = qkv[..., (hq + hkv) * d:].unflatten(-1, (hkv, d))
    return q, k, v


def _bhtd(b, t, h, d, seed, dtype):
    return syn.normal(seed, (b, h, t, d), "cuda").to(dtype).permute(0, 2, 1, 3)


def _both(q, k, v, do, mask, opts):
    out = []
    for args in ((q, k, v, do), tuple(x.contiguous() for x in (q, k, v, do))):
        o, lse = dm.attention_with_lse(*args[:3], mask, opts)
        g = dm.attention_backward(*args[:3], o, lse, args[3], mask, opts)
        out.append((o, lse) + g)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [128, 64, 256])
def test_fused_projection_slices(dtype, d):
    b, t, hq, hkv = 2, 300, 8, 2
    q, k, v = _fused(b, t, hq, hkv, d, 5, dtype)
    assert not q.is_contiguous() and q.stride()[1] == (hq + 2 * hkv) * d
    do = _bhtd(b, t, hq, d, 9, dtype)
    opts = dm.AttentionOptions(causal=True)
    _lib.probe_reset()
    strided, contig = _both(q, k, v, do, None, opts)
    pc = _lib.probe_counts()
    assert pc["attn_fwd_generic"] == 0 and pc["attn_bwd_generic"] == 0, pc
    for a, e in zip(strided, contig):
        assert torch.equal(a, e)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bhtd_permutations_packed(dtype):
    lens = [70, 1, 200, 33]
    cu = torch.tensor([0, 70, 71, 271, 304], dtype=torch.int32, device="cuda")
    t, hq, hkv, d = sum(lens), 4, 2, 128
    q, k, v = (_bhtd(1, t, h, d, s, dtype) for h, s in ((hq, 1), (hkv, 2), (hkv, 3)))
    do = _bhtd(1, t, hq, d, 4, dtype)
    mask = dm.AttentionMask.packed(cu, cu)
    opts = dm.AttentionOptions(causal=True, window=dm.Window(50, 0))
    strided, contig = _both(q, k, v, do, mask, opts)
    for a, e in zip(strided, contig):
        assert torch.equal(a, e)


def test_unaligned_views_are_copied_and_still_match():
    """A view whose strides are not multiples of 16 bytes is copied by the host mirror (as the
    reference copies what its kernels cannot read in place): same results."""
    b, t, h, d = 1, 130, 2, 128
    base = syn.normal(7, (b, t, h * d + 4), "cuda").bfloat16()
    q = base[..., 4:].unflatten(-1, (h, d))  # offset by 8 bytes
    k = syn.normal(8, (b, t, h, d), "cuda").bfloat16()
    v = syn.normal(9, (b, t, h, d), "cuda").bfloat16()
    do = syn.normal(10, (b, t, h, d), "cuda").bfloat16()
    strided, contig = _both(q, k, v, do, None, dm.AttentionOptions(causal=True))
    for a, e in zip(strided, contig):
        assert torch.equal(a, e)


@pytest.mark.parametrize("d", [128, 64])
def test_decode_cache_views(d):
    b, s, hq, hkv = 6, 1000, 8, 2
    q = syn.normal(1, (b, 2 * hq, d), "cuda").bfloat16()[:, ::2]  # every other head: h stride 2D
    kc = syn.normal(2, (b, hkv, s, d), "cuda").bfloat16().transpose(1, 2)  # [B, S, Hkv, D] view
    vc = syn.normal(3, (b, hkv, s, d), "cuda").bfloat16().transpose(1, 2)
    lens = torch.tensor([1000, 1, 517, 0, 999, 64], dtype=torch.int32, device="cuda")
    _lib.probe_reset()
    o1 = dm.attention_decode(q, kc, vc, lens)
    assert _lib.probe_counts()["decode_split"] > 0
    o2 = dm.attention_decode(q.contiguous(), kc.contiguous(), vc.contiguous(), lens)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    if d == 128:
        # the paged form: pages of 16 keys as [P, Hkv, 16, D] permuted to [P, 16, Hkv, D]
        ps, npg = 16, (s + 15) // 16
        kpad = torch.zeros(b, npg * ps, hkv, d, dtype=kc.dtype, device="cuda")
        vpad = torch.zeros_like(kpad)
        kpad[:, :s], vpad[:, :s] = kc, vc
        kp = kpad.reshape(b * npg, ps, hkv, d).permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
        vp = vpad.reshape(b * npg, ps, hkv, d).permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
        table = torch.arange(b * npg, dtype=torch.int32, device="cuda").reshape(b, npg)
        o3 = dm.attention_decode_paged(q, kp, vp, table, lens)
        o4 = dm.attention_decode_paged(q.contiguous(), kp.contiguous(), vp.contiguous(), table,
                                       lens)
        torch.cuda.synchronize()
        assert torch.equal(o3, o4)


def test_decode_packed_cache_view():
    b, s, hq, hkv, d = 4, 300, 8, 2, 128
    q = syn.normal(11, (b, hq, d), "cuda").bfloat16()
    kv = syn.normal(12, (b * s, 2, hkv, d), "cuda").bfloat16()  # keys and values interleaved
    k, v = kv[:, 0], kv[:, 1]
    cu = torch.arange(b + 1, dtype=torch.int32, device="cuda") * s
    o1 = dm.attention_decode_packed(q, k, v, cu)
    o2 = dm.attention_decode_packed(q, k.contiguous(), v.contiguous(), cu)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def _gdr_inputs(t, h, dk, dv, dtype, seed, fused=True):
    """q, k, v as slices of one fused projection [1, T, H (2 Dk + Dv)] (or [1, H, T, D]
    permutations), g and beta as slices of one [1, T, 2 H] f32 tensor."""
    if fused:
        qkv = syn.normal(seed, (1, t, h * (2 * dk + dv)), "cuda").to(dtype)
        q = qkv[..., :h * dk].unflatten(-1, (h, dk))
        k = qkv[..., h * dk:2 * h * dk].unflatten(-1, (h, dk))
        v = qkv[..., 2 * h * dk:].unflatten(-1, (h, dv))
    else:
        q = syn.normal(seed, (1, h, t, dk), "cuda").to(dtype).transpose(1, 2)
        k = syn.normal(seed + 1, (1, h, t, dk), "cuda").to(dtype).transpose(1, 2)
        v = syn.normal(seed + 2, (1, h, t, dv), "cuda").to(dtype).transpose(1, 2)
    gb = syn.normal(seed + 3, (1, t, 2 * h), "cuda")
    gb = torch.cat([-torch.nn.functional.softplus(gb[..., :h]), torch.sigmoid(gb[..., h:])], -1)
    return q, k, v, gb[..., :h], gb[..., h:]


@pytest.mark.parametrize("dtype,fused", [(torch.bfloat16, True), (torch.bfloat16, False),
                                         (torch.float32, True), (torch.float32, False)])
def test_gdr_chunk_views(dtype, fused):
    lens = [70, 1, 200, 64]
    cu = torch.tensor([0, 70, 71, 271, 335], dtype=torch.int32, device="cuda")
    t, h, d = sum(lens), 2, 128 if dtype != torch.float32 else 32
    q, k, v, g, beta = _gdr_inputs(t, h, d, d, dtype, 31, fused)
    assert not q.is_contiguous() and not g.is_contiguous()
    h0 = syn.normal(37, (len(lens), h, d, d), "cuda", std=0.1)
    do = syn.normal(38, (1, h, t, d), "cuda").to(dtype).transpose(1, 2)
    opts = dm.ChunkGatedDeltaOptions(qk_l2norm=True, output_final_state=True)
    _lib.probe_reset()
    r1 = dm.chunk_gated_delta_rule(q, k, v, g, beta, h0, cu, opts)
    b1 = dm.chunk_gated_delta_rule_backward(q, k, v, g, beta, h0, cu, do, None, opts)
    if dtype != torch.float32:
        pc = _lib.probe_counts()
        assert pc["gdr_chunk_fwd_mfma"] > 0 and pc["gdr_chunk_bwd_mfma"] > 0, pc
    c = [x.contiguous() for x in (q, k, v, g, beta)]
    r2 = dm.chunk_gated_delta_rule(*c, h0, cu, opts)
    b2 = dm.chunk_gated_delta_rule_backward(*c, h0, cu, do.contiguous(), None, opts)
    torch.cuda.synchronize()
    for a_, e_ in zip(list(r1) + list(b1), list(r2) + list(b2)):
        assert torch.equal(a_, e_)


def test_gdr_step_views():
    b, h, d = 5, 3, 128
    x = syn.normal(41, (b, 3 * h, d), "cuda").bfloat16()
    q, k, v = x[:, :h], x[:, h:2 * h], x[:, 2 * h:]
    gb = syn.normal(42, (b, 2 * h), "cuda")
    gb = torch.cat([-torch.nn.functional.softplus(gb[:, :h]), torch.sigmoid(gb[:, h:])], -1)
    g, beta = gb[:, :h], gb[:, h:]
    st = syn.normal(43, (b, h, d, d), "cuda", std=0.1)
    opts = dm.GatedDeltaStepOptions(True)
    o1, s1 = dm.gated_delta_step(q, k, v, g, beta, st, None, opts)
    o2, s2 = dm.gated_delta_step(q.contiguous(), k.contiguous(), v.contiguous(), g.contiguous(),
                                 beta.contiguous(), st, None, opts)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_gdr_chunk_refuses_misaligned_bases():
    """Through the C ABI: bf16 heads that the MFMA kernels take (multiples of 8 wide) with q's
    base 2 elements (4 bytes) past a 16-byte boundary are refused with the op's name, forward and
    backward, before any launch; the aligned call on the same data runs."""
    import ctypes
    from dashmag_amd import ops
    lib = _lib.lib()
    t, h, dk = 128, 2, 64
    buf = syn.normal(40, (t * h * dk + 8,), "cuda").bfloat16()
    q_bad = buf[2:2 + t * h * dk].view(1, t, h, dk)
    k = syn.normal(41, (1, t, h, dk), "cuda").bfloat16()
    v = syn.normal(42, (1, t, h, dk), "cuda").bfloat16()
    g = -torch.nn.functional.softplus(syn.normal(43, (1, t, h), "cuda"))
    beta = torch.sigmoid(syn.normal(44, (1, t, h), "cuda"))
    desc, _, _ = ops._gdr_desc("chunk_gated_delta_rule", q_bad, k, v, g, beta, None, True, None,
                               False, [])
    out = torch.empty_like(v)
    dq, dk_, dv = torch.empty_like(k), torch.empty_like(k), torch.empty_like(v)
    dg, db = torch.empty_like(g), torch.empty_like(beta)
    nf = lib.dm_gdr_chunk_fwd_workspace(ctypes.byref(desc))
    nb = lib.dm_gdr_chunk_bwd_workspace(ctypes.byref(desc))
    ws = torch.empty(max(nf, nb, 1), dtype=torch.uint8, device="cuda")
    p = lambda x: ctypes.c_void_p(None if x is None else x.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.probe_reset()
    rc = lib.dm_gdr_chunk_fwd(ctypes.byref(desc), p(q_bad), p(k), p(v), p(g), p(beta), p(None),
                              p(out), p(None), p(ws), ws.numel(), st)
    assert rc == _lib.DM_ERR_REFUSED
    assert _lib.last_error().startswith("chunk_gated_delta_rule: "), _lib.last_error()
    rc = lib.dm_gdr_chunk_bwd(ctypes.byref(desc), p(q_bad), p(k), p(v), p(g), p(beta), p(None),
                              p(out), p(None), p(dq), p(dk_), p(dv), p(dg), p(db), p(None), p(ws),
                              ws.numel(), st)
    assert rc == _lib.DM_ERR_REFUSED
    assert _lib.last_error().startswith("chunk_gated_delta_rule_backward: "), _lib.last_error()
    assert _lib.probe_counts()["gdr_chunk_fwd"] == 0
    # the operations copy such a view and run
    o, _ = dm.chunk_gated_delta_rule(q_bad, k, v, g, beta, None, None,
                                     dm.ChunkGatedDeltaOptions(qk_l2norm=True))
    o2, _ = dm.chunk_gated_delta_rule(q_bad.contiguous(), k, v, g, beta, None, None,
                                      dm.ChunkGatedDeltaOptions(qk_l2norm=True))
    assert torch.equal(o, o2)
