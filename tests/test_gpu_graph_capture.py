"""The hot path under HIP graph capture: callers that replay a captured step (serving loops,
training steps under torch.cuda.graphs) call the C ABI with descriptors and workspaces prepared
beforehand, on the capturing stream. Each op is run eagerly once (the library's one-time set-up:
kernel attributes), captured, then the graph is replayed several times with other device work and
synchronisations between the replays; every replay must equal the eager call to the bit (the
kernels are deterministic and none of them records a memset)."""
import ctypes

import pytest
import torch

import dashmag_amd as dm
from dashmag_amd import _lib, ops, synthetic as syn

pytestmark = pytest.mark.gpu


def _check(rc, lib):
    assert rc == 0, lib.dm_last_error().decode()


def _replays(fn, outs, n=3):
    """Eager outputs, then n graph replays of fn compared with them bit for bit."""
    fn()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    for o in outs:
        o.fill_(float("nan")) if o.is_floating_point() else o.zero_()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            fn()
    torch.cuda.synchronize()
    for r in range(n):
        for o in outs:
            o.fill_(float("nan")) if o.is_floating_point() else o.zero_()
        junk = torch.randn(1 << 20, device="cuda") * (r + 1)  # other device work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, e in zip(outs, eager):
            assert torch.equal(a, e), f"replay {r} differs"
        del junk


def test_attention_fwd_bwd_packed_graph():
    lib = _lib.lib()
    c = syn.config2("cuda", total=2048)
    q, k, v, do, cu = c["q"], c["k"], c["v"], c["do"], c["cu_seqlens"]
    keep = []
    mask = dm.AttentionMask.packed(cu, cu)
    desc = ops._attention_desc("attention", q, k, v, mask, dm.AttentionOptions(causal=True), keep)
    o, lse = torch.empty_like(q), torch.empty(q.shape[:3], dtype=torch.float32, device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    nb = max(lib.dm_attention_fwd_workspace(ctypes.byref(desc)),
             lib.dm_attention_bwd_workspace(ctypes.byref(desc)), 1)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    P = [ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, o, lse, do, dq, dk, dv, ws)]

    def fn():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _check(lib.dm_attention_fwd(ctypes.byref(desc), P[0], P[1], P[2], P[3], P[4], P[9], nb, st), lib)
        _check(lib.dm_attention_bwd(ctypes.byref(desc), P[0], P[1], P[2], P[3], P[4], P[5], P[6],
                                    P[7], P[8], P[9], nb, st), lib)

    _replays(fn, [o, lse, dq, dk, dv])


def test_attention_fwd_bwd_d256_graph():
    """Head width 256 (the reference's shape, Hq = 8, Hkv = 2, causal): the backward's dV and dK
    passes in one launch, split over the query heads, their partials added by a second kernel."""
    lib = _lib.lib()
    t, hq, hkv, d = 1024, 8, 2, 256
    q = syn.normal(41, (1, t, hq, d), "cuda").to(torch.bfloat16)
    k = syn.normal(42, (1, t, hkv, d), "cuda").to(torch.bfloat16)
    v = syn.normal(43, (1, t, hkv, d), "cuda").to(torch.bfloat16)
    do = syn.normal(44, (1, t, hq, d), "cuda").to(torch.bfloat16)
    keep = []
    desc = ops._attention_desc("attention", q, k, v, dm.AttentionMask.none(),
                               dm.AttentionOptions(causal=True), keep)
    o, lse = torch.empty_like(q), torch.empty(q.shape[:3], dtype=torch.float32, device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    nb = max(lib.dm_attention_fwd_workspace(ctypes.byref(desc)),
             lib.dm_attention_bwd_workspace(ctypes.byref(desc)), 1)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    P = [ctypes.c_void_p(x.data_ptr()) for x in (q, k, v, o, lse, do, dq, dk, dv, ws)]

    def fn():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _check(lib.dm_attention_fwd(ctypes.byref(desc), P[0], P[1], P[2], P[3], P[4], P[9], nb, st), lib)
        _check(lib.dm_attention_bwd(ctypes.byref(desc), P[0], P[1], P[2], P[3], P[4], P[5], P[6],
                                    P[7], P[8], P[9], nb, st), lib)

    _lib.probe_reset()
    _replays(fn, [o, lse, dq, dk, dv])
    assert _lib.probe_counts()["attn_bwd_mfma"] > 0


def test_gdr_chunk_fwd_bwd_graph():
    lib = _lib.lib()
    c = syn.config4("cuda", total=3000, nseq=3)
    keep = []
    args_t = [c[x] for x in ("q", "k", "v", "g", "beta")]
    desc, _, _ = ops._gdr_desc("chunk_gated_delta_rule", *args_t, c["cu_seqlens"], False, None,
                               False, keep)
    out, fin = torch.empty_like(c["v"]), torch.empty_like(c["h0"])
    dq, dk, dv = (torch.empty_like(x) for x in args_t[:3])
    dg, db, dh0 = torch.empty_like(c["g"]), torch.empty_like(c["beta"]), torch.empty_like(c["h0"])
    nf = max(lib.dm_gdr_chunk_fwd_workspace(ctypes.byref(desc)), 1)
    nbw = max(lib.dm_gdr_chunk_bwd_workspace(ctypes.byref(desc)), 1)
    wf = torch.empty(nf, dtype=torch.uint8, device="cuda")
    wb = torch.empty(nbw, dtype=torch.uint8, device="cuda")
    p = [ctypes.c_void_p(x.data_ptr()) for x in args_t + [c["h0"], out, fin, wf]]
    pb = [ctypes.c_void_p(x.data_ptr()) for x in
          args_t + [c["h0"], c["do"], fin, dq, dk, dv, dg, db, dh0, wb]]

    def fn():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _check(lib.dm_gdr_chunk_fwd(ctypes.byref(desc), *p[:8], p[8], nf, st), lib)
        _check(lib.dm_gdr_chunk_bwd(ctypes.byref(desc), *pb[:14], pb[14], nbw, st), lib)

    _lib.probe_reset()
    _replays(fn, [out, fin, dq, dk, dv, dg, db, dh0])
    pc = _lib.probe_counts()
    assert pc["gdr_chunk_fwd_mfma"] > 0 and pc["gdr_chunk_bwd_mfma"] > 0, pc


def test_decode_graph():
    lib = _lib.lib()
    c = syn.config3("cuda", b=8, s=2048, lo=100)
    q, k, v, lens = c["q"], c["k"], c["v"], c["lengths"]
    keep = []
    desc = ops._attention_desc("attention_decode", q.unsqueeze(1), k, v, dm.AttentionMask.none(),
                               dm.AttentionOptions(), keep)
    o = torch.empty_like(q)
    nb = max(lib.dm_attention_decode_workspace(ctypes.byref(desc)), 1)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    P = [ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, lens, o, ws)]

    def fn():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _check(lib.dm_attention_decode(ctypes.byref(desc), *P[:5], P[5], nb, st), lib)

    _replays(fn, [o])


def _into(bufs):
    """Copies of an op's outputs into buffers made once, so that a captured op's outputs (new
    tensors in the graph's pool) are compared across replays through fixed tensors."""
    def put(*outs):
        for b, o in zip(bufs, outs):
            if o is not None:
                b.copy_(o)
    return put


def test_conv1d_fwd_bwd_update_graph():
    """The conv1d forward (final states in its launch), backward (initial states' gradient in
    its launch, then the segments' sums) and decoding step, batched (no offsets to check on the
    host), with bias, SiLU and states."""
    b, t, c, k, w = 3, 700, 256, 4, 3
    x = syn.normal(11, (b, t, c), "cuda").to(torch.bfloat16)
    wt = (syn.normal(12, (c, k), "cuda") * 0.5).to(torch.bfloat16)
    bias = syn.normal(13, (c,), "cuda").to(torch.bfloat16)
    h0 = syn.normal(14, (b, w, c), "cuda")
    go = syn.normal(15, (b, t, c), "cuda").to(torch.bfloat16)
    gf = syn.normal(16, (b, w, c), "cuda")
    xs = syn.normal(17, (b, c), "cuda").to(torch.bfloat16)
    opts = dm.CausalConv1dOptions(activation=dm.Activation.SILU).with_final_state_len(w)
    step = dm.contract.CausalConv1dStepOptions.from_sequence(opts)
    bufs = [torch.empty_like(x), torch.empty((b, w, c), device="cuda"), torch.empty_like(x),
            torch.empty_like(wt), torch.empty_like(bias), torch.empty_like(h0),
            torch.empty_like(xs), torch.empty_like(h0)]
    put = _into(bufs)

    def fn():
        out, fin = dm.causal_conv1d(x, wt, bias, h0, None, opts)
        grads = dm.causal_conv1d_backward(x, wt, bias, h0, None, go, gf, opts)
        ys, hs = dm.causal_conv1d_update(xs, wt, bias, h0, step)
        put(out, fin, *grads, ys, hs)

    _lib.probe_reset()
    _replays(fn, bufs)
    pc = _lib.probe_counts()
    assert pc["conv1d_fwd"] > 0 and pc["conv1d_bwd"] > 0, pc


def test_gdr_step_fwd_bwd_graph():
    """The recurrent step out of place and its backward (per-slice sums, then the finishing
    pass), batched, with the l2 normalisation."""
    c = syn.config5("cuda", b=16, h=4)
    args = [c[x] for x in ("q", "k", "v", "g", "beta")]
    st = c["state"]
    do = syn.normal(21, tuple(c["v"].shape), "cuda").to(torch.bfloat16)
    dst = syn.normal(22, tuple(st.shape), "cuda", std=0.1)
    opts = dm.GatedDeltaStepOptions().with_qk_l2norm(True)
    bufs = [torch.empty_like(c["v"]), torch.empty_like(st)] + \
        [torch.empty_like(x) for x in args] + [torch.empty_like(st)]
    put = _into(bufs)

    def fn():
        out, st_out = dm.gated_delta_step(*args, st, None, opts)
        grads = dm.gated_delta_step_backward(*args, st, None, do, dst, opts)
        put(out, st_out, *grads)

    _replays(fn, bufs)
