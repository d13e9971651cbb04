"""The no-allocation decode entry point (``dm_attention_decode_noalloc``, its scratch a static
device array) against ``dm_attention_decode`` with a caller's workspace, through the C ABI: the
same kernels on the same inputs, so the outputs must agree to the bit, on two calls in a row, the
second with a smaller input (the scratch keeps the first call's partials), and on a packed cache."""
import ctypes

import pytest
import torch

import dashmag_amd as dm
from dashmag_amd import _lib, ops, synthetic as syn

pytestmark = pytest.mark.gpu


def _inputs(b, s, hq, hkv, d, seed, dtype=torch.bfloat16):
    q = syn.normal(seed, (b, hq, d), "cuda").to(dtype)
    k = syn.normal(seed + 1, (b, s, hkv, d), "cuda").to(dtype)
    v = syn.normal(seed + 2, (b, s, hkv, d), "cuda").to(dtype)
    lens = (syn.uniform(seed + 3, b, "cuda") * s).to(torch.int32).clamp(min=1)
    return q, k, v, lens


def _both(q, k, v, lens, desc):
    lib = _lib.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    nbytes = lib.dm_attention_decode_workspace(ctypes.byref(desc))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    o1, o2 = torch.empty_like(q), torch.empty_like(q)
    rc = lib.dm_attention_decode(ctypes.byref(desc), p(q), p(k), p(v), p(lens), p(o1), p(ws),
                                 nbytes, st)
    assert rc == 0, _lib.last_error()
    rc = lib.dm_attention_decode_noalloc(ctypes.byref(desc), p(q), p(k), p(v), p(lens), p(o2), st)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return o1, o2, nbytes


def _desc(q, k, v):
    return ops._attention_desc("attention_decode", q.unsqueeze(1), k, v, dm.AttentionMask.none(),
                               dm.AttentionOptions(), [])


@pytest.mark.parametrize("d", [128, 64])
def test_noalloc_decode_equals_workspace_decode_twice(d):
    # config 3's shape (8 MiB of partials at D = 128), then a smaller call on the same scratch
    for b, s, hq, hkv, seed in [(64, 8192, 32, 8, 11), (5, 700, 8, 2, 12)]:
        print(f"no-alloc decode B={b} S={s} Hq={hq} Hkv={hkv} D={d}", flush=True)
        q, k, v, lens = _inputs(b, s, hq, hkv, d, seed)
        o1, o2, nbytes = _both(q, k, v, lens, _desc(q, k, v))
        assert nbytes > 0
        assert torch.equal(o1, o2)


def test_noalloc_decode_packed_cache():
    b, s, hq, hkv, d = 6, 900, 8, 2, 128
    q, k, v, lens = _inputs(b, s, hq, hkv, d, 21)
    cu = torch.arange(b + 1, dtype=torch.int32, device="cuda") * s
    kp, vp = k.reshape(b * s, hkv, d), v.reshape(b * s, hkv, d)
    desc = ops._decode_desc("attention_decode", q, kp, vp, s, dm.AttentionOptions())
    desc.cu_seqlens_k, desc.nseq = cu.data_ptr(), b
    o1, o2, _ = _both(q, kp, vp, lens, desc)
    assert torch.equal(o1, o2)
    # and the dense cache's own result, to the bit
    o3, _, _ = _both(q, k, v, lens, _desc(q, k, v))
    assert torch.equal(o1, o3)


def test_noalloc_decode_under_graph_capture():
    """An eager call first (the device's array looked up outside capture), then the call captured
    in a HIP graph and replayed three times, other device work between the replays: every replay
    equals the eager output to the bit."""
    lib = _lib.lib()
    b, s, hq, hkv, d = 8, 2048, 8, 2, 128
    q, k, v, lens = _inputs(b, s, hq, hkv, d, 31)
    desc = _desc(q, k, v)
    o = torch.empty_like(q)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def fn():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.dm_attention_decode_noalloc(ctypes.byref(desc), p(q), p(k), p(v), p(lens), p(o),
                                             st)
        assert rc == 0, _lib.last_error()

    fn()
    torch.cuda.synchronize()
    eager = o.clone()
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        with torch.cuda.graph(g, stream=cs):
            fn()
    torch.cuda.synchronize()
    for r in range(3):
        o.fill_(float("nan"))
        junk = torch.randn(1 << 20, device="cuda") * (r + 1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, eager), f"replay {r} differs"
        del junk
