"""Attention decode (attention.rs:732, reference.rs:433-467) over the shapes the split kernel
takes on MFMA (head dimensions 64/128/256, query groups 1/2/4/8, bf16/f16; a probe shows it ran) and the generic one (f32, a
group of 3), with cache lengths at the split boundaries (0, 1, a split less one, a split, a split
plus one, a ragged tail) and left windows, against the f64 oracle on the same rounded inputs.

Tolerance: relative error max|a - e| / max|e| at most 1e-2 for 16-bit inputs (f32 accumulation,
one 16-bit rounding of the output) and 1e-5 for f32; an empty cache gives exact zeros.
"""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
import oracle
from dashmag_amd import _lib
from fixtures import errors

pytestmark = pytest.mark.gpu

LENGTHS = [0, 1, 1023, 1024, 1025, 2900]


def _case(dtype, d, hkv, g, window, seed):
    gen = torch.Generator().manual_seed(seed)
    b, s = len(LENGTHS), max(LENGTHS) + 7
    q = torch.randn(b, hkv * g, d, generator=gen).to(dtype)
    k = torch.randn(b, s, hkv, d, generator=gen).to(dtype)
    v = torch.randn(b, s, hkv, d, generator=gen).to(dtype)
    lengths = torch.tensor(LENGTHS, dtype=torch.int32)
    opts = dm.AttentionOptions(window=None if window is None else dm.Window(window, 0))
    print(f"decode case dtype={dtype} d={d} hkv={hkv} g={g} window={window} seed={seed}",
          flush=True)
    out = dm.attention_decode(q.cuda(), k.cuda(), v.cuda(), lengths.cuda(), opts)
    torch.cuda.synchronize()
    e = oracle.attention_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                lengths.numpy(), left=window, precision="f64")
    return out.float().cpu().numpy(), e


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d,hkv,g", [(64, 2, 1), (128, 2, 4), (128, 1, 8), (256, 2, 2), (256, 1, 8),
                                     (64, 1, 8)])
@pytest.mark.parametrize("window", [None, 700])
def test_split_decode(dtype, d, hkv, g, window):
    _lib.probe_reset()
    a, e = _case(dtype, d, hkv, g, window, seed=d * 100 + g * 10 + (window is None))
    assert _lib.probe_counts()["decode_split"] > 0, "the MFMA split pass did not run"
    assert np.all(a[0] == 0.0), "an empty cache gives zeros"
    r = errors(a, e)[1]
    print(f"rel {r:.2e}")
    assert r <= 1e-2


@pytest.mark.parametrize("dtype,d,hkv,g", [(torch.float32, 128, 2, 4), (torch.bfloat16, 96, 1, 3)])
def test_generic_decode(dtype, d, hkv, g):
    a, e = _case(dtype, d, hkv, g, None, seed=7)
    r = errors(a, e)[1]
    print(f"rel {r:.2e}")
    assert r <= (1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("d,g", [(64, 4), (128, 4), (256, 2)])
def test_single_split_writes_the_output(d, g):
    """A cache of at most one split's keys (128): the split kernel writes the output itself and no
    merge runs."""
    gen = torch.Generator().manual_seed(d + g)
    lengths = torch.tensor([0, 1, 77, 128], dtype=torch.int32)
    b, s, hkv = 4, 128, 2
    q = torch.randn(b, hkv * g, d, generator=gen).bfloat16()
    k = torch.randn(b, s, hkv, d, generator=gen).bfloat16()
    v = torch.randn(b, s, hkv, d, generator=gen).bfloat16()
    _lib.probe_reset()
    out = dm.attention_decode(q.cuda(), k.cuda(), v.cuda(), lengths.cuda())
    torch.cuda.synchronize()
    pc = _lib.probe_counts()
    assert pc["decode_split"] == 1 and pc["decode_merge"] == 0, pc
    e = oracle.attention_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                lengths.numpy(), precision="f64")
    a = out.float().cpu().numpy()
    assert np.all(a[0] == 0.0)
    assert errors(a, e)[1] <= 1e-2


def _decode_c(q, k, v, lens, ws, opts=None):
    """dm_attention_decode through the C ABI with the caller's workspace tensor `ws`."""
    import ctypes
    from dashmag_amd import ops
    lib = _lib.lib()
    desc = ops._attention_desc("attention_decode", q.unsqueeze(1), k, v, dm.AttentionMask.none(),
                               opts or dm.AttentionOptions(), [])
    nbytes = lib.dm_attention_decode_workspace(ctypes.byref(desc))
    assert ws.numel() >= nbytes
    o = torch.empty_like(q)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.dm_attention_decode(ctypes.byref(desc), p(q), p(k), p(v), p(lens), p(o), p(ws),
                                 nbytes, st)
    assert rc == 0, _lib.last_error()
    return o


@pytest.mark.parametrize("window", [None, 1024])
def test_result_does_not_depend_on_the_workspace(window):
    """The reference's small decode shape (B = 8, S = 6144, Hq = 8, Hkv = 2, D = 256, a window of
    1024 or none): the same result, to the bit, from a zeroed workspace, from one filled with 0xff
    bytes, from the previous call's leftovers, and after a call of another shape on the same
    workspace; and it matches the f64 oracle."""
    gen = torch.Generator().manual_seed(61)
    b, s, hq, hkv, d = 8, 6144, 8, 2, 256
    q = torch.randn(b, hq, d, generator=gen).bfloat16().cuda()
    k = torch.randn(b, s, hkv, d, generator=gen).bfloat16().cuda()
    v = torch.randn(b, s, hkv, d, generator=gen).bfloat16().cuda()
    lens = torch.tensor([100, 6144, 3000, 1, 4097, 2048, 5999, 777], dtype=torch.int32).cuda()
    opts = dm.AttentionOptions(window=None if window is None else dm.Window(window, 0))
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    print(f"decode B={b} S={s} D={d} window={window}, workspace contents", flush=True)
    _lib.probe_reset()
    o0 = _decode_c(q, k, v, lens, ws, opts)
    torch.cuda.synchronize()
    pc = _lib.probe_counts()
    assert pc["decode_split"] == 1 and pc["decode_merge"] == 1, pc
    o1 = _decode_c(q, k, v, lens, ws, opts)
    ws.fill_(0xFF)
    o2 = _decode_c(q, k, v, lens, ws, opts)
    # another shape on the same workspace (fewer sequences, D = 128), then this one again
    _decode_c(q[:3, :, :128].contiguous(), k[:3, :, :, :128].contiguous(),
              v[:3, :, :, :128].contiguous(), lens[:3], ws)
    o3 = _decode_c(q, k, v, lens, ws, opts)
    torch.cuda.synchronize()
    for o in (o1, o2, o3):
        assert torch.equal(o0, o)
    e = oracle.attention_decode(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                v.float().cpu().numpy(), lens.cpu().numpy(), left=window,
                                precision="f64")
    r = errors(o0.float().cpu().numpy(), e)[1]
    print(f"rel {r:.2e}")
    assert r <= 1e-2


def test_config3_shape_splits_and_merges():
    """Config 3's shape (4096 split workgroups) through the C ABI: the split and merge kernels run,
    and sampled sequences match the f64 oracle."""
    gen = torch.Generator().manual_seed(62)
    b, s, hq, hkv, d = 64, 8192, 32, 8, 128
    q = torch.randn(b, hq, d, generator=gen).bfloat16().cuda()
    k = torch.randn(b, s, hkv, d, generator=gen).bfloat16().cuda()
    v = torch.randn(b, s, hkv, d, generator=gen).bfloat16().cuda()
    lens = torch.randint(512, s + 1, (b,), generator=gen, dtype=torch.int32).cuda()
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    _lib.probe_reset()
    o = _decode_c(q, k, v, lens, ws)
    torch.cuda.synchronize()
    pc = _lib.probe_counts()
    assert pc["decode_split"] == 1 and pc["decode_merge"] == 1, pc
    rows = [0, 31, 63]
    e = oracle.attention_decode(q[rows].float().cpu().numpy(), k[rows].float().cpu().numpy(),
                                v[rows].float().cpu().numpy(), lens[rows].cpu().numpy(),
                                precision="f64")
    assert errors(o[rows].float().cpu().numpy(), e)[1] <= 1e-2
