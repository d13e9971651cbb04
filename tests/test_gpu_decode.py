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
