"""Decoding over the other key-value cache layouts: the packed cache (sequence b's rows at an
offset, cu_seqlens_k) and the paged cache (pages of page_size keys and a block table). Both are
the dense decode (attention.rs:732, reference.rs:433-467) over the cache their offsets or table
describe, so the check is the f64 oracle's dense decode of that cache:

- relative error max|a - e| / max|e| at most 1e-2 for 16-bit inputs and 1e-5 for f32, the
  tolerances of the dense decode tests;
- every cache row the query does not see (past a sequence's length, before its window, on pages
  no sequence uses) holds NaN, so a read of any of them shows in the output;
- the packed cache with offsets b * S gives the dense call's bits, and two block tables over
  differently shuffled pages give the same bits (the kernels see the same keys in the same
  order);
- a page index out of range for a visible key reads as zeros (the oracle's cache holds zeros
  there), never outside the pages.
"""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
from dashmag_amd import _lib
import oracle
from fixtures import errors

pytestmark = pytest.mark.gpu

LENGTHS = [0, 1, 15, 16, 17, 1023, 1024, 1025, 2900]


def _qkv(dtype, d, hkv, g, s, seed):
    gen = torch.Generator().manual_seed(seed)
    b = len(LENGTHS)
    q = torch.randn(b, hkv * g, d, generator=gen).to(dtype)
    k = torch.randn(b, s, hkv, d, generator=gen).to(dtype)
    v = torch.randn(b, s, hkv, d, generator=gen).to(dtype)
    return q, k, v


def _poison(k, lengths, window):
    """NaN in every row of the dense cache the query of its sequence does not see."""
    k = k.clone()
    for b, n in enumerate(lengths):
        k[b, n:] = float("nan")
        if window is not None and n - 1 - window > 0:
            k[b, :n - 1 - window] = float("nan")
    return k


def _expect(q, k, v, lengths, window):
    # the oracle reads only the visible rows, so the NaN rows are replaced by anything finite
    kk, vv = torch.nan_to_num(k).float().numpy(), torch.nan_to_num(v).float().numpy()
    return oracle.attention_decode(q.float().numpy(), kk, vv, np.asarray(lengths), left=window,
                                   precision="f64")


def _bound(dtype):
    return 1e-5 if dtype == torch.float32 else 1e-2


@pytest.mark.parametrize("dtype,d,hkv,g", [(torch.bfloat16, 128, 2, 4), (torch.float16, 64, 2, 2),
                                           (torch.bfloat16, 256, 2, 8), (torch.float32, 128, 1, 4)])
@pytest.mark.parametrize("window", [None, 700])
def test_packed_cache(dtype, d, hkv, g, window):
    s = max(LENGTHS) + 7
    q, k, v = _qkv(dtype, d, hkv, g, s, seed=11 * d + g)
    k, v = _poison(k, LENGTHS, window), _poison(v, LENGTHS, window)
    print(f"packed decode dtype={dtype} d={d} hkv={hkv} g={g} window={window}", flush=True)
    opts = dm.AttentionOptions(window=None if window is None else dm.Window(window, 0))
    lengths = torch.tensor(LENGTHS, dtype=torch.int32)
    # each sequence's span: its length plus a ragged slack of NaN rows, packed back to back
    rng = np.random.default_rng(d + g)
    spans = [n + int(rng.integers(0, 40)) for n in LENGTHS]
    cu = np.concatenate([[0], np.cumsum(spans)]).astype(np.int32)
    kp = torch.full((int(cu[-1]), hkv, d), float("nan"), dtype=dtype)
    vp = kp.clone()
    for b, n in enumerate(LENGTHS):
        kp[cu[b]:cu[b] + n] = k[b, :n]
        vp[cu[b]:cu[b] + n] = v[b, :n]
    out = dm.attention_decode_packed(q.cuda(), kp.cuda(), vp.cuda(), torch.from_numpy(cu),
                                     lengths.cuda(), opts)
    torch.cuda.synchronize()
    a = out.float().cpu().numpy()
    e = _expect(q, k, v, LENGTHS, window)
    assert np.all(a[0] == 0.0), "an empty cache gives zeros"
    r = errors(a, e)[1]
    print(f"rel {r:.2e}")
    assert r <= _bound(dtype)

    # offsets b * S over the dense cache: the dense call's bits
    dense = dm.attention_decode(q.cuda(), k.cuda(), v.cuda(), lengths.cuda(), opts)
    cu_dense = torch.arange(len(LENGTHS) + 1, dtype=torch.int32) * s
    packed = dm.attention_decode_packed(q.cuda(), k.reshape(-1, hkv, d).cuda(),
                                        v.reshape(-1, hkv, d).cuda(), cu_dense, lengths.cuda(),
                                        opts, max_len=s)
    torch.cuda.synchronize()
    assert torch.equal(dense.cpu(), packed.cpu())


def _paged(k, v, lengths, page_size, rng, extra=3):
    """The dense cache cut into pages, shuffled among `extra` unused NaN pages; returns the
    pages and the block table (unused table slots hold -1)."""
    b, s, hkv, d = k.shape
    max_pages = -(-s // page_size)
    used = [-(-n // page_size) for n in lengths]
    npages = sum(used) + extra
    perm = rng.permutation(npages)
    kp = torch.full((npages, page_size, hkv, d), float("nan"), dtype=k.dtype)
    vp = kp.clone()
    table = np.full((b, max_pages), -1, np.int32)
    nxt = 0
    for i, n in enumerate(lengths):
        for p in range(used[i]):
            pg = int(perm[nxt])
            nxt += 1
            table[i, p] = pg
            rows = min(page_size, s - p * page_size)
            kp[pg, :rows] = k[i, p * page_size:p * page_size + rows]
            vp[pg, :rows] = v[i, p * page_size:p * page_size + rows]
    return kp, vp, table


@pytest.mark.parametrize("dtype,d,hkv,g,page_size", [
    (torch.bfloat16, 128, 2, 4, 16), (torch.bfloat16, 128, 1, 8, 64),
    (torch.float16, 128, 2, 2, 32), (torch.bfloat16, 128, 2, 4, 5),
    (torch.bfloat16, 64, 2, 2, 16), (torch.float32, 128, 1, 4, 16),
    (torch.bfloat16, 256, 2, 4, 16),
])
@pytest.mark.parametrize("window", [None, 700])
def test_paged_cache(dtype, d, hkv, g, page_size, window):
    s = max(LENGTHS) + 7
    q, k, v = _qkv(dtype, d, hkv, g, s, seed=7 * d + g + page_size)
    k, v = _poison(k, LENGTHS, window), _poison(v, LENGTHS, window)
    print(f"paged decode dtype={dtype} d={d} hkv={hkv} g={g} page_size={page_size} "
          f"window={window}", flush=True)
    opts = dm.AttentionOptions(window=None if window is None else dm.Window(window, 0))
    lengths = torch.tensor(LENGTHS, dtype=torch.int32)
    rng = np.random.default_rng(page_size)
    kp, vp, table = _paged(k, v, LENGTHS, page_size, rng)
    _lib.probe_reset()
    out = dm.attention_decode_paged(q.cuda(), kp.cuda(), vp.cuda(), torch.from_numpy(table),
                                    lengths.cuda(), opts)
    torch.cuda.synchronize()
    # the MFMA split pass for 16-bit pages of a multiple of 16 keys, the generic kernel otherwise
    split = dtype != torch.float32 and page_size % 16 == 0
    pc = _lib.probe_counts()
    assert (pc["decode_split"] > 0) == split and (pc["attn_fwd_generic"] > 0) != split, pc
    a = out.float().cpu().numpy()
    e = _expect(q, k, v, LENGTHS, window)
    assert np.all(a[0] == 0.0), "an empty cache gives zeros"
    r = errors(a, e)[1]
    print(f"rel {r:.2e}")
    assert r <= _bound(dtype)

    # another shuffle of the pages: the same bits
    kp2, vp2, table2 = _paged(k, v, LENGTHS, page_size, np.random.default_rng(page_size + 99), 5)
    out2 = dm.attention_decode_paged(q.cuda(), kp2.cuda(), vp2.cuda(), torch.from_numpy(table2),
                                     lengths.cuda(), opts)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out2.cpu())


@pytest.mark.parametrize("page_size,d", [(16, 128), (5, 128), (16, 256)])
def test_paged_bad_page_reads_zeros(page_size, d):
    dtype, hkv, g = torch.bfloat16, 2, 4
    s = max(LENGTHS) + 7
    q, k, v = _qkv(dtype, d, hkv, g, s, seed=3)
    print(f"paged decode, page index out of range, page_size={page_size} d={d}", flush=True)
    lengths = torch.tensor(LENGTHS, dtype=torch.int32)
    kp, vp, table = _paged(k, v, LENGTHS, page_size, np.random.default_rng(1))
    # the last sequence's third page: below zero; the one before's second: past the pages
    bad = [(len(LENGTHS) - 1, 2, -7), (len(LENGTHS) - 2, 1, kp.shape[0] + 1000)]
    kz, vz = k.clone(), v.clone()
    for b, p, idx in bad:
        table[b, p] = idx
        kz[b, p * page_size:(p + 1) * page_size] = 0
        vz[b, p * page_size:(p + 1) * page_size] = 0
    out = dm.attention_decode_paged(q.cuda(), kp.cuda(), vp.cuda(), torch.from_numpy(table),
                                    lengths.cuda())
    torch.cuda.synchronize()
    a = out.float().cpu().numpy()
    e = _expect(q, kz, vz, LENGTHS, None)
    r = errors(a, e)[1]
    print(f"rel {r:.2e}")
    assert r <= 1e-2
