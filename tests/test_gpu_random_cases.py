"""Seeded random shapes, masks and packings for the hot path's operations on the GPU, each
against the f64 oracle with the bounds of its dedicated tests: attention forward and backward
(test_gpu_attention_sweep.py), the chunked gated delta rule forward (test_gpu_gdr_mfma.py),
decode (test_gpu_decode.py). Each case prints its draw before the GPU call, so a failure names
its shape."""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
import oracle
from dashmag_amd import _lib, synthetic as syn
from conformance import BF16, F16
from fixtures import errors
from test_gpu_attention_sweep import PARTS, U, _build, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.set_threads(16)


def _attention_case(seed):
    rng = np.random.default_rng(seed)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2]))
    g = int(rng.choice([1, 2, 4]))
    kind = str(rng.choice(["none", "causal", "window", "padding", "packed"]))
    b = int(rng.integers(1, 3))
    tq = int(rng.integers(1, 400))
    tk = tq if rng.random() < 0.6 else int(rng.integers(1, 400))
    causal = kind == "causal" or (kind in ("window", "packed") and rng.random() < 0.5)
    window = None
    mspec = None
    if kind == "window":
        left = U if rng.random() < 0.3 else int(rng.integers(0, 200))
        right = U if (left != U and rng.random() < 0.3) else int(rng.integers(0, 100))
        window = (left, right)
    elif kind == "padding":
        mspec = "padding"
    elif kind == "packed":
        n = int(rng.integers(1, 5))
        lq = [int(x) for x in rng.integers(0, 200, n)]
        lk = lq if rng.random() < 0.5 else [int(x) for x in rng.integers(0, 200, n)]
        if sum(lq) == 0:
            lq[0] = 1
        if sum(lk) == 0:
            lk[0] = 1
        mspec = ("packed", lq, lk)
        b = 1
    scale = None if rng.random() < 0.7 else float(rng.uniform(0.05, 0.5))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    name = f"attn{seed}"
    return (name, b, tq, tk, hkv * g, hkv, mspec, causal, window, scale), dtype, d


@pytest.mark.parametrize("seed", range(40))
def test_random_attention(seed):
    case, dtype, d = _attention_case(7000 + seed)
    print(f"random attention {case} {dtype} D={d}", flush=True)
    (q, k, v, do), mask, opts, mk = _build(case, dtype, d, 9000 + seed)
    _lib.probe_reset()
    o, lse = dm.attention_with_lse(q, k, v, mask, opts)
    dq, dk, dv = dm.attention_backward(q, k, v, o, lse, do, mask, opts)
    torch.cuda.synchronize()
    pc = _lib.probe_counts()
    assert pc["attn_fwd_mfma"] > 0 and pc["attn_bwd_mfma"] > 0, pc
    call = mk(host(q), host(k), host(v))
    eo, el = oracle.attention_fwd(call, "f64")
    gq, gk, gv = oracle.attention_bwd(call, host(o), host(lse), host(do), "f64")
    bounds = (BF16 if dtype == torch.bfloat16 else F16).masks
    got = [host(o), host(lse), host(dq), host(dk), host(dv)]
    for name, a, e, bound in zip(PARTS, got, [eo, el, gq, gk, gv], bounds):
        ab, err = errors(a, e)
        if name != "lse" and np.max(np.abs(e[np.isfinite(e)]), initial=0.0) < 1e-3:
            err = ab
        tol = 2 * bound * (max(1.0, np.sqrt(k.shape[1] / 64)) if name == "lse" else 1.0)
        print(f"  {name}: rel {err:.2e} (bound {tol:.1e})")
        assert err <= tol, (case, name, err)
    empty = el == -np.inf
    if empty.any():
        assert np.all(got[0][empty] == 0.0) and np.all(got[2][empty] == 0.0)


@pytest.mark.parametrize("seed", range(16))
def test_random_chunk_gated_delta_rule(seed):
    rng = np.random.default_rng(7100 + seed)
    n = int(rng.integers(1, 5))
    lens = [int(x) for x in rng.integers(0, 300, n)]
    if sum(lens) == 0:
        lens[-1] = 1
    h = int(rng.integers(1, 4))
    dk = int(rng.choice([32, 64, 96, 128]))
    dv = int(rng.choice([32, 64, 128]))
    l2norm = bool(rng.random() < 0.5)
    has_h0 = bool(rng.random() < 0.5)
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    print(f"random chunk GDR lens={lens} h={h} dk={dk} dv={dv} l2norm={l2norm} h0={has_h0} "
          f"{dtype}", flush=True)
    T = sum(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    s0 = 7200 + seed * 10
    q = syn.normal(s0, (1, T, h, dk), "cuda")
    k = syn.normal(s0 + 1, (1, T, h, dk), "cuda")
    if not l2norm:
        q, k = syn.l2norm(q), syn.l2norm(k)
    v = syn.normal(s0 + 2, (1, T, h, dv), "cuda")
    g = -torch.nn.functional.softplus(syn.normal(s0 + 3, (1, T, h), "cuda"))
    beta = torch.sigmoid(syn.normal(s0 + 4, (1, T, h), "cuda"))
    st = syn.normal(s0 + 5, (n, h, dk, dv), "cuda", std=0.1) if has_h0 else None
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    _lib.probe_reset()
    opts = dm.ChunkGatedDeltaOptions(qk_l2norm=l2norm, output_final_state=True)
    out, fin = dm.chunk_gated_delta_rule(q, k, v, g, beta, st, cu.cuda(), opts)
    torch.cuda.synchronize()
    assert _lib.probe_counts()["gdr_chunk_fwd_mfma"] > 0
    eo, ef = oracle.gdr_chunk_fwd(host(q), host(k), host(v), host(g), host(beta),
                                  None if st is None else host(st), cu.numpy(), l2norm,
                                  precision="f64")
    ro, rf = errors(host(out), eo)[1], errors(host(fin), ef)[1]
    print(f"  out {ro:.2e} final {rf:.2e}")
    assert ro <= 1e-2 and rf <= 1e-2


@pytest.mark.parametrize("seed", range(16))
def test_random_decode(seed):
    rng = np.random.default_rng(7300 + seed)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4]))
    g = int(rng.choice([1, 2, 4, 8]))
    b = int(rng.integers(1, 9))
    s = int(rng.integers(1, 3000))
    lens = [int(x) for x in rng.integers(0, s + 1, b)]
    window = None if rng.random() < 0.5 else int(rng.integers(0, 1500))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    print(f"random decode B={b} S={s} hkv={hkv} g={g} D={d} lens={lens} window={window} {dtype}",
          flush=True)
    gen = torch.Generator().manual_seed(7400 + seed)
    q = torch.randn(b, hkv * g, d, generator=gen).to(dtype)
    k = torch.randn(b, s, hkv, d, generator=gen).to(dtype)
    v = torch.randn(b, s, hkv, d, generator=gen).to(dtype)
    lengths = torch.tensor(lens, dtype=torch.int32)
    opts = dm.AttentionOptions(window=None if window is None else dm.Window(window, 0))
    _lib.probe_reset()
    out = dm.attention_decode(q.cuda(), k.cuda(), v.cuda(), lengths.cuda(), opts)
    torch.cuda.synchronize()
    assert _lib.probe_counts()["decode_split"] > 0
    e = oracle.attention_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                lengths.numpy(), left=window, precision="f64")
    a = out.float().cpu().numpy()
    for i, n in enumerate(lens):
        if n == 0:
            assert np.all(a[i] == 0.0)
    r = errors(a, e)[1]
    print(f"  rel {r:.2e}")
    assert r <= 1e-2
