"""The MFMA attention kernels (forward ``attn_fwd_mfma``, backward ``bwd_dkdv``/``bwd_dq``) at the
head widths they take, D = 128 and 64, in bf16 and f16, against the CPU oracle over every mask
kind of the contract: no mask, sliding windows (left, right, both, with and without causality),
key padding, packed sequences with different query and key lengths (bottom-right alignment),
Tq < Tk and Tq > Tk, an explicit scale, and lengths that cut the 32-, 64-, 128- and 256-row tiles
(1, 31, 33, 127, 129, 4097). One packed case has sequences longer than the query tiles, an empty one
and query rows after the last sequence.

Rows that see no key must give lse = -inf, o = 0 and dq = 0 exactly
(crates/dash-contract/src/attention.rs:56-71); a launch probe shows that the MFMA kernels, not the
generic ones, ran.

Inputs are rounded to the dtype before the oracle sees them, and the oracle's backward takes the
GPU's o and lse (as dash-conformance's adapter composes the backward). Bounds: dash-conformance's
for the masked fixtures (crates/dash-conformance/src/attention.rs:70-108: bf16 about 4e-3, f16
about 7e-4, relative to the largest reference magnitude), doubled for the sums over up to 4097
keys that the fixtures' 40-key sequences do not reach; lse's further by sqrt(Tk / 64), the growth
of an f32 sum's rounding with its length.
"""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
import oracle
from dashmag_amd import _lib, synthetic as syn
from conformance import BF16, F16
from fixtures import errors

pytestmark = pytest.mark.gpu
U = dm.contract.UNBOUNDED
PARTS = ["o", "lse", "dq", "dk", "dv"]


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.set_threads(16)


def host(x):
    return x.detach().float().cpu().numpy()


# (name, B, Tq, Tk, Hq, Hkv, mask spec, causal, window (left, right) or None, scale)
CASES = [
    ("none_129", 1, 129, 129, 4, 2, None, False, None, None),
    ("none_cross_33x127", 2, 33, 127, 4, 1, None, False, None, None),
    ("causal_1", 1, 1, 1, 2, 1, None, True, None, None),
    ("causal_31", 1, 31, 31, 4, 2, None, True, None, None),
    ("causal_127_scale", 1, 127, 127, 4, 2, None, True, None, 0.3),
    ("causal_tq33_tk129", 1, 33, 129, 4, 2, None, True, None, None),
    ("causal_tq127_tk33_empty_rows", 1, 127, 33, 4, 2, None, True, None, None),
    ("window_left_257", 1, 257, 257, 4, 2, None, False, (64, U), None),
    ("window_right_200", 1, 200, 200, 4, 2, None, False, (U, 10), None),
    ("window_both_300", 1, 300, 300, 4, 2, None, False, (50, 20), None),
    ("causal_window_left_129", 2, 129, 129, 4, 2, None, True, (40, U), None),
    ("window_narrow_empty_rows", 1, 96, 40, 2, 1, None, False, (3, 0), None),
    ("key_padding_160", 3, 160, 160, 4, 2, "padding", False, None, None),
    ("key_padding_causal_133", 2, 133, 133, 4, 2, "padding", True, None, None),
    ("packed_cross", 1, None, None, 4, 2, ("packed", [1, 31, 33, 127, 0, 129], [5, 31, 129, 127, 3, 70]),
     True, None, None),
    ("packed_window", 1, None, None, 4, 2, ("packed", [64, 200, 17], [64, 200, 17]), True, (30, U),
     None),
    ("packed_no_causal", 1, None, None, 2, 1, ("packed", [40, 1, 90], [100, 7, 90]), False, None,
     None),
    ("causal_4097", 1, 4097, 4097, 4, 2, None, True, None, None),
    # sequences longer than the query tiles, an empty one, one row, and rows after the last
    ("packed_tiles_tail", 1, None, None, 4, 2,
     ("packed", [300, 700, 0, 257, 129, 1], [300, 700, 0, 257, 129, 1], 77), True, None, None),
]


def _build(case, dtype, d, seed):
    name, b, tq, tk, hq, hkv, mspec, causal, window, scale = case
    cu_q = cu_k = pad = None
    if isinstance(mspec, tuple):
        lq, lk = mspec[1], mspec[2]
        cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
        cu_k = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
        tq, tk = int(cu_q[-1]), int(cu_k[-1])
        if len(mspec) > 3:
            tq += mspec[3]  # query rows after the last sequence: they see no key
    q = syn.normal(seed, (b, tq, hq, d), "cuda").to(dtype)
    k = syn.normal(seed + 1, (b, tk, hkv, d), "cuda").to(dtype)
    v = syn.normal(seed + 2, (b, tk, hkv, d), "cuda").to(dtype)
    do = syn.normal(seed + 3, (b, tq, hq, d), "cuda").to(dtype)
    if mspec == "padding":
        rng = np.random.default_rng(seed)
        pad = rng.random((b, tk)) < 0.3
        pad[-1, :] = True  # one batch row with every key left out: every query row empty
        pad[0, :5] = False
    opts = dm.AttentionOptions(causal=causal, scale=scale,
                               window=None if window is None else dm.contract.Window(*window))
    if cu_q is not None:
        mask = dm.AttentionMask.packed(torch.from_numpy(cu_q).cuda(), torch.from_numpy(cu_k).cuda())
        omask = ("packed", cu_q, cu_k)
    elif pad is not None:
        mask = dm.AttentionMask.key_padding(torch.from_numpy(pad).cuda())
        omask = ("padding", pad)
    else:
        mask, omask = dm.AttentionMask.none(), None
    left = None if window is None or window[0] == U else window[0]
    right = None if window is None or window[1] == U else window[1]
    call = lambda qq, kk, vv: oracle.AttentionCall(qq, kk, vv, omask, causal, scale, left, right)  # noqa: E731
    return (q, k, v, do), mask, opts, call


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_mfma_attention_matches_oracle(case, dtype, d):
    print(f"case {case[0]} {dtype} D={d}", flush=True)
    seed = 1000 + 17 * CASES.index(case) + d
    (q, k, v, do), mask, opts, mk = _build(case, dtype, d, seed)
    _lib.probe_reset()
    o, lse = dm.attention_with_lse(q, k, v, mask, opts)
    dq, dk, dv = dm.attention_backward(q, k, v, o, lse, do, mask, opts)
    torch.cuda.synchronize()
    pc = _lib.probe_counts()
    assert pc["attn_fwd_mfma"] > 0 and pc["attn_fwd_generic"] == 0, pc
    assert pc["attn_bwd_mfma"] > 0 and pc["attn_bwd_generic"] == 0, pc
    call = mk(host(q), host(k), host(v))
    prec = "f64"
    eo, el = oracle.attention_fwd(call, prec)
    gq, gk, gv = oracle.attention_bwd(call, host(o), host(lse), host(do), prec)
    bounds = (BF16 if dtype == torch.bfloat16 else F16).masks
    got = [host(o), host(lse), host(dq), host(dk), host(dv)]
    want = [eo, el, gq, gk, gv]
    for name, a, e, bound in zip(PARTS, got, want, bounds):
        ab, err = errors(a, e)
        if name != "lse" and np.max(np.abs(e[np.isfinite(e)]), initial=0.0) < 1e-3:
            # zero in exact arithmetic (a single visible key makes dS = P (dP - delta) vanish):
            # the rounding left over is measured against the inputs' unit scale
            err = ab
        tol = 2 * bound
        if name == "lse":
            # an f32 sum of n exponentials carries about sqrt(n) roundings: the fixtures' bound
            # is for 40 keys
            tol *= max(1.0, np.sqrt(k.shape[1] / 64))
        print(f"  {name}: rel {err:.2e} (bound {tol:.1e})")
        assert err <= tol, (case[0], name, err)
    # rows that see no key: lse = -inf (checked by errors), o = 0 and dq = 0 exactly
    empty = el == -np.inf
    if empty.any():
        print(f"  {int(empty.sum())} empty rows")
        assert np.all(got[0][empty] == 0.0) and np.all(got[2][empty] == 0.0)


def test_mfma_attention_nondeterministic_flag_matches():
    """``deterministic = false`` gives results within the same bounds (the contract allows a
    different summation order for dq only; dk and dv are the deterministic mode's)."""
    case = CASES[4]
    (q, k, v, do), mask, opts, mk = _build(case, torch.bfloat16, 128, 77)
    o, lse = dm.attention_with_lse(q, k, v, mask, opts)
    r1 = dm.attention_backward(q, k, v, o, lse, do, mask, opts)
    r2 = dm.attention_backward(q, k, v, o, lse, do, mask, opts.with_deterministic(False))
    assert torch.equal(r1[1], r2[1]) and torch.equal(r1[2], r2[2])
    err = errors(host(r2[0]), host(r1[0]))[1]
    assert err <= 2 * BF16.masks[2]


D256_CASES = [c for c in CASES if c[0] in (
    "none_129", "causal_1", "causal_31", "causal_127_scale", "causal_tq127_tk33_empty_rows",
    "window_both_300", "key_padding_160", "packed_cross", "packed_no_causal",
    "packed_tiles_tail")] + [
    # the reference's head shape (Hq = 8, Hkv = 2) over a longer causal sequence: dK/dV work
    # items of both passes in one launch, split over the query heads
    ("causal_1024_gqa4", 1, 1024, 1024, 8, 2, None, True, None, None),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", D256_CASES, ids=[c[0] for c in D256_CASES])
def test_mfma_attention_d256_matches_oracle(case, dtype):
    """Head width 256 (the reference's published attention shapes): forward and backward on the
    MFMA kernels (4-wavefront forms; probes show them), against the f64 oracle."""
    print(f"case {case[0]} {dtype} D=256", flush=True)
    seed = 3000 + 17 * (CASES.index(case) if case in CASES else len(CASES) + D256_CASES.index(case))
    (q, k, v, do), mask, opts, mk = _build(case, dtype, 256, seed)
    _lib.probe_reset()
    o, lse = dm.attention_with_lse(q, k, v, mask, opts)
    torch.cuda.synchronize()
    pc = _lib.probe_counts()
    assert pc["attn_fwd_mfma"] > 0 and pc["attn_fwd_generic"] == 0, pc
    dq, dk, dv = dm.attention_backward(q, k, v, o, lse, do, mask, opts)
    torch.cuda.synchronize()
    pc = _lib.probe_counts()
    assert pc["attn_bwd_mfma"] > 0 and pc["attn_bwd_generic"] == 0, pc
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
        assert err <= tol, (case[0], name, err)
    empty = el == -np.inf
    if empty.any():
        assert np.all(got[0][empty] == 0.0) and np.all(got[2][empty] == 0.0)

