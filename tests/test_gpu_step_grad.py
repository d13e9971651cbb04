"""The recurrent step's backward (dm_gdr_step_bwd) and the step forward at widths the fixtures
leave open, through the C ABI, against the CPU oracle in float64 (itself pinned to the
reference's recorded gradients and to finite differences, tests/test_oracle.py).

Tolerances: relative error max|a - e| / max|e| at most 1e-5 where the inputs are f32, 1e-2 where
they are bf16 (each gradient rounded once to bf16, 2^-9 relative, from f32 arithmetic).
"""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
import oracle
from dashmag_amd import _lib, synthetic as syn
from fixtures import errors

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def host(x):
    return x.detach().float().cpu().numpy()


def rel(a, e):
    return errors(a, e)[1]


def inputs(seed, cu, h, dk, dv, dtype, nseq=None):
    """Packed tokens (cu given) or one token per sequence: q, k, v, g, beta, state, d_out,
    d_state on the GPU."""
    gen = torch.Generator().manual_seed(seed)
    t = int(cu[-1]) if cu is not None else nseq
    s = len(cu) - 1 if cu is not None else nseq
    rn = lambda *shape: torch.randn(*shape, generator=gen)  # noqa: E731
    q, k = rn(t, h, dk), rn(t, h, dk)
    v = rn(t, h, dv)
    g = -torch.nn.functional.softplus(rn(t, h))
    beta = torch.sigmoid(rn(t, h))
    st = 0.3 * rn(s, h, dk, dv)
    do = rn(t, h, dv)
    dst = rn(s, h, dk, dv)
    cast = lambda x: x.to(dtype).cuda()  # noqa: E731
    return dict(q=cast(q), k=cast(k), v=cast(v), g=g.cuda(), beta=cast(beta), state=st.cuda(),
                d_out=cast(do), d_state=dst.cuda())


CASES = [
    # (h, dk, dv, sequence lengths or None for one token per sequence of `nseq`)
    (2, 16, 24, [1, 3, 0, 2]),
    (2, 32, 13, [5, 0, 1]),          # Dv not a multiple of 4: element-wise state rows
    (3, 64, 12, None),
    (4, 128, 128, [1, 7, 0, 40, 2]),  # two 64-column slices per (sequence, head)
    (1, 256, 256, [3, 1]),           # four slices, 16 rows a thread
    (2, 96, 200, [2, 4]),            # one slice of 200 columns
    (3, 128, 256, None),             # one token per sequence at Dk = 128: the compile-time form
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("l2norm", [True, False])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_step_backward_against_oracle(case, l2norm, dtype):
    h, dk, dv, lens = CASES[case]
    cu = None if lens is None else np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    x = inputs(100 + case, cu, h, dk, dv, dtype, nseq=5)
    cu_d = None if cu is None else torch.as_tensor(cu, dtype=torch.int32).cuda()
    opts = dm.GatedDeltaStepOptions(qk_l2norm=l2norm, scale=None if l2norm else 0.45)
    args = [x[n] for n in ("q", "k", "v", "g", "beta", "state")]
    print(f"step backward case {case} h={h} dk={dk} dv={dv} lens={lens} l2norm={l2norm} {dtype}",
          flush=True)
    _lib.probe_reset()
    r = dm.gated_delta_step_backward(*args, cu_d, x["d_out"], x["d_state"], opts)
    torch.cuda.synchronize()
    assert _lib.probe_counts()["gdr_step_bwd"] == 1
    scale = 0.45 if not l2norm else float(np.float32(1 / np.sqrt(dk)))
    e = oracle.gdr_step_bwd(*(host(a) for a in args), host(x["d_out"]), host(x["d_state"]),
                            cu=cu, l2norm=l2norm, scale=scale, precision="f64")
    for name, a, ee, want_dt in zip(["dq", "dk", "dv", "dg", "dbeta", "d_state"], r, e,
                                    [dtype, dtype, dtype, torch.float32, dtype, torch.float32]):
        assert a.dtype == want_dt, (name, a.dtype)
        rr = rel(host(a), ee)
        print(f"  {name}: rel {rr:.2e}")
        assert rr <= TOL[dtype], (name, rr)
    # the forward at the same widths
    out, ns = dm.gated_delta_step(*args, cu_d, opts)
    eo, es = oracle.gdr_step(*(host(a) for a in args), cu=cu, l2norm=l2norm, scale=scale,
                             precision="f64")
    assert rel(host(out), eo) <= TOL[dtype] and rel(host(ns), es) <= 1e-5


def test_step_backward_without_cotangents():
    """d_out or d_state absent reads as zeros: with both absent every gradient is zero."""
    cu = np.array([0, 2, 5], np.int64)
    x = inputs(7, cu, 2, 16, 8, torch.float32)
    cu_d = torch.as_tensor(cu, dtype=torch.int32).cuda()
    args = [x[n] for n in ("q", "k", "v", "g", "beta", "state")]
    r0 = dm.gated_delta_step_backward(*args, cu_d, None, None)
    assert all(float(t.abs().max()) == 0.0 for t in r0)
    r1 = dm.gated_delta_step_backward(*args, cu_d, x["d_out"], None)
    r2 = dm.gated_delta_step_backward(*args, cu_d, x["d_out"], torch.zeros_like(x["d_state"]))
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


def test_config5_step_backward():
    """Config 5 (128 sequences x 16 heads, Dk = Dv = 128, bf16 inputs, f32 states) at full size,
    with N(0, 1) cotangents of the output and the new states; checked on three sequences."""
    c = syn.config5("cuda")
    args = [c[x] for x in ("q", "k", "v", "g", "beta")] + [c["state"]]
    gen = torch.Generator().manual_seed(55)
    do = torch.randn(c["v"].shape, generator=gen).to(torch.bfloat16).cuda()
    dst = torch.randn(c["state"].shape, generator=gen).cuda()
    r = dm.gated_delta_step_backward(*args, None, do, dst)
    torch.cuda.synchronize()
    rows = [0, 77, 127]
    e = oracle.gdr_step_bwd(*(host(x[rows]) for x in args), host(do[rows]), host(dst[rows]),
                            precision="f64")
    for name, a, ee in zip(["dq", "dk", "dv", "dg", "dbeta", "d_state"], r, e):
        rr = rel(host(a[rows]), ee)
        print(f"config 5 backward {name}: rel {rr:.2e}")
        assert rr <= (1e-5 if name == "d_state" else 2e-2), (name, rr)


@pytest.mark.parametrize("dk", [128, 256])
def test_wide_step_packed_equals_token_by_token(dk):
    """With the l2 normalisation at Dk = 256 every wavefront of a workgroup holds part of q's and
    k's squared sums: they are added in a fixed order, so a packed call equals its tokens run one
    call at a time, and a repeated call itself, to the bit (gated_delta_packed.rs:459-502)."""
    cu = [0, 3, 4]
    x = inputs(91 + dk, cu, 2, dk, 64, torch.bfloat16)
    args = [x[n] for n in ("q", "k", "v", "g", "beta")]
    opts = dm.GatedDeltaStepOptions().with_qk_l2norm(True)
    cut = torch.tensor(cu, dtype=torch.int32)
    out, st = dm.gated_delta_step(*args, x["state"], cut, opts)
    out2, st2 = dm.gated_delta_step(*args, x["state"], cut, opts)
    assert torch.equal(out, out2) and torch.equal(st, st2)
    for s in range(len(cu) - 1):
        state = x["state"][s:s + 1].clone()
        for t in range(cu[s], cu[s + 1]):
            o1, state = dm.gated_delta_step(*(a[t:t + 1] for a in args), state, None, opts)
            assert torch.equal(o1[0], out[t]), (s, t)
        assert torch.equal(state[0], st[s]), s


@pytest.mark.parametrize("l2norm", [True, False])
def test_one_token_form_equals_the_general_form(l2norm):
    """One token per sequence at Dk = 128 runs the compile-time form of the step and its backward;
    the same rows as packed sequences of one token each run the general form. The arithmetic is
    the same, in the same order: the results agree to the bit."""
    b, h = 12, 3
    x = inputs(505, None, h, 128, 128, torch.bfloat16, nseq=b)
    args = [x[n] for n in ("q", "k", "v", "g", "beta")]
    opts = dm.GatedDeltaStepOptions(qk_l2norm=l2norm, scale=None if l2norm else 0.45)
    cut = torch.arange(b + 1, dtype=torch.int32)
    print(f"one-token form against the general form, l2norm={l2norm}", flush=True)
    o1, s1 = dm.gated_delta_step(*args, x["state"], None, opts)
    o2, s2 = dm.gated_delta_step(*args, x["state"], cut, opts)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    g1 = dm.gated_delta_step_backward(*args, x["state"], None, x["d_out"], x["d_state"], opts)
    g2 = dm.gated_delta_step_backward(*args, x["state"], cut, x["d_out"], x["d_state"], opts)
    torch.cuda.synchronize()
    for name, a, e in zip(["dq", "dk", "dv", "dg", "dbeta", "d_state"], g1, g2):
        assert torch.equal(a, e), name
