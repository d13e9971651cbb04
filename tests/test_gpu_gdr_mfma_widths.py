"""The MFMA chunked gated delta rule at head widths below 128 and with Dk != Dv (the reference's
kernels take any Dk, Dv: crates/dash-ops/src/gated_delta/chunk.rs; its conformance fixtures run
at Dk = Dv = 32). The kernels keep their 128-wide products and hold the columns past each width
at zero; a probe shows the MFMA kernels ran. Bounds as at Dk = Dv = 128: 1e-2 for the forward,
the reference's tensor-core backward bounds (7.5e-3 with the l2 normalisation, 1.2e-2 without,
crates/dash-ops/tests/gated_delta_chunk.rs:510-531) for the backward."""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
import oracle
from dashmag_amd import _lib, synthetic as syn
from fixtures import errors

pytestmark = pytest.mark.gpu
WIDTHS = [(32, 32), (64, 64), (32, 64), (64, 32), (128, 64), (64, 128), (96, 48)]


def host(x):
    return x.detach().float().cpu().numpy()


def _inputs(lens, h, dk, dv, dtype, seed, l2norm):
    T = sum(lens)
    q = syn.normal(seed, (1, T, h, dk), "cuda")
    k = syn.normal(seed + 1, (1, T, h, dk), "cuda")
    if not l2norm:
        q, k = syn.l2norm(q), syn.l2norm(k)
    v = syn.normal(seed + 2, (1, T, h, dv), "cuda")
    g = -torch.nn.functional.softplus(syn.normal(seed + 3, (1, T, h), "cuda"))
    beta = torch.sigmoid(syn.normal(seed + 4, (1, T, h), "cuda"))
    h0 = syn.normal(seed + 5, (len(lens), h, dk, dv), "cuda", std=0.1)
    do = syn.normal(seed + 6, (1, T, h, dv), "cuda").to(dtype)
    dfin = syn.normal(seed + 7, (len(lens), h, dk, dv), "cuda", std=0.1)
    return q.to(dtype), k.to(dtype), v.to(dtype), g, beta, h0, do, dfin


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dk,dv", WIDTHS, ids=[f"{a}x{b}" for a, b in WIDTHS])
@pytest.mark.parametrize("l2norm", [True, False])
def test_mfma_widths_match_oracle(dtype, dk, dv, l2norm):
    lens = [37, 64, 0, 130, 1]
    h = 2
    print(f"widths {dk}x{dv} l2norm {l2norm} {dtype}", flush=True)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    q, k, v, g, beta, h0, do, dfin = _inputs(lens, h, dk, dv, dtype, 500 + dk + 3 * dv, l2norm)
    opts = dm.ChunkGatedDeltaOptions(qk_l2norm=l2norm, output_final_state=True)
    _lib.probe_reset()
    out, fin = dm.chunk_gated_delta_rule(q, k, v, g, beta, h0, cu.cuda(), opts)
    r = dm.chunk_gated_delta_rule_backward(q, k, v, g, beta, h0, cu.cuda(), do, dfin, opts)
    torch.cuda.synchronize()
    pc = _lib.probe_counts()
    assert pc["gdr_chunk_fwd_mfma"] > 0 and pc["gdr_chunk_bwd_mfma"] > 0, pc
    assert out.shape == (1, sum(lens), h, dv) and fin.shape == (len(lens), h, dk, dv)
    args = (host(q), host(k), host(v), host(g), host(beta), host(h0))
    eo, ef = oracle.gdr_chunk_fwd(*args, cu.numpy(), l2norm, precision="f64")
    ro, rf = errors(host(out), eo)[1], errors(host(fin), ef)[1]
    print(f"  out {ro:.2e} final {rf:.2e}")
    assert ro <= 1e-2 and rf <= 1e-2
    e = oracle.gdr_chunk_bwd(*args, host(do), host(dfin), cu.numpy(), l2norm, precision="f64")
    tol = 7.5e-3 if l2norm else 1.2e-2
    for name, a_, e_ in zip(["dq", "dk", "dv", "dg", "dbeta", "dh0"], r, e):
        rr = errors(host(a_), e_)[1]
        print(f"  {name}: rel {rr:.2e}")
        assert rr <= tol, (name, rr)


def test_mfma_widths_fused_views_equal_contiguous():
    """q, k, v as slices of one fused projection at Dk = 64, Dv = 32: read in place, equal to
    the contiguous call to the bit."""
    lens, h, dk, dv = [70, 1, 130], 2, 64, 32
    T = sum(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32).cuda()
    qkv = syn.normal(61, (1, T, h * (2 * dk + dv)), "cuda").bfloat16()
    q = qkv[..., :h * dk].unflatten(-1, (h, dk))
    k = qkv[..., h * dk:2 * h * dk].unflatten(-1, (h, dk))
    v = qkv[..., 2 * h * dk:].unflatten(-1, (h, dv))
    g = -torch.nn.functional.softplus(syn.normal(62, (1, T, h), "cuda"))
    beta = torch.sigmoid(syn.normal(63, (1, T, h), "cuda"))
    opts = dm.ChunkGatedDeltaOptions(qk_l2norm=True, output_final_state=True)
    do = syn.normal(64, (1, T, h, dv), "cuda").bfloat16()
    r1 = dm.chunk_gated_delta_rule(q, k, v, g, beta, None, cu, opts)
    b1 = dm.chunk_gated_delta_rule_backward(q, k, v, g, beta, None, cu, do, None, opts)
    c = [x.contiguous() for x in (q, k, v)]
    r2 = dm.chunk_gated_delta_rule(*c, g, beta, None, cu, opts)
    b2 = dm.chunk_gated_delta_rule_backward(*c, g, beta, None, cu, do, None, opts)
    torch.cuda.synchronize()
    for a_, e_ in zip(list(r1) + list(b1), list(r2) + list(b2)):
        if a_ is None:
            assert e_ is None
        else:
            assert torch.equal(a_, e_)
