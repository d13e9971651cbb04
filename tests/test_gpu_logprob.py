"""The chosen-token log-probability on the GPU (rocBLAS GEMMs for the logits and the gradient's
products, this library's kernels for the online log-sum-exp between them), through the C ABI,
against dash-conformance's bodies and bounds (crates/dash-conformance/src/logprob.rs) on the
reference's PyTorch-float64 recordings, in f32 and bf16:

- `matches_pytorch`: each case with its masked ids in small chunks; bounds [logprob, entropy,
  grad] relative to max|want|: f32 [2e-7, 2e-6, 1e-6], bf16 [2e-7, 2e-6, 4e-3] (the bf16
  gradient rounded to bf16 on the way out, as the reference's backward casts it);
- without the mask, against PyTorch without it;
- chunking (one chunk, tiny chunks, uneven row blocks, the default) leaves the answer within the
  bounds;
- a call without the gradient gives the same log-probabilities and entropies, to the bit;
- an empty batch gives empty outputs.
Beyond the recordings: a larger call (several row blocks and vocabulary chunks, masked ids, a
masked and an out-of-range target) against the f64 oracle with bounds 1e-6 (logprob), 1e-5
(entropy, gradient); mixed bf16/f32 operands, taken as f32; the refusals.
"""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
import oracle
from fixtures import round_bf16
from logprob_cases import CASES, SMALL_CHUNKS, Case, bounds, rel_error

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _call(c, dtype, masked, options, grad=True):
    h = torch.from_numpy(c.hidden).to(DT[dtype]).cuda()
    w = torch.from_numpy(c.weight).to(DT[dtype]).cuda()
    t = torch.from_numpy(c.targets).cuda()
    if grad:
        lp, ent, g = dm.chosen_logprob_with_grad(h, w, t, masked, options)
    else:
        (lp, ent), g = dm.chosen_logprob(h, w, t, masked, options), None
    torch.cuda.synchronize()
    g = None if g is None else g.cpu().numpy() * c.upstream[:, None]
    if g is not None and dtype == "bf16":
        g = round_bf16(g)
    return lp.cpu().numpy(), ent.cpu().numpy(), g


def _check(got, want, dtype):
    for part, g, w, b in zip(["logprob", "entropy", "grad"], got, want, bounds(dtype)):
        r = rel_error(g, w)
        print(f"{part}: {r:.2e} (bound {b:.0e})")
        assert r <= b, (part, r, b)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("name", CASES)
def test_matches_pytorch(name, dtype):
    print(f"logprob case {name} {dtype} masked, small chunks", flush=True)
    c = Case(name)
    _check(_call(c, dtype, c.masked, dm.LogprobOptions(**SMALL_CHUNKS)), c.masked_reference,
           dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("name", CASES)
def test_masked_tokens_leave_the_softmax(name, dtype):
    print(f"logprob case {name} {dtype} unmasked", flush=True)
    c = Case(name)
    _check(_call(c, dtype, [], dm.LogprobOptions(**SMALL_CHUNKS)), c.unmasked_reference, dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("opts", [dict(vocab_chunk=10_000, row_chunk=3072),
                                  dict(vocab_chunk=7, row_chunk=5),
                                  dict(vocab_chunk=300, row_chunk=7), dict()])
def test_chunking_does_not_change_the_answer(opts, dtype):
    print(f"logprob peaked {dtype} {opts}", flush=True)
    c = Case("peaked")
    _check(_call(c, dtype, c.masked, dm.LogprobOptions(**opts)), c.masked_reference, dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_without_gradients_same_values(dtype):
    print(f"logprob basic {dtype} with and without the gradient", flush=True)
    c = Case("basic")
    opts = dm.LogprobOptions(**SMALL_CHUNKS)
    a = _call(c, dtype, c.masked, opts)
    b = _call(c, dtype, c.masked, opts, grad=False)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def test_empty_batch():
    h = torch.zeros(0, 8, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(5, 8, device="cuda", dtype=torch.bfloat16)
    lp, ent, g = dm.chosen_logprob_with_grad(h, w, torch.zeros(0, dtype=torch.int64), [1])
    torch.cuda.synchronize()
    assert lp.shape == (0,) and ent.shape == (0,) and g.shape == (0, 8)


@pytest.mark.parametrize("dtype", ["bf16", "f32", "mixed"])
def test_larger_call_against_the_oracle(dtype):
    print(f"logprob larger call {dtype}", flush=True)
    rng = np.random.default_rng(17)
    n, v, d = 300, 5000, 256
    h = round_bf16(rng.standard_normal((n, d)) * 0.3)
    w = round_bf16(rng.standard_normal((v, d)) * 0.3)
    masked = rng.choice(v, 40, replace=False)
    t = rng.integers(0, v, n)
    t[3] = masked[5]
    t[7] = v + 11
    opts = dict(vocab_chunk=1024, row_chunk=128)
    lp_e, ent_e, g_e = oracle.chosen_logprob(h, w, t, masked, **opts, precision="f64")
    hd = torch.float32 if dtype == "f32" else torch.bfloat16
    wd = torch.bfloat16 if dtype == "bf16" else torch.float32
    lp, ent, g = dm.chosen_logprob_with_grad(torch.from_numpy(h).to(hd).cuda(),
                                             torch.from_numpy(w).to(wd).cuda(),
                                             torch.from_numpy(t), masked.tolist(),
                                             dm.LogprobOptions(**opts))
    torch.cuda.synchronize()
    for part, a, e, b in [("logprob", lp, lp_e, 1e-6), ("entropy", ent, ent_e, 1e-5),
                          ("grad", g, g_e, 1e-5)]:
        r = rel_error(a.cpu().numpy(), e)
        print(f"{part}: {r:.2e}")
        assert r <= b, (part, r)


def test_refusals():
    h = torch.zeros(4, 8, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(5, 8, device="cuda", dtype=torch.bfloat16)
    t = torch.zeros(4, dtype=torch.int64)
    with pytest.raises(dm.Unsupported, match="chosen_logprob: masked token id 5"):
        dm.chosen_logprob(h, w, t, [5])
    with pytest.raises(dm.Unsupported, match="at least one token must stay unmasked"):
        dm.chosen_logprob(h, w, t, [0, 1, 2, 3, 4, 4])
    with pytest.raises(dm.Unsupported, match="bf16 or f32"):
        dm.chosen_logprob(h.half(), w.half(), t)
    with pytest.raises(dm.Unsupported, match="row_chunk"):
        dm.chosen_logprob(h, w, t, [], dm.LogprobOptions(row_chunk=0))
