"""The fused linear cross-entropy on the GPU through the C ABI (hipBLASLt GEMMs for the logits and
the gradients' products, this library's kernels for the online log-sum-exp, the per-row outputs,
the coefficients and the logits' gradient), against the reference's PyTorch-float64 recordings
(crates/dash-ops/tests/fixtures/loss) with the bounds of dash-ops' own kernel tests
(crates/dash-ops/tests/loss.rs:983-992), [loss, logprob, entropy, grad_hidden, grad_weight]
relative to max|want|: f32 [2e-7, 2e-7, 1e-6, 4e-6, 4e-6]; bf16 [2e-7, 2e-7, 3e-7, 5e-3, 5e-3]
(the logits' gradient rounded to bf16 for the products, the gradients returned in bf16). Also:
each term's gradient alone, chunking, f16 inputs against f32 inputs of the same values
(loss.rs:934: [2e-7, 2e-7, 1e-6, 1e-3, 1e-3]), an empty batch, every row ignored, agreement with
the chosen-token log-probability, the refusals."""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
from fixtures import round_f16
from loss_cases import BOUNDS, CASES, PARTS, SMALL_CHUNKS, Case, rel_error

pytestmark = pytest.mark.gpu

PARAMS = [(c, v) for c in CASES for v in Case(c).variants]
DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _options(case, variant, chunks=SMALL_CHUNKS):
    o = case.options(variant)
    return dm.CrossEntropyOptions(reduction=dm.Reduction(o["reduction"]),
                                  ignore_index=o["ignore_index"], label_smoothing=o["eps"],
                                  z_loss=o["lam"], masked=tuple(o["masked"]), entropy=True,
                                  chunks=dm.LogprobOptions(**chunks))


def _run(case, precision, variant, dtype=None, term=None, chunks=SMALL_CHUNKS, values=None):
    h, w = case.inputs(precision) if values is None else values
    dt = DT[dtype or precision]
    opts = _options(case, variant, chunks)
    hd, wd = torch.from_numpy(h).to(dt).cuda(), torch.from_numpy(w).to(dt).cuda()
    t = torch.from_numpy(case.targets)
    loss, lp, ent, rows = dm.linear_cross_entropy(hd, wd, t, opts)
    up = case.upstream(opts.reduction.value, rows[6].cpu().numpy(), term)
    gh, gw = dm.linear_cross_entropy_backward(hd, wd, t, rows, torch.from_numpy(up), opts)
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy()  # noqa: E731
    return [f(loss), f(lp), f(ent), f(gh), f(gw)]


def _check(got, want, bounds):
    for part, g, w, b in zip(PARTS, got, want, bounds):
        r = rel_error(g, w)
        print(f"{part}: {r:.2e} (bound {b:.0e})")
        assert r <= b, (part, r, b)


@pytest.mark.parametrize("precision", ["f32", "bf16"])
@pytest.mark.parametrize("name,variant", PARAMS)
def test_matches_pytorch(name, variant, precision):
    print(f"loss case {name} {variant} {precision}", flush=True)
    c = Case(name)
    _check(_run(c, precision, variant), c.want(precision, variant), BOUNDS[precision])


@pytest.mark.parametrize("precision", ["f32", "bf16"])
@pytest.mark.parametrize("term", ["loss", "lp", "ent"])
@pytest.mark.parametrize("name", ["basic", "peaked"])
def test_each_term_has_its_gradient(name, term, precision):
    print(f"loss case {name} smooth, the {term} term alone, {precision}", flush=True)
    c = Case(name)
    got = _run(c, precision, "smooth", term=term)
    want = c.want(precision, "smooth", term)
    for part, g, w, b in zip(PARTS[3:], got[3:], want[3:], BOUNDS[precision][3:]):
        r = rel_error(g, w)
        print(f"{part}: {r:.2e}")
        assert r <= b, (part, r, b)


@pytest.mark.parametrize("chunks", [dict(vocab_chunk=10_000, row_chunk=3072),
                                    dict(vocab_chunk=7, row_chunk=3), dict(vocab_chunk=0,
                                                                           row_chunk=3072)])
def test_chunking_does_not_change_the_answer(chunks):
    print(f"loss peaked smooth f32 {chunks}", flush=True)
    c = Case("peaked")
    _check(_run(c, "f32", "smooth", chunks=chunks), c.want("f32", "smooth"), BOUNDS["f32"])


@pytest.mark.parametrize("name", CASES)
def test_f16_inputs_against_f32(name):
    """f16 inputs are computed in f32 (loss.rs:911-934): against f32 inputs of the same values,
    [2e-7, 2e-7, 1e-6, 1e-3, 1e-3]."""
    print(f"loss case {name} f16 against f32", flush=True)
    c = Case(name)
    vals = (round_f16(c.hidden), round_f16(c.weight))
    got = _run(c, "f32", "smooth", dtype="f16", values=vals)
    want = _run(c, "f32", "smooth", dtype="f32", values=vals)
    _check(got, want, [2e-7, 2e-7, 1e-6, 1e-3, 1e-3])


def test_agrees_with_chosen_logprob():
    c = Case("basic")
    opts = _options(c, "smooth")
    h, w = torch.from_numpy(c.hidden).cuda(), torch.from_numpy(c.weight).cuda()
    t = torch.from_numpy(c.targets)
    _, lp, ent, rows = dm.linear_cross_entropy(h, w, t, opts)
    lp2, ent2 = dm.chosen_logprob(h, w, t, list(opts.masked), opts.chunks)
    torch.cuda.synchronize()
    counted = rows[6] > 0.5
    assert torch.equal(lp[counted], lp2[counted]) and torch.equal(ent[counted], ent2[counted])


def test_empty_batch_and_all_ignored():
    print("loss: empty batch, every row ignored", flush=True)
    w = torch.randn(50, 16, device="cuda")
    h0 = torch.zeros(0, 16, device="cuda")
    opts = dm.CrossEntropyOptions(entropy=True)
    loss, lp, ent, rows = dm.linear_cross_entropy(h0, w, torch.zeros(0, dtype=torch.int64), opts)
    gh, gw = dm.linear_cross_entropy_backward(h0, w, torch.zeros(0, dtype=torch.int64), rows,
                                              torch.zeros(3, 0), opts)
    torch.cuda.synchronize()
    assert lp.shape == (0,) and gh.shape == (0, 16) and torch.all(gw == 0)
    assert torch.isnan(loss).all()  # the mean over no counted row
    h = torch.randn(6, 16, device="cuda")
    t = torch.full((6,), -100, dtype=torch.int64)
    opts = dm.CrossEntropyOptions(entropy=True, z_loss=1e-2, label_smoothing=0.1)
    loss, lp, ent, rows = dm.linear_cross_entropy(h, w, t, opts)
    gh, gw = dm.linear_cross_entropy_backward(h, w, t, rows, torch.ones(3, 6), opts)
    torch.cuda.synchronize()
    assert torch.isnan(loss).all() and torch.all(lp == 0) and torch.all(ent == 0)
    assert torch.all(gh == 0) and torch.all(gw == 0)


def test_refusals():
    h = torch.zeros(4, 8, device="cuda")
    w = torch.ones(5, 8, device="cuda")
    t = torch.zeros(4, dtype=torch.int64)
    with pytest.raises(dm.Unsupported, match="label_smoothing must be in 0..=1"):
        dm.linear_cross_entropy(h, w, t, dm.CrossEntropyOptions(label_smoothing=1.5))
    with pytest.raises(dm.Unsupported, match="z_loss must be finite and at least 0"):
        dm.linear_cross_entropy(h, w, t, dm.CrossEntropyOptions(z_loss=-1.0))
    with pytest.raises(dm.Unsupported, match="masked token id 9 is not below"):
        dm.linear_cross_entropy(h, w, t, dm.CrossEntropyOptions(masked=(9,)))
    with pytest.raises(dm.Unsupported, match="share one dtype"):
        dm.linear_cross_entropy(h, w.bfloat16(), t)
