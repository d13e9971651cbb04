"""The CPU oracle's chosen-token log-probability (oracle/oracle_logprob.h, a restatement of
crates/dash-ops/src/logprob/reference.rs) pinned to the reference's PyTorch-float64 recordings
with dash-conformance's bounds and bodies (crates/dash-conformance/src/logprob.rs), and to
torch's float64 log_softmax and autograd on the masked logits (the definition the contract
gives, crates/dash-contract/src/logprob.rs:4-15)."""
import numpy as np
import pytest
import torch

import oracle
from fixtures import round_bf16
from logprob_cases import CASES, SMALL_CHUNKS, Case, bounds, rel_error


def _check(got, want, dtype):
    lp, ent, grad = got
    for part, g, w, b in zip(["logprob", "entropy", "grad"], [lp, ent, grad], want,
                             bounds(dtype)):
        r = rel_error(g, w)
        assert r <= b, (part, r, b)


@pytest.mark.parametrize("precision", ["f32", "f64"])
@pytest.mark.parametrize("name", CASES)
def test_matches_pytorch(name, precision):
    """logprob.rs `matches_pytorch`: each case with its masked ids in small chunks."""
    c = Case(name)
    lp, ent, g = oracle.chosen_logprob(c.hidden, c.weight, c.targets, c.masked, **SMALL_CHUNKS,
                                       precision=precision)
    _check((lp, ent, g * c.upstream[:, None]), c.masked_reference, "f32")
    assert np.isneginf(lp[-1]), "the last row's target is masked"


@pytest.mark.parametrize("name", CASES)
def test_masked_tokens_leave_the_softmax(name):
    """logprob.rs `masked_tokens_leave_the_softmax`: without the mask, against PyTorch without
    it."""
    c = Case(name)
    lp, ent, g = oracle.chosen_logprob(c.hidden, c.weight, c.targets, (), **SMALL_CHUNKS)
    _check((lp, ent, g * c.upstream[:, None]), c.unmasked_reference, "f32")


@pytest.mark.parametrize("opts", [dict(vocab_chunk=10_000, row_chunk=3072),
                                  dict(vocab_chunk=7, row_chunk=5),
                                  dict(vocab_chunk=300, row_chunk=7), dict()])
def test_chunking_does_not_change_the_answer(opts):
    c = Case("peaked")
    lp, ent, g = oracle.chosen_logprob(c.hidden, c.weight, c.targets, c.masked, **opts)
    _check((lp, ent, g * c.upstream[:, None]), c.masked_reference, "f32")


def test_without_gradients_same_values():
    c = Case("basic")
    a = oracle.chosen_logprob(c.hidden, c.weight, c.targets, c.masked, **SMALL_CHUNKS)
    b = oracle.chosen_logprob(c.hidden, c.weight, c.targets, c.masked, **SMALL_CHUNKS,
                              with_grad=False)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    assert b[2] is None


def test_empty_batch():
    lp, ent, g = oracle.chosen_logprob(np.zeros((0, 8)), np.ones((5, 8)), np.zeros(0), [1])
    assert lp.shape == (0,) and ent.shape == (0,) and g.shape == (0, 8)


@pytest.mark.parametrize("seed", range(4))
def test_against_torch_log_softmax(seed):
    """torch float64: log_softmax over the logits with the masked ids at -inf, the entropy of
    that distribution, and autograd's gradient of each row's log-probability; targets out of
    range or masked give -inf."""
    rng = np.random.default_rng(seed)
    n, v, d = 19, 333, 24
    h = round_bf16(rng.standard_normal((n, d)) * (1 + seed))
    w = round_bf16(rng.standard_normal((v, d)) * 0.5)
    masked = rng.choice(v, size=seed * 5, replace=False)
    t = rng.integers(0, v, n)
    t[0] = v + 3
    if seed:
        t[1] = masked[0]
    lp, ent, g = oracle.chosen_logprob(h, w, t, masked, vocab_chunk=50, row_chunk=4,
                                       precision="f64")
    ht = torch.from_numpy(h).double().requires_grad_()
    z = ht @ torch.from_numpy(w).double().T
    keep = torch.ones(v, dtype=torch.bool)
    keep[torch.from_numpy(masked.astype(np.int64))] = False
    z = z.masked_fill(~keep, float("-inf"))
    logp = torch.log_softmax(z, 1)
    p = logp.exp()
    ent_t = -(p * logp.masked_fill(~keep, 0)).sum(1)
    ok = torch.from_numpy((t >= 0) & (t < v)) & keep[torch.from_numpy(np.clip(t, 0, v - 1))]
    chosen = logp.gather(1, torch.from_numpy(np.clip(t, 0, v - 1))[:, None])[:, 0]
    want = torch.where(ok, chosen, torch.tensor(float("-inf"), dtype=torch.float64))
    up = torch.from_numpy(rng.standard_normal(n))
    # a row whose target is masked or out of range keeps the gradient of -lse: its target
    # term drops out of (r found weight[t] - o) / s (reference.rs:108-117), as in the
    # recordings, whose last row has a masked target
    lse = torch.logsumexp(z, 1)
    (torch.where(ok, chosen, -lse) * up).sum().backward()
    assert rel_error(lp, want.detach().numpy()) <= 1e-7
    assert rel_error(ent, ent_t.detach().numpy()) <= 1e-7
    assert rel_error(g * up.numpy()[:, None], ht.grad.numpy()) <= 1e-7
