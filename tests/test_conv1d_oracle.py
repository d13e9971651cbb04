"""The CPU oracle's causal conv1d (oracle/oracle_conv1d.h, a restatement of
crates/dash-ops/src/conv1d/reference.rs) pinned to the reference's recordings with
dash-conformance's bounds (conv1d.rs, conv1d_state.rs), to torch's conv1d in float64 (a library
routine the contract names, crates/dash-contract/src/conv1d.rs:24-29), and to the invariants the
contract states: packed equals one call per sequence, a sequence in two pieces equals the whole,
a decoding step continues a prefill."""
import numpy as np
import pytest
import torch

import oracle
from conv1d_cases import bound, cases, state_bound, state_cases, to_dtype
from fixtures import errors, round_bf16

SEQ = [c for c in cases() if not c.step]
STEP = [c for c in cases() if c.step]


@pytest.mark.parametrize("case", SEQ, ids=lambda c: c.name)
def test_sequences_against_recordings(case):
    x, w = case["x"], case["weight"]
    out, _ = oracle.conv1d_fwd(x, w, case.bias, silu=case.silu)
    gx, gw, gb, _ = oracle.conv1d_bwd(x, w, case.bias, None, case["grad_out"], silu=case.silu)
    parts = {"out": out, "grad_x": gx, "grad_weight": gw}
    if case.has_bias:
        parts["grad_bias"] = gb
    for part, value in parts.items():
        _, rel = errors(to_dtype(value, case.dtype), case[part])
        assert rel <= bound(case.dtype, part), (part, rel)


@pytest.mark.parametrize("case", STEP, ids=lambda c: c.name)
def test_steps_against_recordings(case):
    out, nxt = oracle.conv1d_update(case["x"], case["weight"], case.bias, case.state,
                                    silu=case.silu)
    _, rel = errors(to_dtype(out, case.dtype), case["out"])
    assert rel <= bound(case.dtype, "step"), rel
    # the state only moves values: exact
    np.testing.assert_array_equal(case.recorded_layout(nxt), case["new_state"])


@pytest.mark.parametrize("case", state_cases(), ids=lambda c: c.name)
def test_states_and_packed_against_recordings(case):
    x, w = case["x"], case["weight"]
    out, fin = oracle.conv1d_fwd(x, w, case.bias, case.h0, case.cu, case.silu, case.w_out)
    gx, gw, gb, gh = oracle.conv1d_bwd(x, w, case.bias, case.h0, case["grad_out"],
                                       case.grad_final, case.cu, case.silu)
    parts = {"out": to_dtype(out, case.dtype), "grad_x": to_dtype(gx, case.dtype),
             "grad_weight": to_dtype(gw, case.dtype)}
    if case.w_out is not None:
        parts["final_state"] = fin
    if case.has_bias:
        parts["grad_bias"] = to_dtype(gb, case.dtype)
    if case.w is not None:
        parts["grad_initial_state"] = gh
    for part, value in parts.items():
        _, rel = errors(value, case[part])
        assert rel <= state_bound(case.dtype, part), (part, rel)


def _torch_reference(x, w, bias, h0, silu, w_out):
    """torch's F.conv1d with groups = C on [state, x] (or x left-padded by K - 1), in float64:
    the definition the contract gives (crates/dash-contract/src/conv1d.rs:24-29)."""
    b, t, c = x.shape
    k = w.shape[1]
    xt = torch.from_numpy(x).double().transpose(1, 2)
    hist = xt if h0 is None else torch.cat([torch.from_numpy(h0).double().transpose(1, 2), xt], 2)
    pad = torch.nn.functional.pad(hist, (k - 1, 0))
    y = torch.nn.functional.conv1d(pad, torch.from_numpy(w).double()[:, None, :],
                                   None if bias is None else torch.from_numpy(bias).double(),
                                   groups=c)[:, :, -t:] if t > 0 else xt
    if silu:
        y = y * torch.sigmoid(y)
    out = y.transpose(1, 2).numpy()
    fin = None
    if w_out is not None:
        full = torch.nn.functional.pad(hist, (w_out, 0))
        fin = full[:, :, full.shape[2] - w_out:].transpose(1, 2).numpy()
    return out, fin


@pytest.mark.parametrize("k,silu,bias,w,w_out,t", [
    (4, True, True, 3, 3, 37), (1, False, False, None, None, 5), (5, True, False, 6, 2, 3),
    (2, False, True, 1, 7, 0), (8, True, True, None, 7, 70), (3, False, False, 4, None, 1),
])
def test_against_torch_conv1d(k, silu, bias, w, w_out, t):
    rng = np.random.default_rng(k * 100 + t)
    b, c = 2, 7
    x = rng.standard_normal((b, t, c)).astype(np.float32)
    wt = rng.standard_normal((c, k)).astype(np.float32)
    bs = rng.standard_normal(c).astype(np.float32) if bias else None
    h0 = rng.standard_normal((b, w, c)).astype(np.float32) if w is not None else None
    out, fin = oracle.conv1d_fwd(x, wt, bs, h0, None, silu, w_out, precision="f64")
    eo, ef = _torch_reference(x, wt, bs, h0, silu, w_out)
    np.testing.assert_allclose(out, eo, rtol=1e-6, atol=1e-6)
    if w_out is not None:
        np.testing.assert_array_equal(fin, ef)
    # gradients against torch's autograd of the same definition
    if t > 0:
        xt = torch.from_numpy(x).double().requires_grad_()
        wtt = torch.from_numpy(wt).double().requires_grad_()
        bst = torch.from_numpy(bs).double().requires_grad_() if bias else None
        h0t = torch.from_numpy(h0).double().requires_grad_() if h0 is not None else None
        hist = xt.transpose(1, 2) if h0t is None else torch.cat([h0t.transpose(1, 2),
                                                                 xt.transpose(1, 2)], 2)
        y = torch.nn.functional.conv1d(torch.nn.functional.pad(hist, (k - 1, 0)), wtt[:, None, :],
                                       bst, groups=c)[:, :, -t:]
        if silu:
            y = y * torch.sigmoid(y)
        go = rng.standard_normal((b, t, c))
        loss = (y.transpose(1, 2) * torch.from_numpy(go)).sum()
        gfin = None
        if w_out is not None:
            full = torch.nn.functional.pad(hist, (w_out, 0))
            gfin = rng.standard_normal((b, w_out, c))
            loss = loss + (full[:, :, full.shape[2] - w_out:].transpose(1, 2) *
                           torch.from_numpy(gfin)).sum()
        loss.backward()
        gx, gw, gb, gh = oracle.conv1d_bwd(x, wt, bs, h0, go, gfin, None, silu, precision="f64")
        np.testing.assert_allclose(gx, xt.grad.numpy(), rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(gw, wtt.grad.numpy(), rtol=1e-6, atol=1e-5)
        if bias:
            np.testing.assert_allclose(gb, bst.grad.numpy(), rtol=1e-6, atol=1e-5)
        if h0 is not None:
            np.testing.assert_allclose(gh, h0t.grad.numpy(), rtol=1e-6, atol=1e-6)


def test_packed_equals_calls_and_splits():
    """Packed sequences against one call each, and a sequence in two pieces against the whole
    (conv1d_state.rs:317-600): outputs and final states exact."""
    rng = np.random.default_rng(3)
    c, k, w = 6, 4, 3
    lens = [0, 37, 3, 0, 64, 1, 29]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    t = int(cu[-1])
    x = round_bf16(rng.standard_normal((1, t, c)))
    wt = round_bf16(rng.standard_normal((c, k)))
    bs = round_bf16(rng.standard_normal(c))
    h0 = rng.standard_normal((len(lens), w, c)).astype(np.float32)
    out, fin = oracle.conv1d_fwd(x, wt, bs, h0, cu, True, w)
    go = rng.standard_normal((1, t, c)).astype(np.float32)
    gf = rng.standard_normal((len(lens), w, c)).astype(np.float32)
    gx, gw, gb, gh = oracle.conv1d_bwd(x, wt, bs, h0, go, gf, cu, True)
    for s, (a, e) in enumerate(zip(cu[:-1], cu[1:])):
        o1, f1 = oracle.conv1d_fwd(x[:, a:e], wt, bs, h0[s:s + 1], None, True, w)
        np.testing.assert_array_equal(out[:, a:e], o1)
        np.testing.assert_array_equal(fin[s:s + 1], f1)
        g1 = oracle.conv1d_bwd(x[:, a:e], wt, bs, h0[s:s + 1], go[:, a:e], gf[s:s + 1], None,
                               True)
        np.testing.assert_array_equal(gx[:, a:e], g1[0])
        np.testing.assert_array_equal(gh[s:s + 1], g1[3])
        if e - a == 0:  # an empty sequence passes its state through
            np.testing.assert_array_equal(f1, h0[s:s + 1])
    # a split sequence
    xs = x[:, :70]
    whole, fw = oracle.conv1d_fwd(xs, wt, bs, h0[:1], None, True, w)
    first, f1 = oracle.conv1d_fwd(xs[:, :33], wt, bs, h0[:1], None, True, w)
    second, f2 = oracle.conv1d_fwd(xs[:, 33:], wt, bs, f1, None, True, w)
    np.testing.assert_array_equal(np.concatenate([first, second], 1), whole)
    np.testing.assert_array_equal(f2, fw)


def test_prefill_then_steps():
    """A prefill then single steps give the sequence's outputs (conv1d.rs:382-486)."""
    rng = np.random.default_rng(5)
    b, t, c, k = 2, 12, 5, 4
    x = rng.standard_normal((b, t, c)).astype(np.float32)
    wt = rng.standard_normal((c, k)).astype(np.float32)
    bs = rng.standard_normal(c).astype(np.float32)
    whole, _ = oracle.conv1d_fwd(x, wt, bs, None, None, True)
    _, state = oracle.conv1d_fwd(x[:, :5], wt, bs, None, None, True, k + 1)
    for i in range(5, t):
        o, state = oracle.conv1d_update(x[:, i], wt, bs, state, silu=True)
        np.testing.assert_allclose(o, whole[:, i], rtol=0, atol=1e-6)
    np.testing.assert_array_equal(state, x[:, t - (k + 1):])
