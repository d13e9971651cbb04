"""The causal conv1d's HIP path through the C ABI (dashmag_amd.ops.causal_conv1d, _backward,
_update): every recorded case of the reference's conv1d and conv1d_state recordings against
dash-conformance's bounds (conv1d.rs:210-229, conv1d_state.rs:230-245); larger packed and batched
calls (every kernel path: 16-byte channel vectors, one channel per thread, widths 1..8 and the
window of 16) against the f64 oracle on the same inputs; determinism; packed against one call per
sequence; a prefill then decoding steps, in place and not.

Tolerance for the larger calls: max|a - e| / max|e| at most 2e-6 for f32 (5e-6 for the weight's
and the bias's sums over thousands of steps), and 1e-2 for bf16/f16 (one rounding of the f32
result, half a bf16 ulp = 2^-9 of the largest value, plus the f32 sums); final states and the
states the step moves are exact.
"""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
import oracle
from conv1d_cases import bound, cases, state_bound, state_cases, to_dtype
from fixtures import errors

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _act(silu):
    return dm.Activation.SILU if silu else dm.Activation.NONE


def _g(a, dtype=torch.float32):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dtype).cuda()


def _n(t):
    return None if t is None else t.float().cpu().numpy()


@pytest.mark.parametrize("case", [c for c in cases() if not c.step], ids=lambda c: c.name)
def test_sequences_against_recordings(case):
    print(f"conv1d sequence case {case.name}", flush=True)
    dt = TD[case.dtype]
    x, w, b = _g(case["x"], dt), _g(case["weight"], dt), _g(case.bias, dt)
    opts = dm.CausalConv1dOptions(activation=_act(case.silu))
    out, _ = dm.causal_conv1d(x, w, b, None, None, opts)
    gx, gw, gb, _ = dm.causal_conv1d_backward(x, w, b, None, None, _g(case["grad_out"]), None,
                                              opts)
    torch.cuda.synchronize()
    assert out.dtype == dt and gx.dtype == dt and gw.dtype == dt
    parts = {"out": out, "grad_x": gx, "grad_weight": gw}
    if case.has_bias:
        parts["grad_bias"] = gb
    for part, value in parts.items():
        _, rel = errors(_n(value), case[part])
        assert rel <= bound(case.dtype, part), (part, rel)


@pytest.mark.parametrize("case", [c for c in cases() if c.step], ids=lambda c: c.name)
def test_steps_against_recordings(case):
    print(f"conv1d step case {case.name}", flush=True)
    dt = TD[case.dtype]
    out, nxt = dm.causal_conv1d_update(_g(case["x"], dt), _g(case["weight"], dt),
                                       _g(case.bias, dt), _g(case.state),
                                       dm.CausalConv1dStepOptions(_act(case.silu)))
    torch.cuda.synchronize()
    _, rel = errors(_n(out), case["out"])
    assert rel <= bound(case.dtype, "step"), rel
    np.testing.assert_array_equal(case.recorded_layout(_n(nxt)), case["new_state"])


@pytest.mark.parametrize("case", state_cases(), ids=lambda c: c.name)
def test_states_and_packed_against_recordings(case):
    print(f"conv1d state case {case.name}", flush=True)
    dt = TD[case.dtype]
    x, w, b = _g(case["x"], dt), _g(case["weight"], dt), _g(case.bias, dt)
    h0 = _g(case.h0)
    cu = None if case.cu is None else torch.from_numpy(case.cu)
    opts = dm.CausalConv1dOptions(activation=_act(case.silu))
    if case.w_out is not None:
        opts = opts.with_final_state_len(case.w_out)
    out, fin = dm.causal_conv1d(x, w, b, h0, cu, opts)
    gx, gw, gb, gh = dm.causal_conv1d_backward(x, w, b, h0, cu, _g(case["grad_out"]),
                                               _g(case.grad_final), opts)
    torch.cuda.synchronize()
    parts = {"out": out, "grad_x": gx, "grad_weight": gw}
    if case.w_out is not None:
        parts["final_state"] = fin
    if case.has_bias:
        parts["grad_bias"] = gb
    if case.w is not None:
        parts["grad_initial_state"] = gh
    for part, value in parts.items():
        _, rel = errors(_n(value), case[part])
        assert rel <= state_bound(case.dtype, part), (part, rel)


def _random_call(seed, dtype, b, t, c, k, lens=None, w=None, w_out=None, bias=True, silu=True):
    rng = np.random.default_rng(seed)
    tt = sum(lens) if lens is not None else t
    bb = 1 if lens is not None else b
    cu = None if lens is None else np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    s = len(lens) if lens is not None else b
    x = to_dtype(rng.standard_normal((bb, tt, c)), dtype)
    wt = to_dtype(rng.standard_normal((c, k)) * 0.5, dtype)
    bs = to_dtype(rng.standard_normal(c), dtype) if bias else None
    h0 = rng.standard_normal((s, w, c)).astype(np.float32) if w is not None else None
    go = rng.standard_normal((bb, tt, c)).astype(np.float32)
    gf = rng.standard_normal((s, w_out, c)).astype(np.float32) if w_out is not None else None
    return x, wt, bs, h0, cu, go, gf


BIG = [
    # dtype, b, t, c, k, packed lengths, W, W', bias, silu
    ("bf16", 2, 1500, 256, 4, None, 3, 3, True, True),         # 16-byte vectors, K = 4
    ("bf16", 1, 0, 96, 3, [0, 700, 3, 0, 129, 1, 64, 2000], 4, 5, False, True),  # packed
    ("f32", 3, 999, 64, 2, None, None, 1, True, False),        # f32 vectors, no states
    ("f16", 2, 517, 100, 5, None, 6, 6, True, True),           # one channel per thread
    ("bf16", 1, 0, 128, 12, [300, 0, 77, 1024], 11, 13, True, True),  # widths above 8
    ("f32", 2, 640, 40, 8, None, 7, 2, False, True),           # K = 8, f32 vectors
    # no steps at all: only the states' rows of the launches run
    ("bf16", 1, 0, 64, 4, [0, 0, 0], 3, 4, True, True),
    # 2500 short sequences: more states' blocks than the launches' 4096 rows of them hold
    ("f16", 1, 0, 16, 3, [i % 5 for i in range(2500)], 2, 3, True, False),
]


@pytest.mark.parametrize("dtype,b,t,c,k,lens,w,w_out,bias,silu", BIG)
def test_larger_calls_against_oracle(dtype, b, t, c, k, lens, w, w_out, bias, silu):
    print(f"conv1d large case {dtype} b={b} t={t} c={c} k={k} lens={lens} w={w} w_out={w_out}",
          flush=True)
    x, wt, bs, h0, cu, go, gf = _random_call(7 + k, dtype, b, t, c, k, lens, w, w_out, bias, silu)
    dt = TD[dtype]
    opts = dm.CausalConv1dOptions(activation=_act(silu))
    if w_out is not None:
        opts = opts.with_final_state_len(w_out)
    cut = None if cu is None else torch.from_numpy(cu)
    out, fin = dm.causal_conv1d(_g(x, dt), _g(wt, dt), _g(bs, dt), _g(h0), cut, opts)
    grads = dm.causal_conv1d_backward(_g(x, dt), _g(wt, dt), _g(bs, dt), _g(h0), cut, _g(go),
                                      _g(gf), opts)
    grads2 = dm.causal_conv1d_backward(_g(x, dt), _g(wt, dt), _g(bs, dt), _g(h0), cut, _g(go),
                                       _g(gf), opts)
    torch.cuda.synchronize()
    eo, ef = oracle.conv1d_fwd(x, wt, bs, h0, cu, silu, w_out, precision="f64")
    eg = oracle.conv1d_bwd(x, wt, bs, h0, go, gf, cu, silu, precision="f64")
    tol = 1e-2 if dtype != "f32" else 2e-6
    _, rel = errors(_n(out), eo)
    assert rel <= tol, ("out", rel)
    if w_out is not None:
        np.testing.assert_array_equal(_n(fin), ef)
    for name, a, e in zip(["grad_x", "grad_weight", "grad_bias", "grad_initial_state"], grads, eg):
        if e is None:
            assert a is None
            continue
        t_ = tol if dtype != "f32" or name == "grad_x" else 5e-6
        if name == "grad_initial_state":
            t_ = 2e-6
        _, rel = errors(_n(a), e)
        assert rel <= t_, (name, rel)
    # deterministic: the same call twice gives the same bits
    for a, a2 in zip(grads, grads2):
        if a is not None:
            assert torch.equal(a, a2)


def test_packed_equals_calls():
    """Packed sequences against one call each: outputs, final states, the input and the initial
    states' gradients bit for bit (each is computed per element the same way)."""
    lens = [0, 300, 1, 0, 64, 129, 7]
    x, wt, bs, h0, cu, go, gf = _random_call(11, "bf16", 1, 0, 64, 4, lens, 3, 3)
    dt = torch.bfloat16
    opts = dm.CausalConv1dOptions(activation=dm.Activation.SILU).with_final_state_len(3)
    out, fin = dm.causal_conv1d(_g(x, dt), _g(wt, dt), _g(bs, dt), _g(h0), torch.from_numpy(cu),
                                opts)
    gx, _, _, gh = dm.causal_conv1d_backward(_g(x, dt), _g(wt, dt), _g(bs, dt), _g(h0),
                                             torch.from_numpy(cu), _g(go), _g(gf), opts)
    for s, (a, e) in enumerate(zip(cu[:-1], cu[1:])):
        o1, f1 = dm.causal_conv1d(_g(x[:, a:e], dt), _g(wt, dt), _g(bs, dt), _g(h0[s:s + 1]),
                                  None, opts)
        g1 = dm.causal_conv1d_backward(_g(x[:, a:e], dt), _g(wt, dt), _g(bs, dt),
                                       _g(h0[s:s + 1]), None, _g(go[:, a:e]), _g(gf[s:s + 1]),
                                       opts)
        assert torch.equal(out[:, a:e], o1)
        assert torch.equal(fin[s:s + 1], f1)
        assert torch.equal(gx[:, a:e], g1[0])
        assert torch.equal(gh[s:s + 1], g1[3])


@pytest.mark.parametrize("in_place", [False, True])
def test_prefill_then_steps(in_place):
    """A prefill's final state, then single steps to the end, give the whole sequence's outputs
    (conv1d.rs:382-486) and leave the last inputs as the state."""
    rng = np.random.default_rng(13)
    b, t, c, k, w = 3, 40, 48, 4, 6
    dt = torch.bfloat16
    x = to_dtype(rng.standard_normal((b, t, c)), "bf16")
    wt = to_dtype(rng.standard_normal((c, k)), "bf16")
    bs = to_dtype(rng.standard_normal(c), "bf16")
    opts = dm.CausalConv1dOptions(activation=dm.Activation.SILU)
    whole, _ = dm.causal_conv1d(_g(x, dt), _g(wt, dt), _g(bs, dt), None, None, opts)
    _, state = dm.causal_conv1d(_g(x[:, :17], dt), _g(wt, dt), _g(bs, dt), None, None,
                                opts.with_final_state_len(w))
    step = dm.CausalConv1dStepOptions.from_sequence(opts)
    outs = []
    for i in range(17, t):
        o, nxt = dm.causal_conv1d_update(_g(x[:, i], dt), _g(wt, dt), _g(bs, dt), state, step,
                                         in_place=in_place)
        if in_place:
            assert nxt.data_ptr() == state.data_ptr()
        state = nxt
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(torch.stack(outs, 1), whole[:, 17:])
    np.testing.assert_array_equal(_n(state), x[:, t - w:])


def test_refusals():
    x = torch.zeros(2, 5, 8, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(8, 4, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(dm.Unsupported, match="causal_conv1d: x and weight must share one dtype"):
        dm.causal_conv1d(x, w.float())
    with pytest.raises(dm.Unsupported, match="cannot feed a kernel of width 4"):
        dm.causal_conv1d(x, w, None, torch.zeros(2, 2, 8, device="cuda"))
    with pytest.raises(dm.Unsupported, match="packed sequences lie along T of a batch of one"):
        dm.causal_conv1d(x, w, None, None, torch.tensor([0, 5]))
    with pytest.raises(dm.Unsupported, match="kernel widths above 16"):
        dm.causal_conv1d(x, torch.zeros(8, 17, dtype=torch.bfloat16, device="cuda"))


def test_update_batch_above_one_launch():
    """A decoding step over 70,000 rows: more rows than one launch's grid holds (65,535), so the
    rows go in two launches; checked against the f64 oracle (1e-2) and the exact next state."""
    b, c, k, w = 70000, 8, 3, 2
    print(f"conv1d update b={b} c={c} k={k} w={w}", flush=True)
    gen = torch.Generator().manual_seed(71)
    x = torch.randn(b, c, generator=gen).to(torch.bfloat16)
    wt = (0.5 * torch.randn(c, k, generator=gen)).to(torch.bfloat16)
    bs = torch.randn(c, generator=gen).to(torch.bfloat16)
    state = torch.randn(b, w, c, generator=gen)
    opts = dm.CausalConv1dStepOptions(activation=dm.Activation.SILU)
    out, nxt = dm.causal_conv1d_update(x.cuda(), wt.cuda(), bs.cuda(), state.cuda(), opts)
    torch.cuda.synchronize()
    eo, en = oracle.conv1d_update(x.float().numpy(), wt.float().numpy(), bs.float().numpy(),
                                  state.numpy(), True, precision="f64")
    _, rel = errors(_n(out), eo)
    assert rel <= 1e-2, rel
    np.testing.assert_array_equal(_n(nxt), en)
