"""Seeded random shapes, masks and packings for the hot path's operations on the GPU, each
against the f64 oracle with the bounds of its dedicated tests: attention forward and backward
(test_gpu_attention_sweep.py), the chunked gated delta rule forward and backward
(test_gpu_gdr_mfma.py), decode (test_gpu_decode.py), the recurrent step (test_gpu_step_grad.py)
and the causal conv1d and its decoding step (test_gpu_conv1d.py). Each case prints its draw before the GPU call, so a failure names
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


@pytest.mark.parametrize("seed", range(8))
def test_random_chunk_gated_delta_rule_backward(seed):
    """Bounds of test_gpu_gdr_mfma.py's backward (the reference's own for its tensor-core kernels
    at [1, 200, 2, 128, 128]: 7.5e-3 with the l2 normalisation, 1.2e-2 without), taken 1.5 times
    for packings of up to four sequences of up to 300 tokens."""
    rng = np.random.default_rng(7500 + seed)
    n = int(rng.integers(1, 5))
    lens = [int(x) for x in rng.integers(0, 300, n)]
    if sum(lens) == 0:
        lens[-1] = 1
    h = int(rng.integers(1, 3))
    l2norm = bool(rng.random() < 0.5)
    states = bool(rng.random() < 0.6)
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    tol = 1.5 * (7.5e-3 if l2norm else 1.2e-2)
    print(f"random chunk GDR backward lens={lens} h={h} l2norm={l2norm} states={states} {dtype}",
          flush=True)
    T, D = sum(lens), 128
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    s0 = 7600 + seed * 10
    q = syn.normal(s0, (1, T, h, D), "cuda")
    k = syn.normal(s0 + 1, (1, T, h, D), "cuda")
    if not l2norm:
        q, k = syn.l2norm(q), syn.l2norm(k)
    v = syn.normal(s0 + 2, (1, T, h, D), "cuda")
    g = -torch.nn.functional.softplus(syn.normal(s0 + 3, (1, T, h), "cuda"))
    beta = torch.sigmoid(syn.normal(s0 + 4, (1, T, h), "cuda"))
    h0 = syn.normal(s0 + 5, (n, h, D, D), "cuda", std=0.1) if states else None
    do = syn.normal(s0 + 6, (1, T, h, D), "cuda").to(dtype)
    dfin = syn.normal(s0 + 7, (n, h, D, D), "cuda", std=0.1) if states else None
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    _lib.probe_reset()
    opts = dm.ChunkGatedDeltaOptions(qk_l2norm=l2norm, output_final_state=True)
    r = dm.chunk_gated_delta_rule_backward(q, k, v, g, beta, h0, cu.cuda(), do, dfin, opts)
    torch.cuda.synchronize()
    assert _lib.probe_counts()["gdr_chunk_bwd_mfma"] > 0
    e = oracle.gdr_chunk_bwd(host(q), host(k), host(v), host(g), host(beta),
                             None if h0 is None else host(h0), host(do),
                             None if dfin is None else host(dfin), cu.numpy(), l2norm,
                             precision="f64")
    names = ["dq", "dk", "dv", "dg", "dbeta", "dh0"]
    if h0 is None:
        names, r, e = names[:5], r[:5], e[:5]
    for name, a_, e_ in zip(names, r, e):
        rr = errors(host(a_), e_)[1]
        print(f"  {name}: rel {rr:.2e} (bound {tol:.1e})")
        assert rr <= tol, (name, rr)


@pytest.mark.parametrize("seed", range(8))
def test_random_conv1d(seed):
    """The conv1d forward and backward (test_gpu_conv1d.py's bounds: 1e-2 for 16-bit inputs,
    2e-6 for f32; the final states bit-equal)."""
    from test_gpu_conv1d import TD, _act, _g, _n, _random_call
    rng = np.random.default_rng(7700 + seed)
    dtype = str(rng.choice(["bf16", "f16", "f32"]))
    k = int(rng.integers(1, 9))
    c = int(rng.choice([8, 40, 64, 96, 128, 264]))
    packed = bool(rng.random() < 0.5)
    lens = [int(x) for x in rng.integers(0, 400, int(rng.integers(1, 5)))] if packed else None
    b = 1 if packed else int(rng.integers(1, 4))
    t = 0 if packed else int(rng.integers(1, 600))
    w = None if rng.random() < 0.3 else int(rng.integers(k - 1 if k > 1 else 1, k + 4))
    w_out = None if rng.random() < 0.3 else int(rng.integers(1, k + 4))
    bias, silu = bool(rng.random() < 0.5), bool(rng.random() < 0.6)
    print(f"random conv1d {dtype} b={b} t={t} c={c} k={k} lens={lens} w={w} w_out={w_out} "
          f"bias={bias} silu={silu}", flush=True)
    x, wt, bs, h0, cu, go, gf = _random_call(7800 + seed, dtype, b, t, c, k, lens, w, w_out, bias,
                                             silu)
    dt = TD[dtype]
    opts = dm.CausalConv1dOptions(activation=_act(silu))
    if w_out is not None:
        opts = opts.with_final_state_len(w_out)
    cut = None if cu is None else torch.from_numpy(cu)
    out, fin = dm.causal_conv1d(_g(x, dt), _g(wt, dt), _g(bs, dt), _g(h0), cut, opts)
    grads = dm.causal_conv1d_backward(_g(x, dt), _g(wt, dt), _g(bs, dt), _g(h0), cut, _g(go),
                                      _g(gf), opts)
    torch.cuda.synchronize()
    eo, ef = oracle.conv1d_fwd(x, wt, bs, h0, cu, silu, w_out, precision="f64")
    eg = oracle.conv1d_bwd(x, wt, bs, h0, go, gf, cu, silu, precision="f64")
    tol = 1e-2 if dtype != "f32" else 2e-6
    assert errors(_n(out), eo)[1] <= tol
    if w_out is not None:
        np.testing.assert_array_equal(_n(fin), ef)
    for name, a, e in zip(["grad_x", "grad_weight", "grad_bias", "grad_initial_state"], grads, eg):
        if e is None:
            assert a is None
            continue
        t_ = tol if dtype != "f32" or name == "grad_x" else 5e-6
        if name == "grad_initial_state":
            t_ = 2e-6
        rel = errors(_n(a), e)[1]
        print(f"  {name}: rel {rel:.2e} (bound {t_:.1e})")
        assert rel <= t_, (name, rel)


@pytest.mark.parametrize("seed", range(8))
def test_random_gated_delta_step(seed):
    """The recurrent step over random packings (several tokens per sequence, empty sequences),
    widths and options, against the f64 oracle (test_gpu_step_grad.py's bounds: 1e-5 for f32
    inputs, 1e-2 for bf16; the new states 1e-5)."""
    rng = np.random.default_rng(7900 + seed)
    n = int(rng.integers(1, 6))
    lens = [int(x) for x in rng.integers(0, 6, n)]
    if sum(lens) == 0:
        lens[0] = 1
    h = int(rng.integers(1, 4))
    dk = int(rng.choice([16, 32, 64, 128]))
    dv = int(rng.choice([8, 13, 64, 96, 128]))
    l2norm = bool(rng.random() < 0.5)
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
    print(f"random step lens={lens} h={h} dk={dk} dv={dv} l2norm={l2norm} {dtype}", flush=True)
    t = sum(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    gen = torch.Generator().manual_seed(8000 + seed)
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    q, k, v = rn(t, h, dk).to(dtype), rn(t, h, dk).to(dtype), rn(t, h, dv).to(dtype)
    g = -torch.nn.functional.softplus(rn(t, h))
    beta = torch.sigmoid(rn(t, h)).to(dtype)
    st = 0.3 * rn(n, h, dk, dv)
    scale = None if l2norm else 0.4
    opts = dm.GatedDeltaStepOptions(qk_l2norm=l2norm, scale=scale)
    args = [x.cuda() for x in (q, k, v, g, beta, st)]
    out, ns = dm.gated_delta_step(*args, torch.as_tensor(cu, dtype=torch.int32).cuda(), opts)
    torch.cuda.synchronize()
    sc = scale if scale is not None else float(np.float32(1 / np.sqrt(dk)))
    eo, es = oracle.gdr_step(*(x.float().numpy() for x in (q, k, v, g, beta, st)), cu=cu,
                             l2norm=l2norm, scale=sc, precision="f64")
    ro, rs = errors(host(out), eo)[1], errors(host(ns), es)[1]
    print(f"  out {ro:.2e} state {rs:.2e}")
    assert ro <= (1e-5 if dtype == torch.float32 else 1e-2) and rs <= 1e-5


@pytest.mark.parametrize("seed", range(6))
def test_random_conv1d_update(seed):
    """The conv1d decoding step against the f64 oracle (1e-2 for 16-bit inputs, 2e-6 for f32;
    the next state exact: it only shifts values)."""
    rng = np.random.default_rng(8100 + seed)
    dtype = str(rng.choice(["bf16", "f16", "f32"]))
    b, c, k = int(rng.integers(1, 9)), int(rng.choice([8, 40, 128, 264])), int(rng.integers(1, 9))
    w = int(rng.integers(max(k - 1, 1), k + 4))
    bias, silu = bool(rng.random() < 0.5), bool(rng.random() < 0.6)
    print(f"random conv1d update {dtype} b={b} c={c} k={k} w={w} bias={bias} silu={silu}",
          flush=True)
    td = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    gen = torch.Generator().manual_seed(8200 + seed)
    x = torch.randn(b, c, generator=gen).to(td)
    wt = (0.5 * torch.randn(c, k, generator=gen)).to(td)
    bs = torch.randn(c, generator=gen).to(td) if bias else None
    state = torch.randn(b, w, c, generator=gen)
    opts = dm.CausalConv1dStepOptions(
        activation=dm.Activation.SILU if silu else dm.Activation.NONE)
    out, nxt = dm.causal_conv1d_update(x.cuda(), wt.cuda(), None if bs is None else bs.cuda(),
                                       state.cuda(), opts)
    torch.cuda.synchronize()
    eo, en = oracle.conv1d_update(x.float().numpy(), wt.float().numpy(),
                                  None if bs is None else bs.float().numpy(), state.numpy(),
                                  silu, precision="f64")
    assert errors(host(out), eo)[1] <= (2e-6 if dtype == "f32" else 1e-2)
    np.testing.assert_array_equal(host(nxt), en)
