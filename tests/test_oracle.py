"""The CPU oracle pinned to the reference's recorded fixtures and to brute force (no GPU).

Each check below fails on a plausible mistake in the restatement: a wrong mask index or
alignment (the 8 mask records, the brute-force mask comparison), a dropped gradient term (every
gradient of every record), a wrong decay, cumsum or inverse (the chunk fixtures against
transformers' and fla's outputs), a wrong packing (packed against per-sequence, to the bit).
"""
import numpy as np
import pytest

import conformance as cf
import oracle
from oracle_adapter import OracleAdapter


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.set_threads(4)


@pytest.mark.parametrize("precision", ["f32", "f64"])
def test_attention_matches_torch_f32(precision):
    # f32 arithmetic in another summation order than Flex's: held to the autotune bounds, the
    # loosest f32 bounds dash-conformance accepts for a reference (attention.rs:94-97)
    worst, compared = cf.matches_torch(OracleAdapter(precision), "oracle", "f32", True,
                                       cf.AUTOTUNE_F32)
    assert compared == 10


@pytest.mark.parametrize("dtype,bounds", [("bf16", cf.BF16), ("f16", cf.F16)])
def test_attention_matches_torch_low_precision(dtype, bounds):
    # the kernels' bounds for the dtype, no tighter than the f32 reference's own rounding
    loose = cf.Bounds(tuple(map(max, bounds.causal, cf.AUTOTUNE_F32.causal)),
                      tuple(map(max, bounds.masks, cf.AUTOTUNE_F32.masks)))
    worst, compared = cf.matches_torch(OracleAdapter("f32"), "oracle", dtype, True, loose)
    assert compared == 10


def test_attention_without_gradients():
    cf.without_gradients(OracleAdapter(), "oracle", cf.AUTOTUNE_F32)


def test_decoding_is_attention_with_one_query():
    # dash-ops' reference decodes to the bit without lengths, within 1e-6 with them
    # (crates/dash-ops/tests/attention_masks.rs:727-732)
    cf.decoding_is_attention_with_one_query(OracleAdapter(), "oracle", [0.0, 1e-6])


def _brute_visible(b, tq, tk, causal, left, right, padding=None, cu_q=None, cu_k=None):
    """Which keys each query sees, from the contract's definitions alone
    (crates/dash-contract/src/attention.rs:33-58), by enumeration."""
    vis = np.zeros((b, tq, tk), bool)
    if cu_q is None:
        seqs = [(0, tq, 0, tk)]
    else:
        seqs = [(cu_q[s], cu_q[s + 1], cu_k[s], cu_k[s + 1]) for s in range(len(cu_q) - 1)]
    for bi in range(b):
        for qs, qe, ks, ke in seqs:
            lq, lk = qe - qs, ke - ks
            for i in range(qs, qe):
                pos = (i - qs) + lk - lq
                for j in range(ks, ke):
                    rel = j - ks
                    if (causal or right is not None) and rel > pos + (0 if causal else right):
                        continue
                    if left is not None and rel < pos - left:
                        continue
                    if padding is not None and padding[bi, j]:
                        continue
                    vis[bi, i, j] = True
    return vis


@pytest.mark.parametrize("case", range(40))
def test_mask_closed_form_against_enumeration(case):
    rng = np.random.default_rng(case)
    tq, tk = int(rng.integers(1, 20)), int(rng.integers(1, 20))
    causal = bool(rng.integers(0, 2))
    left = None if rng.random() < 0.4 else int(rng.integers(0, 8))
    right = None if rng.random() < 0.4 else int(rng.integers(0, 8))
    kind = case % 3
    padding = cu_q = cu_k = None
    b = 1
    if kind == 1:
        b = 2
        padding = rng.random((b, tk)) < 0.3
        mask = ("padding", padding)
    elif kind == 2:
        s = int(rng.integers(1, 4))
        cu_q = np.concatenate([[0], np.sort(rng.integers(0, tq + 1, s))]).astype(np.int64)
        cu_k = np.concatenate([[0], np.sort(rng.integers(0, tk + 1, s))]).astype(np.int64)
        mask = ("packed", cu_q, cu_k)
    else:
        mask = None
    q = np.zeros((b, tq, 1, 8), np.float32)
    k = np.zeros((b, tk, 1, 8), np.float32)
    call = oracle.AttentionCall(q, k, k, mask, causal, None, left, right)
    want = _brute_visible(b, tq, tk, causal, left, right, padding, cu_q, cu_k)
    for bi in range(b):
        assert np.array_equal(call.visible_matrix(bi), want[bi])


def test_chunk_f32_cases():
    cf.check_chunk_f32_cases(OracleAdapter("f32"), "oracle-f32")


def test_chunk_f32_cases_f64_oracle():
    cf.check_chunk_f32_cases(OracleAdapter("f64"), "oracle-f64")


def test_chunk_bf16_case():
    cf.check_chunk_bf16_case(OracleAdapter("f32"), "oracle", cf.CHUNK_BF16_TOL)


def test_chunk_packed_f32():
    cf.check_chunk_packed_f32(OracleAdapter("f32"), "oracle")


def test_chunk_packed_bf16():
    cf.check_chunk_packed_bf16(OracleAdapter("f32"), "oracle", cf.BF16_VS_F64)


@pytest.mark.parametrize("name", cf.CHUNK_PACKED_F32)
def test_chunk_packed_equals_per_sequence(name):
    assert cf.packed_against_sequences(OracleAdapter("f32"), name, "oracle") == 0.0


def test_steps():
    cf.check_steps(OracleAdapter("f32"), "oracle")
    cf.check_f32_steps(OracleAdapter("f32"), "oracle")
    cf.check_prefill_then_decode(OracleAdapter("f32"), "oracle")
    cf.check_bf16_step(OracleAdapter("f32"), "oracle")


def test_chunk_continues_into_step():
    """The state a chunked pass leaves is what the step continues from: chunked over T tokens
    equals chunked over T-1 then one step (crates/dash-contract/src/gated_delta.rs:11-30)."""
    rng = np.random.default_rng(7)
    t, h, dk, dv = 70, 2, 16, 8
    q, k = rng.standard_normal((2, 1, t, h, dk)).astype(np.float32)
    v = rng.standard_normal((1, t, h, dv)).astype(np.float32)
    g = -np.log1p(np.exp(rng.standard_normal((1, t, h)))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((1, t, h))))).astype(np.float32)
    h0 = (0.1 * rng.standard_normal((1, h, dk, dv))).astype(np.float32)
    out, fin = oracle.gdr_chunk_fwd(q, k, v, g, beta, h0, l2norm=True, precision="f64")
    out1, fin1 = oracle.gdr_chunk_fwd(q[:, :-1], k[:, :-1], v[:, :-1], g[:, :-1], beta[:, :-1],
                                      h0, l2norm=True, precision="f64")
    o2, st = oracle.gdr_step(q[:, -1], k[:, -1], v[:, -1], g[:, -1], beta[:, -1], fin1,
                             l2norm=True, precision="f64")
    np.testing.assert_allclose(out[:, :-1], out1, rtol=0, atol=1e-5)
    np.testing.assert_allclose(out[:, -1], o2, rtol=0, atol=1e-5)
    np.testing.assert_allclose(fin, st, rtol=0, atol=1e-5)


@pytest.mark.parametrize("precision", ["f32", "f64"])
def test_step_gradients(precision):
    """dash-conformance's check_gradients (torch autograd through one step) and
    check_step_gradients (packed steps against float64) on the oracle's step backward."""
    assert cf.check_gradients(OracleAdapter(precision), f"oracle-{precision}")
    assert cf.check_step_gradients(OracleAdapter(precision), f"oracle-{precision}") == 2


def test_default_scale():
    assert cf.the_default_scale_is_one_over_the_root_of_dk(OracleAdapter("f32"), "oracle")


@pytest.mark.parametrize("l2norm", [False, True])
def test_step_gradients_finite_differences(l2norm):
    """The step backward in f64 against central differences of the f64 step: the loss
    sum(out * d_out) + sum(new_state * d_state) over packed sequences of 3, 0, 1 and 4 tokens,
    each input perturbed one element at a time. Independent of the fixtures: a dropped term, a
    wrong sign or a transposed product shows here."""
    rng = np.random.default_rng(11)
    cu = np.array([0, 3, 3, 4, 8], np.int64)
    t, s, h, dk, dv = 8, 4, 2, 5, 3
    q, k = rng.standard_normal((2, t, h, dk))
    v = rng.standard_normal((t, h, dv))
    g = -np.log1p(np.exp(rng.standard_normal((t, h))))
    beta = 1 / (1 + np.exp(-rng.standard_normal((t, h))))
    st = 0.3 * rng.standard_normal((s, h, dk, dv))
    d_out = rng.standard_normal((t, h, dv))
    d_st = rng.standard_normal((s, h, dk, dv))
    scale = 0.7
    inputs = [q, k, v, g, beta, st]

    def loss(xs):
        # the f64 oracle takes f32 arrays: keep the perturbation exact in f32 by scaling the
        # inputs to values f32 holds exactly is not needed, the tolerance covers it
        out, ns = oracle.gdr_step(*xs, cu=cu, l2norm=l2norm, scale=scale, precision="f64")
        return float(np.sum(out.astype(np.float64) * d_out) + np.sum(ns.astype(np.float64) * d_st))

    grads = oracle.gdr_step_bwd(*inputs, d_out, d_st, cu=cu, l2norm=l2norm, scale=scale,
                                precision="f64")
    eps = 1e-3
    for which, (x, gx) in enumerate(zip(inputs, grads)):
        flat = x.reshape(-1)
        num = np.zeros(flat.size)
        for i in range(flat.size):
            keep = flat[i]
            flat[i] = keep + eps
            lp = loss(inputs)
            flat[i] = keep - eps
            lm = loss(inputs)
            flat[i] = keep
            num[i] = (lp - lm) / (2 * eps)
        np.testing.assert_allclose(gx.reshape(-1), num, rtol=2e-3, atol=2e-3,
                                   err_msg=f"input {which}")
    # the empty sequence passes the state's gradient through
    np.testing.assert_array_equal(grads[5][1], d_st[1].astype(np.float32))
