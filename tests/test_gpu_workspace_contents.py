"""Results do not depend on what the caller's workspace held: each entry point runs twice, once
with its workspace filled with 0xFF bytes (NaN as f32, -1 as int32) and once with zeros, and the
two results must be equal to the bit. This covers the accumulators that the first product writes
with beta = 0 (the linear cross-entropy's weight and hidden gradients, never cleared), the
partials, plans and per-chunk intermediates of every other workspace user."""
import pytest
import torch

import dashmag_amd as dm
from dashmag_amd import ops, synthetic as syn

pytestmark = pytest.mark.gpu


def _twice(fn):
    """fn() under a workspace of 0xFF bytes, then of zeros."""
    real = ops._workspace
    out = []
    for fill in (0xFF, 0):
        def ws(nbytes, device, fill=fill):
            return torch.full((max(int(nbytes), 1),), fill, dtype=torch.uint8, device=device)
        ops._workspace = ws
        try:
            r = fn()
            torch.cuda.synchronize()
            out.append(r)
        finally:
            ops._workspace = real
    return out


def _equal(a, b):
    if isinstance(a, (tuple, list)):
        assert len(a) == len(b)
        for x, y in zip(a, b):
            _equal(x, y)
    elif a is None:
        assert b is None
    else:
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_linear_cross_entropy(dtype):
    n, d, v = 300, 256, 5000
    h = syn.normal(1, (n, d), "cuda").to(dtype)
    w = (0.05 * syn.normal(2, (v, d), "cuda")).to(dtype)
    t = (torch.arange(n, device="cuda") * 37 % v).to(torch.int64)
    opts = dm.CrossEntropyOptions(label_smoothing=0.1, z_loss=1e-4, masked=(3, 7),
                                  chunks=dm.LogprobOptions(vocab_chunk=1024, row_chunk=128))
    _, _, _, rows = dm.linear_cross_entropy(h, w, t, opts)
    up = torch.ones(3, n)

    def run():
        return dm.linear_cross_entropy_backward(h, w, t, rows, up, opts)
    a, b = _twice(run)
    _equal(a, b)
    assert torch.isfinite(a[0].float()).all() and torch.isfinite(a[1].float()).all()


def test_logprob_with_grad():
    n, d, v = 200, 128, 3000
    h = syn.normal(3, (n, d), "cuda").bfloat16()
    w = (0.05 * syn.normal(4, (v, d), "cuda")).bfloat16()
    t = (torch.arange(n, device="cuda") * 13 % v).to(torch.int64)
    opts = dm.LogprobOptions(vocab_chunk=1024, row_chunk=64)
    a, b = _twice(lambda: dm.chosen_logprob_with_grad(h, w, t, (5,), opts))
    _equal(a, b)


def test_attention_and_decode():
    q = syn.normal(5, (1, 700, 4, 128), "cuda").bfloat16()
    k = syn.normal(6, (1, 700, 2, 128), "cuda").bfloat16()
    v = syn.normal(7, (1, 700, 2, 128), "cuda").bfloat16()
    do = syn.normal(8, (1, 700, 4, 128), "cuda").bfloat16()
    cu = torch.tensor([0, 300, 700], dtype=torch.int32, device="cuda")
    mask = dm.AttentionMask.packed(cu, cu)
    opts = dm.AttentionOptions(causal=True)

    def attn():
        o, lse = dm.attention_with_lse(q, k, v, mask, opts)
        return (o, lse) + tuple(dm.attention_backward(q, k, v, o, lse, do, mask, opts))
    a, b = _twice(attn)
    _equal(a, b)
    lens = torch.tensor([700, 1, 0, 333], dtype=torch.int32, device="cuda")
    qd = syn.normal(9, (4, 8, 256), "cuda").bfloat16()
    kc = syn.normal(10, (4, 700, 2, 256), "cuda").bfloat16()
    vc = syn.normal(11, (4, 700, 2, 256), "cuda").bfloat16()
    a, b = _twice(lambda: dm.attention_decode(qd, kc, vc, lens))
    _equal(a, b)


def test_gated_delta_rule_and_conv1d():
    lens = [70, 1, 200, 130]
    t = sum(lens)
    cu = torch.tensor([0, 70, 71, 271, 401], dtype=torch.int32, device="cuda")
    q = syn.normal(12, (1, t, 2, 128), "cuda").bfloat16()
    k = syn.normal(13, (1, t, 2, 128), "cuda").bfloat16()
    v = syn.normal(14, (1, t, 2, 128), "cuda").bfloat16()
    g = -torch.nn.functional.softplus(syn.normal(15, (1, t, 2), "cuda"))
    beta = torch.sigmoid(syn.normal(16, (1, t, 2), "cuda"))
    h0 = syn.normal(17, (4, 2, 128, 128), "cuda", std=0.1)
    do = syn.normal(18, (1, t, 2, 128), "cuda").bfloat16()
    opts = dm.ChunkGatedDeltaOptions(qk_l2norm=True, output_final_state=True)

    def gdr():
        return (tuple(dm.chunk_gated_delta_rule(q, k, v, g, beta, h0, cu, opts)) +
                tuple(dm.chunk_gated_delta_rule_backward(q, k, v, g, beta, h0, cu, do, None, opts)))
    a, b = _twice(gdr)
    _equal(a, b)
    x = syn.normal(19, (1, t, 256), "cuda").bfloat16()
    wc = syn.normal(20, (256, 4), "cuda").bfloat16()
    gy = syn.normal(21, (1, t, 256), "cuda").bfloat16()
    copts = dm.CausalConv1dOptions(activation=dm.Activation.SILU)
    a, b = _twice(lambda: dm.causal_conv1d_backward(x, wc, None, None, cu, gy, None, copts))
    _equal(a, b)


def test_gated_delta_step_backward():
    """The step backward's kept states and per-slice partial sums."""
    cu = torch.tensor([0, 3, 3, 4, 9], dtype=torch.int32, device="cuda")
    q = syn.normal(22, (9, 2, 128), "cuda").bfloat16()
    k = syn.normal(23, (9, 2, 128), "cuda").bfloat16()
    v = syn.normal(24, (9, 2, 128), "cuda").bfloat16()
    g = -torch.nn.functional.softplus(syn.normal(25, (9, 2), "cuda"))
    beta = torch.sigmoid(syn.normal(26, (9, 2), "cuda"))
    st = syn.normal(27, (4, 2, 128, 128), "cuda", std=0.1)
    do = syn.normal(28, (9, 2, 128), "cuda").bfloat16()
    dst = syn.normal(29, (4, 2, 128, 128), "cuda")
    opts = dm.GatedDeltaStepOptions(qk_l2norm=True)
    a, b = _twice(lambda: dm.gated_delta_step_backward(q, k, v, g, beta, st, cu, do, dst, opts))
    _equal(a, b)
