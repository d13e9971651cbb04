"""The host mirror's refusals of malformed offsets and ids, without a GPU: every offset array the
kernels would index rows with is checked on the host first, as dash-ops' ``read_cu_seqlens``
checks it (crates/dash-ops/src/sequences.rs:49-67), and int64 values are never wrapped by the
int32 (or uint32) arrays the C ABI takes. The descriptor builders are called directly with CPU
tensors (they launch nothing)."""
import pytest
import torch

import dashmag_amd as dm
from dashmag_amd import ops
from dashmag_amd.contract import Unsupported


def _attn(cu_q, cu_k, tq=10, tk=10):
    q = torch.zeros(1, tq, 2, 8)
    k = torch.zeros(1, tk, 1, 8)
    mask = dm.AttentionMask.packed(torch.tensor(cu_q), torch.tensor(cu_k))
    return ops._attention_desc("attention", q, k, k, mask, dm.AttentionOptions(), [])


def test_attention_packed_offsets_accepted():
    _attn([0, 4, 10], [0, 3, 10])
    _attn([0, 4, 6], [0, 3, 7])  # positions past the last offset belong to no sequence


@pytest.mark.parametrize("cu_q,cu_k,what", [
    ([1, 4, 10], [0, 3, 10], "cu_seqlens_q"),
    ([0, 6, 4], [0, 3, 10], "cu_seqlens_q"),
    ([0, 4, 11], [0, 3, 10], "cu_seqlens_q"),
    ([0, 4, 10], [0, 3, 12], "cu_seqlens_k"),
    ([0, 4, 10], [0, -1, 10], "cu_seqlens_k"),
])
def test_attention_packed_offsets_refused(cu_q, cu_k, what):
    with pytest.raises(Unsupported, match=f"^attention: {what} must go from 0 to at most T"):
        _attn(cu_q, cu_k)


def _gdr(cu, t=12, step=False):
    if step:
        q = torch.zeros(t, 2, 8)
        g = torch.zeros(t, 2)
    else:
        q = torch.zeros(1, t, 2, 8)
        g = torch.zeros(1, t, 2)
    return ops._gdr_desc("chunk_gated_delta_rule", q, q, q, g, g, torch.tensor(cu), False, None,
                         step, [])


def test_gdr_offsets():
    _gdr([0, 5, 5, 12])
    for bad in ([0, 5, 11], [0, 7, 5, 12], [2, 12], [0, 5, 13]):
        with pytest.raises(Unsupported, match="^chunk_gated_delta_rule: cu_seqlens must go from "
                                              "0 to T = 12 without decreasing"):
            _gdr(bad)
    _gdr([0, 3, 4], t=4, step=True)
    with pytest.raises(Unsupported, match="T = 4"):
        _gdr([0, 3, 5], t=4, step=True)


def test_conv1d_offsets():
    x = torch.zeros(1, 9, 4)
    w = torch.zeros(4, 3)
    ops._conv1d_desc("causal_conv1d", x, w, None, [], torch.tensor([0, 2, 9]), dm.Activation.NONE,
                     [])
    with pytest.raises(Unsupported, match="^causal_conv1d: cu_seqlens must go from 0 to T = 9"):
        ops._conv1d_desc("causal_conv1d", x, w, None, [], torch.tensor([0, 5, 2, 9]),
                         dm.Activation.NONE, [])


def test_int64_offsets_are_not_wrapped():
    big = torch.tensor([0, 1 << 32], dtype=torch.int64)
    with pytest.raises(Unsupported, match="must fit in int32"):
        ops._offsets(big, "cpu", "attention_decode_paged", "the block table")
    with pytest.raises(Unsupported, match="must go from 0 to"):
        _attn([0, (1 << 32) + 4], [0, 10])


def test_cache_lengths():
    assert ops._cache_lengths("attention_decode", torch.tensor([3, 0]), 2, "cpu").tolist() == [3, 0]
    with pytest.raises(Unsupported, match="not negative"):
        ops._cache_lengths("attention_decode", torch.tensor([3, -1]), 2, "cpu")
    with pytest.raises(Unsupported, match="fit in int32"):
        ops._cache_lengths("attention_decode", torch.tensor([1 << 31, 1]), 2, "cpu")


def test_masked_ids_checked_before_the_uint32_cast():
    assert ops._masked_ids("chosen_logprob", [0, 5, 9], 10) == [0, 5, 9]
    with pytest.raises(Unsupported, match="masked token id 4294967299 is not below the "
                                          "vocabulary size 10"):
        ops._masked_ids("chosen_logprob", [(1 << 32) + 3], 10)
    with pytest.raises(Unsupported, match="not negative"):
        ops._masked_ids("linear_cross_entropy", [-1], 10)
