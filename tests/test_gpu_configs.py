"""The HIP path against the CPU oracle on the benchmark's synthetic configs (BASELINE.json
``configs``), at the benchmark's full sizes on the GPU, checked on slices the oracle finishes in
seconds (heads and sequences are independent, so a slice of the full call is a complete check of
those rows), plus size-independent properties at full size.

Tolerances (north star): relative error max|a - e| / max|e| at most 1e-5 for the f32 config and
2e-2 for bf16 inputs with f32 accumulation; integer work (cu_seqlens, cache lengths) exact.
"""
import numpy as np
import pytest
import torch

import dashmag_amd as dm
import oracle
from dashmag_amd import _lib, synthetic as syn
from fixtures import errors

pytestmark = pytest.mark.gpu
BF16_TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.set_threads(16)


def host(x):
    return x.detach().float().cpu().numpy()


def rel(a, e):
    return errors(a, e)[1]


def test_config1_f32_causal_forward():
    q, k, v = (x.cuda() for x in syn.config1())
    o, lse = dm.attention_with_lse(q, k, v, None, dm.AttentionOptions(causal=True))
    call = oracle.AttentionCall(host(q), host(k), host(v), None, True)
    eo, el = oracle.attention_fwd(call, "f64")
    print("config 1 o", rel(host(o), eo), "lse", rel(host(lse), el))
    assert rel(host(o), eo) <= 1e-5
    assert rel(host(lse), el) <= 1e-5


def _attention_slice_check(c, seqs, heads_kv, label):
    """The full call on the GPU; the oracle per sequence (the packed contract is per-sequence
    attention) on the query heads of key-value heads `heads_kv`."""
    q, k, v, do = c["q"], c["k"], c["v"], c["do"]
    cu = c.get("cu_seqlens")
    mask = None if cu is None else dm.AttentionMask.packed(cu, cu)
    opts = dm.AttentionOptions(causal=True)
    o, lse = dm.attention_with_lse(q, k, v, mask, opts)
    dq, dk, dv = dm.attention_backward(q, k, v, o, lse, do, mask, opts)
    torch.cuda.synchronize()
    hq, hkv = q.shape[2], k.shape[2]
    g = hq // hkv
    cuh = [0, q.shape[1]] if cu is None else cu.tolist()
    for s in seqs:
        a, b = cuh[s], cuh[s + 1]
        for kh in heads_kv:
            hs = slice(kh * g, (kh + 1) * g)
            sl = lambda x, h: np.ascontiguousarray(host(x[:, a:b, h]))  # noqa: E731
            call = oracle.AttentionCall(sl(q, hs), sl(k, slice(kh, kh + 1)),
                                        sl(v, slice(kh, kh + 1)), None, True)
            eo, el = oracle.attention_fwd(call)
            gq, gk, gv = oracle.attention_bwd(call, sl(o, hs), host(lse[:, a:b, hs]), sl(do, hs))
            for name, x, e in [("o", sl(o, hs), eo), ("lse", host(lse[:, a:b, hs]), el),
                               ("dq", sl(dq, hs), gq), ("dk", sl(dk, slice(kh, kh + 1)), gk),
                               ("dv", sl(dv, slice(kh, kh + 1)), gv)]:
                r = rel(x, e)
                print(f"{label} seq {s} ({b - a} tokens) kv head {kh} {name}: rel {r:.2e}")
                assert r <= (1e-5 if name == "lse" else BF16_TOL), (label, s, kh, name, r)


def test_config2_packed_varlen_forward_backward():
    c = syn.config2("cuda")
    assert c["cu_seqlens"].tolist()[-1] == 16384
    _attention_slice_check(c, seqs=[0, len(c["lengths"]) - 1], heads_kv=[0, 7], label="config 2")


def test_config2_single_sequence_4096():
    c = syn.config2_single("cuda")
    _attention_slice_check(c, seqs=[0], heads_kv=[3], label="T=4096")


def test_config3_decode():
    c = syn.config3("cuda")
    out = dm.attention_decode(c["q"], c["k"], c["v"], c["lengths"])
    torch.cuda.synchronize()
    lens = c["lengths"].cpu().numpy()
    for b in [0, 17, 63]:
        ln = int(lens[b])
        e = oracle.attention_decode(host(c["q"][b:b + 1]), host(c["k"][b:b + 1, :ln]),
                                    host(c["v"][b:b + 1, :ln]))
        r = rel(host(out[b:b + 1]), e)
        print(f"config 3 sequence {b} ({ln} keys): rel {r:.2e}")
        assert r <= BF16_TOL


def test_config3_decode_equals_attention_with_one_query():
    """attention_decode is attention with the one query after the sequence's keys
    (crates/dash-conformance/src/attention.rs:484-565), at the config's sizes for a few rows."""
    c = syn.config3("cuda")
    out = dm.attention_decode(c["q"], c["k"], c["v"], c["lengths"])
    for b in [3, 40]:
        ln = int(c["lengths"][b])
        full = dm.attention(c["q"][b:b + 1, None], c["k"][b:b + 1, :ln], c["v"][b:b + 1, :ln],
                            None, dm.AttentionOptions(causal=True))
        r = rel(host(out[b]), host(full[0, 0]))
        print(f"decode vs attention, sequence {b}: rel {r:.2e}")
        assert r <= 1e-2


def test_config4_chunk_forward():
    c = syn.config4("cuda")
    opts = dm.ChunkGatedDeltaOptions(output_final_state=True)
    out, fin = dm.chunk_gated_delta_rule(c["q"], c["k"], c["v"], c["g"], c["beta"], c["h0"],
                                         c["cu_seqlens"], opts)
    torch.cuda.synchronize()
    cu = c["cu_seqlens"].tolist()
    for s in [0, 7]:
        a, b = cu[s], cu[s + 1]
        for h in [0, 15]:
            sl = lambda x: host(x[:, a:b, h:h + 1])  # noqa: E731
            eo, ef = oracle.gdr_chunk_fwd(sl(c["q"]), sl(c["k"]), sl(c["v"]), sl(c["g"]),
                                          sl(c["beta"]), host(c["h0"][s:s + 1, h:h + 1]))
            r1 = rel(host(out[:, a:b, h:h + 1]), eo)
            r2 = rel(host(fin[s:s + 1, h:h + 1]), ef)
            print(f"config 4 seq {s} ({b - a} tokens) head {h}: out {r1:.2e} final {r2:.2e}")
            assert r1 <= BF16_TOL and r2 <= BF16_TOL


def test_config4_chunk_backward_slice():
    """The backward at a slice of config 4 (two sequences of its packing, two heads)."""
    c = syn.config4("cuda", total=2048, nseq=8)
    opts = dm.ChunkGatedDeltaOptions(output_final_state=True)
    args = [c[x] for x in ("q", "k", "v", "g", "beta")]
    dfin = syn.normal(77, tuple(c["h0"].shape), "cuda", std=0.1)
    r = dm.chunk_gated_delta_rule_backward(*args, c["h0"], c["cu_seqlens"], c["do"], dfin, opts)
    torch.cuda.synchronize()
    e = oracle.gdr_chunk_bwd(*(host(x) for x in args), host(c["h0"]), host(c["do"]), host(dfin),
                             c["cu_seqlens"].cpu().numpy())
    for name, a_, e_ in zip(["dq", "dk", "dv", "dg", "dbeta", "dh0"], r, e):
        rr = rel(host(a_), e_)
        print(f"config 4 (2048 tokens) {name}: rel {rr:.2e}")
        assert rr <= BF16_TOL


def test_config4_chunk_backward_full():
    """The backward at config 4's full size (32768 tokens, 8 sequences, H = 16), checked on
    oracle slices of two sequences x two heads: sequences and heads are independent, so each
    slice's gradients (and its initial state's) are that sequence's own backward."""
    c = syn.config4("cuda")
    opts = dm.ChunkGatedDeltaOptions(output_final_state=True)
    args = [c[x] for x in ("q", "k", "v", "g", "beta")]
    dfin = syn.normal(78, tuple(c["h0"].shape), "cuda", std=0.1)
    _lib.probe_reset()
    r = dm.chunk_gated_delta_rule_backward(*args, c["h0"], c["cu_seqlens"], c["do"], dfin, opts)
    torch.cuda.synchronize()
    assert _lib.probe_counts()["gdr_chunk_bwd_mfma"] > 0, "the MFMA backward did not run"
    cu = c["cu_seqlens"].tolist()
    for s in [1, 6]:
        a, b = cu[s], cu[s + 1]
        for h in [2, 13]:
            sl = lambda x: host(x[:, a:b, h:h + 1])  # noqa: E731
            e = oracle.gdr_chunk_bwd(*(sl(x) for x in args), host(c["h0"][s:s + 1, h:h + 1]),
                                     sl(c["do"]), host(dfin[s:s + 1, h:h + 1]))
            got = [sl(x) for x in r[:5]] + [host(r[5][s:s + 1, h:h + 1])]
            for name, a_, e_ in zip(["dq", "dk", "dv", "dg", "dbeta", "dh0"], got, e):
                rr = rel(a_, e_)
                print(f"config 4 seq {s} ({b - a} tokens) head {h} {name}: rel {rr:.2e}")
                assert rr <= BF16_TOL, (s, h, name, rr)


def test_config5_step():
    c = syn.config5("cuda")
    args = [c[x] for x in ("q", "k", "v", "g", "beta")]
    out, st = dm.gated_delta_step(*args, c["state"])
    torch.cuda.synchronize()
    rows = [0, 77, 127]
    eo, es = oracle.gdr_step(*(host(x[rows]) for x in args), host(c["state"][rows]))
    print("config 5 out", rel(host(out[rows]), eo), "state", rel(host(st[rows]), es))
    assert rel(host(out[rows]), eo) <= BF16_TOL
    assert rel(host(st[rows]), es) <= 1e-5


def test_config5_step_in_place_equals_out_of_place():
    c = syn.config5("cuda")
    args = [c[x] for x in ("q", "k", "v", "g", "beta")]
    o1, s1 = dm.gated_delta_step(*args, c["state"])
    s2 = c["state"].clone()
    o2, s2r = dm.gated_delta_step(*args, s2, in_place=True)
    assert s2r.data_ptr() == s2.data_ptr()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
