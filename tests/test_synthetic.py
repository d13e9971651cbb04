"""The benchmark's generator (dashmag_amd/synthetic.py) against a plain-integer splitmix64."""
import math

import torch

from dashmag_amd import synthetic as syn


def splitmix64_py(seed, n):
    out, s = [], seed
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & (2**64 - 1)
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        out.append(z ^ (z >> 31))
    return out


def test_splitmix64_matches_plain_integers():
    assert splitmix64_py(0, 1)[0] == 0xE220A8397B1DCDAF  # the published first output
    for seed in [0, 1, syn.seed_of(2, syn.Q), 2**63 + 5]:
        got = [x & (2**64 - 1) for x in syn.splitmix64(seed, 50).tolist()]
        assert got == splitmix64_py(seed, 50)


def test_normal_moments_and_uniform_range():
    u = syn.uniform(7, 100000)
    assert float(u.min()) >= 0.0 and float(u.max()) < 1.0
    z = syn.normal(7, (200000,))
    assert abs(float(z.mean())) < 0.01 and abs(float(z.std()) - 1.0) < 0.01


def test_attention_lengths():
    lens, cu = syn.attention_lengths()
    assert sum(lens) == 16384 and cu[-1] == 16384
    assert all(256 <= l <= 4096 for l in lens[:-1]) and 1 <= lens[-1] <= 4096
    assert syn.visible_pairs([4096]) == 8390656


def test_config4_cuts():
    c = syn.config4(total=1024, h=1, dk=8, dv=8)
    cu = c["cu_seqlens"].tolist()
    assert cu[0] == 0 and cu[-1] == 1024 and len(cu) == 9
    assert all(b > a for a, b in zip(cu, cu[1:]))
