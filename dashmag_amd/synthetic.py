"""The benchmark's synthetic inputs, identical wherever they are drawn.

Each tensor comes from splitmix64 seeded with ``0xDA5A0000 + 16 * config + tensor_index``
(tensor indices: q 0, k 1, v 2, dO 3, g 4, beta 5, state 6, lengths 7): 53-bit uniforms, normal
variates by Box-Muller in f64 (pairs ``r cos t``, ``r sin t``), then cast to f32 and, where the
input is bf16, rounded to nearest even. Generated with torch integer and f64 arithmetic on the
device the tensors are wanted on.

Configs (BASELINE.json ``configs``):
  1. causal attention forward, f32, B=1, H=4, T=256, D=64;
  2. packed varlen attention forward + backward, bf16, Hq=32, Hkv=8, D=128, 16384 tokens,
     lengths uniform in [256, 4096] (the last trimmed), causal per sequence; plus one causal
     sequence of 4096 tokens;
  3. decode, bf16, B=64, Hq=32, Hkv=8, D=128, cache lengths uniform in [512, 8192];
  4. chunked gated delta rule, bf16, 32768 tokens in 8 sequences, H=16, Dk=Dv=128;
  5. gated delta step, 128 sequences, H=16, Dk=Dv=128, f32 state;
  6. (beside them, no BASELINE config) the causal conv1d of a Gated DeltaNet layer over config 4's
     packing: C = 6144 channels (q, k and v of 16 heads of 128), K = 4, SiLU, bf16, initial and
     final states of 3 steps; and its decoding step over 128 sequences (config 5's batch).
"""
from __future__ import annotations

import math

import torch

GAMMA = 0x9E3779B97F4A7C15
M1 = 0xBF58476D1CE4E5B9
M2 = 0x94D049BB133111EB
Q, K, V, DO, G, BETA, STATE, LENGTHS = range(8)


def _i64(x: int) -> int:
    x &= (1 << 64) - 1
    return x - (1 << 64) if x >= (1 << 63) else x


def _shr(x, s):
    """Logical right shift of int64 tensors holding uint64 bits."""
    return (x >> s) & ((1 << (64 - s)) - 1)


def seed_of(config: int, tensor: int) -> int:
    return 0xDA5A0000 + 16 * config + tensor


def splitmix64(seed: int, n: int, device="cpu") -> torch.Tensor:
    """The first ``n`` outputs of splitmix64 from ``seed``, as int64 tensors of uint64 bits."""
    i = torch.arange(1, n + 1, dtype=torch.int64, device=device)
    z = i * _i64(GAMMA) + _i64(seed)  # wraps modulo 2^64
    z = (z ^ _shr(z, 30)) * _i64(M1)
    z = (z ^ _shr(z, 27)) * _i64(M2)
    return z ^ _shr(z, 31)


def uniform(seed: int, n: int, device="cpu") -> torch.Tensor:
    """53-bit uniforms in [0, 1), f64."""
    return _shr(splitmix64(seed, n, device), 11).to(torch.float64) * (2.0 ** -53)


def normal(seed: int, shape, device="cpu", std=1.0) -> torch.Tensor:
    """N(0, std^2) by Box-Muller in f64, cast to f32."""
    n = int(math.prod(shape))
    m = (n + 1) // 2
    u = uniform(seed, 2 * m, device)
    u1, u2 = 1.0 - u[0::2], u[1::2]  # u1 in (0, 1]
    r = torch.sqrt(-2.0 * torch.log(u1))
    t = 2.0 * math.pi * u2
    z = torch.stack([r * torch.cos(t), r * torch.sin(t)], 1).reshape(-1)[:n]
    return (z * std).to(torch.float32).reshape(shape)


def as_input(x: torch.Tensor, dtype) -> torch.Tensor:
    return x.to(dtype)  # f32 -> bf16 rounds to nearest even


def l2norm(x: torch.Tensor) -> torch.Tensor:
    return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def attention_lengths(total=16384, lo=256, hi=4096, config=2):
    """Lengths ``lo + floor(u * (hi - lo + 1))`` drawn until they reach ``total``, the last
    trimmed; returns (lengths, cu_seqlens int32)."""
    u = uniform(seed_of(config, LENGTHS), 4096).tolist()
    lens, s = [], 0
    for x in u:
        ln = lo + int(math.floor(x * (hi - lo + 1)))
        if s + ln >= total:
            lens.append(total - s)
            break
        lens.append(ln)
        s += ln
    cu = [0]
    for ln in lens:
        cu.append(cu[-1] + ln)
    return lens, torch.tensor(cu, dtype=torch.int32)


def config1(device="cpu"):
    shape = (1, 256, 4, 64)
    return [normal(seed_of(1, i), shape, device) for i in (Q, K, V)]


def config2(device="cpu", dtype=torch.bfloat16, total=16384, hq=32, hkv=8, d=128):
    lens, cu = attention_lengths(total)
    q = as_input(normal(seed_of(2, Q), (1, total, hq, d), device), dtype)
    k = as_input(normal(seed_of(2, K), (1, total, hkv, d), device), dtype)
    v = as_input(normal(seed_of(2, V), (1, total, hkv, d), device), dtype)
    do = as_input(normal(seed_of(2, DO), (1, total, hq, d), device), dtype)
    return dict(q=q, k=k, v=v, do=do, lengths=lens, cu_seqlens=cu.to(device))


def config2_single(device="cpu", dtype=torch.bfloat16, t=4096, hq=32, hkv=8, d=128):
    """The north-star target shape: one causal sequence of 4096 tokens (seeds of config 2)."""
    q = as_input(normal(seed_of(2, Q), (1, t, hq, d), device), dtype)
    k = as_input(normal(seed_of(2, K), (1, t, hkv, d), device), dtype)
    v = as_input(normal(seed_of(2, V), (1, t, hkv, d), device), dtype)
    do = as_input(normal(seed_of(2, DO), (1, t, hq, d), device), dtype)
    return dict(q=q, k=k, v=v, do=do)


def config3(device="cpu", dtype=torch.bfloat16, b=64, hq=32, hkv=8, d=128, s=8192, lo=512):
    u = uniform(seed_of(3, LENGTHS), b)
    lengths = (lo + torch.floor(u * (s - lo + 1))).to(torch.int32)
    q = as_input(normal(seed_of(3, Q), (b, hq, d), device), dtype)
    k = as_input(normal(seed_of(3, K), (b, s, hkv, d), device), dtype)
    v = as_input(normal(seed_of(3, V), (b, s, hkv, d), device), dtype)
    return dict(q=q, k=k, v=v, lengths=lengths.to(device))


def gdr_gates(config, shape, device):
    g = -torch.nn.functional.softplus(normal(seed_of(config, G), shape, device))
    beta = torch.sigmoid(normal(seed_of(config, BETA), shape, device))
    return g, beta


def config4(device="cpu", dtype=torch.bfloat16, total=32768, nseq=8, h=16, dk=128, dv=128):
    """7 distinct uniform cut points, sorted, every length >= 1."""
    u = uniform(seed_of(4, LENGTHS), 1024).tolist()
    cuts = set()
    for x in u:
        c = 1 + int(math.floor(x * (total - 1)))
        cuts.add(c)
        if len(cuts) == nseq - 1:
            break
    cu = torch.tensor([0] + sorted(cuts) + [total], dtype=torch.int32)
    q = as_input(l2norm(normal(seed_of(4, Q), (1, total, h, dk), device)), dtype)
    k = as_input(l2norm(normal(seed_of(4, K), (1, total, h, dk), device)), dtype)
    v = as_input(normal(seed_of(4, V), (1, total, h, dv), device), dtype)
    do = as_input(normal(seed_of(4, DO), (1, total, h, dv), device), dtype)
    g, beta = gdr_gates(4, (1, total, h), device)
    h0 = normal(seed_of(4, STATE), (nseq, h, dk, dv), device, std=0.1)
    return dict(q=q, k=k, v=v, do=do, g=g, beta=as_input(beta, dtype), h0=h0,
                cu_seqlens=cu.to(device))


def config5(device="cpu", dtype=torch.bfloat16, b=128, h=16, dk=128, dv=128):
    q = as_input(l2norm(normal(seed_of(5, Q), (b, h, dk), device)), dtype)
    k = as_input(l2norm(normal(seed_of(5, K), (b, h, dk), device)), dtype)
    v = as_input(normal(seed_of(5, V), (b, h, dv), device), dtype)
    g, beta = gdr_gates(5, (b, h), device)
    state = normal(seed_of(5, STATE), (b, h, dk, dv), device, std=0.1)
    return dict(q=q, k=k, v=v, g=g, beta=as_input(beta, dtype), state=state)


def conv1d_config(device="cpu", dtype=torch.bfloat16, c=6144, k=4, w=3, b_step=128):
    """Config 6: x [1, 32768, C] over config 4's 8 sequences, weight [C, K] (std 1/2), output
    gradient, initial states [8, W, C] f32; the step's token [b_step, C] and state [b_step, W, C]
    (tensor indices: x 0, weight 1, output gradient 3, states 6, step token 2)."""
    cu = _config4_cuts()
    total, nseq = int(cu[-1]), len(cu) - 1
    x = as_input(normal(seed_of(6, Q), (1, total, c), device), dtype)
    weight = as_input(normal(seed_of(6, K), (c, k), device, std=0.5), dtype)
    go = as_input(normal(seed_of(6, DO), (1, total, c), device), dtype)
    h0 = normal(seed_of(6, STATE), (nseq, w, c), device)
    xs = as_input(normal(seed_of(6, V), (b_step, c), device), dtype)
    state = normal(seed_of(6, STATE), (b_step, w, c), device)
    return dict(x=x, weight=weight, go=go, h0=h0, cu_seqlens=cu.to(device), step_x=xs,
                step_state=state)


def logprob_config(device="cpu", dtype=torch.bfloat16, n=4096, d=4096, v=151936, n_masked=64):
    """Config 7: the chosen-token log-probability after a model's last layer. hidden [n, D]
    N(0, 1), the output weight [V, D] N(0, 0.02^2) (V = 151936, a Qwen-family vocabulary; logits
    of standard deviation about 1.3), targets uniform in [0, V), n_masked distinct masked ids
    (tensor indices: hidden 0, weight 1, targets 7, masked ids 2)."""
    hidden = as_input(normal(seed_of(7, Q), (n, d), device), dtype)
    weight = as_input(normal(seed_of(7, K), (v, d), device, std=0.02), dtype)
    targets = (uniform(seed_of(7, LENGTHS), n, device) * v).to(torch.int64).clamp_(0, v - 1)
    order = torch.argsort(uniform(seed_of(7, V), v))
    masked = sorted(order[:n_masked].tolist())
    return dict(hidden=hidden, weight=weight, targets=targets, masked=masked)


def _config4_cuts(total=32768, nseq=8):
    """Config 4's sequence boundaries (see config4)."""
    u = uniform(seed_of(4, LENGTHS), 1024).tolist()
    cuts = set()
    for x in u:
        cuts.add(1 + int(math.floor(x * (total - 1))))
        if len(cuts) == nseq - 1:
            break
    return torch.tensor([0] + sorted(cuts) + [total], dtype=torch.int32)


def visible_pairs(lengths) -> int:
    """P = sum L (L + 1) / 2, the (query, key) pairs causal attention computes."""
    return sum(l * (l + 1) // 2 for l in lengths)
