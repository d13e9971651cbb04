"""Benchmark of the attention and gated-delta-rule hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

A step is one pass of the hot path over one batch of synthetic input (dashmag_amd/synthetic.py).
The headline (``value``) is BASELINE.json's first metric on its config 2: causal packed-varlen
attention forward + backward, bf16, Hq=32, Hkv=8, D=128, 16384 tokens, as algorithmic TFLOP/s
(14 P D Hq per step, P the visible pairs). The other metrics of the same line, under
``secondary``: the north-star T=4096 single sequence, KV-cache decode (config 3, HBM GB/s),
the chunked gated delta rule forward and backward (config 4, tokens/s and TFLOP/s) and the
recurrent step (config 5, HBM GB/s). Inputs are resident in HBM before the timed region; every
call goes through libdashmi.so's C ABI with descriptors and buffers prepared beforehand, timed
with HIP events on the stream the kernels run on.

``cpu_baseline`` is the CPU oracle (the C restatement of dash-ops' reference, OpenMP) on a
bounded sample of the same workload, on this host's cores.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", default="",
                   help="comma list: attn,attn4096,attn256,decode,gdr,step,conv1d,logprob,refshapes")
    p.add_argument("--copy-probe", action="store_true",
                   help="also run a plain 1 GiB device copy (torch copy_), 5 times: the known-size "
                        "kernel that scales the FETCH_SIZE / WRITE_SIZE counters of a --pmc run")
    return p.parse_args()


class Timed:
    """Times a C-ABI call on the current stream: `steps` back-to-back calls between two HIP
    events, after `warmup` untimed ones. Over the same timed region the library's kernel timers
    (HIP event pairs around each launch, on the launch stream) give each kernel's average launch
    duration, in ``kernel_ms`` {name: (ms per launch, launches)}. A second run of as many calls
    with the kernel timers off gives ``ms_plain``, the call's time without the timers' event
    records between its launches, which ``run`` returns (``ms_timers`` keeps the first)."""

    def __init__(self, torch, fn):
        self.torch, self.fn = torch, fn
        self.kernel_ms = {}
        self.ms_plain = None

    def run(self, steps, warmup):
        from dashmag_amd import _lib
        torch = self.torch
        for _ in range(warmup):
            self.fn()
        torch.cuda.synchronize()
        _lib.kernel_timing(True)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            self.fn()
        end.record()
        torch.cuda.synchronize()
        self.kernel_ms = {k: (ms / n, n) for k, (ms, n) in _lib.kernel_times().items() if n}
        _lib.kernel_timing(False)
        ms = start.elapsed_time(end) / steps  # ms per call
        start.record()
        for _ in range(steps):
            self.fn()
        end.record()
        torch.cuda.synchronize()
        self.ms_plain = start.elapsed_time(end) / steps
        self.ms_timers = ms
        return self.ms_plain


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (a line ``traffic_bytes_per_launch <kernel>: N``), or None when it has none."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_per_kernel.md")
    try:
        for line in open(path):
            if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def check(rc, lib):
    if rc != 0:
        raise RuntimeError(lib.dm_last_error().decode())


def bench_attention(torch, dm, ops, lib, data, steps, warmup, cu=None, opts=None):
    """Forward + backward of one batch; returns (ms_step, ms_fwd, ms_bwd)."""
    from dashmag_amd import _lib
    q, k, v, do = data["q"], data["k"], data["v"], data["do"]
    mask = dm.AttentionMask.none() if cu is None else dm.AttentionMask.packed(cu, cu)
    opts = opts or dm.AttentionOptions(causal=True)
    keep = []
    desc = ops._attention_desc("attention", q, k, v, mask, opts, keep)
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    fws = lib.dm_attention_fwd_workspace(ctypes.byref(desc))
    bws = lib.dm_attention_bwd_workspace(ctypes.byref(desc))
    ws = torch.empty(max(fws, bws, 1), dtype=torch.uint8, device=q.device)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = [ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, o, lse, do, dq, dk, dv, ws)]
    d = ctypes.byref(desc)

    def fwd():
        check(lib.dm_attention_fwd(d, P[0], P[1], P[2], P[3], P[4], P[9], fws, st), lib)

    def bwd():
        check(lib.dm_attention_bwd(d, P[0], P[1], P[2], P[3], P[4], P[5], P[6], P[7], P[8],
                                   P[9], bws, st), lib)

    def step():
        fwd()
        bwd()

    ms_fwd = Timed(torch, fwd).run(steps, warmup)
    ms_bwd = Timed(torch, bwd).run(steps, warmup)
    t = Timed(torch, step)
    t.run(steps, warmup)
    # the step's time over the region the kernel timers measured (the headline's roofline
    # reads those timers), and beside it the same steps without the timers
    ms_step = t.ms_timers
    bench_attention.ms_plain = t.ms_plain
    return ms_step, ms_fwd, ms_bwd, _lib.probe_counts(), t.kernel_ms


def ref_shapes(torch, dm, ops, lib, syn, dev, args):
    """dash-ops' published device times (crates/dash-ops/README.md:72-88, RTX 5070 Ti, bf16) and
    this build's for the same work on one MI355X, in ms per call (back-to-back calls between
    HIP events; inputs from the synthetic generator at those shapes)."""
    from dashmag_amd import _lib
    out = {}
    steps = max(3, args.steps // 2)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def note(name, ms, ref_ms, shape, tm=None, n=None):
        # short calls: the device's time (the library's kernel timers, summed per call) beside
        # the back-to-back call time, which the host's dispatch bounds at these sizes; dash-ops'
        # figures are device times too (sums over nsys's kernels)
        dev_ms = None
        if tm is not None:
            dev_ms = sum(v[0] * v[1] for v in tm.kernel_ms.values()) / n
        t = dev_ms if dev_ms is not None else ms
        out[name] = dict(ms=round(t, 4), reference_ms=ref_ms,
                         reference_over_this=round(ref_ms / t, 2), shape=shape)
        if dev_ms is not None:
            out[name]["call_ms_back_to_back"] = round(ms, 4)
            out[name]["timing"] = "device time (kernel timers)"
        print(f"reference shape {name}: {t:.4f} ms (dash-ops on an RTX 5070 Ti: {ref_ms} ms)",
              file=sys.stderr, flush=True)

    # attention forward + backward, T=6144, Hq=8, Hkv=2, D=256 (README.md:83): causal; no mask;
    # 4 packed sequences of 1536 (causal within each); causal within a window of 1024
    c = syn.config2_single(dev, t=6144, hq=8, hkv=2, d=256)
    cu4 = torch.tensor([0, 1536, 3072, 4608, 6144], dtype=torch.int32, device=dev)
    for name, cu, opts, ref in [
            ("attention_fwd_bwd_D256_causal", None, dm.AttentionOptions(causal=True), 9.17),
            ("attention_fwd_bwd_D256_no_mask", None, dm.AttentionOptions(), 17.6),
            ("attention_fwd_bwd_D256_packed_4x1536", cu4, dm.AttentionOptions(causal=True), 2.59),
            ("attention_fwd_bwd_D256_window_1024", None,
             dm.AttentionOptions(causal=True, window=dm.Window(1024, 0)), 3.07)]:
        ms, _, _, _, _ = bench_attention(torch, dm, ops, lib, c, steps, 1, cu, opts)
        note(name, ms, ref, "T=6144, Hq=8, Hkv=2, D=256, bf16, deterministic backward")
    del c
    # attention forward, T=6144, Hq=8, Hkv=2, D=64 (README.md:84)
    c = syn.config2_single(dev, t=6144, hq=8, hkv=2, d=64)
    for name, cu, opts, ref in [
            ("attention_fwd_D64_causal", None, dm.AttentionOptions(causal=True), 0.528),
            ("attention_fwd_D64_no_mask", None, dm.AttentionOptions(), 0.902),
            ("attention_fwd_D64_packed_4x1536", cu4, dm.AttentionOptions(causal=True), 0.145),
            ("attention_fwd_D64_window_1024", None,
             dm.AttentionOptions(causal=True, window=dm.Window(1024, 0)), 0.163)]:
        _, mf, _, _, _ = bench_attention(torch, dm, ops, lib, c, steps, 1, cu, opts)
        note(name, mf, ref, "T=6144, Hq=8, Hkv=2, D=64, bf16, forward only")
    del c
    # attention decoding, batch 8, 6144 cached keys, Hq=8, Hkv=2, D=256 (README.md:85): the
    # whole cache; lengths from 100 to 6144; a window of 1024
    c = syn.config3(dev, b=8, hq=8, hkv=2, d=256, s=6144, lo=6144)
    q, k, v = c["q"], c["k"], c["v"]
    o = torch.empty_like(q)
    for name, lens, opts, ref in [
            ("decode_D256_whole_cache", [6144] * 8, dm.AttentionOptions(), 0.131),
            ("decode_D256_lengths_100_to_6144", [100 + (6044 * i) // 7 for i in range(8)],
             dm.AttentionOptions(), 0.036),
            ("decode_D256_window_1024", [6144] * 8, dm.AttentionOptions(window=dm.Window(1024, 0)),
             0.015)]:
        lt = torch.tensor(lens, dtype=torch.int32, device=dev)
        keep = []
        desc = ops._attention_desc("attention_decode", q.unsqueeze(1), k, v,
                                   dm.AttentionMask.none(), opts, keep)
        nb = lib.dm_attention_decode_workspace(ctypes.byref(desc))
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        ptrs = [ctypes.c_void_p(t_.data_ptr()) for t_ in (q, k, v, lt, o, ws)]
        fn = lambda: check(lib.dm_attention_decode(ctypes.byref(desc), *ptrs[:5], ptrs[5], nb,  # noqa
                                                   st), lib)
        n_ = max(args.steps, 50)
        tm = Timed(torch, fn)
        ms = tm.run(n_, args.warmup)
        note(name, ms, ref, "B=8, S=6144, Hq=8, Hkv=2, D=256, bf16", tm, n_)
    del c, q, k, v, o
    # chunked gated delta rule forward, and forward + backward, 6144 tokens, 16 heads of 128
    # (README.md:80): one sequence; four packed sequences of 1536
    for label, cuts, ref_f, ref_fb in [("1x6144", [0, 6144], 0.81, 2.57),
                                       ("4x1536", [0, 1536, 3072, 4608, 6144], 0.79, 2.44)]:
        c = syn.config4(dev, total=6144, nseq=len(cuts) - 1)
        c["cu_seqlens"] = torch.tensor(cuts, dtype=torch.int32, device=dev)
        c["h0"] = c["h0"][:len(cuts) - 1].contiguous()
        keep = []
        args_t = [c[x] for x in ("q", "k", "v", "g", "beta")]
        desc, _, _ = ops._gdr_desc("chunk_gated_delta_rule", *args_t, c["cu_seqlens"], False,
                                   None, False, keep)
        outg, fin = torch.empty_like(c["v"]), torch.empty_like(c["h0"])
        nb = lib.dm_gdr_chunk_fwd_workspace(ctypes.byref(desc))
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        p = [ctypes.c_void_p(x.data_ptr()) for x in args_t + [c["h0"], outg, fin, ws]]
        fwd = lambda: check(lib.dm_gdr_chunk_fwd(ctypes.byref(desc), *p[:8], p[8], nb, st), lib)  # noqa
        dq, dk_, dv_ = (torch.empty_like(x) for x in args_t[:3])
        dg, db, dh0 = torch.empty_like(c["g"]), torch.empty_like(c["beta"]), torch.empty_like(c["h0"])
        nbb = lib.dm_gdr_chunk_bwd_workspace(ctypes.byref(desc))
        wsb = torch.empty(max(nbb, 1), dtype=torch.uint8, device=dev)
        pb = [ctypes.c_void_p(x.data_ptr()) for x in
              args_t + [c["h0"], c["do"], fin, dq, dk_, dv_, dg, db, dh0, wsb]]
        bwd = lambda: check(lib.dm_gdr_chunk_bwd(ctypes.byref(desc), *pb[:14], pb[14], nbb, st),  # noqa
                            lib)

        def both():
            fwd()
            bwd()

        ms_f = Timed(torch, fwd).run(steps, 1)
        ms_fb = Timed(torch, both).run(steps, 1)
        note(f"gdr_chunk_fwd_{label}", ms_f, ref_f, "6144 tokens, H=16, Dk=Dv=128, bf16")
        note(f"gdr_chunk_fwd_bwd_{label}", ms_fb, ref_fb, "6144 tokens, H=16, Dk=Dv=128, bf16")
        del c, ws, wsb
    # the recurrent decoding step, batch 8, 16 heads of 128 (README.md:82)
    c = syn.config5(dev, b=8)
    keep = []
    args_t = [c[x] for x in ("q", "k", "v", "g", "beta")]
    desc, _, _ = ops._gdr_desc("gated_delta_step", *args_t, None, False, None, True, keep)
    outs = torch.empty_like(c["v"])
    p = [ctypes.c_void_p(x.data_ptr()) for x in args_t + [c["state"], c["state"], outs]]
    fn = lambda: check(lib.dm_gdr_step(ctypes.byref(desc), *p, st), lib)  # noqa
    n_ = max(args.steps, 100)
    tm = Timed(torch, fn)
    ms = tm.run(n_, args.warmup)
    note("gdr_step_B8", ms, 0.0217, "B=8, H=16, Dk=Dv=128, f32 state, bf16 inputs", tm, n_)
    del c
    # causal conv1d forward + backward, 6144 steps, 6144 channels, width 4, SiLU (README.md:88)
    c = syn.conv1d_config(dev)
    x = c["x"][:, :6144].contiguous()
    wt, go = c["weight"], c["go"][:, :6144].contiguous()
    _, t, ch = x.shape
    kw = wt.shape[1]
    desc = _lib.Conv1dDesc(b=1, t=t, c=ch, k=kw, dtype=_lib.DM_BF16, has_bias=0,
                           activation=_lib.DM_ACT_SILU)
    outc, gx, gw = torch.empty_like(x), torch.empty_like(x), torch.empty_like(wt)
    ws = torch.empty(max(lib.dm_causal_conv1d_bwd_workspace(ctypes.byref(desc)), 1),
                     dtype=torch.uint8, device=dev)
    P = lambda tt: None if tt is None else ctypes.c_void_p(tt.data_ptr())  # noqa: E731

    def conv():
        check(lib.dm_causal_conv1d_fwd(ctypes.byref(desc), P(x), P(wt), None, None, P(outc), None,
                                       st), lib)
        check(lib.dm_causal_conv1d_bwd(ctypes.byref(desc), P(x), P(wt), None, None, P(go),
                                       _lib.DM_BF16, None, P(gx), P(gw), None, None, P(ws),
                                       ws.numel(), st), lib)

    ms = Timed(torch, conv).run(max(args.steps, 50), args.warmup)
    note("conv1d_fwd_bwd", ms, 0.56, "T=6144, C=6144, K=4, SiLU, bf16")
    del c, x, go
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not run (every GPU "
              "box here has one GPU; the hot path shards over sequences and heads with no exchange)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import dashmag_amd as dm
    from dashmag_amd import _lib, ops, synthetic as syn

    lib = _lib.lib()
    dev = torch.device("cuda:0")
    only = set(filter(None, args.only.split(",")))
    want = lambda name: not only or name in only  # noqa: E731
    secondary = {}
    print(f"device: {_lib.describe()}", file=sys.stderr, flush=True)
    if args.copy_probe:
        x = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print("copy probe: 5 copies of 1 GiB (read 1048576 KiB, write 1048576 KiB each)",
              file=sys.stderr, flush=True)
        del x, y

    # ---- headline: attention fwd+bwd, config 2 ----
    c2 = syn.config2(dev)
    P2 = syn.visible_pairs(c2["lengths"])
    flop2 = 14 * P2 * 128 * 32
    head = None
    if want("attn"):
        ms, mf, mb, probes, kms = bench_attention(torch, dm, ops, lib, c2, args.steps, args.warmup,
                                             c2["cu_seqlens"])
        head = dict(ms=ms, ms_fwd=mf, ms_bwd=mb, probes=probes, kernel_ms=kms)
        secondary["attention_config2_ms_per_step_kernel_timers_off"] = round(
            bench_attention.ms_plain, 4)
        secondary["attention_config2_kernel_us"] = {k: round(v[0] * 1e3, 2)
                                                    for k, v in kms.items()}
        print("attention config 2 kernels: " + ", ".join(
            f"{k} {v[0] * 1e3:.1f} us" for k, v in kms.items()), file=sys.stderr, flush=True)
        print(f"attention config 2: {ms:.3f} ms/step (fwd {mf:.3f}, bwd {mb:.3f}), "
              f"{flop2 / ms / 1e9:.1f} TFLOP/s", file=sys.stderr, flush=True)
    del c2
    if want("attn4096"):
        c = syn.config2_single(dev)
        ms, mf, mb, _, kms4 = bench_attention(torch, dm, ops, lib, c, args.steps, args.warmup)
        P = syn.visible_pairs([4096])
        secondary["attention_fwd_bwd_T4096"] = dict(
            unit="TFLOP/s", value=14 * P * 128 * 32 / ms / 1e9, ms_per_step=ms,
            fwd_tflops=4 * P * 128 * 32 / mf / 1e9, bwd_tflops=10 * P * 128 * 32 / mb / 1e9,
            frac_of_bf16_peak=14 * P * 128 * 32 / ms / 1e9 / BF16_PEAK_TFLOPS,
            kernel_us={k: round(v[0] * 1e3, 2) for k, v in kms4.items()})
        print("attention T=4096 kernels: " + ", ".join(
            f"{k} {v[0] * 1e3:.1f} us" for k, v in kms4.items()), file=sys.stderr, flush=True)
        print(f"attention T=4096: {ms:.3f} ms/step, "
              f"{secondary['attention_fwd_bwd_T4096']['value']:.1f} TFLOP/s", file=sys.stderr,
              flush=True)
        del c

    # ---- the reference's own attention shape: T=6144, Hq=8, Hkv=2, D=256, causal ----
    if want("attn256"):
        c = syn.config2_single(dev, t=6144, hq=8, hkv=2, d=256)
        ms, mf, mb, _, kms = bench_attention(torch, dm, ops, lib, c, args.steps, args.warmup)
        P = syn.visible_pairs([6144])
        fl = lambda n: n * P * 256 * 8  # noqa: E731
        secondary["attention_fwd_bwd_T6144_D256"] = dict(
            unit="TFLOP/s", value=fl(14) / ms / 1e9, ms_per_step=ms, ms_fwd=mf, ms_bwd=mb,
            fwd_tflops=fl(4) / mf / 1e9, bwd_tflops=fl(10) / mb / 1e9,
            frac_of_bf16_peak=fl(14) / ms / 1e9 / BF16_PEAK_TFLOPS,
            kernel_us={k_: round(v_[0] * 1e3, 2) for k_, v_ in kms.items()},
            shape="causal, T=6144, Hq=8, Hkv=2, D=256, bf16 (crates/dash-ops/README.md:83-84)")
        print("attention T=6144 D=256 kernels: " + ", ".join(
            f"{k_} {v_[0] * 1e3:.1f} us" for k_, v_ in kms.items()), file=sys.stderr, flush=True)
        print(f"attention T=6144 D=256: {ms:.3f} ms/step (fwd {mf:.3f} = {fl(4) / mf / 1e9:.1f}, "
              f"bwd {mb:.3f} = {fl(10) / mb / 1e9:.1f} TFLOP/s)", file=sys.stderr, flush=True)
        del c

    # ---- decode, config 3 ----
    if want("decode"):
        c = syn.config3(dev)
        q, k, v, lens = c["q"], c["k"], c["v"], c["lengths"]
        keep = []
        desc = ops._attention_desc("attention_decode", q.unsqueeze(1), k, v,
                                   dm.AttentionMask.none(), dm.AttentionOptions(), keep)
        o = torch.empty_like(q)
        nb = lib.dm_attention_decode_workspace(ctypes.byref(desc))
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        ptrs = [ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, lens, o, ws)]
        fn = lambda: check(lib.dm_attention_decode(ctypes.byref(desc), *ptrs[:5], ptrs[5], nb,  # noqa
                                                   st), lib)
        tm = Timed(torch, fn)
        ms = tm.run(max(args.steps, 50), args.warmup)
        sum_l = int(lens.sum())
        nbytes = 4 * 8 * 128 * sum_l + 4 * 64 * 32 * 128 + 4 * 64
        secondary["decode"] = dict(unit="GB/s", value=nbytes / ms / 1e6, us_per_call=ms * 1e3,
                                   bytes=nbytes, frac_of_hbm_peak=nbytes / ms / 1e6 / HBM_PEAK_GBS,
                                   kernel_us={k: round(v[0] * 1e3, 2) for k, v in tm.kernel_ms.items()})
        if "decode_split" in tm.kernel_ms:
            ks = tm.kernel_ms["decode_split"][0]
            secondary["decode"]["split_kernel_GBps"] = nbytes / ks / 1e6
        print(f"decode: {ms * 1e3:.1f} us, {nbytes / ms / 1e6:.0f} GB/s", file=sys.stderr,
              flush=True)

        # the same keys in the other cache layouts: packed back to back (offsets cu_seqlens_k)
        # and in shuffled pages of 16 keys (a block table)
        bsz, S, hkv, d = k.shape
        lens_h = lens.to("cpu", torch.int64)
        starts = torch.arange(bsz, dtype=torch.int64) * S
        rows = torch.cat([starts[b] + torch.arange(int(lens_h[b])) for b in range(bsz)]).to(dev)
        kpk, vpk = k.reshape(-1, hkv, d)[rows], v.reshape(-1, hkv, d)[rows]
        cu = torch.zeros(bsz + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(lens_h, 0).to(torch.int32)
        cu = cu.to(dev)
        pdesc = ops._decode_desc("attention_decode", q, kpk, vpk, S, dm.AttentionOptions())
        pdesc.cu_seqlens_k, pdesc.nseq = cu.data_ptr(), bsz
        pnb = lib.dm_attention_decode_workspace(ctypes.byref(pdesc))
        pws = torch.empty(max(pnb, 1), dtype=torch.uint8, device=dev)
        pp = [ctypes.c_void_p(t.data_ptr()) for t in (q, kpk, vpk, o, pws)]
        fn = lambda: check(lib.dm_attention_decode(ctypes.byref(pdesc), pp[0], pp[1], pp[2],  # noqa
                                                   None, pp[3], pp[4], pnb, st), lib)
        tm = Timed(torch, fn)
        ms_p = tm.run(max(args.steps, 50), args.warmup)
        secondary["decode_packed"] = dict(unit="GB/s", value=nbytes / ms_p / 1e6,
                                          us_per_call=ms_p * 1e3, layout="packed, cu_seqlens_k",
                                          frac_of_hbm_peak=nbytes / ms_p / 1e6 / HBM_PEAK_GBS)
        del kpk, vpk
        ps = 16
        npg = [-(-int(n) // ps) for n in lens_h]
        total = sum(npg)
        perm = torch.from_numpy(np.random.default_rng(3).permutation(total)).to(torch.int64)
        table = torch.full((bsz, S // ps), -1, dtype=torch.int32)
        src = []
        i = 0
        for b in range(bsz):
            table[b, :npg[b]] = perm[i:i + npg[b]].to(torch.int32)
            src.append(starts[b] + torch.arange(npg[b] * ps))
            i += npg[b]
        src = torch.cat(src).to(dev)
        kpg = torch.empty(total, ps, hkv, d, dtype=k.dtype, device=dev)
        vpg = torch.empty_like(kpg)
        kpg[perm.to(dev)] = k.reshape(-1, hkv, d)[src].reshape(total, ps, hkv, d)
        vpg[perm.to(dev)] = v.reshape(-1, hkv, d)[src].reshape(total, ps, hkv, d)
        table = table.to(dev)
        gdesc = ops._decode_desc("attention_decode_paged", q, kpg, vpg, S, dm.AttentionOptions())
        gnb = lib.dm_attention_decode_paged_workspace(ctypes.byref(gdesc), ps)
        gws = torch.empty(max(gnb, 1), dtype=torch.uint8, device=dev)
        gp = [ctypes.c_void_p(t.data_ptr()) for t in (q, kpg, vpg, table, lens, o, gws)]
        fn = lambda: check(lib.dm_attention_decode_paged(  # noqa
            ctypes.byref(gdesc), gp[0], gp[1], gp[2], total, ps, gp[3], S // ps, gp[4], gp[5],
            gp[6], gnb, st), lib)
        tm = Timed(torch, fn)
        ms_g = tm.run(max(args.steps, 50), args.warmup)
        secondary["decode_paged"] = dict(unit="GB/s", value=nbytes / ms_g / 1e6,
                                         us_per_call=ms_g * 1e3,
                                         layout=f"pages of {ps} keys, shuffled, block table",
                                         frac_of_hbm_peak=nbytes / ms_g / 1e6 / HBM_PEAK_GBS,
                                         kernel_us={k: round(v[0] * 1e3, 2)
                                                    for k, v in tm.kernel_ms.items()})
        print(f"decode packed: {ms_p * 1e3:.1f} us; paged ({ps}): {ms_g * 1e3:.1f} us, "
              f"{nbytes / ms_g / 1e6:.0f} GB/s", file=sys.stderr, flush=True)
        del c, k, v, kpg, vpg

        # the reference's attention head shape (Hq = 8, Hkv = 2, D = 256) over config 3's cache
        # lengths
        c = syn.config3(dev, hq=8, hkv=2, d=256)
        q, k, v, lens = c["q"], c["k"], c["v"], c["lengths"]
        desc = ops._attention_desc("attention_decode", q.unsqueeze(1), k, v,
                                   dm.AttentionMask.none(), dm.AttentionOptions(), keep)
        o = torch.empty_like(q)
        nb = lib.dm_attention_decode_workspace(ctypes.byref(desc))
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        ptrs = [ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, lens, o, ws)]
        fn = lambda: check(lib.dm_attention_decode(ctypes.byref(desc), *ptrs[:5], ptrs[5], nb,  # noqa
                                                   st), lib)
        tm = Timed(torch, fn)
        ms = tm.run(max(args.steps, 50), args.warmup)
        nbytes = 4 * 2 * 256 * int(lens.sum()) + 4 * 64 * 8 * 256 + 4 * 64
        secondary["decode_d256"] = dict(
            unit="GB/s", value=nbytes / ms / 1e6, us_per_call=ms * 1e3, bytes=nbytes,
            frac_of_hbm_peak=nbytes / ms / 1e6 / HBM_PEAK_GBS,
            kernel_us={k_: round(v_[0] * 1e3, 2) for k_, v_ in tm.kernel_ms.items()},
            shape="config 3's lengths, B=64, S=8192, Hq=8, Hkv=2, D=256, bf16")
        print(f"decode D=256 (Hq=8, Hkv=2): {ms * 1e3:.1f} us, {nbytes / ms / 1e6:.0f} GB/s",
              file=sys.stderr, flush=True)
        del c, q, k, v, o, ws

    # ---- gated delta rule chunked, config 4 ----
    if want("gdr"):
        c = syn.config4(dev)
        opts = dm.ChunkGatedDeltaOptions(output_final_state=True)
        keep = []
        args_t = [c[x] for x in ("q", "k", "v", "g", "beta")]
        desc, nseq, (b, t, h, dk, dv) = ops._gdr_desc("chunk_gated_delta_rule", *args_t,
                                                      c["cu_seqlens"], False, None, False, keep)
        out = torch.empty_like(c["v"])
        fin = torch.empty_like(c["h0"])
        nb = lib.dm_gdr_chunk_fwd_workspace(ctypes.byref(desc))
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        p = [ctypes.c_void_p(x.data_ptr()) for x in args_t + [c["h0"], out, fin, ws]]
        fn = lambda: check(lib.dm_gdr_chunk_fwd(ctypes.byref(desc), *p[:8], p[8], nb, st), lib)  # noqa
        tm = Timed(torch, fn)
        ms = tm.run(max(3, args.steps // 4), 1)
        cu = c["cu_seqlens"].tolist()
        nch = h * sum((cu[i + 1] - cu[i] + 63) // 64 for i in range(len(cu) - 1))
        flop = 11534336 * nch
        secondary["gdr_chunk_fwd"] = dict(unit="tokens/s", value=t / ms * 1e3, ms_per_call=ms,
                                          tflops=flop / ms / 1e9,
                                          frac_of_bf16_peak=flop / ms / 1e9 / BF16_PEAK_TFLOPS,
                                          kernel_us={k: round(v[0] * 1e3, 2)
                                                     for k, v in tm.kernel_ms.items()})
        print(f"gdr chunk fwd: {ms:.3f} ms, {t / ms * 1e3:.3e} tokens/s, "
              f"{flop / ms / 1e9:.2f} TFLOP/s", file=sys.stderr, flush=True)
        # backward (reported)
        dq, dk_, dv_ = (torch.empty_like(x) for x in args_t[:3])
        dg, db = torch.empty_like(c["g"]), torch.empty_like(c["beta"])
        dh0 = torch.empty_like(c["h0"])
        nbb = lib.dm_gdr_chunk_bwd_workspace(ctypes.byref(desc))
        wsb = torch.empty(max(nbb, 1), dtype=torch.uint8, device=dev)
        pb = [ctypes.c_void_p(x.data_ptr()) for x in
              args_t + [c["h0"], c["do"], fin, dq, dk_, dv_, dg, db, dh0, wsb]]
        fnb = lambda: check(lib.dm_gdr_chunk_bwd(ctypes.byref(desc), *pb[:14], pb[14], nbb, st),  # noqa
                            lib)
        tmb = Timed(torch, fnb)
        msb = tmb.run(max(3, args.steps // 4), 1)
        secondary["gdr_chunk_bwd"] = dict(unit="tokens/s", value=t / msb * 1e3, ms_per_call=msb,
                                          tflops=32.5e6 * nch / msb / 1e9,
                                          kernel_us={k: round(v[0] * 1e3, 2)
                                                     for k, v in tmb.kernel_ms.items()})
        print(f"gdr chunk bwd: {msb:.3f} ms, kernels (us) "
              f"{secondary['gdr_chunk_bwd']['kernel_us']}", file=sys.stderr, flush=True)
        del c, ws, wsb

    # ---- gated delta step, config 5 ----
    if want("step"):
        c = syn.config5(dev)
        keep = []
        args_t = [c[x] for x in ("q", "k", "v", "g", "beta")]
        desc, nseq, (b, _, h, dk, dv) = ops._gdr_desc("gated_delta_step", *args_t, None, False,
                                                      None, True, keep)
        st_in = c["state"]
        out = torch.empty_like(c["v"])
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        p = [ctypes.c_void_p(x.data_ptr()) for x in args_t + [st_in, st_in, out]]
        fn = lambda: check(lib.dm_gdr_step(ctypes.byref(desc), *p, st), lib)  # noqa
        tm = Timed(torch, fn)
        ms = tm.run(max(args.steps, 100), args.warmup)
        nbytes = 8 * b * h * dk * dv + (3 * 2 * h * 128 + 2 * 4 * h) * b
        secondary["gdr_step"] = dict(unit="GB/s", value=nbytes / ms / 1e6, us_per_call=ms * 1e3,
                                     bytes=nbytes,
                                     frac_of_hbm_peak=nbytes / ms / 1e6 / HBM_PEAK_GBS,
                                     kernel_us={k: round(v[0] * 1e3, 2)
                                                for k, v in tm.kernel_ms.items()})
        print(f"gdr step: {ms * 1e3:.1f} us, {nbytes / ms / 1e6:.0f} GB/s", file=sys.stderr,
              flush=True)
        # the step's backward on the same inputs, N(0, 1) cotangents of the output and the new
        # states: the state and its gradient read, the state's gradient written, plus the tokens'
        # inputs and gradients
        gen = torch.Generator().manual_seed(55)
        d_out = torch.randn(c["v"].shape, generator=gen).to(c["v"].dtype).to(dev)
        d_st = torch.randn(st_in.shape, generator=gen).to(dev)
        gq, gk, gv = torch.empty_like(c["q"]), torch.empty_like(c["k"]), torch.empty_like(c["v"])
        gg, gb = torch.empty_like(c["g"]), torch.empty_like(c["beta"])
        gst = torch.empty_like(st_in)
        wsb = lib.dm_gdr_step_bwd_workspace(ctypes.byref(desc))
        wst = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        pb = [ctypes.c_void_p(x.data_ptr())
              for x in args_t + [st_in, d_out, d_st, gq, gk, gv, gg, gb, gst, wst]]
        fnb = lambda: check(lib.dm_gdr_step_bwd(ctypes.byref(desc), *pb, wsb, st), lib)  # noqa
        tmb = Timed(torch, fnb)
        msb = tmb.run(max(args.steps, 100), args.warmup)
        nb_b = 3 * 4 * b * h * dk * dv + (8 * 2 * h * 128 + 4 * 4 * h) * b
        secondary["gdr_step_bwd"] = dict(unit="GB/s", value=nb_b / msb / 1e6,
                                         us_per_call=msb * 1e3, bytes=nb_b,
                                         frac_of_hbm_peak=nb_b / msb / 1e6 / HBM_PEAK_GBS,
                                         kernel_us={k: round(v[0] * 1e3, 2)
                                                    for k, v in tmb.kernel_ms.items()})
        print(f"gdr step backward: {msb * 1e3:.1f} us, {nb_b / msb / 1e6:.0f} GB/s",
              file=sys.stderr, flush=True)
        del c

    # ---- causal conv1d, config 6 (beside config 4: a Gated DeltaNet layer's conv) ----
    if want("conv1d"):
        c = syn.conv1d_config(dev)
        x, wt, go, h0, cu = c["x"], c["weight"], c["go"], c["h0"], c["cu_seqlens"]
        _, t, ch = x.shape
        kw, nseq, w = wt.shape[1], h0.shape[0], h0.shape[1]
        desc = _lib.Conv1dDesc(b=1, t=t, c=ch, k=kw, dtype=_lib.DM_BF16,
                               cu_seqlens=cu.data_ptr(), nseq=nseq, has_bias=0,
                               activation=_lib.DM_ACT_SILU, has_initial=1, w=w, has_final=1,
                               w_out=w)
        out, gx, gw = torch.empty_like(x), torch.empty_like(x), torch.empty_like(wt)
        fin, gh = torch.empty_like(h0), torch.empty_like(h0)
        gfin = torch.ones_like(h0)
        ws = torch.empty(max(lib.dm_causal_conv1d_bwd_workspace(ctypes.byref(desc)), 1),
                         dtype=torch.uint8, device=dev)
        P = lambda tt: None if tt is None else ctypes.c_void_p(tt.data_ptr())  # noqa: E731
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        fwd = lambda: check(lib.dm_causal_conv1d_fwd(  # noqa: E731
            ctypes.byref(desc), P(x), P(wt), None, P(h0), P(out), P(fin), st), lib)
        bwd = lambda: check(lib.dm_causal_conv1d_bwd(  # noqa: E731
            ctypes.byref(desc), P(x), P(wt), None, P(h0), P(go), _lib.DM_BF16, P(gfin), P(gx),
            P(gw), None, P(gh), P(ws), ws.numel(), st), lib)
        tf, tb = Timed(torch, fwd), Timed(torch, bwd)
        ms_f = tf.run(max(args.steps, 50), args.warmup)
        ms_b = tb.run(max(args.steps, 50), args.warmup)
        # algorithmic bytes: x read and the output written (forward); x and the output's
        # gradient read and the input's written (backward); the f32 states in and out
        sb = nseq * w * ch * 4
        fwd_bytes = 2 * t * ch * 2 + 2 * sb + ch * kw * 2
        bwd_bytes = 3 * t * ch * 2 + 3 * sb + ch * kw * 2
        bs, sx, sst = c["step_x"].shape[0], c["step_x"], c["step_state"]
        sdesc = _lib.Conv1dDesc(b=bs, t=1, c=ch, k=kw, dtype=_lib.DM_BF16, has_bias=0,
                                activation=_lib.DM_ACT_SILU, w=w)
        sout = torch.empty_like(sx)
        upd = lambda: check(lib.dm_causal_conv1d_update(  # noqa: E731
            ctypes.byref(sdesc), P(sx), P(wt), None, P(sst), P(sout), P(sst), st), lib)
        tu = Timed(torch, upd)
        ms_u = tu.run(max(args.steps, 100), args.warmup)
        upd_bytes = 2 * bs * ch * 2 + 2 * bs * w * ch * 4
        kus = {k: round(v[0] * 1e3, 2) for k, v in {**tf.kernel_ms, **tb.kernel_ms,
                                                    **tu.kernel_ms}.items()}
        secondary["conv1d"] = dict(
            unit="GB/s", workload="causal conv1d, bf16, 32768 tokens in config 4's 8 sequences, "
            "C=6144, K=4, SiLU, initial and final states of 3 steps; step: 128 sequences",
            fwd_GBps=fwd_bytes / ms_f / 1e6, fwd_us=ms_f * 1e3,
            fwd_frac_of_hbm_peak=fwd_bytes / ms_f / 1e6 / HBM_PEAK_GBS,
            bwd_GBps=bwd_bytes / ms_b / 1e6, bwd_us=ms_b * 1e3,
            bwd_frac_of_hbm_peak=bwd_bytes / ms_b / 1e6 / HBM_PEAK_GBS,
            step_GBps=upd_bytes / ms_u / 1e6, step_us=ms_u * 1e3, kernel_us=kus)
        print(f"conv1d: fwd {ms_f * 1e3:.1f} us ({fwd_bytes / ms_f / 1e6:.0f} GB/s), bwd "
              f"{ms_b * 1e3:.1f} us ({bwd_bytes / ms_b / 1e6:.0f} GB/s), step {ms_u * 1e3:.1f} us",
              file=sys.stderr, flush=True)
        del c, x, go, out, gx

    # ---- the shapes dash-ops publishes its own device times for (crates/dash-ops/README.md:72-88,
    #      one RTX 5070 Ti; context, not a target): the same work here, per call ----
    if want("refshapes"):
        secondary["reference_shapes"] = ref_shapes(torch, dm, ops, lib, syn, dev, args)

    # ---- chosen-token log-probability, config 7 (after the model: the next row) ----
    if want("logprob"):
        c = syn.logprob_config(dev)
        h, wt, tg, masked = c["hidden"], c["weight"], c["targets"], c["masked"]
        n, d = h.shape
        v = wt.shape[0]
        desc = _lib.LogprobDesc(n=n, v=v, d=d, hidden_dtype=_lib.DM_BF16,
                                weight_dtype=_lib.DM_BF16, vocab_chunk=0, row_chunk=3072)
        ids = (ctypes.c_uint32 * len(masked))(*masked)
        lp = torch.empty(n, dtype=torch.float32, device=dev)
        ent, grad = torch.empty_like(lp), torch.empty(n, d, dtype=torch.float32, device=dev)
        nb = lib.dm_chosen_logprob_workspace(ctypes.byref(desc), 1)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        P = lambda tt: None if tt is None else ctypes.c_void_p(tt.data_ptr())  # noqa: E731
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

        def lp_call(g):
            check(lib.dm_chosen_logprob(ctypes.byref(desc), P(h), P(wt), P(tg),
                                        ctypes.cast(ids, ctypes.c_void_p), len(masked), P(lp),
                                        P(ent), P(g), P(ws), nb, st), lib)

        tfw, tgr = Timed(torch, lambda: lp_call(None)), Timed(torch, lambda: lp_call(grad))
        ms_f = tfw.run(max(args.steps, 5), args.warmup)
        ms_g = tgr.run(max(args.steps, 5), args.warmup)
        # algorithmic flops: the logits (2 n V D) and, with the gradient, its product (2 n V D)
        fl = 2 * n * v * d
        kus = {k: round(v_[0] * 1e3, 2) for k, v_ in tgr.kernel_ms.items()}
        secondary["logprob"] = dict(
            unit="TFLOP/s", workload=f"chosen-token logprob, bf16, n={n}, D={d}, V={v}, "
            f"{len(masked)} masked ids, default chunking",
            fwd_ms=ms_f, fwd_TFLOPs=fl / ms_f / 1e9, fwd_frac_of_mfma_peak=fl / ms_f / 1e9 / BF16_PEAK_TFLOPS,
            grad_ms=ms_g, grad_TFLOPs=2 * fl / ms_g / 1e9,
            grad_frac_of_mfma_peak=2 * fl / ms_g / 1e9 / BF16_PEAK_TFLOPS,
            rows_per_s=n / ms_g * 1e3, kernel_us=kus)
        print(f"logprob: fwd {ms_f:.2f} ms ({fl / ms_f / 1e9:.0f} TFLOP/s), with gradient "
              f"{ms_g:.2f} ms ({2 * fl / ms_g / 1e9:.0f} TFLOP/s)", file=sys.stderr, flush=True)
        del grad, ws

        # the fused linear cross-entropy on the same inputs: label smoothing 0.1, z-loss 1e-4,
        # the 64 masked ids; forward, then the gradients of hidden and of a trained weight
        opts = dm.CrossEntropyOptions(label_smoothing=0.1, z_loss=1e-4, masked=tuple(masked))
        up = torch.zeros(3, n)
        up[0] = 1.0 / n
        rows_box = {}

        def lce_fwd():
            rows_box["rows"] = dm.linear_cross_entropy(h, wt, tg, opts)[3]

        def lce_step():
            lce_fwd()
            dm.linear_cross_entropy_backward(h, wt, tg, rows_box["rows"], up, opts)

        tlf, tls = Timed(torch, lce_fwd), Timed(torch, lce_step)
        ms_lf = tlf.run(max(args.steps, 5), args.warmup)
        ms_ls = tls.run(max(args.steps, 5), args.warmup)
        # forward: the logits (2 n V D); backward: the logits again, grad_hidden and grad_weight
        secondary["linear_cross_entropy"] = dict(
            unit="TFLOP/s", workload=f"fused linear cross-entropy, bf16, n={n}, D={d}, V={v}, "
            "label smoothing 0.1, z-loss 1e-4, 64 masked ids, gradients of hidden and weight",
            fwd_ms=ms_lf, fwd_TFLOPs=fl / ms_lf / 1e9, step_ms=ms_ls,
            step_TFLOPs=4 * fl / ms_ls / 1e9,
            step_frac_of_mfma_peak=4 * fl / ms_ls / 1e9 / BF16_PEAK_TFLOPS)
        print(f"linear cross-entropy: fwd {ms_lf:.2f} ms, fwd+bwd {ms_ls:.2f} ms "
              f"({4 * fl / ms_ls / 1e9:.0f} TFLOP/s)", file=sys.stderr, flush=True)
        del c, h, wt, rows_box

    # ---- CPU baseline: the oracle on a bounded sample of config 2 ----
    cpu = None
    if not args.no_cpu_baseline and want("attn"):

        import oracle
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        oracle.set_threads(threads)
        c = syn.config2("cpu", dtype=torch.float32)
        lens = c["lengths"]
        s = 1  # sequence 1 of config 2
        a, e = sum(lens[:s]), sum(lens[:s + 1])
        sl = lambda x: np.ascontiguousarray(x[:, a:e].numpy())  # noqa: E731
        q, k, v, do = (sl(c[x].to(torch.bfloat16).float()) for x in ("q", "k", "v", "do"))
        call = oracle.AttentionCall(q, k, v, None, True)
        t0 = time.time()
        o, l = oracle.attention_fwd(call)
        oracle.attention_bwd(call, o, l, do)
        sec = time.time() - t0
        L = e - a
        flop = 14 * syn.visible_pairs([L]) * 128 * 32
        cpu = dict(value=flop / sec / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                   sample=f"config 2 sequence {s} alone ({L} tokens, causal, Hq=32, Hkv=8, "
                          f"D=128, f32 values of the bf16 inputs), forward + backward, "
                          f"{sec:.1f} s")
        print(f"cpu baseline: {cpu['value'] * 1e3:.2f} GFLOP/s on {threads} threads "
              f"({sec:.1f} s)", file=sys.stderr, flush=True)

    if head is None:
        print(json.dumps({"secondary": secondary}))
        return
    ms = head["ms"]
    value = flop2 / ms / 1e9
    # dominant kernel: the one with the most time per step, with the GEMMs it performs as its
    # algorithmic work (2 P D Hq FLOP per GEMM): forward QK^T and PV (2 GEMMs); dk/dv kernel
    # QK^T, dO V^T, P^T dO, dS^T Q (4); dq kernel QK^T, dO V^T, dS K (3)
    gemms = {"attn_fwd": 2, "attn_bwd_dkdv": 4, "attn_bwd_dq": 3}
    kms = {k: v for k, v in head["kernel_ms"].items() if k in gemms}
    dom = max(kms, key=lambda k: kms[k][0] * kms[k][1])
    dom_ms = kms[dom][0]
    dom_flop = gemms[dom] * 2 * P2 * 128 * 32
    achieved = dom_flop / dom_ms / 1e9
    traffic = measured_traffic(dom)
    line = {
        "metric": "attn fwd+bwd TFLOP/s; GDR chunk tokens/s; decode HBM GB/s (% of roofline)",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (splitmix64 + Box-Muller, the benchmark configs' seeds)",
        "config": {"workload": "attention fwd+bwd, packed varlen causal, 16384 tokens in "
                               f"{len(syn.attention_lengths()[0])} sequences, Hq=32, Hkv=8, "
                               "D=128 (BASELINE config 2)",
                   "tokens": 16384, "hq": 32, "hkv": 8, "d": 128,
                   "visible_pairs": P2, "flop_per_step": flop2},
        "roofline": {"bound": "mfma", "kernel": dom, "kernel_us": round(dom_ms * 1e3, 2),
                     "flop_per_launch": dom_flop, "achieved": round(achieved, 2),
                     "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
