#!/usr/bin/env python3
"""Decode-step benchmark of the quantized Nemotron-H-8B paths on one MI355X.

One step = the quantized work of one decode step of the hybrid stack at batch 64, context 16384:
  4 attention layers:  INT4 pack of the new K and V token (one lq_int4_pack_kv_pair call, as the
                       module's _pack_kv_into_cache makes it) + q_len=1 decode attention
                       over the packed cache (32 query / 8 KV heads, head_dim 128, group 32)
  24 Mamba2 layers:    fused MX4 selective-state update (128 heads x 64 x 128, 8 groups,
                       stochastic writeback from the counter generator)
Every layer owns its own cache / state (about 8 GB in total), so no buffer is reused within a
step and the 256 MB Infinity Cache cannot hold a layer's data between its uses. Inputs are
synthetic (random packed caches with fp32 scales, N(0, 0.5) states, N(0, 1) activations) and
resident in HBM before the timed region.

Prints one JSON line: value = microseconds per step (lower is better), per-kernel HIP-event
timings over the timed steps, the roofline of the dominant kernel, and the CPU oracle timed on a
bounded sample of the same work on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = ("µs/decode-step & achieved HBM GB/s (frac of 8 TB/s): INT4 attn, MX8/MX4 state")
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=16384)
    ap.add_argument("--group", type=int, default=32)
    ap.add_argument("--attn-layers", type=int, default=4)
    ap.add_argument("--mamba-layers", type=int, default=24)
    ap.add_argument("--state-bits", type=int, default=4, choices=[4, 8])
    ap.add_argument("--state-layout", default="reference", choices=["reference", "compact"],
                    help="MX cache layout: the reference's tensors (default) or the compact one "
                         "(bit micro-exponents, MX4 nibble mantissas; same arithmetic)")
    ap.add_argument("--cpu-baseline", choices=["on", "off"], default="on")
    ap.add_argument("--sweep", nargs="?", const="all", default=None,
                    choices=["all", "attention", "state", "prefill"],
                    help="instead of the decode step, time each kernel alone over the BASELINE "
                         "configurations (attention: batch 1/8/64 x ctx 1K/4K/16K; MX8, MX4 and "
                         "bf16 state updates: batch 1/8/64; INT4 prefill: L 1K/4K/16K), each call "
                         "after a 512 MB scratch read so that nothing is cache-resident; prints "
                         "one JSON line. An argument restricts it to one kernel family")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 1 GiB device-to-device copy, the reference kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return ap.parse_args()


class Events:
    """Pairs of timing events recorded on the current stream around each kernel call."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs: dict[str, list] = {}

    def around(self, name, fn):
        t = self.torch
        a = t.cuda.Event(enable_timing=True)
        b = t.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        self.pairs.setdefault(name, []).append((a, b))

    def mean_us(self, name):
        pairs = self.pairs.get(name, [])
        if not pairs:
            return None
        return 1000.0 * sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)


def _mx_tensors(torch, shape, bits, layout, dev):
    """Empty MX state tensors (q_state, shared_exp, micro_exp) in the given layout."""
    b, h, p, n = shape
    if layout == "compact":
        q = torch.empty(b, h, p, n // 2 if bits == 4 else n,
                        dtype=torch.uint8 if bits == 4 else torch.int8, device=dev)
        m = torch.empty(b, h, p, n // 16, dtype=torch.uint8, device=dev)
    else:
        q = torch.empty(shape, dtype=torch.int8, device=dev)
        m = torch.empty(b, h, p, n // 2, dtype=torch.uint8, device=dev)
    return q, torch.empty(b, h, p, n // 16, dtype=torch.uint8, device=dev), m


def build_workload(torch, args, dev):
    from layer_quant_amd import _abi
    from layer_quant_amd.traffic import attention_bytes, mx_update_bytes, pack_bytes

    B, S, g = args.batch, args.ctx, args.group
    hq, hkv, d = 32, 8, 128
    nh, p_, n, ng = 128, 64, 128, 8
    gen = torch.Generator(device=dev).manual_seed(0)
    attn = []
    for _ in range(args.attn_layers):
        layer = dict(
            k_packed=torch.randint(0, 256, (B, hkv, S, d // 2), dtype=torch.uint8, device=dev,
                                   generator=gen),
            v_packed=torch.randint(0, 256, (B, hkv, S, d // 2), dtype=torch.uint8, device=dev,
                                   generator=gen),
            k_scale=torch.rand(B, hkv, S, d // g, device=dev, generator=gen) * 0.5 + 0.01,
            v_scale=torch.rand(B, hkv, S, d // g, device=dev, generator=gen) * 0.5 + 0.01,
            q=torch.randn(B, hq, 1, d, device=dev, generator=gen).to(torch.bfloat16),
            k_new=torch.randn(B, hkv, 1, d, device=dev, generator=gen).to(torch.bfloat16),
            v_new=torch.randn(B, hkv, 1, d, device=dev, generator=gen).to(torch.bfloat16),
            out=torch.empty(B, hq, d, device=dev, dtype=torch.bfloat16),
            pos=torch.full((1,), S - 1, dtype=torch.long, device=dev),
        )
        attn.append(layer)
    mamba = []
    for _ in range(args.mamba_layers):
        h0 = torch.randn(B, nh, p_, n, device=dev, generator=gen) * 0.5
        st = _mx_tensors(torch, (B, nh, p_, n), args.state_bits, args.state_layout, dev)
        _abi.mx_encode(h0, *st, args.state_bits, _abi.ROUND_NEAREST_EVEN)
        del h0
        layer = dict(
            st=st,
            x=torch.randn(B, nh, p_, device=dev, generator=gen).to(torch.bfloat16),
            dt=torch.randn(B, nh, device=dev, generator=gen).to(torch.bfloat16)[:, :, None]
            .expand(B, nh, p_),
            A=(-torch.exp(torch.rand(nh, device=dev, generator=gen) * 2))[:, None, None]
            .expand(nh, p_, n),
            B=torch.randn(B, ng, n, device=dev, generator=gen).to(torch.bfloat16),
            C=torch.randn(B, ng, n, device=dev, generator=gen).to(torch.bfloat16),
            D=torch.randn(nh, device=dev, generator=gen)[:, None].expand(nh, p_),
            dt_bias=(torch.randn(nh, device=dev, generator=gen) * 0.1)[:, None].expand(nh, p_),
            out=torch.empty(B, nh, p_, device=dev, dtype=torch.bfloat16),
            step=0,
        )
        mamba.append(layer)
    torch.cuda.synchronize()
    sizes = dict(
        attention=attention_bytes(B, hq, hkv, d, S, g),
        pack=2 * pack_bytes(B, hkv, 1, d, g),  # K and V in one call
        mx_update=mx_update_bytes(B, nh, p_, n, ng, format_bits=args.state_bits,
                                  layout=args.state_layout),
    )
    return attn, mamba, sizes


def run_step(torch, args, attn, mamba, ev=None):
    from layer_quant_amd import _abi

    B, S, g = args.batch, args.ctx, args.group
    total_state = B * 128 * 64 * 128

    def call(name, fn):
        if ev is None:
            fn()
        else:
            ev.around(name, fn)

    for L in attn:
        call("pack", lambda: _abi.int4_pack_kv_pair(L["k_new"], L["v_new"], L["k_packed"],
                                                    L["v_packed"], L["k_scale"], L["v_scale"],
                                                    L["pos"], g))
        call("attention", lambda: _abi.int4_decode_attention(
            L["q"], L["k_packed"], L["v_packed"], L["k_scale"], L["v_scale"], None, L["out"], S,
            4, g))
    for M in mamba:
        off = M["step"] * total_state
        call("mx_update", lambda: _abi.mx_state_update(
            *M["st"], M["x"], M["dt"], M["dt_bias"], M["A"], M["B"], M["C"], M["D"], None,
            M["out"], args.state_bits, True, _abi.ROUND_SR_COUNTER, seed=1234, rng_offset=off))
        M["step"] += 1


def sweep(torch, dev, which: str = "all", reps: int = 20):
    """Per-kernel cold-cache timings over the BASELINE configurations."""
    from layer_quant_amd import _abi
    from layer_quant_amd.traffic import (attention_bytes, mx_update_bytes, prefill_flops,
                                         ssm_update_bytes)

    scratch = torch.ones(512 << 20, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    cache_bytes = 256 << 20

    def timed(fn):
        fn()
        ts = []
        for i in range(reps):
            scratch.max()  # reads 512 MB: evicts L2 and the Infinity Cache, leaves no dirty lines
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            ts.append((a, b))
        torch.cuda.synchronize()
        us = sorted(1000.0 * a.elapsed_time(b) for a, b in ts)
        return us[len(us) // 2], sum(us) / len(us)

    def row(kernel, nbytes, med, mean, **cfg):
        gbs = nbytes / (med * 1e-6) / 1e9
        r = dict(kernel=kernel, **cfg, median_us=round(med, 2), mean_us=round(mean, 2),
                 algorithmic_bytes=nbytes, GB_s=round(gbs, 1),
                 frac_of_peak=round(gbs / PEAK_HBM_GBS, 4), fits_in_infinity_cache=nbytes <= cache_bytes)
        log(f"{kernel} {cfg}: {med:.1f} us, {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%})")
        return r

    rows = []
    hq, hkv, d, g = 32, 8, 128, 32
    shapes = [(B, S, g) for B in (1, 8, 64) for S in (1024, 4096, 16384)]
    shapes.append((8, 2072, 64))  # the shape of the reference's own published figure (A100)
    shapes.append((64, 16384, 64))  # the reference driver's default group (--kv-group-size 64)
    for B, S, gs in (shapes if which in ("all", "attention") else ()):
        kp = torch.randint(0, 256, (B, hkv, S, d // 2), dtype=torch.uint8, device=dev, generator=gen)
        vp = torch.randint(0, 256, (B, hkv, S, d // 2), dtype=torch.uint8, device=dev, generator=gen)
        ks = torch.rand(B, hkv, S, d // gs, device=dev, generator=gen) + 0.01
        vs = torch.rand(B, hkv, S, d // gs, device=dev, generator=gen) + 0.01
        q = torch.randn(B, hq, 1, d, device=dev, generator=gen).to(torch.bfloat16)
        out = torch.empty(B, hq, d, device=dev, dtype=torch.bfloat16)
        med, mean = timed(lambda: _abi.int4_decode_attention(q, kp, vp, ks, vs, None, out, S, 4, gs))
        rows.append(row("int4_decode_attention", attention_bytes(B, hq, hkv, d, S, gs), med, mean,
                        batch=B, ctx=S, group=gs))
        del kp, vp, ks, vs
    nh, p_, n, ng = 128, 64, 128, 8
    for B in ((1, 8, 64) if which in ("all", "state") else ()):
        x = torch.randn(B, nh, p_, device=dev, generator=gen).to(torch.bfloat16)
        dt = torch.randn(B, nh, device=dev, generator=gen).to(torch.bfloat16)[:, :, None].expand(B, nh, p_)
        A = (-torch.exp(torch.rand(nh, device=dev, generator=gen) * 2))[:, None, None].expand(nh, p_, n)
        Bm = torch.randn(B, ng, n, device=dev, generator=gen).to(torch.bfloat16)
        Cm = torch.randn(B, ng, n, device=dev, generator=gen).to(torch.bfloat16)
        D = torch.randn(nh, device=dev, generator=gen)[:, None].expand(nh, p_)
        dtb = (torch.randn(nh, device=dev, generator=gen) * 0.1)[:, None].expand(nh, p_)
        out = torch.empty(B, nh, p_, device=dev, dtype=torch.bfloat16)
        h0 = torch.randn(B, nh, p_, n, device=dev, generator=gen) * 0.5
        for bits, layout in ((8, "reference"), (4, "reference"), (8, "compact"), (4, "compact")):
            st = _mx_tensors(torch, (B, nh, p_, n), bits, layout, dev)
            _abi.mx_encode(h0, *st, bits, _abi.ROUND_NEAREST_EVEN)
            step = [0]

            def upd():
                _abi.mx_state_update(*st, x, dt, dtb, A, Bm, Cm, D, None, out, bits, True,
                                     _abi.ROUND_SR_COUNTER, seed=1234,
                                     rng_offset=step[0] * B * nh * p_ * n)
                step[0] += 1
            med, mean = timed(upd)
            rows.append(row(f"mx{bits}_state_update", mx_update_bytes(
                B, nh, p_, n, ng, format_bits=bits, layout=layout), med, mean, batch=B,
                layout=layout, rounding="stochastic (counter)"))
        # the BASELINE configurations' seeded uniform tensor (reference formula, bit-exact mode):
        # the fp32 tensor adds 4 bytes per state element to the traffic
        uni = torch.rand(B, nh, p_, n, device=dev, generator=gen)
        for bits in (8, 4):
            st = _mx_tensors(torch, (B, nh, p_, n), bits, "reference", dev)
            _abi.mx_encode(h0, *st, bits, _abi.ROUND_NEAREST_EVEN)
            med, mean = timed(lambda: _abi.mx_state_update(*st, x, dt, dtb, A, Bm, Cm, D, None, out,
                                                           bits, True, _abi.ROUND_SR_UNIFORM,
                                                           uniform=uni))
            rows.append(row(f"mx{bits}_state_update", mx_update_bytes(
                B, nh, p_, n, ng, format_bits=bits) + 4 * uni.numel(), med, mean, batch=B,
                layout="reference", rounding="stochastic (supplied uniform tensor)"))
        del uni
        state = h0.to(torch.bfloat16)
        med, mean = timed(lambda: _abi.selective_state_update(state, x, dt, dtb, A, Bm, Cm, D, None,
                                                              out, True))
        rows.append(row("bf16_selective_state_update", ssm_update_bytes(B, nh, p_, n, ng), med, mean,
                        batch=B))
    for L in ((1024, 4096, 16384) if which in ("all", "prefill") else ()):
        # causal prefill over the packed cache of one attention layer, batch 1 (MFMA-bound)
        kp = torch.randint(0, 256, (1, hkv, L, d // 2), dtype=torch.uint8, device=dev, generator=gen)
        vp = torch.randint(0, 256, (1, hkv, L, d // 2), dtype=torch.uint8, device=dev, generator=gen)
        ks = torch.rand(1, hkv, L, d // g, device=dev, generator=gen) + 0.01
        vs = torch.rand(1, hkv, L, d // g, device=dev, generator=gen) + 0.01
        q = torch.randn(1, hq, L, d, device=dev, generator=gen).to(torch.bfloat16)
        out = torch.empty(1, hq, L, d, device=dev, dtype=torch.bfloat16)
        med, mean = timed(lambda: _abi.int4_prefill_attention(q, kp, vp, ks, vs, out, 4, g))
        fl = prefill_flops(1, hq, L, d)
        tfs = fl / (med * 1e-6) / 1e12
        rows.append(dict(kernel="int4_prefill_attention", batch=1, q_len=L, group=g,
                         median_us=round(med, 2), mean_us=round(mean, 2), algorithmic_flops=fl,
                         TFLOP_s=round(tfs, 1), frac_of_peak=round(tfs / PEAK_BF16_TFLOPS, 4),
                         peak="bf16 dense MFMA"))
        log(f"int4_prefill_attention L={L}: {med:.1f} us, {tfs:.0f} TFLOP/s "
            f"({tfs / PEAK_BF16_TFLOPS:.1%} of bf16 MFMA)")
        del kp, vp, ks, vs, q, out
    return {"sweep": rows, "reps": reps, "timing": "median of per-call HIP events, each call after a "
            "512 MB scratch read (a read evicts the caches without leaving dirty lines whose "
            "write-back would compete with the timed kernel)", "peak_GB_s": PEAK_HBM_GBS}


def config1_gpu(torch, dev, reps: int = 20) -> float:
    """BASELINE config 1 on the GPU through the C ABI: pack a 1024-token K/V cache (one
    lq_int4_pack_kv_pair call) and attend once (lq_int4_decode_attention), batch 1, 32 q / 8 KV
    heads, group 32; median us per repetition (HIP events)."""
    from layer_quant_amd import _abi

    hq, hkv, d, g, S = 32, 8, 128, 32, 1024
    gen = torch.Generator(device=dev).manual_seed(0)
    k = torch.randn(1, hkv, S, d, device=dev, generator=gen).to(torch.bfloat16)
    v = torch.randn(1, hkv, S, d, device=dev, generator=gen).to(torch.bfloat16)
    q = torch.randn(1, hq, 1, d, device=dev, generator=gen).to(torch.bfloat16)
    kp = torch.empty(1, hkv, S, d // 2, dtype=torch.uint8, device=dev)
    vp = torch.empty_like(kp)
    ks = torch.empty(1, hkv, S, d // g, device=dev)
    vs = torch.empty_like(ks)
    pos = torch.arange(S, device=dev)
    out = torch.empty(1, hq, d, device=dev, dtype=torch.bfloat16)

    def once():
        _abi.int4_pack_kv_pair(k, v, kp, vp, ks, vs, pos, g)
        _abi.int4_decode_attention(q, kp, vp, ks, vs, None, out, S, hq // hkv, g)

    once()
    ts = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        once()
        b.record()
        ts.append((a, b))
    torch.cuda.synchronize()
    us = sorted(1000.0 * a.elapsed_time(b) for a, b in ts)
    return us[len(us) // 2]


def cpu_baseline(args):
    """The CPU oracle (torch fp32/fp64 restatement of the reference formulas) on a bounded
    sample of the same step, on this host's cores, scaled linearly to the full step."""
    import numpy as np
    import torch

    from oracle import int4_kv as oik
    from oracle import mx_state as omx

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(0)
    hq, hkv, d, g = 32, 8, 128, args.group
    s_sample = args.ctx
    ba_sample = min(args.batch, 2)
    cache = oik.allocate_cache(ba_sample, hkv, s_sample, d, g)
    kv = torch.randn(ba_sample, hkv, s_sample, d, generator=gen).to(torch.bfloat16)
    oik.pack_kv_into_cache(cache, kv, kv, torch.arange(s_sample), g)
    del kv
    q = torch.randn(ba_sample, hq, 1, d, generator=gen).to(torch.bfloat16)
    new = torch.randn(ba_sample, hkv, 1, d, generator=gen).to(torch.bfloat16)

    def attn_once():
        oik.pack_into(cache["k_packed"], cache["k_scale"], new, torch.tensor([s_sample - 1]), g)
        oik.pack_into(cache["v_packed"], cache["v_scale"], new, torch.tensor([s_sample - 1]), g)
        oik.decode_attention(q, cache["k_packed"], cache["v_packed"], cache["k_scale"],
                             cache["v_scale"], s_sample, 4, g)

    b_sample = min(args.batch, 8)
    shape = (b_sample, 128, 64, 128)
    qs, es, ms_ = omx.mx_encode((torch.randn(shape, generator=gen) * 0.5).numpy(), args.state_bits)
    x = torch.randn(b_sample, 128, 64, generator=gen).to(torch.bfloat16)
    dt = torch.randn(b_sample, 128, 64, generator=gen).to(torch.bfloat16)
    A = -torch.rand(128, generator=gen)[:, None, None].expand(128, 64, 128)
    Bm = torch.randn(b_sample, 8, 128, generator=gen).to(torch.bfloat16)
    D = torch.randn(128, generator=gen)[:, None].expand(128, 64)

    def mx_once():
        omx.mx_update(qs, es, ms_, x, dt, A, Bm, Bm, D=D, dt_bias=D * 0.1, dt_softplus=True,
                      format_bits=args.state_bits, round_mode=omx.ROUND_SR_COUNTER, seed=1234)

    def timed(fn, reps):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    # BASELINE config 1 (the reference's CPU-runnable case): pack a 1024-token K/V cache and
    # attend once, batch 1, 32 q / 8 KV heads, group 32, seed 0
    g1 = 32
    kv1 = torch.randn(2, 1, hkv, 1024, d, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    q1 = torch.randn(1, hq, 1, d, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)

    def config1_once():
        c1 = oik.allocate_cache(1, hkv, 1024, d, g1)
        oik.pack_kv_into_cache(c1, kv1[0], kv1[1], torch.arange(1024), g1)
        oik.decode_attention(q1, c1["k_packed"], c1["v_packed"], c1["k_scale"], c1["v_scale"],
                             1024, 4, g1)

    reps = 3
    t_cfg1 = timed(config1_once, 5)
    t_attn = timed(attn_once, reps)
    t_mx = timed(mx_once, reps)
    scale_attn = (args.batch / ba_sample) * (args.ctx / s_sample)
    scale_mx = args.batch / b_sample
    step_s = args.attn_layers * t_attn * scale_attn + args.mamba_layers * t_mx * scale_mx
    return {
        "value": round(step_s * 1e6, 1),
        "unit": "us/step",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle (torch/numpy CPU, torch threads = cores; numpy elementwise work "
                   f"single-threaded) on 1 attention layer at batch {ba_sample}, ctx {s_sample} "
                   f"(pack K,V + attend) and 1 MX{args.state_bits} update at batch {b_sample}, "
                   f"median of {reps} after one warm-up, scaled linearly to {args.attn_layers} "
                   f"layers x batch {args.batch} x ctx {args.ctx} and {args.mamba_layers} layers x "
                   f"batch {args.batch}; attention {t_attn * 1e3:.1f} ms, update "
                   f"{t_mx * 1e3:.1f} ms per sample call"),
        "config1_us": round(t_cfg1 * 1e6, 1),
    }


def load_traffic(kernel: str, workload: str):
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        data = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    entry = data.get(kernel, {})
    if entry.get("workload") != workload:
        return None
    return entry.get("bytes_per_launch")


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path has no multi-GPU component in this build)", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.sweep:
        print(json.dumps(sweep(torch, dev, args.sweep)), flush=True)
        return
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log(f"building workload: batch {args.batch}, ctx {args.ctx}, {args.attn_layers} attention "
        f"+ {args.mamba_layers} MX{args.state_bits} layers")
    attn, mamba, sizes = build_workload(torch, args, dev)
    log("warmup")
    for _ in range(args.warmup):
        run_step(torch, args, attn, mamba)
    torch.cuda.synchronize()

    # timed region 1: whole steps, no per-kernel events
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(torch, args, attn, mamba)
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / args.steps
    log(f"step: {step_s * 1e6:.1f} us")

    # timed region 2: the same steps with HIP events around every kernel call
    ev = Events(torch)
    for _ in range(args.steps):
        run_step(torch, args, attn, mamba, ev)
    torch.cuda.synchronize()
    kernels = {}
    for name, nbytes in sizes.items():
        us = ev.mean_us(name)
        if us is None:  # no such layer in this configuration
            continue
        gbs = nbytes / (us * 1e-6) / 1e9
        kernels[name] = {"us": round(us, 2), "algorithmic_bytes": nbytes,
                         "GB_s": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
                         "calls_per_step": {"attention": args.attn_layers,
                                            "pack": args.attn_layers,
                                            "mx_update": args.mamba_layers}[name]}
        log(f"{name}: {us:.1f} us/call, {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%})")
    dominant = max(kernels, key=lambda k: kernels[k]["us"] * kernels[k]["calls_per_step"])
    dk = kernels[dominant]
    workload = f"b{args.batch}_ctx{args.ctx}_g{args.group}_mx{args.state_bits}" + (
        "_compact" if args.state_layout == "compact" else "")
    roofline = {
        "kernel": {"attention": "lq_int4_decode_attention (attn_fast_kernel, + attn_merge_kernel "
                                "when split)",
                   "mx_update": f"lq_mx_state_update (mx_update_rows_kernel MX{args.state_bits})",
                   "pack": "lq_int4_pack_kv_pair"}[dominant],
        "bound": "hbm",
        "achieved": dk["GB_s"],
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": dk["frac_of_peak"],
        "traffic": load_traffic(dominant, workload),
    }
    cfg1_gpu = config1_gpu(torch, dev)
    cpu = None
    cfg1 = None
    if args.cpu_baseline == "on":
        log("cpu baseline")
        cpu = cpu_baseline(args)
        cfg1_cpu = cpu.pop("config1_us")
        cfg1 = {"workload": "BASELINE config 1: pack a 1024-token INT4 K/V cache + one q_len=1 "
                            "decode attention, batch 1, 32 q / 8 KV heads, head_dim 128, group 32",
                "gpu_us": round(cfg1_gpu, 1), "cpu_us": cfg1_cpu, "cpu_cores": cpu["cores"],
                "cpu_kind": "port (oracle)"}
    line = {
        "metric": METRIC,
        "value": round(step_s * 1e6, 1),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"Nemotron-H-8B decode step, quantized paths only: {args.attn_layers} "
                         f"INT4-KV attention layers (32q/8kv heads, head_dim 128, group "
                         f"{args.group}, ctx {args.ctx}) with their K/V packs + "
                         f"{args.mamba_layers} MX{args.state_bits} Mamba2 state updates "
                         "(128 heads x 64 x 128, 8 groups, stochastic writeback"
                         + (", compact cache layout)" if args.state_layout == "compact" else ")")),
            "batch": args.batch,
            "ctx": args.ctx,
            "group_size": args.group,
            "state_format": f"mx{args.state_bits}",
            "state_layout": args.state_layout,
        },
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "config1_cpu_vs_gpu": cfg1,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
