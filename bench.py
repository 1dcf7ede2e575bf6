#!/usr/bin/env python3
"""Decode-step benchmark of the quantized Nemotron-H-8B paths on one MI355X.

One step = the quantized work of one decode step of the hybrid stack at batch 64, context 16384:
  4 attention layers:  INT4 pack of the new K and V token into cache row S - 1 + q_len=1 decode
                       attention over the packed cache (32 query / 8 KV heads, head_dim 128,
                       group 32): one lq_int4_decode_attention_pack call, as the module's
                       decode branch makes it (one kernel: the attention packs the token)
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
    ap.add_argument("--steps", type=int, default=20)
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
    ap.add_argument("--settle-seconds", type=float, default=0.3,
                    help="after the warmup steps, keep running untimed steps until this much "
                         "time has passed: under sustained load the GPU clocks ramp up over the "
                         "first ~50 ms, and the VALU-heavy MX update runs 20-25 %% slower "
                         "before they settle")
    ap.add_argument("--cpu-baseline", choices=["on", "off"], default="on")
    ap.add_argument("--layout-pair", choices=["on", "off"], default="on",
                    help="after the timed steps, time the same MX updates on compact-layout "
                         "states (layout_pair in the line; reference-layout runs only)")
    ap.add_argument("--sweep", nargs="?", const="all", default=None,
                    choices=["all", "attention", "state", "prefill", "pack"],
                    help="instead of the decode step, time each kernel alone over the BASELINE "
                         "configurations (attention: batch 1/8/64 x ctx 1K/4K/16K; MX8, MX4 and "
                         "bf16 state updates: batch 1/8/64; INT4 prefill: L 1K/4K/16K; the K+V "
                         "pack of a prompt, L 1K/4K/16K, and of one decode token), each call "
                         "after a 512 MB scratch read so that nothing is cache-resident; prints "
                         "one JSON line. An argument restricts it to one kernel family")
    ap.add_argument("--batches", default=None,
                    help="--sweep: comma-separated batch sizes to keep (default: all)")
    ap.add_argument("--ctxs", default=None,
                    help="--sweep attention: comma-separated contexts to keep (default: all)")
    ap.add_argument("--lengths", default=None,
                    help="--sweep prefill / pack: comma-separated prompt lengths (default 1024,4096,16384)")
    ap.add_argument("--reps", type=int, default=20,
                    help="--sweep: timed calls per configuration (median reported)")
    ap.add_argument("--cpu-pairs", choices=["on", "off"], default="on",
                    help="--sweep: time the CPU oracle on the same inputs next to each "
                         "attention (batch 1 and 8) and MX-update configuration")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 1 GiB device-to-device copy, the reference kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return ap.parse_args()


class Events:
    """Pairs of timing events recorded on the current stream around each kernel call."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs: dict[str, list] = {}

    def around(self, name, fn, calls: int = 1):
        """Time fn() (which makes `calls` launches of kernel `name`, back to back) with one
        event pair; its launches count as `calls` calls of equal duration."""
        t = self.torch
        a = t.cuda.Event(enable_timing=True)
        b = t.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        self.pairs.setdefault(name, []).append((a, b, calls))

    def mean_us(self, name):
        pairs = self.pairs.get(name, [])
        if not pairs:
            return None
        return 1000.0 * sum(a.elapsed_time(b) for a, b, _ in pairs) / sum(c for *_, c in pairs)

    def spread_us(self, name):
        """min / median / max of the per-call durations (us; per event pair divided by its
        launches) and the number of calls."""
        pairs = self.pairs.get(name, [])
        us = sorted(1000.0 * a.elapsed_time(b) / c for a, b, c in pairs)
        if not us:
            return None
        return {"min": round(us[0], 2), "median": round(us[len(us) // 2], 2),
                "max": round(us[-1], 2), "calls": sum(c for *_, c in pairs),
                "event_pairs": len(us)}


def cpu_cores() -> tuple[int, str]:
    """Host threads the CPU baseline uses: every core in this process's affinity set, limited by
    the cgroup CPU quota when one is set (the share a container or job actually gets)."""
    cores = len(os.sched_getaffinity(0))
    how = f"{cores} cores in the affinity set"
    quota = None
    try:
        text = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if text and text[0] != "max":
            quota = int(text[0]) / int(text[1])
    except (OSError, ValueError, IndexError):
        try:
            q = int(Path("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read_text())
            per = int(Path("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read_text())
            quota = q / per if q > 0 else None
        except (OSError, ValueError):
            quota = None
    if quota is not None and int(quota) < cores:
        cores = max(1, int(quota))
        how += f", cgroup CPU quota {quota:g}"
    return cores, how


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_time(fn, min_reps: int = 3, max_reps: int = 5, long_s: float = 3.0) -> float:
    """Median seconds of fn() on the host after one warm-up call: max_reps repetitions, or
    min_reps when one call takes longer than long_s."""
    import statistics

    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    reps = min_reps if first > long_s else max_reps
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def oracle_mx_update_threaded(pool, workers, q, e, m, x, dt, A, B, C, D, dt_bias, bits, seed,
                              rng_offset):
    """The CPU oracle's MX update (oracle.mx_state.mx_update, counter rounding) split over batch
    chunks run on `workers` threads (rows are independent; each chunk's counter offset is its
    first element's index, so the draws are the same as one call's). numpy and torch release the
    GIL inside their kernels, so the chunks run in parallel."""
    from oracle import mx_state as omx

    bsz = q.shape[0]
    per = q[0].size
    bounds = [(bsz * i // workers, bsz * (i + 1) // workers) for i in range(workers)]
    bounds = [(a, b) for a, b in bounds if b > a]

    def one(ab):
        a, b = ab
        return omx.mx_update(q[a:b], e[a:b], m[a:b], x[a:b], dt[a:b], A, B[a:b], C[a:b], D=D,
                             dt_bias=dt_bias, dt_softplus=True, format_bits=bits,
                             round_mode=omx.ROUND_SR_COUNTER, seed=seed,
                             rng_offset=rng_offset + a * per)

    return list(pool.map(one, bounds))


def oracle_attention_threaded(pool, cache, q, new, seq_len, nrep, g):
    """One decode-attention layer of the CPU oracle at the full batch: per batch element, pack
    the new K and V token into cache row seq_len - 1 (oracle.int4_kv.pack_into) and attend over
    the context (oracle.int4_kv.decode_attention, float64); the batch elements run as separate
    tasks on the pool's threads (each task single-threaded; torch releases the GIL in its
    kernels). Batch elements are independent, so the result is the one-call result."""
    import torch

    from oracle import int4_kv as oik

    pos = torch.tensor([seq_len - 1])

    def one(b):
        sl = slice(b, b + 1)
        oik.pack_into(cache["k_packed"][sl], cache["k_scale"][sl], new[sl], pos, g)
        oik.pack_into(cache["v_packed"][sl], cache["v_scale"][sl], new[sl], pos, g)
        return oik.decode_attention(q[sl], cache["k_packed"][sl], cache["v_packed"][sl],
                                    cache["k_scale"][sl], cache["v_scale"][sl], seq_len, nrep, g)

    return list(pool.map(one, range(q.shape[0])))


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
        # the fused call: the attention's reads plus the new K and V token's pack
        attention=attention_bytes(B, hq, hkv, d, S, g) + 2 * pack_bytes(B, hkv, 1, d, g),
        mx_update=mx_update_bytes(B, nh, p_, n, ng, format_bits=args.state_bits,
                                  layout=args.state_layout),
    )
    return attn, mamba, sizes


def run_step(torch, args, attn, mamba, ev=None, round_mode=None):
    from layer_quant_amd import _abi

    mode = _abi.ROUND_SR_COUNTER if round_mode is None else round_mode

    B, S, g = args.batch, args.ctx, args.group
    total_state = B * 128 * 64 * 128

    def call(name, fn, calls=1):
        if ev is None:
            fn()
        else:
            ev.around(name, fn, calls)

    # attention layers: pack the new token into row S - 1 and attend, one call per layer, each
    # timed by its own event pair (1-3 % of event overhead on the 210 us call)
    for L in attn:
        call("attention", lambda: _abi.int4_decode_attention_pack(
            L["q"], L["k_new"], L["v_new"], L["k_packed"], L["v_packed"], L["k_scale"],
            L["v_scale"], None, L["out"], S, 4, g))

    # the Mamba layers' updates run back to back and are timed as one run per step: an event
    # pair around every 40 us update adds its own dispatch time (per-call events read 1-2.5 us
    # above the kernel trace's durations), one pair per run of 24 spreads it over 24 calls
    def updates():
        for M in mamba:
            off = M["step"] * total_state
            _abi.mx_state_update(
                *M["st"], M["x"], M["dt"], M["dt_bias"], M["A"], M["B"], M["C"], M["D"], None,
                M["out"], args.state_bits, True, mode, seed=1234, rng_offset=off)
            M["step"] += 1

    if mamba:
        call("mx_update", updates, len(mamba))


def _ints(text):
    return None if not text else [int(v) for v in str(text).split(",") if v.strip()]


def sweep(torch, dev, args):
    """Per-kernel cold-cache timings over the BASELINE configurations, each with the CPU oracle
    timed on the same inputs (attention at batch 1 and 8, every state update) unless
    --cpu-pairs off."""
    from concurrent.futures import ThreadPoolExecutor

    from layer_quant_amd import _abi
    from layer_quant_amd.traffic import (attention_bytes, mx_update_bytes, pack_bytes,
                                         prefill_flops, ssm_update_bytes)
    from oracle import int4_kv as oik
    from oracle import mx_state as omx

    which, reps = args.sweep, args.reps
    keep_b, keep_s = _ints(args.batches), _ints(args.ctxs)
    lengths = _ints(args.lengths) or [1024, 4096, 16384]
    pairs = args.cpu_pairs == "on"
    cores, how = cpu_cores()
    torch.set_num_threads(cores)
    pool = ThreadPoolExecutor(max_workers=cores) if pairs else None
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

    def cpu_pair(r, fn, what):
        sec = cpu_time(fn)
        r["cpu_baseline"] = {"us": round(sec * 1e6, 1), "cores": cores, "kind": "port",
                             "what": what, "cpu_over_gpu": round(sec * 1e6 / r["median_us"], 1)}
        log(f"  cpu oracle: {sec * 1e3:.1f} ms ({r['cpu_baseline']['cpu_over_gpu']}x the GPU)")

    def want(b, s=None):
        return (keep_b is None or b in keep_b) and (s is None or keep_s is None or s in keep_s)

    rows = []
    hq, hkv, d, g = 32, 8, 128, 32
    shapes = [(B, S, g) for B in (1, 8, 64) for S in (1024, 4096, 16384)]
    shapes.append((8, 2072, 64))  # the shape of the reference's own published figure (A100)
    shapes.append((64, 16384, 64))  # the reference driver's default group (--kv-group-size 64)
    for B, S, gs in (shapes if which in ("all", "attention") else ()):
        if not want(B, S):
            continue
        kp = torch.randint(0, 256, (B, hkv, S, d // 2), dtype=torch.uint8, device=dev, generator=gen)
        vp = torch.randint(0, 256, (B, hkv, S, d // 2), dtype=torch.uint8, device=dev, generator=gen)
        ks = torch.rand(B, hkv, S, d // gs, device=dev, generator=gen) + 0.01
        vs = torch.rand(B, hkv, S, d // gs, device=dev, generator=gen) + 0.01
        q = torch.randn(B, hq, 1, d, device=dev, generator=gen).to(torch.bfloat16)
        out = torch.empty(B, hq, d, device=dev, dtype=torch.bfloat16)
        med, mean = timed(lambda: _abi.int4_decode_attention(q, kp, vp, ks, vs, None, out, S, 4, gs))
        r = row("int4_decode_attention", attention_bytes(B, hq, hkv, d, S, gs), med, mean,
                batch=B, ctx=S, group=gs)
        if pairs and B <= 8:
            c = [t.cpu() for t in (q, kp, vp, ks, vs)]
            cpu_pair(r, lambda: oik.decode_attention(*c, S, 4, gs),
                     "oracle.int4_kv.decode_attention (float64, dequantizes the packed cache as "
                     "the reference's kernel does) on the same cache and queries")
        rows.append(r)
        del kp, vp, ks, vs
    nh, p_, n, ng = 128, 64, 128, 8
    for B in ((1, 8, 64) if which in ("all", "state") else ()):
        if not want(B):
            continue
        x = torch.randn(B, nh, p_, device=dev, generator=gen).to(torch.bfloat16)
        dt = torch.randn(B, nh, device=dev, generator=gen).to(torch.bfloat16)[:, :, None].expand(B, nh, p_)
        A = (-torch.exp(torch.rand(nh, device=dev, generator=gen) * 2))[:, None, None].expand(nh, p_, n)
        Bm = torch.randn(B, ng, n, device=dev, generator=gen).to(torch.bfloat16)
        Cm = torch.randn(B, ng, n, device=dev, generator=gen).to(torch.bfloat16)
        D = torch.randn(nh, device=dev, generator=gen)[:, None].expand(nh, p_)
        dtb = (torch.randn(nh, device=dev, generator=gen) * 0.1)[:, None].expand(nh, p_)
        out = torch.empty(B, nh, p_, device=dev, dtype=torch.bfloat16)
        h0 = torch.randn(B, nh, p_, n, device=dev, generator=gen) * 0.5
        host = [t.cpu() for t in (x, dt, A, Bm, Cm, D, dtb)] if pairs else None
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
            r = row(f"mx{bits}_state_update", mx_update_bytes(
                B, nh, p_, n, ng, format_bits=bits, layout=layout), med, mean, batch=B,
                layout=layout, rounding="stochastic (counter)")
            if pairs and layout == "reference":
                qh, eh, mh = (t.cpu().numpy() for t in st)
                hx, hdt, hA, hB, hC, hD, hdtb = host

                def cpu_upd():
                    torch.set_num_threads(1)
                    try:
                        oracle_mx_update_threaded(pool, cores, qh, eh, mh, hx, hdt, hA, hB, hC,
                                                  hD, hdtb, bits, 1234, 0)
                    finally:
                        torch.set_num_threads(cores)
                cpu_pair(r, cpu_upd, "oracle.mx_state.mx_update (decode, fp32 update, counter "
                                     "writeback), batch chunks on every thread, same state and "
                                     "inputs")
            rows.append(r)
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
        # the reference's own draws (tl.rand's Philox4x32-10 per element, generated in the kernel)
        for bits in (8, 4):
            st = _mx_tensors(torch, (B, nh, p_, n), bits, "reference", dev)
            _abi.mx_encode(h0, *st, bits, _abi.ROUND_NEAREST_EVEN)
            med, mean = timed(lambda: _abi.mx_state_update(*st, x, dt, dtb, A, Bm, Cm, D, None, out,
                                                           bits, True, _abi.ROUND_SR_PHILOX,
                                                           seed=1234))
            rows.append(row(f"mx{bits}_state_update", mx_update_bytes(
                B, nh, p_, n, ng, format_bits=bits), med, mean, batch=B, layout="reference",
                rounding="stochastic (Philox, the reference's tl.rand stream)"))
        state = h0.to(torch.bfloat16)
        med, mean = timed(lambda: _abi.selective_state_update(state, x, dt, dtb, A, Bm, Cm, D, None,
                                                              out, True))
        r = row("bf16_selective_state_update", ssm_update_bytes(B, nh, p_, n, ng), med, mean,
                batch=B)
        if pairs:
            hs = state.cpu()
            hx, hdt, hA, hB, hC, hD, hdtb = host
            cpu_pair(r, lambda: omx.bf16_state_update(hs, hx, hdt, hA, hB, hC, D=hD,
                                                      dt_bias=hdtb, dt_softplus=True),
                     "oracle.mx_state.bf16_state_update (torch fp32, intra-op threads), same "
                     "state and inputs")
        rows.append(r)
    # the K+V pack of one attention layer (lq_int4_pack_kv_pair, one launch): a prompt's tokens
    # at batch 1 (the prefill's pack, int4_8b_attention.py:477-515 with q_len = L) and one decode
    # token at batch 64 (the standalone pack; the decode step packs inside the attention)
    for B, T in ([(1, L) for L in lengths] + [(64, 1)] if which in ("all", "pack") else ()):
        if not want(B):
            continue
        kx = torch.randn(B, hkv, T, d, device=dev, generator=gen).to(torch.bfloat16)
        vx = torch.randn(B, hkv, T, d, device=dev, generator=gen).to(torch.bfloat16)
        cap = T if T > 1 else 16384
        kp = torch.empty(B, hkv, cap, d // 2, dtype=torch.uint8, device=dev)
        vp = torch.empty_like(kp)
        ks = torch.empty(B, hkv, cap, d // g, device=dev)
        vs = torch.empty_like(ks)
        pos = torch.arange(T, device=dev) + (cap - T)
        med, mean = timed(lambda: _abi.int4_pack_kv_pair(kx, vx, kp, vp, ks, vs, pos, g))
        rows.append(row("int4_pack_kv_pair", 2 * pack_bytes(B, hkv, T, d, g), med, mean,
                        batch=B, tokens=T, group=g))
        del kx, vx, kp, vp, ks, vs
    for L in (lengths if which in ("all", "prefill") else ()):
        # causal prefill over the packed cache of one attention layer, batch 1 (MFMA-bound); no
        # CPU pair: the float64 oracle's L x L scores at L = 16384 need 69 GB
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
    if pool is not None:
        pool.shutdown()
    return {"sweep": rows, "reps": reps, "timing": "median of per-call HIP events, each call after a "
            "512 MB scratch read (a read evicts the caches without leaving dirty lines whose "
            "write-back would compete with the timed kernel)", "peak_GB_s": PEAK_HBM_GBS,
            "cpu": {"cores": cores, "how": how, "model": cpu_model(),
                    "timing": "median of 5 calls after one warm-up (3 when a call takes over 3 s)",
                    "inputs": "host copies of the GPU row's inputs, already in memory"}
            if pairs else None}


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


# The reference's own published per-call kernel times (A100 80GB PCIe, nsys, Nemotron-H-8B, batch
# 8, context 2048 + 8 warmup over 32 profiled decode steps, i.e. about 2072 keys on average, KV
# group 64): reference results/kernel_latency/data/
# nemotron_8b_kv_int4_state_mx8_nsys_cuda_gpu_kern_sum.csv:3-4.
REF_A100_ATTENTION_US = 1185.3
REF_A100_MX8_UPDATE_US = 187.2


def reference_shape(torch, dev, passes: int = 6):
    """The reference's published shape on this GPU: the INT4 decode attention at batch 8, 32 q /
    8 KV heads, ctx 2072, group 64 (lq_int4_decode_attention: the attention kernel alone, as the
    reference's figure is; its two pack launches are listed apart), and the MX8 update at batch 8 (counter stochastic writeback, as the reference's default
    stochastic=True). Each kernel runs over 16 layers of its own data back to back (307 MB and
    424 MB, more than the 256 MB Infinity Cache, so every call reads its layer cold), one event
    pair around each pass of 16 calls, enqueued behind a spin kernel so that the pass runs on
    the GPU back to back; the mean per call over `passes` passes after one untimed pass."""
    from layer_quant_amd import _abi
    from layer_quant_amd.traffic import attention_bytes, mx_update_bytes

    gen = torch.Generator(device=dev).manual_seed(2072)
    B, hq, hkv, d, S, g, layers = 8, 32, 8, 128, 2072, 64, 16
    attn = []
    for _ in range(layers):
        attn.append(dict(
            kp=torch.randint(0, 256, (B, hkv, S, d // 2), dtype=torch.uint8, device=dev, generator=gen),
            vp=torch.randint(0, 256, (B, hkv, S, d // 2), dtype=torch.uint8, device=dev, generator=gen),
            ks=torch.rand(B, hkv, S, d // g, device=dev, generator=gen) + 0.01,
            vs=torch.rand(B, hkv, S, d // g, device=dev, generator=gen) + 0.01,
            q=torch.randn(B, hq, 1, d, device=dev, generator=gen).to(torch.bfloat16),
            out=torch.empty(B, hq, d, device=dev, dtype=torch.bfloat16)))
    nh, p_, n, ng = 128, 64, 128, 8
    mx = []
    for _ in range(layers):
        h0 = torch.randn(B, nh, p_, n, device=dev, generator=gen) * 0.5
        st = _mx_tensors(torch, (B, nh, p_, n), 8, "reference", dev)
        _abi.mx_encode(h0, *st, 8, _abi.ROUND_NEAREST_EVEN)
        mx.append(dict(
            st=st, x=torch.randn(B, nh, p_, device=dev, generator=gen).to(torch.bfloat16),
            dt=torch.randn(B, nh, device=dev, generator=gen).to(torch.bfloat16)[:, :, None].expand(B, nh, p_),
            A=(-torch.exp(torch.rand(nh, device=dev, generator=gen) * 2))[:, None, None].expand(nh, p_, n),
            B=torch.randn(B, ng, n, device=dev, generator=gen).to(torch.bfloat16),
            C=torch.randn(B, ng, n, device=dev, generator=gen).to(torch.bfloat16),
            D=torch.randn(nh, device=dev, generator=gen)[:, None].expand(nh, p_),
            dtb=(torch.randn(nh, device=dev, generator=gen) * 0.1)[:, None].expand(nh, p_),
            out=torch.empty(B, nh, p_, device=dev, dtype=torch.bfloat16)))
        del h0
    step = [0]

    def attn_pass():
        for L in attn:
            _abi.int4_decode_attention(L["q"], L["kp"], L["vp"], L["ks"], L["vs"], None,
                                       L["out"], S, hq // hkv, g)

    def mx_pass():
        for L in mx:
            _abi.mx_state_update(*L["st"], L["x"], L["dt"], L["dtb"], L["A"], L["B"], L["C"],
                                 L["D"], None, L["out"], 8, True, _abi.ROUND_SR_COUNTER,
                                 seed=1234, rng_offset=step[0] * B * nh * p_ * n)
            step[0] += 1

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        ev = []
        for _ in range(passes):
            # a spin kernel ahead of each pass holds the GPU while the host enqueues the pass: the
            # calls' host-side cost (about 20 us of Python and ctypes each) exceeds these small
            # kernels, and without it the events would time the host's launch rate
            torch.cuda._sleep(2_000_000)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            ev.append((a, b))
            torch.cuda.synchronize()
        return sum(1000.0 * a.elapsed_time(b) for a, b in ev) / (passes * layers)

    a_us = timed(attn_pass)
    m_us = timed(mx_pass)
    a_bytes = attention_bytes(B, hq, hkv, d, S, g)
    m_bytes = mx_update_bytes(B, nh, p_, n, ng, format_bits=8, layout="reference")
    del attn, mx
    entry = lambda us, nbytes, ref: {
        "us": round(us, 2), "algorithmic_bytes": nbytes,
        "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
        "frac_of_peak": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
        "reference_a100_us": ref, "reference_over_this": round(ref / us, 1)}
    return {
        "what": ("the reference's published shape (A100 80GB PCIe, nsys: batch 8, ctx ~2072, "
                 "group 64; reference results/kernel_latency/data/"
                 "nemotron_8b_kv_int4_state_mx8_nsys_cuda_gpu_kern_sum.csv:3-4) on this GPU, "
                 "16 layers of data per kernel called back to back (each call reads its layer "
                 "cold; the pass enqueued behind a spin kernel, so no host gaps), mean us per "
                 "call; different hardware, so not a vs_baseline figure"),
        "int4_decode_attention_b8_ctx2072_g64": entry(a_us, a_bytes, REF_A100_ATTENTION_US),
        "mx8_state_update_b8": entry(m_us, m_bytes, REF_A100_MX8_UPDATE_US),
    }


def cpu_baseline(args):
    """The CPU oracle (torch/numpy restatement of the reference formulas, tests' checker) timed on
    this host at the step's full batch: one attention layer (pack the new K and V token, attend
    over the full context) with the batch elements as tasks on every core, and one MX update with
    batch chunks on every core; both times the step's layer counts. Inputs are host tensors
    already in memory (the attention's packed cache is random bytes and scales, as the GPU
    workload's is)."""
    from concurrent.futures import ThreadPoolExecutor

    import torch

    from oracle import int4_kv as oik
    from oracle import mx_state as omx

    cores, how = cpu_cores()
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(0)
    hq, hkv, d, g = 32, 8, 128, args.group
    S = args.ctx
    ba = args.batch
    cache = {
        "k_packed": torch.randint(0, 256, (ba, hkv, S, d // 2), dtype=torch.uint8, generator=gen),
        "v_packed": torch.randint(0, 256, (ba, hkv, S, d // 2), dtype=torch.uint8, generator=gen),
        "k_scale": torch.rand(ba, hkv, S, d // g, generator=gen) * 0.5 + 0.01,
        "v_scale": torch.rand(ba, hkv, S, d // g, generator=gen) * 0.5 + 0.01,
    }
    q = torch.randn(ba, hq, 1, d, generator=gen).to(torch.bfloat16)
    new = torch.randn(ba, hkv, 1, d, generator=gen).to(torch.bfloat16)
    pool = ThreadPoolExecutor(max_workers=cores)

    def attn_once():
        torch.set_num_threads(1)  # one thread per batch element; the pool supplies the parallelism
        try:
            oracle_attention_threaded(pool, cache, q, new, S, hq // hkv, g)
        finally:
            torch.set_num_threads(cores)

    bm = args.batch
    nh, p_, n, ng = 128, 64, 128, 8
    qs, es, ms_ = omx.mx_encode((torch.randn(bm, nh, p_, n, generator=gen) * 0.5).numpy(),
                                args.state_bits)
    x = torch.randn(bm, nh, p_, generator=gen).to(torch.bfloat16)
    dt = torch.randn(bm, nh, 1, generator=gen).to(torch.bfloat16).expand(bm, nh, p_)
    A = (-torch.exp(torch.rand(nh, generator=gen) * 2))[:, None, None].expand(nh, p_, n)
    Bm = torch.randn(bm, ng, n, generator=gen).to(torch.bfloat16)
    Cm = torch.randn(bm, ng, n, generator=gen).to(torch.bfloat16)
    D = torch.randn(nh, generator=gen)[:, None].expand(nh, p_)
    dtb = (torch.randn(nh, generator=gen) * 0.1)[:, None].expand(nh, p_)

    def mx_once():
        torch.set_num_threads(1)  # one thread per chunk; the pool supplies the parallelism
        try:
            oracle_mx_update_threaded(pool, cores, qs, es, ms_, x, dt, A, Bm, Cm, D, dtb,
                                      args.state_bits, 1234, 0)
        finally:
            torch.set_num_threads(cores)

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

    t_cfg1 = cpu_time(config1_once)
    t_attn = cpu_time(attn_once, min_reps=1, max_reps=3)
    t_mx = cpu_time(mx_once)
    pool.shutdown()
    del cache
    step_s = args.attn_layers * t_attn + args.mamba_layers * t_mx
    return {
        "value": round(step_s * 1e6, 1),
        "unit": "us/step",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle (torch/numpy CPU) on {cores} threads ({how}; {cpu_model()}), both "
                   f"legs at the full batch {args.batch}: one attention layer at ctx {S} (pack "
                   f"the new K and V token + attend, float64; the batch elements as tasks on "
                   f"{cores} threads) {t_attn * 1e3:.1f} ms; one MX{args.state_bits} update "
                   f"(batch chunks on {cores} threads) {t_mx * 1e3:.1f} ms; medians after one "
                   f"warm-up (one timed attention call when a call exceeds 3 s); step = "
                   f"{args.attn_layers} x attention + {args.mamba_layers} x update"),
        "legs_ms": {"attention_layer_full_batch": round(t_attn * 1e3, 2),
                    "mx_update_full_batch": round(t_mx * 1e3, 2)},
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


def layout_pair(torch, args, dev, mamba, ref_us):
    """The step's MX updates on compact-layout states: the same inputs, layer count, rounding
    and timing (one event pair around each step's run of back-to-back updates) as the timed
    region, with fresh states encoded from h0 ~ N(0, 0.5)."""
    from layer_quant_amd import _abi
    from layer_quant_amd.traffic import mx_update_bytes

    B, nh, p_, n, ng = args.batch, 128, 64, 128, 8
    gen = torch.Generator(device=dev).manual_seed(1)
    layers = []
    for M in mamba:
        h0 = torch.randn(B, nh, p_, n, device=dev, generator=gen) * 0.5
        st = _mx_tensors(torch, (B, nh, p_, n), args.state_bits, "compact", dev)
        _abi.mx_encode(h0, *st, args.state_bits, _abi.ROUND_NEAREST_EVEN)
        del h0
        layers.append(dict(M, st=st, step=0))
    for _ in range(3):
        run_step(torch, args, [], layers)
    torch.cuda.synchronize()
    ev = Events(torch)
    for _ in range(args.steps):
        run_step(torch, args, [], layers, ev)
    torch.cuda.synchronize()
    us = ev.mean_us("mx_update")
    nbytes = mx_update_bytes(B, nh, p_, n, ng, format_bits=args.state_bits, layout="compact")
    del layers
    return {"what": (f"the step's {len(mamba)} MX{args.state_bits} updates on compact-layout "
                     "states (nibble mantissas, bit micro-exponents; same values), timed as the "
                     "reference-layout updates of the line"),
            "reference_us": round(ref_us, 2), "compact_us": round(us, 2),
            "compact_algorithmic_bytes": nbytes,
            "compact_GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
            "compact_over_reference_time": round(us / ref_us, 4)}


def rng_pair(torch, args, mamba, ref_us):
    """The step's MX updates on the line's own states with the reference's rounding stream
    (LQ_ROUND_SR_PHILOX: Triton's tl.rand per element, generated in the kernel), timed as the
    line's counter-mode updates (one event pair around each step's run of back-to-back
    updates)."""
    from layer_quant_amd import _abi

    for _ in range(3):
        run_step(torch, args, [], mamba, round_mode=_abi.ROUND_SR_PHILOX)
    torch.cuda.synchronize()
    ev = Events(torch)
    for _ in range(args.steps):
        run_step(torch, args, [], mamba, ev, round_mode=_abi.ROUND_SR_PHILOX)
    torch.cuda.synchronize()
    us = ev.mean_us("mx_update")
    return {"what": (f"the step's {len(mamba)} MX{args.state_bits} updates with the reference's "
                     "own stochastic-rounding stream (Triton tl.rand, Philox4x32-10, per element "
                     "in the kernel; bit-exact with the reference's draws) instead of the "
                     "library's counter generator"),
            "counter_us": round(ref_us, 2), "philox_us": round(us, 2),
            "philox_over_counter_time": round(us / ref_us, 3)}


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
        print(json.dumps(sweep(torch, dev, args)), flush=True)
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
    # settle: untimed steps until the clocks have ramped up (in kernel traces of this workload
    # the MX update took ~50 us in the first steps and ~40 us from about the 25th on, while the
    # HBM-bound attention stayed flat)
    settle_steps = 0
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < args.settle_seconds:
        for _ in range(5):
            run_step(torch, args, attn, mamba)
            settle_steps += 1
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_settle
    log(f"settle: {settle_steps} steps in {settle_s:.3f} s")

    # timed region 1: whole steps, no per-kernel events
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(torch, args, attn, mamba)
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / args.steps
    log(f"step: {step_s * 1e6:.1f} us")

    # timed region 2: the same steps with HIP events around the kernel calls (see run_step)
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
                                            "mx_update": args.mamba_layers}[name],
                         "per_call_us": ev.spread_us(name)}
        log(f"{name}: {us:.1f} us/call, {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%})")
    dominant = max(kernels, key=lambda k: kernels[k]["us"] * kernels[k]["calls_per_step"])
    dk = kernels[dominant]
    workload = f"b{args.batch}_ctx{args.ctx}_g{args.group}_mx{args.state_bits}" + (
        "_compact" if args.state_layout == "compact" else "")
    roofline = {
        "kernel": {"attention": "lq_int4_decode_attention_pack (attn_fast_kernel with the "
                                "token's pack, + attn_merge_kernel when split)",
                   "mx_update": f"lq_mx_state_update (mx_update_rows_kernel MX{args.state_bits})",
                   }[dominant],
        "bound": "hbm",
        "achieved": dk["GB_s"],
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": dk["frac_of_peak"],
        "traffic": load_traffic(dominant, workload),
        "timing": (f"HIP events on the launch stream over the {args.steps} timed steps, "
                   + ("one pair around each call" if dominant != "mx_update" else
                      f"one pair around each step's {args.mamba_layers} back-to-back updates")
                   + f" ({dk['per_call_us']['calls']} calls; per-pair mean per call min / "
                   f"median / max {dk['per_call_us']['min']} / {dk['per_call_us']['median']} / "
                   f"{dk['per_call_us']['max']} us)"),
    }
    pair = None
    if args.layout_pair == "on" and args.state_layout == "reference" and mamba:
        log("compact-layout MX updates")
        pair = layout_pair(torch, args, dev, mamba, kernels["mx_update"]["us"])
        log(f"compact layout: {pair['compact_us']} us/call against {pair['reference_us']} us")
    rng = None
    if mamba and args.state_layout == "reference":
        log("MX updates with the reference's Philox stream")
        rng = rng_pair(torch, args, mamba, kernels["mx_update"]["us"])
        log(f"Philox rounding: {rng['philox_us']} us/call against {rng['counter_us']} us")
    cfg1_gpu = config1_gpu(torch, dev)
    log("the reference's published shape")
    ref_shape = reference_shape(torch, dev)
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
        "settle": {"steps": settle_steps, "seconds": round(settle_s, 3),
                   "note": "untimed steps after the warmup until the GPU clocks settle"},
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "dtype_note": ("fp32 accumulation and softmax; the attention's MFMA operands are exact "
                       "bf16 values (queries, nibbles as offset integers) except the P V weights "
                       "p * vscale, which enter as a bf16 hi + lo pair (about 16 significant "
                       "bits); the MX update is fp32 VALU"),
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
        "layout_pair": pair,
        "rng_pair": rng,
        "reference_shape": ref_shape,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
