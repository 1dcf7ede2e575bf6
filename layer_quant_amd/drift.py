"""Long-chain state drift of the MX4 / MX8 recurrent state against an unquantized state.

    python -m layer_quant_amd.drift [--batch 8] [--steps 2048] [--checkpoints 128,256,512,1024,2048]
                                    [--rounding counter|philox|uniform]

Runs one Mamba2 layer of Nemotron-H-8B's shape (128 heads x 64 x 128, 8 groups) for --steps
decode steps from one initial state h0 ~ N(0, 0.5), along four paths that see identical inputs:

    mx4   the MX4 state, fused update with stochastic writeback (counter generator, seed 1234,
          the reference's step offsets; with --rounding philox the reference's own tl.rand
          stream at those offsets; or, with --rounding uniform, a seeded uniform tensor drawn
          per step and applied by the reference's floor(q) + (u < frac) rule)
                                                                 -- lq_mx_state_update
    mx8   the same with the MX8 format                             -- lq_mx_state_update
    bf16  a bf16 state, fp32 update, rounded back each step        -- lq_selective_state_update
    fp32  an fp32 state                                            -- lq_selective_state_update

Per step the inputs are drawn fresh from one seeded generator: x ~ N(0, 1) bf16 [B,H,P],
dt = softplus(N(0, 1)) one value per (batch, head) (passed with dt_softplus=False, no dt_bias),
B, C ~ N(0, 1) bf16 [B,G,N]; A = -exp(U(0, 2)) and D ~ N(0, 1) per head are fixed. At each
checkpoint the MX states are decoded and compared with the bf16 state (the baseline the
experiment names) and with the fp32 state, as relative Frobenius norms
||deq(h_mx) - h_ref|| / ||h_ref||, together with the relative error of that step's output y.
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import torch

from . import _abi

HEADS, DIM, DSTATE, GROUPS = 128, 64, 128, 8


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double()
    b = b.double()
    return float((a - b).norm() / b.norm())


def run(batch: int = 8, steps: int = 2048, checkpoints=(128, 256, 512, 1024, 2048),
        seed: int = 0, device: str = "cuda:0", record: dict | None = None,
        rounding: str = "counter", record_states: int = 0,
        record_steps: int | None = None) -> dict:
    """The experiment; `record`, when given, receives CPU copies of h0, A, D and the inputs of
    the first `record_steps` steps (all steps by default) for replaying a short chain elsewhere,
    and with record_states = k the MX4 and MX8 states (q, shared_exp, micro_exp) after each of
    the first k steps in record["states"]. `rounding` is "counter" (the library's generator),
    "philox" (the reference's tl.rand stream) or "uniform" (a uniform tensor per step from the
    seeded generator)."""
    if rounding not in ("counter", "philox", "uniform"):
        raise ValueError(f"rounding must be 'counter', 'philox' or 'uniform', got {rounding!r}")
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    shape = (batch, HEADS, DIM, DSTATE)
    h0 = torch.randn(shape, device=dev, generator=gen) * 0.5
    A = (-torch.exp(torch.rand(HEADS, device=dev, generator=gen) * 2))[:, None, None].expand(
        HEADS, DIM, DSTATE)
    D = torch.randn(HEADS, device=dev, generator=gen)[:, None].expand(HEADS, DIM)
    if record is not None:
        record.update(h0=h0.cpu(), A=A.cpu(), D=D.cpu(), steps=[], states=[])

    mx = {}
    for bits in (4, 8):
        st = (torch.empty(shape, dtype=torch.int8, device=dev),
              torch.empty(*shape[:3], DSTATE // 16, dtype=torch.uint8, device=dev),
              torch.empty(*shape[:3], DSTATE // 2, dtype=torch.uint8, device=dev))
        _abi.mx_encode(h0, *st, bits, _abi.ROUND_NEAREST_EVEN)
        mx[bits] = st
    plain = {"bf16": h0.to(torch.bfloat16), "fp32": h0.clone()}
    outs = {k: torch.empty(batch, HEADS, DIM, device=dev, dtype=torch.bfloat16)
            for k in ("mx4", "mx8", "bf16", "fp32")}
    deq = torch.empty(shape, device=dev)
    total = batch * HEADS * DIM * DSTATE
    marks = sorted(set(int(c) for c in checkpoints if 0 < int(c) <= steps))
    rows = []
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for step in range(1, steps + 1):
        x = torch.randn(batch, HEADS, DIM, device=dev, generator=gen).to(torch.bfloat16)
        dt = torch.nn.functional.softplus(
            torch.randn(batch, HEADS, device=dev, generator=gen))[:, :, None].expand(
                batch, HEADS, DIM)
        Bm = torch.randn(batch, GROUPS, DSTATE, device=dev, generator=gen).to(torch.bfloat16)
        Cm = torch.randn(batch, GROUPS, DSTATE, device=dev, generator=gen).to(torch.bfloat16)
        uni = (torch.rand(shape, device=dev, generator=gen) if rounding == "uniform" else None)
        if record is not None and (record_steps is None or step <= record_steps):
            record["steps"].append(dict(x=x.cpu(), dt=dt.cpu(), B=Bm.cpu(), C=Cm.cpu(),
                                        uniform=None if uni is None else uni.cpu()))
        for bits in (4, 8):
            if uni is None:
                mode = _abi.ROUND_SR_PHILOX if rounding == "philox" else _abi.ROUND_SR_COUNTER
                _abi.mx_state_update(*mx[bits], x, dt, None, A, Bm, Cm, D, None,
                                     outs[f"mx{bits}"], bits, False, mode,
                                     seed=1234, rng_offset=(step - 1) * total)
            else:
                _abi.mx_state_update(*mx[bits], x, dt, None, A, Bm, Cm, D, None,
                                     outs[f"mx{bits}"], bits, False, _abi.ROUND_SR_UNIFORM,
                                     uniform=uni)
        for name, state in plain.items():
            _abi.selective_state_update(state, x, dt, None, A, Bm, Cm, D, None, outs[name], False)
        if record is not None and step <= record_states:
            record["states"].append({bits: tuple(t.cpu() for t in mx[bits]) for bits in (4, 8)})
        if step in marks:
            row = {"step": step}
            for bits in (4, 8):
                _abi.mx_decode(*mx[bits], deq)
                row[f"mx{bits}_state_vs_bf16"] = _rel(deq, plain["bf16"])
                row[f"mx{bits}_state_vs_fp32"] = _rel(deq, plain["fp32"])
                row[f"mx{bits}_y_vs_bf16"] = _rel(outs[f"mx{bits}"], outs["bf16"])
            row["bf16_state_vs_fp32"] = _rel(plain["bf16"], plain["fp32"])
            row["state_rms_fp32"] = float(plain["fp32"].double().pow(2).mean().sqrt())
            rows.append(row)
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    return {
        "experiment": "MX state drift against an unquantized state (Nemotron-H-8B Mamba2 layer)",
        "batch": batch,
        "steps": steps,
        "shape": list(shape),
        "groups": GROUPS,
        "rounding": {
            "counter": "stochastic writeback, counter generator, seed 1234",
            "philox": "stochastic writeback, the reference's tl.rand (Philox4x32-10) stream, seed 1234",
            "uniform": "stochastic writeback, seeded uniform tensor per step (floor(q) + (u < frac))",
        }[rounding],
        "inputs": "fresh per step: x ~ N(0,1) bf16, dt = softplus(N(0,1)) per (batch, head), "
                  "B, C ~ N(0,1) bf16; fixed A = -exp(U(0,2)), D ~ N(0,1) per head; "
                  f"h0 ~ N(0, 0.5); generator seed {seed}",
        "drift": rows,
        "seconds": round(elapsed, 3),
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--checkpoints", default="128,256,512,1024,2048")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--rounding", choices=["counter", "philox", "uniform"], default="counter")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("the drift experiment needs a GPU", file=sys.stderr)
        return 1
    res = run(args.batch, args.steps, [int(c) for c in args.checkpoints.split(",") if c],
              args.seed, rounding=args.rounding)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
