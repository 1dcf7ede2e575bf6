"""Seeded random sweep of MX state updates through the C ABI against the CPU oracle.

Each case draws the format (MX8 / MX4), the rounding mode (nearest-even, half-up, supplied
uniforms, counter; 24 further cases all take the reference's own Philox stream), d_state (64, 128, 256 on the row kernel's layout; 96 on the general kernel),
head_dim (ragged against the row kernel's 64-row workgroups), batch, groups and heads per group,
the dtypes of x and of the output, whether dt is constant along head_dim (the model's layout,
taken by the row kernel) or not (general kernel), whether A varies along head_dim, whether
dt_bias, D and z are present, softplus, the seed and the counter offset. The update follows
hybrid_quant/mamba_state_8b_kernel.py:97-222 (MX8) and :289-544 (MX4); y within the stated
tolerance, the writeback equal to the oracle's except at encoder decision boundaries
(tests/helpers.py: assert_mx_writeback)."""
import random

import pytest
import torch

from helpers import assert_close_rel, assert_mx_writeback, to_device, update_term_magnitudes
from layer_quant_amd import _abi
from oracle import mx_state as omx

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
Y_RTOL = {"f32": 2e-3, "f16": 3e-3, "bf16": 8e-3}  # the output's own rounding on top of 2e-3


def _draw_cases(n, seed, mode=None):
    rng = random.Random(seed)
    cases = []
    for i in range(n):
        c = dict(
            fb=rng.choice([8, 4]),
            mode=rng.choice([0, 1, 2, 3]) if mode is None else mode,
            n=rng.choice([64, 128, 256, 128, 96]),
            p=rng.choice([16, 40, 64, 100]),
            bsz=rng.randint(1, 3),
            ng=rng.choice([1, 2, 4]),
            ratio=rng.choice([1, 2, 4]),
            xdt=rng.choice(["bf16", "f16", "f32"]),
            odt=rng.choice(["f32", "bf16", "f16"]),
            head_dt=rng.random() < 0.7,
            a_rows=rng.random() < 0.2,
            dtb=rng.random() < 0.7,
            has_d=rng.random() < 0.7,
            has_z=rng.random() < 0.3,
            softplus=rng.random() < 0.7,
            seed=rng.randint(0, 2**31),
            off=16 * rng.randint(0, 10**6) + rng.choice([0, 0, 0, 2]),  # +2: general kernel
        )
        cases.append((i, c))
    return cases


CASES = _draw_cases(96, 1202)
# the reference's own stream (LQ_ROUND_SR_PHILOX), numbered after the cases above
CASES += [(96 + i, c) for i, c in _draw_cases(24, 1303, mode=4)]


@pytest.mark.parametrize("i,c", CASES, ids=[f"case{i}" for i, _ in CASES])
def test_mx_update_random(gpu, diag, i, c):
    # the row kernel's layout: dt and A constant along head_dim, d_state 64/128/256, and in
    # counter mode an offset that is a multiple of 16; the library must then take that kernel
    rows = (c["head_dt"] and not c["a_rows"] and c["n"] != 96
            and not (c["mode"] == 3 and c["off"] % 16 != 0))
    if rows:
        diag.set("LQ_MX_REQUIRE_ROWS")
    print(f"[case {i}] {'rows' if rows else 'general'} {c}", flush=True)
    g = torch.Generator().manual_seed(5000 + i)
    bsz, nh, p_, n, ng = c["bsz"], c["ng"] * c["ratio"], c["p"], c["n"], c["ng"]
    shape = (bsz, nh, p_, n)
    h0 = torch.randn(*shape, generator=g) * 0.5 * torch.exp(torch.randn(*shape[:-1], 1, generator=g))
    q, e, m = omx.mx_encode(h0.numpy(), c["fb"], 0)
    xdt = DTYPES[c["xdt"]]
    dt_shape = (bsz, nh, 1) if c["head_dt"] else (bsz, nh, p_)
    dt = torch.nn.functional.softplus(torch.randn(*dt_shape, generator=g)).to(xdt).expand(bsz, nh, p_)
    if c["a_rows"]:
        A = -torch.exp(torch.rand(nh, p_, 1, generator=g) * 2).expand(nh, p_, n)
    else:
        A = (-torch.exp(torch.rand(nh, generator=g) * 2))[:, None, None].expand(nh, p_, n)
    t = dict(
        x=torch.randn(bsz, nh, p_, generator=g).to(xdt),
        dt=dt,
        A=A,
        B=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
        C=torch.randn(bsz, ng, n, generator=g).to(torch.bfloat16),
        D=torch.randn(nh, generator=g)[:, None].expand(nh, p_) if c["has_d"] else None,
        dt_bias=((torch.randn(nh, generator=g) * 0.1)[:, None].expand(nh, p_)
                 if c["dtb"] else None),
        z=torch.randn(bsz, nh, p_, generator=g).to(xdt) if c["has_z"] else None,
    )
    uni = torch.rand(*shape, generator=g) if c["mode"] == 2 else None
    st = [torch.from_numpy(a).to(gpu) for a in (q, e, m)]
    out = torch.empty(bsz, nh, p_, dtype=DTYPES[c["odt"]], device=gpu)
    dev = {k: to_device(v, gpu) for k, v in t.items()}
    _abi.mx_state_update(*st, dev["x"], dev["dt"], dev["dt_bias"], dev["A"], dev["B"], dev["C"],
                         dev["D"], dev["z"], out, c["fb"], c["softplus"], c["mode"],
                         uniform=None if uni is None else uni.to(gpu), seed=c["seed"],
                         rng_offset=c["off"])
    torch.cuda.synchronize()
    rq, re_, rm, ry, rh = omx.mx_update(q, e, m, t["x"], t["dt"], t["A"], t["B"], t["C"],
                                        D=t["D"], z=t["z"], dt_bias=t["dt_bias"],
                                        dt_softplus=c["softplus"], format_bits=c["fb"],
                                        round_mode=c["mode"], uniform=uni, seed=c["seed"],
                                        rng_offset=c["off"])
    assert_close_rel(out.float().cpu(), ry, rtol=Y_RTOL[c["odt"]], what=f"y case {i}")
    mag = update_term_magnitudes(omx.mx_decode(q, e, m), t["x"], t["dt"], t["A"], t["B"],
                                 t["C"], dt_bias=t["dt_bias"], dt_softplus=c["softplus"])
    assert_mx_writeback([a.cpu().numpy() for a in st], (rq, re_, rm), rh, mag, c["fb"],
                        c["mode"], uniform=uni, seed=c["seed"], rng_offset=c["off"],
                        what=f"state case {i}")
