"""Algorithmic (unique) HBM bytes of one call of each kernel: every input read once, every output
written once, and the algorithmic flops of the MFMA-bound prefill. These are the figures behind
the GB/s, TFLOP/s and roofline fractions bench.py reports."""
from __future__ import annotations


def attention_bytes(batch: int, n_q_heads: int, n_kv_heads: int, head_dim: int, seq_len: int,
                    group_size: int, q_bytes: int = 2, out_bytes: int = 2,
                    mask: bool = False) -> int:
    """q_len=1 decode attention over the packed INT4 cache: K and V nibbles (head_dim/2 bytes
    per key each), their fp32 group scales, q and out (+ an fp32 mask row)."""
    kv = 2 * batch * n_kv_heads * seq_len * (head_dim // 2)
    scales = 2 * batch * n_kv_heads * seq_len * (head_dim // group_size) * 4
    qo = batch * n_q_heads * head_dim * (q_bytes + out_bytes)
    return kv + scales + qo + (batch * seq_len * 4 if mask else 0)


def pack_bytes(batch: int, n_kv_heads: int, n_tokens: int, head_dim: int, group_size: int,
               x_bytes: int = 2) -> int:
    """One INT4 pack call (K or V): read the new tokens, write their bytes and scales."""
    return batch * n_kv_heads * n_tokens * (head_dim * x_bytes + head_dim // 2
                                            + 4 * (head_dim // group_size))


def mx_state_bytes(elems: int, format_bits: int = 8, layout: str = "reference") -> int:
    """Bytes of an MX state of `elems` values: one exponent byte per 16 values, plus one byte per
    mantissa and one per pair (reference layout), or nibble mantissas for MX4 and one micro bit per
    pair (compact layout)."""
    if layout == "compact":
        return (elems // 2 if format_bits == 4 else elems) + elems // 16 + elems // 16
    return elems + elems // 16 + elems // 2


def mx_update_bytes(batch: int, nheads: int, dim: int, dstate: int, ngroups: int,
                    x_bytes: int = 2, out_bytes: int = 2, dt_bytes: int = 2,
                    format_bits: int = 8, layout: str = "reference") -> int:
    """One MX8/MX4 state update: the state read and written once (mx_state_bytes), x and y per
    row, B and C per group, dt per (batch, head), A, D and dt_bias per head."""
    elems = batch * nheads * dim * dstate
    state = 2 * mx_state_bytes(elems, format_bits, layout)
    io = batch * nheads * dim * (x_bytes + out_bytes)
    bc = 2 * batch * ngroups * dstate * 2
    scalars = batch * nheads * dt_bytes + 3 * nheads * 4
    return state + io + bc + scalars


def ssm_update_bytes(batch: int, nheads: int, dim: int, dstate: int, ngroups: int,
                     state_bytes: int = 2, x_bytes: int = 2, out_bytes: int = 2,
                     dt_bytes: int = 2) -> int:
    """One unquantized selective-state update: the state read and written once, plus the same
    per-row, per-group and per-head inputs as the MX update."""
    elems = batch * nheads * dim * dstate
    io = batch * nheads * dim * (x_bytes + out_bytes)
    bc = 2 * batch * ngroups * dstate * 2
    scalars = batch * nheads * dt_bytes + 3 * nheads * 4
    return 2 * elems * state_bytes + io + bc + scalars


def prefill_flops(batch: int, n_q_heads: int, q_len: int, head_dim: int) -> int:
    """Causal prefill attention: 2*D flops for q.k and 2*D for p*v per visible (query, key)
    pair, L (L + 1) / 2 pairs per (batch, head)."""
    return 4 * head_dim * batch * n_q_heads * (q_len * (q_len + 1) // 2)
