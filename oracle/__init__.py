"""CPU oracle for the two decode-path kernels -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithms on the CPU (PyTorch fp32/fp64 for the float
math, numpy for bits and bytes). It is the checker that the HIP kernels are compared against:

    int4_kv   INT4 group quantization, nibble packing, cache pack, decode attention, mask
    mx_state  MX8/MX4 block encoders (nearest-even, half-up, stochastic), decoder, the fused
              selective-state update, and the bf16-state baseline update used for drift
    rng       the counter-based uniform generator of LQ_ROUND_SR_COUNTER

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only as
the checker or the timed CPU baseline. The product path (layer_quant_amd, hybrid_quant) never
imports it and fails loudly when the HIP library is missing.

Pinning status of every function is recorded in each module's docstring.
"""
