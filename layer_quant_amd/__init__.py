"""MI355X-native (gfx950) kernels for Layer_Quant's two quantized decode paths.

    layer_quant_amd.int4_8b_attention     INT4 KV cache + fused q_len=1 decode attention
    layer_quant_amd.mamba_state_8b_kernel MX8/MX4 Mamba2 state + fused selective-state update

Both call hand-written HIP kernels through the C ABI of include/layer_quant.h
(layer_quant_amd/lib/liblayer_quant.so, built by `python -m layer_quant_amd.build`).
The top-level package `hybrid_quant` aliases these modules under the reference's import paths.
"""
