"""``fp8_flow_moe.flow_moe`` (reference fp8/flow_moe.py:3-15, fp8/__init__.py:24)."""

from nanopysche_amd.flow_moe import (  # noqa: F401
    FP8_BLOCK_SIZE,
    FP8FlowMoECompute,
    FP8FlowMoEConfig,
    FP8SharedExpertCompute,
    dequantize_from_fp8,
    fp8_grouped_gemm,
    fused_permute_pad,
    fused_silu_multiply_quantize,
    fused_swiglu_quantize,
    fused_unpermute_unpad,
    quantize_to_fp8,
    scaling_aware_transpose,
)
