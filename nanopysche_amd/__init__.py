"""MI355X-native fp8_flow_moe operator path (hand-written HIP for gfx950).

Exports the names nanopsyche imports from ``fp8_flow_moe`` (reference
``fp8/__init__.py:8-24``) plus the routing kernels.  All compute runs in
libfm_hip.so; see ``nanopysche_amd.build`` to compile it.
"""

from .recipes import BlockScalingGranularity, FP8RecipeConfig, FP8RecipeType
from .flow_moe import (
    FP8_BLOCK_SIZE,
    ExpertWeights,
    FP8FlowMoECompute,
    FP8FlowMoEConfig,
    FP8SharedExpertCompute,
    FP8Tensor,
    PermutedTokens,
    dequantize_from_fp8,
    fp8_grouped_gemm,
    fused_permute_pad,
    fused_silu_multiply_quantize,
    fused_swiglu_quantize,
    fused_unpermute_unpad,
    quantize_to_fp8,
    scaling_aware_transpose,
)
from .graph import GraphedStep
from .moe_layer import FP8FlowMoELayer
from .norm import NormOutput, RMSNorm, rmsnorm, rmsnorm_backward, rmsnorm_quantize
from .routing import (ExpertLoadTracker, RoutingPlan, expert_counts, load_balancing_loss, route, route_tokens,
                      router_logits, topk_gating)

__all__ = [
    "FP8FlowMoEConfig",
    "FP8FlowMoECompute",
    "FP8SharedExpertCompute",
    "FP8RecipeConfig",
    "FP8RecipeType",
    "BlockScalingGranularity",
    "quantize_to_fp8",
    "dequantize_from_fp8",
    "scaling_aware_transpose",
    "fused_swiglu_quantize",
    "fused_silu_multiply_quantize",
    "fused_permute_pad",
    "fused_unpermute_unpad",
    "fp8_grouped_gemm",
    "FP8_BLOCK_SIZE",
    "FP8Tensor",
    "PermutedTokens",
    "ExpertWeights",
    "RoutingPlan",
    "route_tokens",
    "topk_gating",
    "load_balancing_loss",
    "route",
    "router_logits",
    "expert_counts",
    "ExpertLoadTracker",
    "FP8FlowMoELayer",
    "GraphedStep",
    "RMSNorm",
    "rmsnorm",
    "rmsnorm_quantize",
    "rmsnorm_backward",
    "NormOutput",
]
