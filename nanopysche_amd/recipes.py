"""FP8 recipe configuration, mirroring the names nanopsyche imports from
``fp8_flow_moe.recipes`` (reference ``fp8/recipes.py:3-7``) and the values its
CLI accepts (reference ``cli.py:49-54``: none, blockwise, mxfp8, flow_moe).

Recipe -> number formats used by the expert block:

============  ===================================  ==============================
recipe        activations / gradients              expert weights
============  ===================================  ==============================
none          bf16                                 bf16
blockwise     e4m3, 1x128 fp32 scales; 128x1       e4m3, 128x128 fp32 scales
              column blocks quantised from the
              bf16 source for the weight grads
flow_moe      e4m3, 1x128 power-of-two scales;     e4m3, 128x128 power-of-two
              column blocks by the scaling-aware   scales
              transpose of the row blocks (no
              second rounding from bf16)
mxfp8         e4m3, 1x32 e8m0 scales (OCP MX);     e4m3, 1x32 e8m0 scales along
              32x1 column blocks                   the contraction dimension
============  ===================================  ==============================
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum

from . import _lib


class FP8RecipeType(str, Enum):
    NONE = "none"
    BLOCKWISE = "blockwise"
    MXFP8 = "mxfp8"
    FLOW_MOE = "flow_moe"


class BlockScalingGranularity(str, Enum):
    """Shape of one scaling block, as rows x columns of the quantised tensor."""

    ROW_1x128 = "1x128"        # activations, scales [rows, cols/128]
    COL_128x1 = "128x1"        # transposed activations, scales [rows/128, cols] of the source
    BLOCK_128x128 = "128x128"  # weights, scales [rows/128, cols/128]
    MX_1x32 = "1x32"           # MXFP8, e8m0 scales [rows, cols/32]
    MX_32x1 = "32x1"           # transposed MXFP8, e8m0 scales [rows/32, cols] of the source


@dataclass
class FP8RecipeConfig:
    enabled: bool = False
    recipe_type: FP8RecipeType = FP8RecipeType.NONE

    def __post_init__(self):
        self.recipe_type = FP8RecipeType(self.recipe_type)

    @property
    def uses_fp8(self) -> bool:
        return self.enabled and self.recipe_type != FP8RecipeType.NONE

    @property
    def act_kind(self) -> int:
        """Quantisation kind of activations and activation gradients."""
        return {
            FP8RecipeType.NONE: _lib.QUANT_BF16,
            FP8RecipeType.BLOCKWISE: _lib.QUANT_BLOCK,
            FP8RecipeType.FLOW_MOE: _lib.QUANT_POW2,
            FP8RecipeType.MXFP8: _lib.QUANT_MX,
        }[self.recipe_type if self.enabled else FP8RecipeType.NONE]

    @property
    def gemm_kind(self) -> int:
        return {
            _lib.QUANT_BF16: _lib.GEMM_BF16,
            _lib.QUANT_BLOCK: _lib.GEMM_FP8_F32,
            _lib.QUANT_POW2: _lib.GEMM_FP8_POW2,
            _lib.QUANT_MX: _lib.GEMM_FP8_MX,
        }[self.act_kind]
