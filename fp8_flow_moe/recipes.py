"""``fp8_flow_moe.recipes`` (reference fp8/recipes.py:3-7)."""

from nanopysche_amd.recipes import (  # noqa: F401
    BlockScalingGranularity,
    FP8RecipeConfig,
    FP8RecipeType,
)
