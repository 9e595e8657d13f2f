"""The drop-in module names (no GPU): every name nanopsyche imports from the
absent ``fp8_flow_moe`` package resolves from this repository's
``fp8_flow_moe`` modules, to the MI355X implementation.

The lists are the import statements of the reference shim, written out here
(the reference is not imported): ``fp8/__init__.py:8-24``,
``fp8/flow_moe.py:3-15``, ``fp8/recipes.py:3-7``; the config and object names
are also those ``model/moe.py:1314-1332`` constructs."""

import importlib

import pytest

# from fp8_flow_moe import (...)                     fp8/__init__.py:8-22
PACKAGE_NAMES = (
    "FP8FlowMoEConfig", "FP8FlowMoECompute", "FP8RecipeConfig", "FP8RecipeType", "BlockScalingGranularity",
    "quantize_to_fp8", "dequantize_from_fp8", "scaling_aware_transpose", "fused_swiglu_quantize",
    "fused_silu_multiply_quantize", "fused_permute_pad", "fused_unpermute_unpad", "fp8_grouped_gemm",
)
# from fp8_flow_moe.flow_moe import (...)            fp8/__init__.py:24, fp8/flow_moe.py:3-15
FLOW_MOE_NAMES = (
    "FP8_BLOCK_SIZE", "FP8FlowMoECompute", "FP8FlowMoEConfig", "dequantize_from_fp8", "fp8_grouped_gemm",
    "fused_permute_pad", "fused_silu_multiply_quantize", "fused_swiglu_quantize", "fused_unpermute_unpad",
    "quantize_to_fp8", "scaling_aware_transpose",
)
# from fp8_flow_moe.recipes import (...)             fp8/recipes.py:3-7
RECIPES_NAMES = ("BlockScalingGranularity", "FP8RecipeConfig", "FP8RecipeType")


@pytest.mark.parametrize("module,names", [
    ("fp8_flow_moe", PACKAGE_NAMES),
    ("fp8_flow_moe.flow_moe", FLOW_MOE_NAMES),
    ("fp8_flow_moe.recipes", RECIPES_NAMES),
])
def test_reference_imports_resolve(module, names):
    import nanopysche_amd

    mod = importlib.import_module(module)
    for n in names:
        obj = getattr(mod, n)
        assert obj is getattr(nanopysche_amd, n), (module, n)


def test_all_fourteen_names_and_values():
    names = set(PACKAGE_NAMES) | set(FLOW_MOE_NAMES) | set(RECIPES_NAMES)
    assert len(names) == 14
    fm = importlib.import_module("fp8_flow_moe")
    assert set(PACKAGE_NAMES) <= set(fm.__all__)
    assert importlib.import_module("fp8_flow_moe.flow_moe").FP8_BLOCK_SIZE == 128
    # the recipe values nanopsyche passes (cli.py:49-54, model/moe.py:1317-1324)
    rt = fm.FP8RecipeType
    assert {rt(v).value for v in ("none", "blockwise", "mxfp8", "flow_moe")} == {"none", "blockwise", "mxfp8",
                                                                                "flow_moe"}
    cfg = fm.FP8FlowMoEConfig(enabled=True, fp8_recipe=fm.FP8RecipeConfig(enabled=True,
                                                                         recipe_type=rt("flow_moe")))
    assert cfg.enabled and cfg.fp8_recipe.recipe_type == rt.FLOW_MOE
