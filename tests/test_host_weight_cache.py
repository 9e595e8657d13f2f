"""Host logic of the expert-weight cache (no GPU): a forward that fails after
its weight quantisation was deferred to the routing sort must not leave a
cache that later calls take as built."""

import types

import pytest
import torch

import nanopysche_amd.flow_moe as fmm
from nanopysche_amd import _lib
from nanopysche_amd.recipes import FP8RecipeConfig, FP8RecipeType


@pytest.mark.parametrize("recipe,kind", [("flow_moe", _lib.QUANT_POW2), ("blockwise", _lib.QUANT_BLOCK)])
def test_failed_forward_invalidates_deferred_weights(monkeypatch, recipe, kind):
    builds = []
    real_build = fmm.ExpertWeights._build

    def counting_build(self, *a, **k):
        builds.append(self.kind)
        return real_build(self, *a, **k)

    def failing_route(*a, **k):
        raise RuntimeError("planted routing failure")

    monkeypatch.setattr(fmm.ExpertWeights, "_build", counting_build)
    monkeypatch.setattr(fmm, "route_tokens", failing_route)
    E, H, D, T, K = 4, 256, 256, 64, 2
    cfg = fmm.FP8FlowMoEConfig(True, FP8RecipeConfig(True, FP8RecipeType(recipe)))
    blk = fmm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=0)
    w1, w2, w3 = (torch.randn(E * H, D).bfloat16() for _ in range(3))
    blk.set_weights(w1, w2, w3)
    blk._record = True
    ctx = types.SimpleNamespace(needs_input_grad=(True,) * 7)
    x = torch.randn(T, D).bfloat16()
    w = torch.rand(T, K)
    idx = torch.randint(0, E, (T, K))
    for attempt in range(2):
        with pytest.raises(RuntimeError, match="planted"):
            blk._forward(ctx, x, w, w1, w2, w3, idx)
        assert blk._cache[kind].key is None
        # every attempt rebuilt the operands instead of trusting the cache
        assert builds == [kind] * (attempt + 1)


def test_refresh_keeps_cache_for_unchanged_weights():
    E, H, D = 2, 256, 256
    w1, w2, w3 = (torch.randn(E * H, D).bfloat16() for _ in range(3))
    ew = fmm.ExpertWeights(_lib.QUANT_POW2)
    jobs = []
    ew.refresh(w1, w2, w3, E, True, defer=jobs)
    assert len(jobs) == 1 and ew.key is not None
    ew.refresh(w1, w2, w3, E, True, defer=jobs)
    assert len(jobs) == 1                      # cached: nothing new to launch
    w2.add_(1.0)                               # an in-place update bumps the version
    ew.refresh(w1, w2, w3, E, True, defer=jobs)
    assert len(jobs) == 2
    ew.invalidate()
    ew.refresh(w1, w2, w3, E, True, defer=jobs)
    assert len(jobs) == 3
