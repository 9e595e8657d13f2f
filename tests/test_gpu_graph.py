"""The MoE layer step captured as a HIP graph (nanopysche_amd.GraphedStep):
every replay, with eager steps and synchronisations between replays, gives
the eager step's outputs and gradients bit for bit (expert-weight
re-quantisation, routing, the expert block, the second stream's dW2 and the
router all inside the graph)."""

import pytest
import torch

import nanopysche_amd as fm
from nanopysche_amd.recipes import FP8RecipeConfig, FP8RecipeType

pytestmark = pytest.mark.gpu


def _cfg(recipe):
    return fm.FP8FlowMoEConfig(enabled=recipe != "none",
                               fp8_recipe=FP8RecipeConfig(recipe != "none", FP8RecipeType(recipe)))


def _check_replays(step, leaves, n_replays=3):
    """step() -> tuple of output tensors (forward + backward done).  Captures
    it, then alternates replays and eager steps, comparing each replay's
    outputs and leaf gradients with the eager step's."""
    def eager():
        for p in leaves:
            p.grad = None
        outs = step()
        snap = [o.detach().clone() for o in outs] + [p.grad.detach().clone() for p in leaves]
        torch.cuda.synchronize()
        return snap

    g = fm.GraphedStep(step, leaves, warmup=2)
    static = list(g.outputs) + list(g.grads)
    ref = None
    for r in range(n_replays):
        keep = list(g.grads)
        ref_r = eager()               # eager work between replays
        ref = ref_r if ref is None else ref
        for a, b in zip(ref_r, ref):
            assert torch.equal(a, b), "eager steps differ"
        for p, k in zip(leaves, keep):
            p.grad = k
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(static, ref)):
            assert torch.equal(a, b), f"replay {r}: tensor {i} differs from the eager step"


@pytest.mark.parametrize("T,D,H,E,K,recipe,extras", [
    (8192, 2048, 1408, 8, 2, "flow_moe", False),   # configs[2]'s layer step (the bench's)
    (1000, 512, 384, 8, 2, "mxfp8", True),         # + pre-norm and a shared expert
])
def test_layer_step_graph_replays_match_eager(dev, T, D, H, E, K, recipe, extras):
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(T, D, device=dev, generator=g).bfloat16().requires_grad_(True)
    gw = (torch.randn(E, D, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True)
    gb = (torch.randn(E, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True)
    ws = [(torch.randn(E * H, D, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True)
          for _ in range(3)]
    go = (torch.randn(T, D, device=dev, generator=g) * 1e-2).bfloat16()
    t = torch.arange(T, device=dev)
    idx = torch.stack([(t + k * (E // K)) % E for k in range(K)], 1)
    extra = []
    if extras:
        layer = fm.FP8FlowMoELayer(_cfg(recipe), D, H, E, K, gating="softmax", fp8_gemm_threshold=0,
                                   shared_hidden_size=256, pre_norm=True)
        sw = [(torch.randn(256, D, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True)
              for _ in range(3)]
        nw = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).requires_grad_(True)
        layer.set_weights(gw, gb, *ws, shared=tuple(sw), norm_weight=nw)
        extra = sw + [nw]
    else:
        layer = fm.FP8FlowMoELayer(_cfg(recipe), D, H, E, K, gating="softmax", fp8_gemm_threshold=0)
        layer.set_weights(gw, gb, *ws)
    one = torch.ones((), device=dev)

    def step():
        layer.block._cache.clear()    # weights re-quantised inside the step
        if layer.shared is not None:
            layer.shared.block._cache.clear()
        out, aux = layer(x, replay_indices=idx)
        torch.autograd.backward([out, aux], [go, one])
        return out, aux

    _check_replays(step, [gw, gb, *ws, x, *extra])


def test_shared_expert_graph_replays_match_eager(dev):
    T, D, H = 2048, 1024, 768
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(T, D, device=dev, generator=g).bfloat16().requires_grad_(True)
    ws = [(torch.randn(H, D, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True) for _ in range(3)]
    go = (torch.randn(T, D, device=dev, generator=g) * 1e-2).bfloat16()
    blk = fm.FP8SharedExpertCompute(_cfg("flow_moe"), D, H)
    blk.set_weights(*ws)

    def step():
        blk.block._cache.clear()
        out = blk(x)
        out.backward(go)
        return (out,)

    _check_replays(step, [*ws, x])


def test_forward_only_graph_replays_match_eager(dev):
    """configs[0]'s shape of step: BF16 layer forward under no_grad, the
    router's own top-1 (no replayed routing)."""
    T, D, H, E, K = 4096, 1024, 1024, 4, 1
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(T, D, device=dev, generator=g).bfloat16()
    gw = (torch.randn(E, D, device=dev, generator=g) * 0.02).bfloat16()
    gb = (torch.randn(E, device=dev, generator=g) * 0.02).bfloat16()
    ws = [(torch.randn(E * H, D, device=dev, generator=g) * 0.02).bfloat16() for _ in range(3)]
    layer = fm.FP8FlowMoELayer(_cfg("none"), D, H, E, K, gating="softmax")
    layer.set_weights(gw, gb, *ws)

    def step():
        with torch.no_grad():
            layer.block._cache.clear()
            out, aux = layer(x)
        return out, aux

    _check_replays(step, [])
