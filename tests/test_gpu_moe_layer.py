"""The MoE layer (router -> expert block -> shared expert, MoEBase.forward of
reference model/moe.py:1338-1393 at expert-parallel size 1) on the GPU:

* BF16 experts against the reference's own op sequence in float64 on the
  CPU -- gate nn.Linear on x.float(), top-k softmax gating, load-balancing
  loss (:133-184, :249-281), the per-expert SwiGLU loop (:1542-1596) -- with
  gradients of out * R + c * aux flowing back into x, the gate weight and
  bias and w1, w2, w3, within the BF16 bar (1e-2);
* FP8 experts: the fused layer against the unfused composition of the same
  kernels (route() then FP8FlowMoECompute, autograd summing the two input
  gradients), and the shared expert added out of place."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import nanopysche_amd as fm
from oracle.layer import max_rel_err
from tests.helpers import randn_bf16

pytestmark = pytest.mark.gpu


def _params(T, D, H, E, seed):
    x = randn_bf16((T, D), seed=seed)
    gw = randn_bf16((E, D), seed=seed + 1, std=0.05)
    gb = randn_bf16((E,), seed=seed + 2, std=0.1)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=seed + s, std=0.02) for s in (3, 4, 5))
    g = torch.Generator().manual_seed(seed + 6)
    R = torch.randn(T, D, generator=g) * 1e-2
    return x, gw, gb, w1, w2, w3, R


def _reference(x, gw, gb, w1, w2, w3, R, E, K, c_aux, replay=None):
    leaves = [t.double().requires_grad_(True) for t in (x, gw, gb, w1, w2, w3)]
    xd, gwd, gbd, a, b, c = leaves
    logits = F.linear(xd, gwd, gbd)                       # gate(x.float()), :151
    if replay is None:
        vals, idx = logits.topk(K, dim=-1)                # _softmax_gating, :249-255
        wts = F.softmax(vals, dim=-1)
    else:                                                 # _routing_replay_gating, :195-247
        mask = torch.zeros_like(logits).scatter_(1, replay, 1.0)
        masked = F.softmax(logits, dim=-1) * mask
        wts, idx = (masked / masked.sum(dim=-1, keepdim=True).clamp(min=1e-8)).topk(K, dim=-1)
    T = xd.shape[0]
    f = F.one_hot(idx, E).sum(dim=1).double().sum(dim=0) / T
    aux = E * (f * F.softmax(logits, dim=-1).mean(dim=0)).sum()   # :267-281
    H = w1.shape[0] // E
    out = torch.zeros_like(xd)
    for e in range(E):                                    # :1565-1594
        tok = (idx == e).any(dim=-1).nonzero(as_tuple=True)[0]
        if tok.numel() == 0:
            continue
        pw = (wts[tok] * (idx[tok] == e).double()).sum(-1)
        sl = slice(e * H, (e + 1) * H)
        h = F.silu(xd[tok] @ a[sl].T) * (xd[tok] @ c[sl].T)
        out = out.index_add(0, tok, pw[:, None] * (h @ b[sl]))
    ((out * R.double()).sum() + c_aux * aux).backward()
    return out.detach(), aux.detach(), [t.grad for t in leaves]


def _layer(recipe, D, H, E, K, shared=None, **kw):
    cfg = fm.FP8FlowMoEConfig(enabled=recipe != "none",
                              fp8_recipe=fm.FP8RecipeConfig(recipe != "none", fm.FP8RecipeType(recipe)))
    return fm.FP8FlowMoELayer(cfg, D, H, E, K, fp8_gemm_threshold=0, shared_hidden_size=shared, **kw)


def test_bf16_layer_matches_reference_ops(dev):
    T, D, H, E, K = 600, 256, 256, 8, 2
    x, gw, gb, w1, w2, w3, R = _params(T, D, H, E, seed=5)
    c_aux = 0.5
    ref_out, ref_aux, ref_grads = _reference(x, gw, gb, w1, w2, w3, R, E, K, c_aux)
    leaves = [t.to(dev).requires_grad_(True) for t in (x, gw, gb, w1, w2, w3)]
    layer = _layer("none", D, H, E, K)
    layer.set_weights(*leaves[1:])
    out, aux = layer(leaves[0])
    ((out.float() * R.to(dev)).sum() + c_aux * aux).backward()
    torch.cuda.synchronize()
    assert max_rel_err(out.detach().float().cpu().numpy(), ref_out.numpy()) < 1e-2
    assert abs(float(aux.detach()) - float(ref_aux)) < 1e-5 * float(ref_aux)
    for name, got, ref in zip(("x", "gate_w", "gate_b", "w1", "w2", "w3"), leaves, ref_grads):
        assert max_rel_err(got.grad.float().cpu().numpy(), ref.numpy()) < 1e-2, name


@pytest.mark.timeout(600)
@pytest.mark.parametrize("replay", [False, True])
def test_bf16_layer_at_c3_shape_takes_the_fused_router(dev, monkeypatch, replay):
    """configs[2]'s layer shape (T=8192, D=2048, E=8, top-2 softmax with the
    load-balancing loss, H=1408) with BF16 experts, so the fused router
    forward (one pass over x), the gating backward that forms the
    router-weight dots itself and the router's dx share folded into the
    unpermute all run -- checked against float64 autograd of the reference
    op sequence (model/moe.py:133-184, :195-247 replay, :249-281,
    :1542-1596) within the BF16 bar, with and without R3 replay.  The test
    records which library entry points ran."""
    from nanopysche_amd import _lib

    T, D, H, E, K = 8192, 2048, 1408, 8, 2
    x, gw, gb, w1, w2, w3, R = _params(T, D, H, E, seed=23)
    c_aux = 0.5
    t = torch.arange(T)
    rep = torch.stack([(t * 5) % E, (t * 5 + 3) % E], 1) if replay else None
    ref_out, ref_aux, ref_grads = _reference(x, gw, gb, w1, w2, w3, R, E, K, c_aux, replay=rep)
    assert _lib.load().fm_router_forward_fused(E, D, _lib.DTYPE_BF16) == 1
    called = []
    real_call = _lib.call

    def spy(name, *args):
        called.append(name)
        return real_call(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    leaves = [t_.to(dev).requires_grad_(True) for t_ in (x, gw, gb, w1, w2, w3)]
    layer = _layer("none", D, H, E, K)
    layer.set_weights(*leaves[1:])
    out, aux = layer(leaves[0], replay_indices=None if rep is None else rep.to(dev))
    fwd = list(called)
    called.clear()
    ((out.float() * R.to(dev)).sum() + c_aux * aux).backward()
    torch.cuda.synchronize()
    bwd = list(called)
    assert "fm_router_forward" in fwd and fwd.count("fm_unpermute") == 1, fwd     # fused router; combine
    for name in ("fm_router_logits", "fm_topk_gating", "fm_expert_counts", "fm_aux_loss"):
        assert name not in fwd, (name, fwd)
    for name in ("fm_gating_grad_dot", "fm_unpermute_router", "fm_router_backward"):
        assert bwd.count(name) == 1, (name, bwd)
    for name in ("fm_gating_grad", "fm_router_weight_grad", "fm_unpermute"):
        assert name not in bwd, (name, bwd)
    assert max_rel_err(out.detach().float().cpu().numpy(), ref_out.numpy()) < 1e-2
    assert abs(float(aux.detach()) - float(ref_aux)) < 1e-5 * float(ref_aux)
    for name, got, ref in zip(("x", "gate_w", "gate_b", "w1", "w2", "w3"), leaves, ref_grads):
        err = max_rel_err(got.grad.float().cpu().numpy(), ref.numpy())
        assert err < 1e-2, (name, err)


@pytest.mark.parametrize("recipe", ["flow_moe", "mxfp8"])
@pytest.mark.parametrize("shared", [None, 256])
def test_fp8_layer_matches_unfused_composition(dev, recipe, shared):
    T, D, H, E, K = 1024, 512, 256, 8, 2
    x, gw, gb, w1, w2, w3, R = _params(T, D, H, E, seed=11)
    sw = None if shared is None else [randn_bf16((shared, D), seed=20 + s, std=0.02) for s in range(3)]
    Rd = R.to(dev)

    def leaves():
        return [t.to(dev).requires_grad_(True) for t in (x, gw, gb, w1, w2, w3)]

    # fused layer
    a = leaves()
    sa = None if sw is None else [t.to(dev).requires_grad_(True) for t in sw]
    layer = _layer(recipe, D, H, E, K, shared=shared)
    layer.set_weights(*a[1:], shared=sa)
    out_a, aux_a = layer(a[0])
    ((out_a.float() * Rd).sum() + 0.3 * aux_a).backward()
    # unfused: route() + expert block (+ shared expert), autograd sums the input gradients
    b = leaves()
    sb = None if sw is None else [t.to(dev).requires_grad_(True) for t in sw]
    wts, idx, aux_b = fm.route(b[0], b[1], b[2], top_k=K, gating="softmax")
    cfg = fm.FP8FlowMoEConfig(True, fm.FP8RecipeConfig(True, fm.FP8RecipeType(recipe)))
    blk = fm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=0)
    blk.set_weights(*b[3:])
    out_b = blk(b[0], wts, idx, 0, E)
    if sw is not None:
        sh = fm.FP8SharedExpertCompute(cfg, D, shared, fp8_gemm_threshold=0)
        sh.set_weights(*sb)
        out_b = out_b + sh(b[0])
    ((out_b.float() * Rd).sum() + 0.3 * aux_b).backward()
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b) and torch.equal(aux_a, aux_b)
    for name, ga, gb_ in zip(("gate_w", "gate_b", "w1", "w2", "w3"), a[1:], b[1:]):
        assert torch.equal(ga.grad, gb_.grad), name
    # the input gradient: one rounding of (router share + expert share) against
    # two roundings and an add
    ea = a[0].grad.float().cpu().numpy()
    eb = b[0].grad.float().cpu().numpy()
    assert max_rel_err(ea, eb) < 1e-2 and np.abs(ea - eb).mean() < 2e-3 * np.abs(eb).mean()
    if sw is not None:
        for ga, gb_ in zip(sa, sb):
            assert torch.equal(ga.grad, gb_.grad)


def test_layer_replay_and_load_tracker(dev):
    """R3 replay through the layer gives the replayed experts; the tracker
    counts them."""
    T, D, H, E, K = 512, 256, 256, 8, 2
    x, gw, gb, w1, w2, w3, _ = _params(T, D, H, E, seed=17)
    t = torch.arange(T)
    rep = torch.stack([t % E, (t + E // 2) % E], 1).to(dev)
    layer = _layer("flow_moe", D, H, E, K)
    layer.set_weights(*(v.to(dev) for v in (gw, gb, w1, w2, w3)))
    tracker = fm.ExpertLoadTracker(E, dev)
    with torch.no_grad():
        out, aux = layer(x.to(dev), replay_indices=rep, load_tracker=tracker)
    assert torch.equal(tracker.tokens_per_expert.cpu(), torch.full((E,), T * K // E, dtype=torch.int64))
    assert int(tracker.total_tokens.item()) == T
    assert out.shape == (T, D) and torch.isfinite(out.float()).all()
