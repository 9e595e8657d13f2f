"""Expert-block parity at the BASELINE configurations' own shapes (the ones
bench.py times), against the CPU oracles:

* T=8192, D=2048, E=8, top-2, H=1408 (an 11-step K on the down
  GEMM), FP8 forced, flow_moe recipe -- stage-synchronised against
  ``oracle.layer.moe_flow_reference`` within 2e-2, and free-running (no shared
  intermediates) with a mean-error bound;
* T=4096, D=2048, 4 experts, top-1 softmax router (weights exactly
  1), H=5632, BF16 -- against the reference's per-expert loop
  (``model/moe.py:1542-1596``) within 1e-2, forward and every gradient;
* configs[4]'s workload at a D / H the CPU oracle carries: one GPU's
  32-expert share of sigmoid top-8 routing over 256 experts with a Zipf(1.2)
  score bias (``model/moe.py:153-162``, ``:257-265``), slots of other GPUs'
  experts passed as out-of-range indices (ignored, ``:1560-1565``), two local
  experts with no tokens, MXFP8.

Each full-shape case runs the oracle once on the host (tens of seconds)."""

import numpy as np
import pytest
import torch

import nanopysche_amd as fm
from oracle import layer as olayer
from oracle import routing as orouting
from tests.helpers import c3_inputs, expert_share_routing, randn_bf16

pytestmark = pytest.mark.gpu

FP8_TOL = 2e-2
BF16_TOL = 1e-2
GRADS = ("x", "weights", "w1", "w2", "w3")


def _block(dev, x, w, idx, w1, w2, w3, go, E, recipe, taps=None, expert_offset=0):
    H = w1.shape[0] // E
    D = x.shape[-1]
    cfg = fm.FP8FlowMoEConfig(enabled=True, fp8_recipe=fm.FP8RecipeConfig(True, fm.FP8RecipeType(recipe)))
    blk = fm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=0)
    blk.capture_intermediates = taps
    p = [t.to(dev).requires_grad_(True) for t in (w1, w2, w3)]
    blk.set_weights(*p)
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    out = blk(xd, wd, idx.to(dev), expert_offset, E)
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    got = {"out": out.detach().float().cpu().numpy()}
    for name, t in zip(GRADS, (xd, wd, *p)):
        got[name] = t.grad.float().cpu().numpy()
    if taps is not None:
        for k in list(taps):
            taps[k] = taps[k].float().cpu().numpy()
    return got


def _errors(got, ref_out, ref_grads):
    errs = {"out": olayer.max_rel_err(got["out"], ref_out)}
    for name in GRADS:
        r = ref_grads[name]
        errs[name] = olayer.max_rel_err(got[name], r.numpy() if torch.is_tensor(r) else r)
    return errs


def _mean_rel(got, ref):
    ref = np.asarray(ref.numpy() if torch.is_tensor(ref) else ref, dtype=np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).mean() / np.abs(ref).mean())


@pytest.mark.timeout(600)
def test_c3_full_shape_stage_synchronised(dev):
    x, w, idx, w1, w2, w3, go = c3_inputs()
    taps = {}
    got = _block(dev, x, w, idx, w1, w2, w3, go, 8, "flow_moe", taps=taps)
    ref_out, ref_grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, 8, go, recipe="flow_moe", taps=taps)
    errs = _errors(got, ref_out, ref_grads)
    assert max(errs.values()) <= FP8_TOL, errs


@pytest.mark.timeout(600)
def test_c3_full_shape_free_running(dev):
    """No shared intermediates: the device's FP8 MFMA sums differ from the
    host's fp32 sums by ~1e-5 relative, which flips a few downstream block
    scales, so the bound here is on the mean error (every tensor within 1% of
    its mean magnitude) with the max-rel bound of the path."""
    x, w, idx, w1, w2, w3, go = c3_inputs()
    got = _block(dev, x, w, idx, w1, w2, w3, go, 8, "flow_moe")
    ref_out, ref_grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, 8, go, recipe="flow_moe")
    errs = _errors(got, ref_out, ref_grads)
    means = {"out": _mean_rel(got["out"], ref_out)}
    means.update({k: _mean_rel(got[k], ref_grads[k]) for k in GRADS})
    assert max(means.values()) <= 1e-2, means
    assert max(errs.values()) <= FP8_TOL, errs


@pytest.mark.timeout(600)
def test_c1_full_shape_bf16_top1(dev):
    T, D, E, K, H = 4096, 2048, 4, 1, 5632
    x = randn_bf16((T, D), seed=0)
    gate_w = randn_bf16((E, D), seed=100, std=0.02)
    gate_b = np.full(E, -1.0, np.float32)   # gate bias init, model/moe.py:107-109
    logits = orouting.router_logits(x.float().numpy(), gate_w.float().numpy(), gate_b)
    w, idx = orouting.softmax_topk(logits, K)
    assert np.all(w == 1.0)                 # top-1 softmax over one logit (model/moe.py:253-254)
    w, idx = torch.from_numpy(w), torch.from_numpy(idx)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=s, std=0.02) for s in (1, 2, 3))
    go = randn_bf16((T, D), seed=4, std=1e-2)
    got = _block(dev, x, w, idx, w1, w2, w3, go, E, "none")
    ref_out, ref_grads = olayer.moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
    errs = _errors(got, ref_out.numpy(), ref_grads)
    assert max(errs.values()) <= BF16_TOL, errs


@pytest.mark.parametrize("local_start", [0, 64])
def test_c5_expert_share_mxfp8(dev, local_start):
    """32 local experts of 256 (rank 0, and rank 2 with expert_offset 64, so
    other ranks' slots arrive both above and below the local range)."""
    E_g, E, K, D, H = 256, 32, 8, 512, 256
    w, idx = expert_share_routing(8192, E_g, E, K, 1.2, seed=4, local_start=local_start, zero_local=(5, 17),
                                  min_local=4000)
    T = idx.shape[0]
    x = randn_bf16((T, D), seed=41)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=s, std=0.02) for s in (42, 43, 44))
    go = randn_bf16((T, D), seed=45, std=1e-2)
    taps = {}
    got = _block(dev, x, w, idx, w1, w2, w3, go, E, "mxfp8", taps=taps, expert_offset=local_start)
    idx_local = idx - local_start
    ref_out, ref_grads = olayer.moe_flow_reference(x, w, idx_local, w1, w2, w3, E, go, recipe="mxfp8", taps=taps)
    errs = _errors(got, ref_out, ref_grads)
    assert max(errs.values()) <= FP8_TOL, errs
    # other ranks' slots get exactly zero router-weight gradient; experts
    # without tokens get exactly zero weight gradients
    nonlocal_ = ((idx_local < 0) | (idx_local >= E)).numpy()
    assert nonlocal_.any() and np.all(got["weights"][nonlocal_] == 0)
    counts = np.bincount(idx_local.numpy()[~nonlocal_], minlength=E)
    assert counts[5] == 0 and counts[17] == 0
    for name in ("w1", "w2", "w3"):
        g = got[name].reshape(E, H, D)
        assert np.all(g[[5, 17]] == 0), name
