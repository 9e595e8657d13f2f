"""Pins the layer oracles (oracle/layer.py): the BF16 per-expert loop against
a dense per-token formulation of ExpertMLP (model/moe.py:1181-1183) with its
own autograd graph, and the FP8-flow oracle's structure against the loop."""

import numpy as np
import torch
import torch.nn.functional as F

from oracle import layer as olayer
from tests.helpers import randn_bf16, zipf_routing


def _case(T=96, D=128, H=128, E=4, K=2, seed=0):
    x = randn_bf16((T, D), seed=seed)
    w, idx = zipf_routing(T, E, K, 0.8, seed=seed + 1, zero_experts=(3,))
    w1, w2, w3 = (randn_bf16((E * H, D), seed=seed + s, std=0.05) for s in (2, 3, 4))
    go = randn_bf16((T, D), seed=seed + 5, std=1e-2)
    return x, w, idx, w1, w2, w3, go


def _dense(x, w, idx, w1, w2, w3, E):
    """out[t] = sum_k w[t,k] * (silu(x w1_e^T) * (x w3_e^T)) w2_e, token by token."""
    H = w1.shape[0] // E
    rows = []
    for t in range(x.shape[0]):
        acc = torch.zeros(x.shape[1], dtype=torch.float64)
        for k in range(idx.shape[1]):
            e = int(idx[t, k])
            sl = slice(e * H, (e + 1) * H)
            h = F.silu(x[t] @ w1[sl].T) * (x[t] @ w3[sl].T)
            acc = acc + w[t, k] * (h @ w2[sl])
        rows.append(acc)
    return torch.stack(rows)


def test_bf16_loop_matches_dense_formulation():
    E = 4
    x, w, idx, w1, w2, w3, go = _case()
    out, grads = olayer.moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
    leaves = [t.detach().double().requires_grad_(True) for t in (x, w, w1, w2, w3)]
    ref = _dense(leaves[0], leaves[1], idx, leaves[2], leaves[3], leaves[4], E)
    ref.backward(go.double())
    assert torch.allclose(out.double(), ref.detach(), rtol=1e-4, atol=1e-6)
    for name, leaf in zip(("x", "weights", "w1", "w2", "w3"), leaves):
        assert torch.allclose(grads[name].double(), leaf.grad, rtol=1e-3, atol=1e-6), name
    # the zero-token expert gets zero weight gradients
    H = w1.shape[0] // E
    assert torch.all(grads["w1"][3 * H:] == 0)


def test_flow_reference_bf16_matches_loop():
    E = 4
    x, w, idx, w1, w2, w3, go = _case(seed=3)
    ref_out, ref_grads = olayer.moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
    out, grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=None)
    assert olayer.max_rel_err(out, ref_out.numpy()) < 1e-2
    for k in ref_grads:
        assert olayer.max_rel_err(grads[k], ref_grads[k].numpy()) < 1e-2, k


def test_flow_reference_fp8_close_to_loop():
    """FP8 quantisation of every GEMM operand: within e4m3 accuracy of the exact
    layer.  A transposed operand or a wrong gradient formula would be O(1) off."""
    E = 4
    x, w, idx, w1, w2, w3, go = _case(seed=5)
    ref_out, ref_grads = olayer.moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
    for recipe in ("blockwise", "flow_moe", "mxfp8"):
        out, grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=recipe)
        assert olayer.max_rel_err(out, ref_out.numpy()) < 0.15, recipe
        for k in ref_grads:
            assert olayer.max_rel_err(grads[k], ref_grads[k].numpy()) < 0.15, (recipe, k)


def test_flow_reference_taps_replace_gemm_outputs():
    E = 4
    x, w, idx, w1, w2, w3, go = _case(seed=7)
    out, grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe="flow_moe")
    # feeding back exactly what the oracle computes is a no-op
    from oracle import routing as orouting

    rt = orouting.sort_assignments(idx.numpy(), E)
    Mp = int(rt["offsets"][-1])
    H = w1.shape[0] // E
    zeros = {"gate_up": np.zeros((Mp, 2 * H), np.float32)}
    out0, _ = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, None, recipe="flow_moe", taps=zeros)
    assert np.all(out0 == 0)  # zero gate|up -> zero hidden -> zero output


def test_max_rel_err_metric():
    assert olayer.max_rel_err(np.array([1.0, 2.0]), np.array([1.0, 2.0])) == 0.0
    assert abs(olayer.max_rel_err(np.array([1.0, 2.1]), np.array([1.0, 2.0])) - 0.05) < 1e-12
