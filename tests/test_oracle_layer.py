"""Pins the layer oracles (oracle/layer.py): the BF16 per-expert loop against
a dense per-token formulation of ExpertMLP (model/moe.py:1181-1183) with its
own autograd graph, and the FP8-flow oracle's structure against the loop."""

import numpy as np
import pytest
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


def _exact_quantisers(monkeypatch):
    """Every FP8 quantisation point of the flow oracle made exact: row and
    weight operands pass through, column operands are the plain transpose."""
    monkeypatch.setattr(olayer, "_q_rows", lambda a, recipe: np.asarray(a, np.float32))
    monkeypatch.setattr(olayer, "_q_cols", lambda a, recipe: np.ascontiguousarray(np.asarray(a, np.float32).T))
    monkeypatch.setattr(olayer, "_q_weight", lambda w, recipe: np.asarray(w, np.float32))


def test_flow_reference_dataflow_with_exact_quantisers(monkeypatch):
    """With every quantiser exact, the FP8 flow's dataflow (operand placement,
    transposed column operands, the router weight on dY, the gradient
    formulas, slot-order combine) must give the reference loop's results up
    to the bf16 rounding of its stored GEMM outputs (the BF16 bar, 1e-2).  A
    transposed operand, a dropped router weight or a wrong gradient is O(1)."""
    E = 4
    x, w, idx, w1, w2, w3, go = _case(seed=5)
    ref_out, ref_grads = olayer.moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
    _exact_quantisers(monkeypatch)
    for recipe in ("blockwise", "flow_moe", "mxfp8"):
        out, grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=recipe)
        assert olayer.max_rel_err(out, ref_out.numpy()) < 1e-2, recipe
        for k in ref_grads:
            assert olayer.max_rel_err(grads[k], ref_grads[k].numpy()) < 1e-2, (recipe, k)


def _rowwise_err(got, ref, axis):
    """Largest relative error of one row (axis=1) or column (axis=0): ||d|| / ||ref||."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float((np.linalg.norm(got - ref, axis=axis) / np.linalg.norm(ref, axis=axis)).max())


def _scaled_case(per_token, seed):
    """C3-like small case whose activations span many octaves, either per
    token (rows of x and of the upstream gradient, 2^-8 .. 2^4) or per feature
    (columns of x and of the upstream gradient, 2^-16 .. 2^4, beyond e4m3's
    range inside one block, and hidden units of w1, w3, 2^-8 .. 2^2)."""
    T, D, H, E, K = 512, 256, 256, 4, 2
    rng = np.random.default_rng(seed)
    x, w, idx, w1, w2, w3, go = _case(T=T, D=D, H=H, E=E, K=K, seed=seed)
    if per_token:
        sx = torch.from_numpy(np.exp2(rng.uniform(-8, 4, (T, 1)))).float()
        sg = torch.from_numpy(np.exp2(rng.uniform(-8, 4, (T, 1)))).float()
    else:
        sx = torch.from_numpy(np.exp2(rng.uniform(-16, 4, (1, D)))).float()
        sg = torch.from_numpy(np.exp2(rng.uniform(-16, 4, (1, D)))).float()
        sh = torch.from_numpy(np.exp2(rng.uniform(-8, 2, (E * H, 1)))).float()
        w1 = (w1.float() * sh).bfloat16()
        w3 = (w3.float() * sh).bfloat16()
    x = (x.float() * sx).bfloat16()
    go = (go.float() * sg).bfloat16()
    return x, w, idx, w1, w2, w3, go, E, H, D


def _plant(monkeypatch, wrong):
    """Plant a quantisation-axis mistake in the oracle (CPU only)."""
    real_rows, real_cols = olayer._q_rows, olayer._q_cols
    if wrong == "rows_across_tokens":     # row operands blocked along the token axis
        monkeypatch.setattr(olayer, "_q_rows", lambda a, recipe: np.ascontiguousarray(real_cols(a, recipe).T))
    else:                                 # column operands blocked along the feature axis
        monkeypatch.setattr(olayer, "_q_cols", lambda a, recipe: np.ascontiguousarray(real_rows(a, recipe).T))


def test_flow_reference_row_operands_blocked_within_a_token(monkeypatch):
    """Tokens whose magnitudes span 12 octaves: row-quantised operands (x and
    dY for the forward and dgrad GEMMs) take their blocks along the
    contraction within one token, so every token's output and input gradient
    keeps e4m3 accuracy relative to its own size (measured 0.09-0.12 of its
    norm, bound 0.25); blocks across tokens flush the small tokens (planting
    that mistake in the oracle gives ~1.0)."""
    x, w, idx, w1, w2, w3, go, E, H, D = _scaled_case(True, seed=21)
    ref_out, ref_grads = olayer.moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
    for recipe in ("blockwise", "flow_moe", "mxfp8"):
        out, grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=recipe)
        assert _rowwise_err(out, ref_out.numpy(), 1) < 0.25, recipe
        assert _rowwise_err(grads["x"], ref_grads["x"].numpy(), 1) < 0.25, recipe
    with monkeypatch.context() as m:
        _plant(m, "rows_across_tokens")
        for recipe in ("blockwise", "flow_moe", "mxfp8"):
            out, _ = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=recipe)
            assert _rowwise_err(out, ref_out.numpy(), 1) > 0.5, recipe


def test_flow_reference_column_operands_blocked_along_tokens(monkeypatch):
    """Features (columns of x and dO, 20 octaves) and hidden units spanning
    many octaves: the weight-gradient GEMMs contract over tokens, and the
    blockwise and MX recipes quantise their column operands (x, dY, h, dg|du)
    from the source in blocks of 128 (32) tokens within one feature, so every
    column of dW1 (a feature of x) and of dW2 (a feature of dY) and every row
    of dW2 (a hidden unit) keeps e4m3 accuracy relative to its own size
    (measured <= 0.21, bound 0.3); blocks along the features would not
    (planted mistake: 0.87-1.4).  The flow_moe recipe's column operands are
    the scaling-aware transpose of its row blocks, so they keep the row
    blocks' per-token scales and lose such features by design (~1.1)."""
    x, w, idx, w1, w2, w3, go, E, H, D = _scaled_case(False, seed=22)
    ref_out, ref_grads = olayer.moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
    r1, r2 = ref_grads["w1"].numpy(), ref_grads["w2"].numpy()
    live = np.repeat(np.bincount(idx.reshape(-1).numpy(), minlength=E) > 0, H)   # experts with tokens

    def errs(recipe):
        _, g = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=recipe)
        return (_rowwise_err(g["w1"], r1, 0), _rowwise_err(g["w2"], r2, 0),
                _rowwise_err(g["w2"][live], r2[live], 1))

    for recipe in ("blockwise", "mxfp8"):
        assert max(errs(recipe)) < 0.3, recipe
    assert errs("flow_moe")[0] > 0.5
    with monkeypatch.context() as m:
        _plant(m, "cols_across_features")
        for recipe in ("blockwise", "mxfp8"):
            assert min(errs(recipe)) > 0.6, recipe


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


def _sampled_case(T, D, H, E, K, seed, zero=()):
    x = randn_bf16((T, D), seed=seed)
    w, idx = zipf_routing(T, E, K, 1.1, seed=seed + 1, zero_experts=zero)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=seed + s, std=0.05) for s in (2, 3, 4))
    go = randn_bf16((T, D), seed=seed + 5, std=1e-2)
    return x, w, idx, w1, w2, w3, go


@pytest.mark.parametrize("recipe", [None, "blockwise", "flow_moe", "mxfp8"])
def test_sampled_oracle_matches_full_oracle(recipe):
    """The sampled restriction of the flow oracle (tokens' outputs and input /
    router-weight gradients, 128 x 128 weight-gradient blocks) against the
    full oracle's rows and blocks.  Only the BLAS summation order differs, so
    nearly every value is identical and none moves by more than a bf16 unit
    passed through one quantiser.  A wrong row map, block offset, expert
    range or operand axis would be O(1) on many values."""
    T, D, H, E, K = 400, 256, 384, 5, 2
    x, w, idx, w1, w2, w3, go = _sampled_case(T, D, H, E, K, seed=21, zero=(4,))
    out, grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=recipe)
    tokens = np.array([0, 3, 17, 111, 250, 399])
    blocks = [("w1", 0, 0, 0), ("w3", 1, 2, 1), ("w2", 2, 1, 1), ("w2", 3, 2, 0), ("w1", 4, 0, 1)]
    s_out, s_g = olayer.moe_flow_sampled(x, w, idx, w1, w2, w3, E, go, recipe, tokens, blocks)
    # bf16-rounded outputs: nearly all identical
    pairs = [(s_out, out[tokens]), (s_g["x"], grads["x"][tokens]), (s_g["weights"], grads["weights"][tokens])]
    for got, ref in pairs:
        got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
        assert got.shape == ref.shape
        assert olayer.max_rel_err(got, ref) < 2e-3
        assert np.mean(got == ref) > 0.9
    # fp32 weight-gradient sums: the same values up to the summation order
    for (name, e, bi, bj), blk in zip(blocks, s_g["blocks"]):
        full = grads[name].reshape(E, H, D)[e, bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
        assert olayer.max_rel_err(blk, full) < 2e-3, (name, e)
    # the expert without tokens has an all-zero block
    assert np.all(s_g["blocks"][-1] == 0)


def test_sampled_oracle_block_index_is_checked():
    """The block comparison tells neighbouring blocks apart: the block one
    hidden block off (an off-by-one in the slices) fails the bound that the
    right block meets."""
    T, D, H, E, K = 256, 256, 256, 4, 2
    x, w, idx, w1, w2, w3, go = _sampled_case(T, D, H, E, K, seed=31)
    _, grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe="flow_moe")
    blocks = [("w1", 1, 1, 0)]
    _, s_g = olayer.moe_flow_sampled(x, w, idx, w1, w2, w3, E, go, "flow_moe", [0], [("w1", 1, 0, 0)])
    full = grads["w1"].reshape(E, H, D)[1, 128:256, 0:128]
    assert olayer.max_rel_err(s_g["blocks"][0], full) > 0.5
    _, s_g = olayer.moe_flow_sampled(x, w, idx, w1, w2, w3, E, go, "flow_moe", [0], blocks)
    assert olayer.max_rel_err(s_g["blocks"][0], full) < 2e-3
