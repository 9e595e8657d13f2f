"""GPU parity of routing: top-k gating, counting sort, permute, unpermute,
router-weight gradient (indices, counts, rows and bytes bit-exact)."""

import numpy as np
import pytest
import torch

import nanopysche_amd as fm
from oracle import fp8 as ofp8
from oracle import routing as orouting
from tests.helpers import randn_bf16, zipf_routing

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("E,K,gating", [(4, 1, "softmax"), (8, 2, "softmax"), (256, 8, "sigmoid"),
                                        (64, 6, "softmax"), (3, 3, "sigmoid"), (1, 1, "softmax"),
                                        (2, 1, "sigmoid"), (12, 3, "softmax"), (16, 4, "sigmoid")])
def test_topk_gating(dev, E, K, gating):
    """T = 4093 tokens: the waves of the E <= 16 kernel (64 / EP tokens at a
    time) end on a partial group."""
    T = 4093
    g = torch.Generator().manual_seed(E * 10 + K)
    logits = torch.randn(T, E, generator=g)
    w, idx, part = fm.topk_gating(logits.to(dev), K, gating, return_prob_partial=True)
    fn = orouting.softmax_topk if gating == "softmax" else orouting.sigmoid_topk
    rw, ridx = fn(logits.numpy(), K)
    assert np.array_equal(_np(idx), ridx)
    assert np.allclose(_np(w), rw, rtol=2e-6, atol=1e-7)
    if gating == "softmax" and K == 1:
        assert np.all(_np(w) == 1.0)  # model/moe.py:253-254 with one selected logit
    plan = fm.route_tokens(idx, E)
    loss = fm.load_balancing_loss(part, plan.counts, T)
    ref = orouting.load_balancing_loss(logits.numpy(), ridx, E)
    assert abs(loss.item() - ref) <= 1e-5 * max(1.0, abs(ref))


def test_topk_ties_go_to_lower_index(dev):
    logits = torch.zeros(64, 16)
    logits[:, 3] = 1.0
    logits[:, 9] = 1.0
    logits[:, 12] = 40.0   # sigmoid saturates to exactly 1.0 ...
    logits[:, 13] = 50.0   # ... for both of these
    _, idx = fm.topk_gating(logits.to(dev), 4, "softmax")
    assert _np(idx).tolist() == [[13, 12, 3, 9]] * 64
    _, idx = fm.topk_gating(logits.to(dev), 4, "sigmoid")
    _, ridx = orouting.sigmoid_topk(logits.numpy(), 4)
    assert np.array_equal(_np(idx), ridx)


CASES = [
    # T, E, K, skew, zero experts
    (4096, 4, 1, 0.0, ()),
    (8192, 8, 2, 0.0, ()),
    (16384, 8, 2, 1.1, ()),
    (8192, 256, 8, 1.2, (0, 5, 17)),
    # the scan folded into the scatter: at most 64 blocks of 1024 assignments
    # and 256 experts (this case at both limits), then just past each
    (8192, 256, 8, 1.2, (0, 5, 255)),
    (8193, 8, 8, 0.0, ()),
    (2000, 300, 4, 1.1, (7,)),
    (1000, 32, 8, 1.2, (1, 2)),
    (7, 8, 2, 0.0, ()),
    (1, 1, 1, 0.0, ()),
]


@pytest.mark.parametrize("T,E,K,s,zeros", CASES)
def test_route_sort_bitexact(dev, T, E, K, s, zeros):
    _, idx = zipf_routing(T, E, K, s, seed=T + E, zero_experts=zeros)
    for dtype in (torch.int64, torch.int32):
        plan = fm.route_tokens(idx.to(dtype).to(dev), E)
        ref = orouting.sort_assignments(idx.numpy(), E)
        assert np.array_equal(_np(plan.counts), ref["counts"])
        assert np.array_equal(_np(plan.offsets), ref["offsets"])
        assert np.array_equal(_np(plan.row_of), ref["row_of"])
        used = int(ref["offsets"][-1])
        aor = _np(plan.assign_of_row)
        assert np.array_equal(aor[:used], ref["assign_of_row"])
        assert np.all(aor[used:] == -1)
        te = _np(plan.tile_expert)
        want = np.full(te.shape, -1)
        for e in range(E):
            want[ref["offsets"][e] // 128: ref["offsets"][e + 1] // 128] = e
        assert np.array_equal(te, want)


def test_route_sort_out_of_range_indices_are_ignored(dev):
    idx = torch.tensor([[0, 5], [1, -1], [2, 1]])
    plan = fm.route_tokens(idx.to(dev), 3)
    assert _np(plan.counts).tolist() == [1, 2, 1]
    assert _np(plan.row_of).tolist() == [0, -1, 128, -1, 256, 129]


def test_route_sort_empty(dev):
    plan = fm.route_tokens(torch.zeros(0, 2, dtype=torch.int64, device=dev), 4)
    assert _np(plan.counts).tolist() == [0, 0, 0, 0]
    assert _np(plan.offsets).tolist() == [0] * 5


@pytest.mark.parametrize("kmajor", [False, True])
@pytest.mark.parametrize("kind", ["bf16", "block", "pow2", "mx"])
def test_permute_bitexact(dev, kind, kmajor):
    T, E, K, D = 3000, 8, 2, 512
    x = randn_bf16((T, D), seed=21)
    w, idx = zipf_routing(T, E, K, 1.1, seed=2, zero_experts=(3,))
    gran = {"bf16": None, "block": fm.BlockScalingGranularity.ROW_1x128,
            "pow2": fm.BlockScalingGranularity.ROW_1x128, "mx": fm.BlockScalingGranularity.MX_1x32}[kind]
    for weights in (None, w):
        pt = fm.fused_permute_pad(x.to(dev), idx.to(dev), E, granularity=gran, pow2_scale=kind == "pow2",
                                  return_transpose=True, kmajor_scales=kmajor,
                                  weights=None if weights is None else weights.to(dev))
        if kmajor and kind != "bf16":
            assert pt.rows.scale.stride(0) == 1  # block-major buffer viewed as [rows, blocks]
        ref = orouting.sort_assignments(idx.numpy(), E)
        xs = x.float().numpy()
        Xp = orouting.permute_pad(xs, ref["assign_of_row"], K)
        if weights is not None:
            wr = np.zeros(Xp.shape[0], np.float32)
            valid = ref["assign_of_row"] >= 0
            wr[valid] = weights.numpy().reshape(-1)[ref["assign_of_row"][valid]]
            Xp = (wr[:, None] * Xp).astype(np.float32)
        used = Xp.shape[0]
        if kind == "bf16":
            assert np.array_equal(pt.rows[:used].float().cpu().numpy(), ofp8.bf16_round(Xp))
            assert np.array_equal(pt.rows_t[:, :used].float().cpu().numpy(), ofp8.bf16_round(Xp).T)
            continue
        if kind == "mx":
            rq, rs = ofp8.quant_mx_1x32(Xp)
            cq, cs = ofp8.quant_mx_32x1(Xp)
        else:
            rq, rs = ofp8.quant_1x128(Xp, pow2=kind == "pow2")
            cq, cs = (ofp8.scaling_aware_transpose(rq, rs) if kind == "pow2" else ofp8.quant_128x1(Xp))
        assert np.array_equal(_np(pt.rows.data)[:used], rq)
        assert np.array_equal(_np(pt.rows.scale)[:used], rs)
        assert np.array_equal(_np(pt.rows_t.data)[:, :used], cq)
        nb = used // (32 if kind == "mx" else 128)
        assert np.array_equal(_np(pt.rows_t.scale)[:nb], cs)


@pytest.mark.parametrize("K,drop", [(1, False), (2, False), (3, True), (4, False), (8, True)])
def test_unpermute_bitexact(dev, K, drop):
    """K = 1, 2, 4, 8 take the kernels that load every slot's row before the
    sums, K = 3 the one-slot-at-a-time loop; `drop`: a third of the slots route
    outside the local experts (no row), as at configs[4]."""
    T, E, D = 2000, 16, 256
    w, idx = zipf_routing(T, E, K, 1.2, seed=7, zero_experts=(2,))
    if drop:
        g = torch.Generator().manual_seed(12)
        idx = torch.where(torch.rand(idx.shape, generator=g) < 0.33, idx + E + 3, idx)
    plan = fm.route_tokens(idx.to(dev), E)
    y = randn_bf16((plan.rows_max, D), seed=8)
    ref = orouting.sort_assignments(idx.numpy(), E, drop_out_of_range=drop)
    for weights in (w, None):
        out = fm.fused_unpermute_unpad(y.to(dev), plan, None if weights is None else weights.to(dev),
                                       out_dtype=torch.float32)
        r = orouting.unpermute_unpad(y.float().numpy(), ref["row_of"],
                                     None if weights is None else weights.numpy(), T, K)
        assert np.array_equal(out.cpu().numpy(), r)
        outb = fm.fused_unpermute_unpad(y.to(dev), plan, None if weights is None else weights.to(dev))
        assert np.array_equal(outb.float().cpu().numpy(), ofp8.bf16_round(r))


def test_router_weight_grad(dev):
    from nanopysche_amd import _lib

    T, E, K, D = 1024, 8, 2, 512
    w, idx = zipf_routing(T, E, K, 0.0, seed=9)
    plan = fm.route_tokens(idx.to(dev), E)
    y = randn_bf16((plan.rows_max, D), seed=10).to(dev)
    dout = randn_bf16((T, D), seed=11).to(dev)
    dw = torch.empty(T * K, dtype=torch.float32, device=dev)
    _lib.call("fm_router_weight_grad", _lib.ptr(dout), D, _lib.ptr(y), D, _lib.ptr(plan.row_of), T, K,
              D, _lib.ptr(dw), _lib.stream_of(dout))
    rows = y.float()[plan.row_of.long()].reshape(T, K, D)
    ref = torch.einsum("td,tkd->tk", dout.float().double(), rows.double()).reshape(-1)
    assert torch.allclose(dw.double(), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("E,K,gating", [(4, 1, "softmax"), (8, 2, "sigmoid"), (16, 4, "softmax"),
                                        (64, 6, "sigmoid"), (256, 8, "softmax")])
def test_topk_replay_and_l2(dev, E, K, gating):
    """R3 replay (model/moe.py:187-247; softmax of the training logits over the
    replayed experts, whatever the gating) and the l2 weight normalisation
    (:167-170) against the oracle; T = 4093 ends the E <= 16 kernel's waves on
    a partial group."""
    T = 4093
    g = torch.Generator().manual_seed(E * 7 + K)
    logits = torch.randn(T, E, generator=g) * 2
    mask = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    w, idx = fm.topk_gating(logits.to(dev), K, gating, replay_indices=mask.to(dev))
    rw, ridx = orouting.replay_gating(logits.numpy(), mask.numpy(), K)
    assert np.array_equal(_np(idx), ridx)
    assert np.allclose(_np(w), rw, rtol=2e-6, atol=1e-7)
    fn = orouting.softmax_topk if gating == "softmax" else orouting.sigmoid_topk
    for replay in (None, mask.to(dev)):
        w2, idx2 = fm.topk_gating(logits.to(dev), K, gating, replay_indices=replay, normalize="l2")
        base = (rw, ridx) if replay is not None else fn(logits.numpy(), K)
        assert np.array_equal(_np(idx2), base[1])
        assert np.allclose(_np(w2), orouting.l2_normalize(base[0]), rtol=3e-6, atol=1e-7)


@pytest.mark.parametrize("E", [8, 64])
def test_topk_nan_and_minus_inf(dev, E):
    """NaN ranks first (torch.topk's order), -inf logits (or a -inf score bias)
    never make an expert win twice: indices equal the oracle's and every row
    holds K distinct experts."""
    K = 4
    T = 256
    g = torch.Generator().manual_seed(E)
    logits = torch.randn(T, E, generator=g)
    logits[::3, : E - 2] = -float("inf")      # only 2 finite experts: K-2 slots among -inf, lower index first
    logits[1::7, 5] = float("nan")
    for gating in ("softmax", "sigmoid"):
        _, idx = fm.topk_gating(logits.to(dev), K, gating)
        scores = logits.numpy() if gating == "softmax" else 1 / (1 + np.exp(-logits.numpy().astype(np.float64)))
        ridx = orouting.topk_lower_index(scores.astype(np.float32), K)
        assert np.array_equal(_np(idx), ridx), gating
        assert all(len(set(r)) == K for r in _np(idx).tolist())
        assert (_np(idx)[1::7, 0] == 5).all()   # NaN first


def test_aux_loss_with_z_loss(dev):
    T, E, K = 3000, 16, 2
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(T, E, generator=g) * 3
    w, idx, part, zpart = fm.topk_gating(logits.to(dev), K, "softmax", True, return_z_partial=True)
    counts = fm.expert_counts(idx, E)
    z_mult = 0.01
    loss = fm.load_balancing_loss(part, counts, T, zpart, z_mult)
    ref = orouting.load_balancing_loss(logits.numpy(), _np(idx), E) + z_mult * orouting.z_loss(logits.numpy())
    assert abs(loss.item() - ref) <= 1e-5 * abs(ref)


def test_router_weight_grad_sparse_slots(dev):
    """A local expert share (8 of 64 experts: most slots have no row) over
    5.6 M slots, more than one batch of 64 candidates per wave (the grid has
    65,536 waves): every slot with a row gets its dot product (float64
    reference on the device), every other slot exactly 0."""
    from nanopysche_amd import _lib

    T, E_local, E_global, K, D = 700_000, 8, 64, 8, 64
    g = torch.Generator(device=dev).manual_seed(12)
    idx = torch.randint(0, E_global, (T, K), generator=g, device=dev)
    plan = fm.route_tokens(idx, E_local)
    y = torch.randn(plan.rows_max, D, generator=g, device=dev).to(torch.bfloat16)
    dout = torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16)
    dw = torch.full((T * K,), float("nan"), dtype=torch.float32, device=dev)
    _lib.call("fm_router_weight_grad", _lib.ptr(dout), D, _lib.ptr(y), D, _lib.ptr(plan.row_of), T, K,
              D, _lib.ptr(dw), _lib.stream_of(dout))
    ro = plan.row_of.long()
    has = ro >= 0
    assert 0 < int(has.sum()) < T * K // 4
    tok = torch.arange(T * K, device=dev) // K
    ref = (dout.double()[tok[has]] * y.double()[ro[has]]).sum(dim=1)
    assert torch.allclose(dw[has].double(), ref, rtol=1e-4, atol=1e-4)
    assert torch.all(dw[~has] == 0)
