"""GPU router gate (fm_router_logits, fm_gating_grad, fm_router_backward via
routing.route) against the oracle's logits and a float64 CPU autograd run of
the reference's own op sequence (model/moe.py:151-154, :249-281)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import nanopysche_amd as fm
from oracle import routing as orouting
from oracle.layer import max_rel_err

pytestmark = pytest.mark.gpu


def _inputs(T, D, E, seed, x_dtype, score_bias):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g).to(x_dtype)
    w = torch.randn(E, D, generator=g) * 0.05
    b = torch.randn(E, generator=g) * 0.1 - 1.0
    sb = torch.randn(E, generator=g) * 0.2 if score_bias else None
    return x, w, b, sb


@pytest.mark.parametrize("T,D,E", [(1000, 512, 4), (333, 2048, 8), (200, 256, 24), (77, 512, 256)])
def test_router_logits(dev, T, D, E):
    x, w, b, sb = _inputs(T, D, E, 1, torch.bfloat16, True)
    got = fm.router_logits(x.to(dev), w.to(dev), b.to(dev), sb.to(dev)).cpu().numpy()
    ref = orouting.router_logits(x.float().numpy(), w.numpy(), b.numpy(), sb.numpy())
    assert max_rel_err(got, ref) < 1e-5
    x32 = x.float()
    got32 = fm.router_logits(x32.to(dev), w.to(dev), b.to(dev)).cpu().numpy()
    assert max_rel_err(got32, orouting.router_logits(x32.numpy(), w.numpy(), b.numpy())) < 1e-5
    # a bf16 gate (E <= 8, D <= 2048 with bf16 x: the matrix-core path)
    wb, bb = w.bfloat16(), b.bfloat16()
    gotb = fm.router_logits(x.to(dev), wb.to(dev), bb.to(dev), sb.to(dev)).cpu().numpy()
    refb = orouting.router_logits(x.float().numpy(), wb.float().numpy(), bb.float().numpy(), sb.numpy())
    assert max_rel_err(gotb, refb) < 1e-5


def _reference(x, w, b, sb, K, gating, R, c_aux):
    """The reference's forward (model/moe.py:151-154, 249-281) and its autograd
    gradients, in float64 on the CPU."""
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    bd = b.double().requires_grad_(True)
    logits = F.linear(xd, wd, bd)
    if sb is not None:
        logits = logits + sb.double()
    E = logits.shape[-1]
    if gating == "softmax":
        vals, idx = logits.topk(K, dim=-1)
        wts = F.softmax(vals, dim=-1)
    else:
        s = torch.sigmoid(logits)
        vals, idx = s.topk(K, dim=-1)
        wts = vals / (vals.sum(dim=-1, keepdim=True) + 1e-8)
    T = logits.shape[0]
    f = F.one_hot(idx, E).sum(dim=1).double().sum(dim=0) / T
    P = F.softmax(logits, dim=-1).mean(dim=0)
    aux = E * (f * P).sum()
    ((wts * R.double()).sum() + c_aux * aux).backward()
    return wts.detach(), idx, aux.detach(), xd.grad, wd.grad, bd.grad


@pytest.mark.parametrize("T,D,E,K,gating,score_bias,x_dtype", [
    (512, 1024, 8, 2, "softmax", False, torch.bfloat16),
    (256, 512, 8, 1, "softmax", False, torch.float32),
    (300, 256, 64, 6, "sigmoid", True, torch.float32),
    (128, 512, 256, 8, "sigmoid", True, torch.bfloat16),
])
def test_route_forward_backward(dev, T, D, E, K, gating, score_bias, x_dtype):
    x, w, b, sb = _inputs(T, D, E, 7, x_dtype, score_bias)
    g = torch.Generator().manual_seed(8)
    R = torch.randn(T, K, generator=g)
    c_aux = 0.3
    rw, ridx, raux, rdx, rdw, rdb = _reference(x, w, b, sb, K, gating, R, c_aux)

    xg = x.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    bg = b.to(dev).requires_grad_(True)
    wts, idx, aux = fm.route(xg, wg, bg, top_k=K, gating=gating, score_bias=None if sb is None else sb.to(dev))
    ((wts * R.to(dev)).sum() + c_aux * aux).backward()
    torch.cuda.synchronize()
    assert torch.equal(idx.cpu(), ridx)
    assert max_rel_err(wts.detach().cpu().numpy(), rw.numpy()) < 1e-5
    assert abs(float(aux.detach()) - float(raux)) <= 1e-5 * abs(float(raux))
    dx_tol = 1e-2 if x_dtype == torch.bfloat16 else 1e-4
    assert xg.grad.dtype == x_dtype
    assert max_rel_err(xg.grad.float().cpu().numpy(), rdx.numpy()) < dx_tol
    assert max_rel_err(wg.grad.cpu().numpy(), rdw.numpy()) < 1e-4
    assert max_rel_err(bg.grad.cpu().numpy(), rdb.numpy()) < 1e-4


def test_expert_counts(dev):
    g = torch.Generator().manual_seed(9)
    idx = torch.randint(-2, 40, (5000, 3), generator=g)
    got = fm.expert_counts(idx.to(dev), 37).cpu().numpy()
    flat = idx.flatten().numpy()
    ref = np.bincount(flat[(flat >= 0) & (flat < 37)], minlength=37)
    assert np.array_equal(got, ref)


def _reference_ext(x, w, b, sb, K, gating, R, c_aux, replay=None, l2=False, z_mult=None):
    """MoERouter.forward's optional stages as torch ops in float64 (reference
    model/moe.py:151-184, :187-247): R3 replay, l2 normalisation, z-loss."""
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    bd = b.double().requires_grad_(True)
    logits = F.linear(xd, wd, bd)
    if sb is not None:
        logits = logits + sb.double()
    E = logits.shape[-1]
    if replay is not None:
        probs = F.softmax(logits, dim=-1)
        mask = torch.zeros_like(probs).scatter(1, replay, 1.0)
        masked = probs * mask
        wts, idx = (masked / masked.sum(dim=-1, keepdim=True).clamp(min=1e-8)).topk(K, dim=-1)
    elif gating == "softmax":
        vals, idx = logits.topk(K, dim=-1)
        wts = F.softmax(vals, dim=-1)
    else:
        vals, idx = torch.sigmoid(logits).topk(K, dim=-1)
        wts = vals / (vals.sum(dim=-1, keepdim=True) + 1e-8)
    if l2:
        wts = wts / (wts.norm(dim=-1, keepdim=True) + 1e-8)
    T = logits.shape[0]
    f = F.one_hot(idx, E).sum(dim=1).double().sum(dim=0) / T
    aux = E * (f * F.softmax(logits, dim=-1).mean(dim=0)).sum()
    if z_mult is not None:
        aux = aux + z_mult * torch.logsumexp(logits, dim=-1).square().mean()
    ((wts * R.double()).sum() + c_aux * aux).backward()
    return wts.detach(), idx, aux.detach(), xd.grad, wd.grad, bd.grad


@pytest.mark.parametrize("E,K,gating,replay,l2,z_mult", [
    (8, 2, "softmax", True, False, None),      # configs[2]'s balanced routing as an R3 replay
    (8, 2, "sigmoid", True, True, 0.001),
    (64, 6, "softmax", False, True, 0.01),
    (256, 8, "sigmoid", False, True, None),
    (16, 4, "sigmoid", False, False, 0.02),
])
def test_route_replay_l2_zloss(dev, E, K, gating, replay, l2, z_mult):
    T, D = 400, 512
    x, w, b, sb = _inputs(T, D, E, 11, torch.bfloat16, gating == "sigmoid")
    g = torch.Generator().manual_seed(12)
    R = torch.randn(T, K, generator=g)
    rep = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]) if replay else None
    c_aux = 0.3
    rw, ridx, raux, rdx, rdw, rdb = _reference_ext(x, w, b, sb, K, gating, R, c_aux, rep, l2, z_mult)
    xg = x.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    bg = b.to(dev).requires_grad_(True)
    wts, idx, aux = fm.route(xg, wg, bg, top_k=K, gating=gating, score_bias=None if sb is None else sb.to(dev),
                             replay_indices=None if rep is None else rep.to(dev),
                             normalize_expert_weights="l2" if l2 else None, z_loss_multiplier=z_mult)
    ((wts * R.to(dev)).sum() + c_aux * aux).backward()
    torch.cuda.synchronize()
    assert torch.equal(idx.cpu(), ridx)
    assert max_rel_err(wts.detach().cpu().numpy(), rw.numpy()) < 1e-5
    assert abs(float(aux.detach()) - float(raux)) <= 2e-5 * abs(float(raux))
    assert max_rel_err(xg.grad.float().cpu().numpy(), rdx.numpy()) < 1e-2
    assert max_rel_err(wg.grad.cpu().numpy(), rdw.numpy()) < 1e-4
    assert max_rel_err(bg.grad.cpu().numpy(), rdb.numpy()) < 1e-4


def test_score_bias_update_on_device(dev):
    """ExpertLoadTracker: counts of two forwards accumulate on the device
    (model/moe.py:284-292), post_batch applies the reference's update
    (:307-317) bit-exactly and clears the totals; a second post_batch with
    nothing accumulated leaves the bias alone."""
    T, D, E, K = 512, 256, 16, 2
    x, w, b, _ = _inputs(T, D, E, 13, torch.bfloat16, False)
    sb = (torch.randn(E, generator=torch.Generator().manual_seed(14)) * 0.1).to(dev)
    tracker = fm.ExpertLoadTracker(E, dev)
    idxs = []
    for i in range(2):
        _, idx, _ = fm.route(x.to(dev) * (1 + i), w.to(dev), b.to(dev), top_k=K, gating="sigmoid", score_bias=sb,
                             load_tracker=tracker)
        idxs.append(idx.cpu().numpy())
    allidx = np.concatenate(idxs)
    counts = np.bincount(allidx.reshape(-1), minlength=E)
    assert np.array_equal(tracker.tokens_per_expert.cpu().numpy(), counts)
    assert int(tracker.total_tokens.item()) == 2 * T
    ref = orouting.score_bias_update(sb.cpu().numpy(), counts, 2 * T, 0.01)
    tracker.post_batch(sb, 0.01)
    assert np.array_equal(sb.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert int(tracker.total_tokens.item()) == 0 and int(tracker.tokens_per_expert.abs().sum().item()) == 0
    tracker.post_batch(sb, 0.01)
    assert np.array_equal(sb.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def _separate(x, w, b, sb, K, gating, replay, normalize, z_mult):
    """The router forward as separate kernels: gate, gating, counts, loss."""
    T, E = x.shape[0], w.shape[0]
    logits = fm.router_logits(x, w, b, sb)
    wts, idx, part, zpart = fm.topk_gating(logits, K, gating, True, replay_indices=replay, normalize=normalize,
                                           return_z_partial=True)
    counts = fm.expert_counts(idx, E)
    aux = fm.load_balancing_loss(part, counts, T, zpart if z_mult else None, z_mult)
    return logits, wts, idx, counts, aux


@pytest.mark.parametrize("T,D,E,K,gating,replay,normalize,z_mult", [
    (8192, 2048, 8, 2, "softmax", False, None, 0.0),     # configs[2]'s router: the fused pass
    (1000, 512, 4, 2, "sigmoid", False, "l2", 1e-3),
    (333, 1536, 8, 8, "softmax", True, None, 1e-2),
    (77, 512, 1, 1, "softmax", False, None, 0.0),
    (500, 256, 8, 2, "softmax", False, None, 0.0),       # D not a multiple of 512: separate kernels
    (300, 512, 24, 4, "sigmoid", True, "l2", 1e-3),      # E > 8: separate kernels
])
@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16])
def test_fused_router_forward_matches_separate_kernels(dev, T, D, E, K, gating, replay, normalize, z_mult, w_dtype):
    """fm_router_forward (one pass over x for small gates, then the counts and
    the loss) against the same steps as separate kernels: logits, weights,
    indices and counts bit for bit, the loss within float32 rounding of its
    per-wave partial sums (grouped differently); the load tracker's totals."""
    from nanopysche_amd.routing import router_forward

    x, w, b, sb = _inputs(T, D, E, 7, torch.bfloat16, True)
    x, w, b, sb = x.to(dev), w.to(w_dtype).to(dev), b.to(w_dtype).to(dev), sb.to(dev)
    rep = None
    if replay:
        g = torch.Generator().manual_seed(8)
        rep = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(dev)
    tracker = fm.ExpertLoadTracker(E, dev)
    wf, idxf, auxf, st = router_forward(x, w, b, sb, K, gating, rep, normalize, z_mult, tracker)
    logits, wts, idx, counts, aux = _separate(x, w, b, sb, K, gating, rep, normalize, z_mult)
    torch.cuda.synchronize()
    assert torch.equal(st.logits, logits)
    assert torch.equal(wf, wts) and torch.equal(idxf, idx)
    assert torch.equal(st.counts, counts)
    assert abs(float(auxf) - float(aux)) <= 1e-6 * abs(float(aux)) + 1e-12
    assert torch.equal(tracker.tokens_per_expert, counts.long()) and int(tracker.total_tokens) == T
    if w_dtype == torch.bfloat16:
        # a bf16 gate is read as stored: its fp32 widening's logits, up to the
        # order of the fp32 sums (bf16 x and gate at D <= 2048 sum on the
        # matrix cores): within D ulps of sum |x w|
        wide = fm.router_logits(x, w.float(), b.float(), sb)
        bound = (x.float().abs() @ w.float().abs().T) * (D * 2.0 ** -24) + 1e-30
        assert torch.all((logits - wide).abs() <= bound)


@pytest.mark.parametrize("E,K,drop", [(8, 2, False), (8, 8, True), (4, 1, False)])
def test_gating_grad_dot_matches_separate_kernels(dev, E, K, drop):
    """fm_gating_grad_dot (the router-weight gradient <dout[t], y[row(t,k)]>
    formed inside the gating backward) against fm_router_weight_grad then
    fm_gating_grad: dlogits and the weight gradient bit for bit, dropped slots
    (row -1) included."""
    from nanopysche_amd import _lib
    from nanopysche_amd.routing import router_forward

    T, D = 1000, 2048
    x, w, b, _ = _inputs(T, D, E, 11, torch.bfloat16, False)
    x, w, b = x.to(dev), w.to(dev), b.to(dev)
    _, idx, _, st = router_forward(x, w, b, None, K, "softmax")
    plan_idx = idx.clone()
    if drop:
        plan_idx[::7, 0] = E + 3       # out-of-range slots: row -1
    plan = fm.route_tokens(plan_idx, E, 0)
    g = torch.Generator().manual_seed(12)
    y = (torch.randn(plan.rows_max, D, generator=g)).bfloat16().to(dev)
    dout = (torch.randn(T, D, generator=g) * 1e-2).bfloat16().to(dev)
    daux = torch.tensor(0.3, device=dev)
    dw = torch.empty(T * K, dtype=torch.float32, device=dev)
    _lib.call("fm_router_weight_grad", _lib.ptr(dout), D, _lib.ptr(y), D, _lib.ptr(plan.row_of), T, K, D,
              _lib.ptr(dw), _lib.stream_of(dout))
    dl1 = torch.empty(T, E, dtype=torch.float32, device=dev)
    _lib.call("fm_gating_grad", _lib.ptr(st.logits), T, E, E, K, st.gating, st.flags, 0, _lib.ptr(idx), 1,
              _lib.ptr(dw), _lib.ptr(daux), _lib.ptr(st.counts), 0.0, _lib.ptr(dl1), E, _lib.stream_of(dout))
    dl2 = torch.empty_like(dl1)
    dw2 = torch.empty_like(dw)
    _lib.call("fm_gating_grad_dot", _lib.ptr(st.logits), T, E, E, K, st.gating, st.flags, 0, _lib.ptr(idx), 1,
              None, _lib.ptr(dout), D, _lib.ptr(y), D, _lib.ptr(plan.row_of), D, _lib.ptr(dw2), _lib.ptr(daux),
              _lib.ptr(st.counts), 0.0, _lib.ptr(dl2), E, _lib.stream_of(dout))
    torch.cuda.synchronize()
    assert torch.equal(dw, dw2) and torch.equal(dl1, dl2)
    if drop:
        assert torch.all(dw2.reshape(T, K)[::7, 0] == 0)


def test_router_backward_writes_parameter_dtypes(dev):
    """dW and db come out in the gate's own dtype: for a bf16 gate, the
    fp32 sums rounded once (equal to the fp32 result rounded to bf16)."""
    from nanopysche_amd.routing import router_backward, router_forward

    T, D, E, K = 2000, 1024, 8, 2
    x, w, b, _ = _inputs(T, D, E, 13, torch.bfloat16, False)
    w, b = w.bfloat16().float(), b.bfloat16().float()   # the same values in both dtypes
    x = x.to(dev)
    daux = torch.tensor(1.0, device=dev)
    dws = torch.randn(T, K, generator=torch.Generator().manual_seed(14)).to(dev)
    out = {}
    for dt in (torch.float32, torch.bfloat16):
        wd, bd = w.to(dt).to(dev), b.to(dt).to(dev)
        _, _, _, st = router_forward(x, wd.float(), bd.float(), None, K, "softmax")
        _, dW, db, _ = router_backward(st, x, wd, dws, daux, need_x=False, bias_dtype=dt)
        out[dt] = (dW, db)
    torch.cuda.synchronize()
    assert out[torch.bfloat16][0].dtype == torch.bfloat16 and out[torch.bfloat16][1].dtype == torch.bfloat16
    assert torch.equal(out[torch.bfloat16][0], out[torch.float32][0].bfloat16())
    assert torch.equal(out[torch.bfloat16][1], out[torch.float32][1].bfloat16())
