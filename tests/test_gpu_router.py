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
