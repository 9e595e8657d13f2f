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
