"""Pins the RMSNorm oracle (oracle/norm.py) against torch's float64 evaluation
of the reference's op sequence (model/norm.py:32-49) and against invariants a
dropped or misplaced term breaks; planted mistakes (in the oracle, on the CPU)
must fail the same checks."""

import numpy as np
import pytest
import torch

from oracle import norm as onorm
from oracle.fp8 import bf16_round


def _ref64(x, w, eps):
    """model/norm.py:40-45 in float64, differentiable in x and w."""
    variance = x.pow(2).mean(dim=-1, keepdim=True)
    return x * torch.rsqrt(variance + eps) * w


def _case(T=64, D=512, seed=0, spread=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g)
    if spread:   # rows spanning many octaves
        x = x * torch.exp2(torch.randint(-12, 8, (T, 1), generator=g).float())
    x = x.bfloat16().float()
    w = (1.0 + 0.1 * torch.randn(D, generator=g)).float()
    dy = (torch.randn(T, D, generator=g) * 1e-2).bfloat16().float()
    return x.numpy(), w.numpy(), dy.numpy()


def _ulps_bf16(a, b):
    """Distance in bf16 units of the last place between bf16 values."""
    ia = torch.from_numpy(np.asarray(a, np.float32)).bfloat16().view(torch.int16).int()
    ib = torch.from_numpy(np.asarray(b, np.float32)).bfloat16().view(torch.int16).int()
    ia = torch.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    return (ia - ib).abs().numpy()


def _check_forward(fn, x, w, eps):
    out, r = fn(x, w, eps)
    ref = _ref64(torch.from_numpy(x).double(), torch.from_numpy(w).double(), eps).numpy()
    # float32 arithmetic: a few float32 roundings of the float64 value
    rel = np.abs(out - ref) / np.maximum(np.abs(ref), 1e-30)
    return float(rel.max()), out, r, ref


@pytest.mark.parametrize("D", [512, 2048, 7168])
def test_forward_matches_float64_reference(D):
    x, w, _, = _case(D=D, seed=D)[:3]
    eps = onorm.DEFAULT_EPS
    rel, out, r, ref = _check_forward(onorm.rmsnorm_f32, x, w, eps)
    assert rel < 8 * 2.0 ** -24
    r64 = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=-1) + eps)
    assert np.abs(r / r64 - 1).max() < 4 * 2.0 ** -24
    # the bf16 output: equal to bf16(float64 value) except at rounding boundaries
    y, _ = onorm.rmsnorm(x, w, eps)
    d = _ulps_bf16(y, bf16_round(ref.astype(np.float32)))
    assert d.max() <= 1 and (d > 0).mean() < 2e-3


def test_invariants():
    x, w, _ = _case(T=32, D=1024, seed=1)
    eps = onorm.DEFAULT_EPS
    ones = np.ones_like(w)
    out, _ = onorm.rmsnorm_f32(x, ones, eps)
    # unit weight: a row of mean square m comes out with mean square m / (m + eps)
    m = np.mean(x.astype(np.float64) ** 2, axis=-1)
    ms = np.mean(out.astype(np.float64) ** 2, axis=-1)
    assert np.abs(ms - m / (m + eps)).max() < 1e-6
    # scale invariance without eps: a power-of-two scale of the input is exact in
    # every float32 step, so the output is unchanged bit for bit
    a, _ = onorm.rmsnorm_f32(x, w, 0.0)
    b, _ = onorm.rmsnorm_f32(x * 4.0, w, 0.0)
    assert np.array_equal(a, b)
    # eps dominates tiny rows: r = 1 / sqrt(eps)
    tiny = np.full((2, 512), 1e-8, np.float32)
    _, r = onorm.rmsnorm_f32(tiny, np.ones(512, np.float32), eps)
    assert np.allclose(r, 1.0 / np.sqrt(1e-16 + eps), rtol=1e-6)


def test_backward_matches_autograd():
    x, w, dy = _case(T=48, D=512, seed=2)
    eps = onorm.DEFAULT_EPS
    xt = torch.from_numpy(x).double().requires_grad_(True)
    wt = torch.from_numpy(w).double().requires_grad_(True)
    _ref64(xt, wt, eps).backward(torch.from_numpy(dy).double())
    dx, dw = onorm.rmsnorm_backward(dy, x, w, eps)
    assert np.allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-12 * np.abs(dx).max())
    assert np.allclose(dw, wt.grad.numpy(), rtol=1e-10, atol=1e-12 * np.abs(dw).max())


def _planted_forward(kind):
    def fn(x, w, eps):
        xf = np.asarray(x, np.float32)
        if kind == "eps_outside_sqrt":
            r = 1.0 / (np.sqrt(np.mean(xf * xf, axis=-1)) + eps)
        elif kind == "sum_not_mean":
            r = 1.0 / np.sqrt(np.sum(xf * xf, axis=-1) + eps)
        else:  # weight dropped
            return (xf / np.sqrt(np.mean(xf * xf, axis=-1, keepdims=True) + eps)).astype(np.float32), None
        return (xf * r[:, None].astype(np.float32) * w).astype(np.float32), r.astype(np.float32)
    return fn


@pytest.mark.parametrize("kind", ["eps_outside_sqrt", "sum_not_mean", "weight_dropped"])
def test_planted_forward_mistakes_fail(kind):
    x, w, _ = _case(T=64, D=512, seed=3)
    x[:4] *= 2.0 ** -14    # rows small enough for eps to matter
    rel, *_ = _check_forward(_planted_forward(kind), x, w, onorm.DEFAULT_EPS)
    assert rel > 1e-3


def test_planted_backward_mistake_fails():
    x, w, dy = _case(T=16, D=512, seed=4)
    eps = onorm.DEFAULT_EPS
    xt = torch.from_numpy(x).double().requires_grad_(True)
    _ref64(xt, torch.from_numpy(w).double(), eps).backward(torch.from_numpy(dy).double())
    r = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True) + eps)
    wrong = r * dy * w                      # the r^3 term dropped
    assert np.abs(wrong - xt.grad.numpy()).max() > 1e-3 * np.abs(xt.grad.numpy()).max()
