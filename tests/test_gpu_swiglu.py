"""GPU parity of the fused SwiGLU(+quant) kernels (fused_silu_multiply_quantize /
fused_swiglu_quantize, reference fp8/__init__.py:17-18, and the backward the
expert block uses) against torch's CPU silu and autograd in fp32.

Spec (the absent fp8_flow_moe package fixes no precision): the kernel's fp32
h = silu(g) * u is within a few ulp of torch's, so its bf16 rounding differs
from torch's by at most one bf16 ulp on a small fraction of elements; the e4m3
row blocks of h match the oracle quantiser applied to torch's h except for
rare one-code (or one-scale-step) flips at rounding boundaries."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import nanopysche_amd as fm
from nanopysche_amd import _lib
from nanopysche_amd.flow_moe import _alloc_quant, _tile_args
from oracle import fp8 as ofp8
from tests.helpers import randn_bf16

pytestmark = pytest.mark.gpu
G = fm.BlockScalingGranularity

M, H = 1200, 1408           # ragged row count, C3 hidden size
MAX_BF16_FLIPS = 2e-3       # fraction of elements allowed one bf16 ulp apart
MAX_CODE_FLIPS = 1e-3       # fraction of e4m3 codes allowed one code apart


def _inputs(seed):
    g = randn_bf16((M, H), seed=seed, std=2.0)
    u = randn_bf16((M, H), seed=seed + 1)
    dh = randn_bf16((M, H), seed=seed + 2, std=0.1)
    return g, u, dh


def _bf16_ulps(a, b):
    """|a - b| in bf16 ulps (bf16 tensors; +0 and -0 are the same point)."""
    def key(t):
        i = t.contiguous().view(torch.int16).to(torch.int32).numpy()
        return np.where(i >= 0, i, -(i & 0x7FFF))
    return np.abs(key(a) - key(b))


def _check_bf16(out, ref):
    d = _bf16_ulps(out, ref)
    assert d.max() <= 1, f"bf16 result {d.max()} ulps from torch"
    assert (d > 0).mean() <= MAX_BF16_FLIPS, f"{(d > 0).mean():.2e} of elements one ulp apart"


def _check_fp8_rows(q, s, h_ref):
    rq, rs = ofp8.quant_1x128(h_ref, pow2=True)
    q, s = q.cpu().numpy(), s.cpu().numpy()
    same = s == rs
    assert same.mean() >= 1 - 1e-3, f"{1 - same.mean():.2e} of block scales differ"
    # where a scale flipped, it is one power of two
    r = s[~same] / rs[~same]
    assert np.all((r == 2.0) | (r == 0.5))
    rows = np.repeat(same, 128, axis=1)
    dq = np.abs(ofp8.e4m3_decode(q)[rows] - ofp8.e4m3_decode(rq)[rows])
    code_d = np.abs(q[rows].astype(np.int32) - rq[rows].astype(np.int32))
    flips = dq > 0
    assert flips.mean() <= MAX_CODE_FLIPS, f"{flips.mean():.2e} of codes differ"
    assert np.all(code_d[flips] == 1), "a code differs by more than one step"


def test_swiglu_forward_bf16(dev):
    g, u, _ = _inputs(seed=31)
    h = fm.fused_silu_multiply_quantize(g.to(dev), u.to(dev), granularity=None)
    ref = (F.silu(g.float()) * u.float()).bfloat16()
    _check_bf16(h.cpu(), ref)


def test_swiglu_forward_packed_matches_split(dev):
    g, u, _ = _inputs(seed=37)
    gu = torch.cat([g, u], dim=1).to(dev)
    a = fm.fused_swiglu_quantize(gu, G.ROW_1x128, pow2_scale=True)
    b = fm.fused_silu_multiply_quantize(g.to(dev), u.to(dev), G.ROW_1x128, pow2_scale=True)
    assert torch.equal(a.data, b.data) and torch.equal(a.scale, b.scale)


def test_swiglu_forward_fp8_rows(dev):
    g, u, _ = _inputs(seed=41)
    t = fm.fused_silu_multiply_quantize(g.to(dev), u.to(dev), G.ROW_1x128, pow2_scale=True)
    h_ref = (F.silu(g.float()) * u.float()).numpy()
    _check_fp8_rows(t.data, t.scale, h_ref)


def _backward(g, u, dh, kind, dev):
    gd, ud, dhd = g.to(dev), u.to(dev), dh.to(dev)
    rows = (M + 127) // 128 * 128
    q, s, qt, st = _alloc_quant(rows, 2 * H, kind, True, False, dev)
    _lib.call("fm_swiglu_backward", _lib.ptr(gd), gd.stride(0), _lib.ptr(ud), ud.stride(0), _lib.ptr(dhd),
              dhd.stride(0), M, H, *_tile_args(kind, q, s, qt, st), None, _lib.stream_of(gd))
    return q[:M], (None if s is None else s[:M])


def _torch_backward(g, u, dh):
    gf = g.float().requires_grad_(True)
    uf = u.float().requires_grad_(True)
    (F.silu(gf) * uf).backward(dh.float())
    return gf.grad, uf.grad


def test_swiglu_backward_bf16(dev):
    g, u, dh = _inputs(seed=43)
    out, _ = _backward(g, u, dh, _lib.QUANT_BF16, dev)
    dg, du = _torch_backward(g, u, dh)
    out = out.cpu()
    _check_bf16(out[:, :H].contiguous(), dg.bfloat16())
    _check_bf16(out[:, H:].contiguous(), du.bfloat16())


def test_swiglu_backward_fp8_rows(dev):
    g, u, dh = _inputs(seed=47)
    q, s = _backward(g, u, dh, _lib.QUANT_POW2, dev)
    dg, du = _torch_backward(g, u, dh)
    _check_fp8_rows(q, s, torch.cat([dg, du], dim=1).numpy())
