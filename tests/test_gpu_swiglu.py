"""GPU parity of the fused SwiGLU(+quant) kernels (fused_silu_multiply_quantize /
fused_swiglu_quantize, reference fp8/__init__.py:17-18, SwiGLU convention
model/moe.py:1181-1183, and the backward the expert block uses).

Spec (the absent fp8_flow_moe package fixes no precision):
  (i)   the kernels' fp32 values -- h = silu(g) u forward, dg and du backward,
        read through fm_swiglu_values, the same device code the fused
        quantisers inline -- are as accurate as torch's CPU silu and autograd
        against the float64 value (worst case within 0.6 ulp of torch's own,
        mean error within 5% of torch's), and within 3 ulp of torch's results
        (dg, whose factor 1 + g (1 - s) cancels near g = -1.28, in ulps of the
        size of its terms);
  (ii)  bf16, e4m3 payloads and scales of every kind (fp32-scale blocks,
        power-of-two blocks, MX 1x32) and of both outputs (row blocks and the
        transposed column blocks) equal the oracle quantiser applied to the
        kernels' own fp32 values, bit for bit;
  (iii) against the oracle quantiser applied to torch's values, at most one
        e4m3 code step on at most 1e-4 of the elements (every element of a
        block whose scale differs counts)."""

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

M, H = 1280, 1408           # C3 hidden size; rows a multiple of 128 for the transposed outputs
MAX_ULP = 2
MAX_CODE_FLIPS = 1e-4       # fraction of e4m3 codes allowed one step apart (iii)
KINDS = {"bf16": _lib.QUANT_BF16, "block": _lib.QUANT_BLOCK, "pow2": _lib.QUANT_POW2, "mx": _lib.QUANT_MX}


def _inputs(seed):
    g = randn_bf16((M, H), seed=seed, std=2.0)
    u = randn_bf16((M, H), seed=seed + 1)
    dh = randn_bf16((M, H), seed=seed + 2, std=0.1)
    return g, u, dh


def _values(g, u, dh, dev):
    """fm_swiglu_values: [M, H] h, or [M, 2H] = [dg | du] when dh is given."""
    gd, ud = g.to(dev), u.to(dev)
    dhd = None if dh is None else dh.to(dev)
    out = torch.empty(M, H if dh is None else 2 * H, dtype=torch.float32, device=dev)
    _lib.call("fm_swiglu_values", _lib.ptr(gd), gd.stride(0), _lib.ptr(ud), ud.stride(0), _lib.ptr(dhd),
              0 if dhd is None else dhd.stride(0), M, H, _lib.ptr(out), out.stride(0), _lib.stream_of(gd))
    return out.cpu().numpy()


def _torch_forward(g, u):
    return (F.silu(g.float()) * u.float()).numpy()


def _torch_backward(g, u, dh):
    gf = g.float().requires_grad_(True)
    uf = u.float().requires_grad_(True)
    (F.silu(gf) * uf).backward(dh.float())
    return np.concatenate([gf.grad.numpy(), uf.grad.numpy()], axis=1)


def _ulp(x):
    """fp32 ulp of |x| (the spacing above it; the smallest subnormal at 0)."""
    a = np.abs(np.asarray(x, np.float32))
    return np.spacing(a).astype(np.float64)


def _fused(g, u, dh, kind, dev):
    """The fused kernel's row and transposed outputs (row scales row-major)."""
    gd, ud = g.to(dev), u.to(dev)
    cols = H if dh is None else 2 * H
    q, s, qt, st = _alloc_quant(M, cols, kind, True, True, dev)
    if dh is None:
        _lib.call("fm_swiglu_quantize", _lib.ptr(gd), gd.stride(0), _lib.ptr(ud), ud.stride(0), M, H,
                  *_tile_args(kind, q, s, qt, st), None, _lib.stream_of(gd))
    else:
        dhd = dh.to(dev)
        _lib.call("fm_swiglu_backward", _lib.ptr(gd), gd.stride(0), _lib.ptr(ud), ud.stride(0), _lib.ptr(dhd),
                  dhd.stride(0), M, H, *_tile_args(kind, q, s, qt, st), None, _lib.stream_of(gd))
    torch.cuda.synchronize()

    def c(t):
        if t is None:
            return None
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).cpu().numpy().view(np.uint16)
        return t.cpu().numpy()

    return c(q), c(s), c(qt), c(st)


def _oracle(v, kind):
    """Oracle quantisation of fp32 values v [M, C]: (q, s, qt, st) in the
    kernels' layouts (row [M, C] + [M, C/blk]; transposed [C, M] + [M/blk, C])."""
    if kind == _lib.QUANT_BF16:
        b = ofp8.bf16_round(v)
        return b, None, np.ascontiguousarray(b.T), None
    if kind == _lib.QUANT_MX:
        q, s = ofp8.quant_mx_1x32(v)
        qt, st = ofp8.quant_mx_32x1(v)
        return q, s, qt, st
    q, s = ofp8.quant_1x128(v, pow2=kind == _lib.QUANT_POW2)
    if kind == _lib.QUANT_POW2:
        qt, st = ofp8.scaling_aware_transpose(q, s)   # the column blocks of the flow_moe recipe
    else:
        qt, st = ofp8.quant_128x1(v)
    return q, s, qt, st


def _exact(g, u, dh):
    """float64 h, or [dg | du], from the bf16 inputs."""
    gf, uf = g.float().numpy().astype(np.float64), u.float().numpy().astype(np.float64)
    s = 1.0 / (1.0 + np.exp(-gf))
    if dh is None:
        return gf * s * uf, None
    df = dh.float().numpy().astype(np.float64)
    dg = df * uf * s * (1.0 + gf * (1.0 - s))
    du = df * gf * s
    # size of dg's terms: its factor 1 + g (1 - s) cancels near g = -1.28
    scale_dg = np.abs(df * uf * s) * (1.0 + np.abs(gf * (1.0 - s)))
    return np.concatenate([dg, du], axis=1), np.concatenate([scale_dg, np.abs(du)], axis=1)


@pytest.mark.parametrize("direction", ["forward", "backward"])
def test_swiglu_values_as_accurate_as_torch(dev, direction):
    """(i): against the float64 value, the kernel's fp32 results are as
    accurate as torch's own CPU results (forward: both 2.5 ulp off at worst,
    mean ~0.47 ulp, on these inputs, each evaluating exp(-g) to ~1 ulp;
    backward: both 8.1 ulp of dg's terms at worst, the rounding of its five
    operations), and the two sit within MAX_ULP + 1 ulp of each other."""
    g, u, dh = _inputs(seed=31)
    dhx = None if direction == "forward" else dh
    got = _values(g, u, dhx, dev).astype(np.float64)
    ref = (_torch_forward(g, u) if dhx is None else _torch_backward(g, u, dh)).astype(np.float64)
    ex, scale = _exact(g, u, dhx)
    ulp = _ulp(ex.astype(np.float32))
    if scale is not None:
        ulp = np.maximum(ulp, _ulp(scale.astype(np.float32)))
    d_k = np.abs(got - ex) / ulp
    d_t = np.abs(ref - ex) / ulp
    assert d_k.max() <= max(MAX_ULP, d_t.max()) + 0.6, f"kernel {d_k.max():.2f} ulp from exact (torch {d_t.max():.2f})"
    assert d_k.mean() <= 1.05 * d_t.mean() + 0.01, f"mean error: kernel {d_k.mean():.3f}, torch {d_t.mean():.3f} ulp"
    d_kt = np.abs(got - ref) / ulp
    assert d_kt.max() <= MAX_ULP + 1, f"kernel {d_kt.max():.2f} ulp from torch"


@pytest.mark.parametrize("direction", ["forward", "backward"])
@pytest.mark.parametrize("kind", ["bf16", "block", "pow2", "mx"])
def test_swiglu_quantised_outputs_bit_exact_on_own_values(dev, kind, direction):
    g, u, dh = _inputs(seed=41)
    k = KINDS[kind]
    dhx = None if direction == "forward" else dh
    v = _values(g, u, dhx, dev)
    q, s, qt, st = _fused(g, u, dhx, k, dev)
    rq, rs, rqt, rst = _oracle(v, k)
    if k == _lib.QUANT_BF16:
        assert np.array_equal(q, (rq.view(np.uint32) >> 16).astype(np.uint16)), "row bf16"
        assert np.array_equal(qt, (rqt.view(np.uint32) >> 16).astype(np.uint16)), "transposed bf16"
        return
    assert np.array_equal(s, rs), "row scales"
    assert np.array_equal(q, rq), "row codes"
    assert np.array_equal(st, rst), "column scales"
    assert np.array_equal(qt, rqt), "column codes"


def _flips(q, s, rq, rs, blk, axis_rows):
    """Fraction of elements whose code differs (every element of a block whose
    scale differs by more than a few fp32 ulp counts: a power-of-two or e8m0
    step, not the last bits of an amax / 448 scale) and the largest code step
    elsewhere."""
    if s.dtype == np.uint8:
        same_s = s == rs
    else:
        same_s = np.abs(s.astype(np.float64) - rs) <= 4 * np.spacing(np.abs(rs)).astype(np.float64)
    mask = np.repeat(same_s, blk, axis=1) if axis_rows else np.repeat(same_s, blk, axis=0).T
    diff = q != rq
    bad = diff | ~mask
    steps = np.abs(q.astype(np.int32) - rq.astype(np.int32))[diff & mask]
    return bad.mean(), (steps.max() if steps.size else 0)


@pytest.mark.parametrize("direction", ["forward", "backward"])
@pytest.mark.parametrize("kind", ["block", "pow2", "mx"])
def test_swiglu_codes_vs_torch_values(dev, kind, direction):
    """(iii): the fused outputs against the oracle quantiser applied to torch's
    own fp32 values (end to end, the kernel's sigmoid included)."""
    g, u, dh = _inputs(seed=47)
    k = KINDS[kind]
    dhx = None if direction == "forward" else dh
    ref = _torch_forward(g, u) if dhx is None else _torch_backward(g, u, dh)
    q, s, qt, st = _fused(g, u, dhx, k, dev)
    rq, rs, rqt, rst = _oracle(ref.astype(np.float32), k)
    blk = 32 if k == _lib.QUANT_MX else 128
    frac, step = _flips(q, s, rq, rs, blk, True)
    assert frac <= MAX_CODE_FLIPS and step <= 1, f"row: {frac:.2e} of codes differ, largest step {step}"
    frac, step = _flips(qt, st, rqt, rst, blk, False)
    assert frac <= MAX_CODE_FLIPS and step <= 1, f"transposed: {frac:.2e} of codes differ, largest step {step}"


def test_swiglu_packed_matches_split(dev):
    g, u, _ = _inputs(seed=37)
    gu = torch.cat([g, u], dim=1).to(dev)
    a = fm.fused_swiglu_quantize(gu, G.ROW_1x128, pow2_scale=True)
    b = fm.fused_silu_multiply_quantize(g.to(dev), u.to(dev), G.ROW_1x128, pow2_scale=True)
    assert torch.equal(a.data, b.data) and torch.equal(a.scale, b.scale)


def test_swiglu_ragged_rows_row_output(dev):
    """A row count that is not a multiple of 128 (row output only)."""
    Mr = 1200
    g, u, _ = _inputs(seed=53)
    g, u = g[:Mr].contiguous(), u[:Mr].contiguous()
    t = fm.fused_silu_multiply_quantize(g.to(dev), u.to(dev), G.ROW_1x128, pow2_scale=True)
    gd, ud = g.to(dev), u.to(dev)
    out = torch.empty(Mr, H, dtype=torch.float32, device=dev)
    _lib.call("fm_swiglu_values", _lib.ptr(gd), gd.stride(0), _lib.ptr(ud), ud.stride(0), None, 0, Mr, H,
              _lib.ptr(out), out.stride(0), _lib.stream_of(gd))
    rq, rs = ofp8.quant_1x128(out.cpu().numpy(), pow2=True)
    assert np.array_equal(t.data.cpu().numpy(), rq) and np.array_equal(t.scale.cpu().numpy(), rs)
