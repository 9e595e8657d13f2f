"""Paired-row operand layout (FM_ROWS_PAIRED / FM_COLS_PAIRED, FM_GEMM_PAIRED).

Rows 2p and 2p + 1 of a paired buffer share one pair row, interleaved in
64-byte pieces.  The producers' paired outputs must be their row-major
outputs in that arrangement, bit for bit (unpairing them on the host gives
the row-major bytes back), and the ring GEMM kernels on paired operands must
give the row-major kernels' results bit for bit -- the fragments, scales and
MFMA order are the same.  Last, the expert block with every operand paired
must produce the bits of the row-major block, forward and all gradients."""

import pytest
import torch

import nanopysche_amd as fm
from nanopysche_amd import _lib
from nanopysche_amd.flow_moe import (ExpertWeights, FP8FlowMoECompute, FP8FlowMoEConfig, _gemm_k, _gemm_m,
                                     _gemm_mk, _swiglu, _wrap, _alloc_quant, _tile_args)
from nanopysche_amd.recipes import FP8RecipeConfig, FP8RecipeType
from tests.helpers import randn_bf16, zipf_routing

pytestmark = pytest.mark.gpu
POW2 = _lib.QUANT_POW2


def unpair(t):
    """Row-major bytes of a paired [R, C] buffer (R even, C a multiple of 64)."""
    R, C = t.shape
    return t.view(R // 2, C // 64, 2, 64).permute(0, 2, 1, 3).reshape(R, C)


def _routing(T, E, seed):
    """Zipf top-2 routing with two zero-token experts."""
    return zipf_routing(T, E, 2, 1.1, seed=seed, zero_experts=(1, 6))


# top-1 expert sizes whose padded groups hold 0, 1, 2, 3 and 16 K steps of
# 128 tokens: the ragged-K ring walks experts of 3+ steps, the rest one at a time
SIZES = (0, 1, 127, 128, 129, 256, 257, 383, 384, 2000)


def _sized_routing(dev):
    idx = torch.cat([torch.full((n,), e, dtype=torch.int64) for e, n in enumerate(SIZES)])
    idx = idx[torch.randperm(idx.numel(), generator=torch.Generator().manual_seed(0))]
    return torch.ones(idx.numel(), 1, device=dev), idx.view(-1, 1).to(dev)


def _equal_rows(a, b, rows):
    return torch.equal(a[:rows].view(torch.uint8), b[:rows].view(torch.uint8))


MX = _lib.QUANT_MX


@pytest.mark.parametrize("kind", [POW2, _lib.QUANT_BLOCK, MX])
def test_producers_paired_layout(dev, kind):
    T, E, D, H = 3000, 8, 512, 384
    x = randn_bf16((T, D), seed=11).to(dev)
    _, idx = _routing(T, E, seed=3)
    idx = idx.to(dev)
    gran, pow2 = "1x32" if kind == MX else "1x128", kind == POW2
    sblk = 32 if kind == MX else 128
    a = fm.fused_permute_pad(x, idx, E, granularity=gran, pow2_scale=pow2, return_transpose=True, kmajor_scales=True)
    b = fm.fused_permute_pad(x, a.plan, E, granularity=gran, pow2_scale=pow2, return_transpose=True,
                             kmajor_scales=True, paired_rows=True, paired_cols=True)
    rows = int(a.plan.offsets[-1])
    assert b.rows.paired and b.rows_t.paired
    assert _equal_rows(unpair(b.rows.data), a.rows.data, rows)
    assert torch.equal(b.rows.scale[:rows], a.rows.scale[:rows])
    assert torch.equal(unpair(b.rows_t.data)[:, :rows], a.rows_t.data[:, :rows])
    assert torch.equal(b.rows_t.scale[:rows // sblk], a.rows_t.scale[:rows // sblk])
    # SwiGLU forward and backward, row and transposed outputs
    R = a.plan.rows_max
    gu = randn_bf16((R, 2 * H), seed=12).to(dev)
    dh = randn_bf16((R, H), seed=13, std=0.1).to(dev)
    outs = []
    for pr in (False, True):
        outs.append(_swiglu(gu[:, :H], gu[:, H:], R, H, kind, True, True, dev, a.plan.tile_expert, kmajor=True,
                            paired=pr, col_paired=pr))
    (q0, s0, qt0, st0), (q1, s1, qt1, st1) = outs
    assert _equal_rows(unpair(q1), q0, rows) and torch.equal(s1[:rows], s0[:rows])
    assert torch.equal(unpair(qt1)[:, :rows], qt0[:, :rows]) and torch.equal(st1[:rows // sblk], st0[:rows // sblk])
    outs = []
    for pr in (False, True):
        gq, gs, gqt, gst = _alloc_quant(R, 2 * H, kind, True, True, dev, kmajor=True)
        _lib.call("fm_swiglu_backward", _lib.ptr(gu), gu.stride(0), _lib.ptr(gu[:, H:]), gu.stride(0),
                  _lib.ptr(dh), dh.stride(0), R, H, *_tile_args(kind, gq, gs, gqt, gst, pr, pr),
                  _lib.ptr(a.plan.tile_expert), _lib.stream_of(gu))
        outs.append((gq, gs, gqt, gst))
    (q0, s0, qt0, st0), (q1, s1, qt1, st1) = outs
    assert _equal_rows(unpair(q1), q0, rows) and torch.equal(s1[:rows], s0[:rows])
    assert torch.equal(unpair(qt1)[:, :rows], qt0[:, :rows]) and torch.equal(st1[:rows // sblk], st0[:rows // sblk])


@pytest.mark.parametrize("kind", [POW2, MX])
def test_weight_quantisation_paired_layout(dev, kind):
    E, H, D = 4, 384, 512
    w1, w2, w3 = (randn_bf16((E * H, D), seed=s, std=0.02).to(dev) for s in (21, 22, 23))
    a = ExpertWeights(kind).refresh(w1, w2, w3, E)
    b = ExpertWeights(kind, paired=True).refresh(w1, w2, w3, E)
    assert b.w13.paired and b.w2.paired and b.w13t.paired and b.w2t.paired and not a.w13.paired
    ops = ((a.w13, b.w13), (a.w2, b.w2))
    if kind == MX:   # the transposed copies too: [D, E*2H] and [D, E*H] matrices
        ops += ((a.w13t, b.w13t), (a.w2t, b.w2t))
    for x, y in ops:
        cols = x.data.shape[-1] if x.data.dim() == 2 else D
        assert torch.equal(unpair(y.data.reshape(-1, cols)), x.data.reshape(-1, cols))
        assert torch.equal(y.scale, x.scale)


def _operands(dev, E=8, T=3000, D=512, H=384, seed=5, sized=False):
    if sized:
        wts, idx = _sized_routing(dev)
        E, T = len(SIZES), idx.shape[0]
    else:
        wts, idx = _routing(T, E, seed=seed)
    x = randn_bf16((T, D), seed=seed).to(dev)
    dO = randn_bf16((T, D), seed=seed + 1, std=0.01).to(dev)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=seed + s, std=0.02).to(dev) for s in (2, 3, 4))
    return x, dO, wts.to(dev), idx.to(dev), (w1, w2, w3)


@pytest.mark.parametrize("kind", [POW2, MX])
@pytest.mark.parametrize("sized", [False, True])
def test_ring_gemms_match_row_major(dev, sized, kind):
    E, T, D, H = 8, 3000, 512, 384
    x, dO, wts, idx, (w1, w2, w3) = _operands(dev, E, T, D, H, sized=sized)
    E = len(SIZES) if sized else E
    ew0 = ExpertWeights(kind).refresh(w1, w2, w3, E)
    ew1 = ExpertWeights(kind, paired=True).refresh(w1, w2, w3, E)
    gran = "1x32" if kind == MX else "1x128"
    kw = dict(granularity=gran, pow2_scale=kind == POW2, return_transpose=True, kmajor_scales=True)
    p0 = fm.fused_permute_pad(x, idx, E, **kw)
    plan = p0.plan
    p1 = fm.fused_permute_pad(x, plan, E, paired_rows=True, paired_cols=True, **kw)
    d0 = fm.fused_permute_pad(dO, plan, E, weights=wts, **kw)
    d1 = fm.fused_permute_pad(dO, plan, E, weights=wts, paired_rows=True, paired_cols=True, **kw)
    R, rows = plan.rows_max, int(plan.offsets[-1])
    h0, hc0 = _wrap(*_swiglu(*(randn_bf16((R, 2 * H), seed=9).to(dev).split(H, 1)), R, H, kind, True, True, dev,
                             plan.tile_expert, kmajor=True), kind)
    h1, hc1 = _wrap(*_swiglu(*(randn_bf16((R, 2 * H), seed=9).to(dev).split(H, 1)), R, H, kind, True, True, dev,
                             plan.tile_expert, kmajor=True, paired=True, col_paired=True), kind, True, True)

    def out(n):
        return torch.zeros(R, n, dtype=torch.bfloat16, device=dev)

    cases = [("gate|up, [N][K] weights", p0.rows, ew0.w13, p1.rows, ew1.w13, 2 * H),
             ("down", h0, ew0.w2t, h1, ew1.w2t, D),
             ("dH, [N][K] weights", d0.rows, ew0.w2, d1.rows, ew1.w2, H)]
    if kind == POW2:
        cases.append(("down, [K][N] weights row-major", h0, ew0.w2t, h1, ew0.w2t, D))
    for name, t0, wa, t1, wb, N in cases:
        o0, o1 = out(N), out(N)
        _gemm_m(kind, t0, wa, plan, o0)
        _gemm_m(kind, t1, wb, plan, o1)
        assert torch.equal(o0[:rows], o1[:rows]), name
    # input gradient through the paired gate|up weights ([K][N] for pow2, the
    # transposed copy for MX); dgu rows
    gq0 = fm.quantize_to_fp8(randn_bf16((R, 2 * H), seed=31).to(dev), gran, pow2_scale=kind == POW2)
    gq1 = fm.FP8Tensor(gq0.data.view(R // 2, 2, 2 * H // 64, 64).permute(0, 2, 1, 3).reshape(R, 2 * H).contiguous(),
                       gq0.scale, gq0.granularity, kind == POW2, True)
    o0, o1 = out(D), out(D)
    _gemm_m(kind, gq0, ew0.w13t, plan, o0)
    _gemm_m(kind, gq1, ew1.w13t, plan, o1)
    assert torch.equal(o0[:rows], o1[:rows]), "dX"
    # weight gradients (ragged-K, experts of 0 to many K steps), and dH + dW2 as one grid
    for a_c, b_c, M, N in (((hc0, d0.rows_t), (hc1, d1.rows_t), H, D), ((p0.rows_t, p0.rows_t), (p1.rows_t, p1.rows_t), D, D)):
        g0 = torch.zeros(E * M, N, dtype=torch.bfloat16, device=dev)
        g1 = torch.zeros_like(g0)
        _gemm_k(kind, a_c[0], a_c[1], plan, M, N, g0, M * N, may_split=False)
        _gemm_k(kind, b_c[0], b_c[1], plan, M, N, g1, M * N, may_split=False)
        assert torch.equal(g0, g1), ("ragged-K", M, N)
    # (MX: the entry point runs dH and dW2 as its two ring launches)
    dh0, dh1 = out(H), out(H)
    dw0 = torch.zeros(E * H, D, dtype=torch.bfloat16, device=dev)
    dw1 = torch.zeros_like(dw0)
    _gemm_mk(kind, d0.rows, ew0.w2, plan, dh0, hc0, d0.rows_t, H, D, dw0, H * D)
    _gemm_mk(kind, d1.rows, ew1.w2, plan, dh1, hc1, d1.rows_t, H, D, dw1, H * D)
    assert torch.equal(dh0[:rows], dh1[:rows]) and torch.equal(dw0, dw1), "dH + dW2 grid"


def _block(E, D, H, threshold=0, recipe=FP8RecipeType.FLOW_MOE):
    cfg = FP8FlowMoEConfig(True, FP8RecipeConfig(True, recipe))
    return FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=threshold)


@pytest.mark.parametrize("E,T,D,H,threshold,balanced,recipe", [
    (8, 3000, 512, 384, 0, False, FP8RecipeType.FLOW_MOE),     # Zipf, zero-token experts: everything paired
    (8, 3000, 512, 384, 400, False, FP8RecipeType.FLOW_MOE),   # threshold split: paired rows, row-major columns
    (8, 8192, 2048, 1408, 0, True, FP8RecipeType.FLOW_MOE),    # configs[2]: dH + dW2 in one paired grid
    (8, 3000, 512, 384, 0, False, FP8RecipeType.MXFP8),        # MX: the paired ring with e8m0 scales
])
def test_block_paired_matches_row_major(dev, E, T, D, H, threshold, balanced, recipe):
    x, dO, wts, idx, ws = _operands(dev, E, T, D, H, seed=7)
    if balanced:
        t = torch.arange(T, device=dev)
        idx = torch.stack([t % E, (t + E // 2) % E], 1)
    res = []
    for paired in (False, True):
        ExpertWeights.PAIRED = paired
        try:
            blk = _block(E, D, H, threshold, recipe)
            p = [w.clone().requires_grad_(True) for w in ws]
            blk.set_weights(*p)
            xi = x.clone().requires_grad_(True)
            wi = wts.clone().requires_grad_(True)
            o = blk(xi, wi, idx, 0, E)
            o.backward(dO)
            torch.cuda.synchronize()
            res.append([o.detach(), xi.grad, wi.grad] + [q.grad for q in p])
        finally:
            ExpertWeights.PAIRED = True
    for name, a, b in zip(("out", "dx", "dweights", "dw1", "dw2", "dw3"), *res):
        assert torch.equal(a, b), name
