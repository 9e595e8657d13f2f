"""GPU grouped GEMM vs dequantise-then-fp32-matmul on CPU (FP8) and fp32
matmul of the bf16 operands (BF16), for ragged-M (forward / dgrad) and
ragged-K (weight gradient) tiles, with zero-token experts and the expert mask."""

import numpy as np
import pytest
import torch

import nanopysche_amd as fm
from nanopysche_amd import _lib
from nanopysche_amd.flow_moe import ExpertWeights, _gemm_k
from oracle import fp8 as ofp8
from oracle.layer import max_rel_err
from tests.helpers import randn_bf16, zipf_routing

pytestmark = pytest.mark.gpu
KINDS = {"bf16": _lib.QUANT_BF16, "block": _lib.QUANT_BLOCK, "pow2": _lib.QUANT_POW2, "mx": _lib.QUANT_MX}


def _deq_rows(t, kind, rows):
    """The first ``rows`` rows of a row-quantised operand (the padded expert
    groups, offsets[E]; the buffer's rows past them are never written)."""
    if kind == "bf16":
        return t[:rows].float().cpu().numpy()
    q, s = t.data[:rows].cpu().numpy(), t.scale[:rows].cpu().numpy()
    return ofp8.dequant_mx_1x32(q, s) if kind == "mx" else ofp8.dequant_1x128(q, s)


def _deq_cols(t, kind, rows):
    """Transposed operand [C, R] with k-major scales [R/blk, C], its first
    ``rows`` columns (source rows)."""
    if kind == "bf16":
        return t[:, :rows].float().cpu().numpy()
    blk = 32 if kind == "mx" else 128
    q = t.data[:, :rows].cpu().numpy()
    s = np.ascontiguousarray(t.scale[:rows // blk].cpu().numpy().T)
    return ofp8.dequant_mx_1x32(q, s) if kind == "mx" else ofp8.dequant_1x128(q, s)


def _weight_values(w, kind):
    """[E*N, K] weights as the GEMM sees them (N rows of each expert, K contiguous)."""
    wf = w.float().numpy()
    if kind == "bf16":
        return ofp8.bf16_round(wf)
    if kind == "mx":
        q, c = ofp8.quant_mx_1x32(wf)
        return ofp8.dequant_mx_1x32(q, c)
    E_N, K = wf.shape
    out = np.empty_like(wf)
    for r0 in range(0, E_N, 128):
        q, s = ofp8.quant_128x128(wf[r0:r0 + 128], pow2=kind == "pow2")
        out[r0:r0 + 128] = ofp8.dequant_128x128(q, s)
    return out


@pytest.mark.parametrize("kind", ["bf16", "block", "pow2", "mx"])
@pytest.mark.parametrize("E,T,K,zeros,D,H", [
    (4, 2048, 2, (), 512, 384), (8, 3000, 2, (2, 5), 512, 384),
    # the non-persistent ragged-M kernel: more than 64 experts (serial walk of
    # the expert table per tile), and a single 128-deep FP8 K step
    (80, 3000, 2, (3, 70), 256, 256), (4, 1000, 2, (1,), 128, 128)])
def test_ragged_m_gate_up_and_down(dev, kind, E, T, K, zeros, D, H):
    k = KINDS[kind]
    x = randn_bf16((T, D), seed=1)
    _, idx = zipf_routing(T, E, K, 1.1, seed=E, zero_experts=zeros)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=s, std=0.02) for s in (2, 3, 4))
    ew = ExpertWeights(k).refresh(w1.to(dev), w2.to(dev), w3.to(dev), E)
    gran = {"bf16": None, "block": "1x128", "pow2": "1x128", "mx": "1x32"}[kind]
    pt = fm.fused_permute_pad(x.to(dev), idx.to(dev), E, granularity=gran, pow2_scale=kind == "pow2")
    plan = pt.plan
    gu = fm.fp8_grouped_gemm(pt.rows, ew.w13, plan, out_dtype=torch.float32)
    offs = plan.offsets.cpu().numpy()
    a = _deq_rows(pt.rows, kind, offs[-1])
    W1v = _weight_values(w1, kind).reshape(E, H, D) if kind != "mx" else None
    if kind == "mx":
        W13 = torch.cat([w1.view(E, H, D), w3.view(E, H, D)], 1).reshape(E * 2 * H, D)
        W13v = _weight_values(W13, kind).reshape(E, 2 * H, D)
    else:
        W13v = np.concatenate([W1v, _weight_values(w3, kind).reshape(E, H, D)], axis=1)
    got = gu.cpu().numpy()
    for e in range(E):
        r0, r1 = offs[e], offs[e + 1]
        if r1 == r0:
            continue
        ref = a[r0:r1] @ W13v[e].T
        assert max_rel_err(got[r0:r1], ref) < 1e-3, (kind, e)
    # down projection: K = H, weights = w2_e^T
    # the rows past the padded groups hold no GEMM output: zeros keep them finite
    gu[int(offs[-1]):] = 0
    hq = fm.quantize_to_fp8(gu[:, :H].bfloat16(), gran, pow2_scale=kind == "pow2") if gran else gu[:, :H].bfloat16()
    y = fm.fp8_grouped_gemm(hq, ew.w2t, plan, out_dtype=torch.float32)
    hv = _deq_rows(hq, kind, offs[-1])
    W2 = w2.float().numpy().reshape(E, H, D)
    got = y.cpu().numpy()
    for e in range(E):
        r0, r1 = offs[e], offs[e + 1]
        if r1 == r0:
            continue
        w2t = np.ascontiguousarray(W2[e].T)
        if kind == "bf16":
            wv = ofp8.bf16_round(w2t)
        elif kind == "mx":
            q, c = ofp8.quant_mx_1x32(w2t)
            wv = ofp8.dequant_mx_1x32(q, c)
        else:
            q, s = ofp8.quant_128x128(w2t, pow2=kind == "pow2")
            wv = ofp8.dequant_128x128(q, s)
        ref = hv[r0:r1] @ wv.T
        assert max_rel_err(got[r0:r1], ref) < 1e-3, (kind, e)


@pytest.mark.parametrize("kind", ["bf16", "block", "pow2", "mx"])
@pytest.mark.parametrize("balanced", [False, True])
@pytest.mark.parametrize("splits", [None, "3"])
def test_ragged_k_weight_grad(dev, kind, balanced, splits, monkeypatch):
    """Skewed routing with a zero-token expert keeps the tiles in launch
    order; balanced routing takes the contiguous per-XCD split.  splits = 3
    forces the split-K form (fp32 partials + ordered reduction; slices of the
    small experts are empty), except for the fp32-scale kind, which has none.
    The a_t-fastest tile order (FM_GEMM_A_FAST) gives the same bits."""
    if splits is not None:
        monkeypatch.setenv("FM_RK_SPLITS", splits)
    E, T, K, D, H = 6, 2500, 2, 256, 256
    k = KINDS[kind]
    x = randn_bf16((T, D), seed=5)
    g = randn_bf16((T, 2 * H), seed=6)
    if balanced:
        t = torch.arange(T)
        idx = torch.stack([t % E, (t + 1) % E], 1)
    else:
        _, idx = zipf_routing(T, E, K, 1.2, seed=3, zero_experts=(4,))
    gran = {"bf16": None, "block": "1x128", "pow2": "1x128", "mx": "1x32"}[kind]
    px = fm.fused_permute_pad(x.to(dev), idx.to(dev), E, granularity=gran, pow2_scale=kind == "pow2",
                              return_transpose=True)
    pg = fm.fused_permute_pad(g.to(dev), px.plan, E, granularity=gran, pow2_scale=kind == "pow2",
                              return_transpose=True)
    plan = px.plan
    for out_dtype in (torch.float32, torch.bfloat16):
        dW1 = torch.full((E * H, D), float("nan"), dtype=out_dtype, device=dev)
        dW3 = torch.full((E * H, D), float("nan"), dtype=out_dtype, device=dev)
        _gemm_k(k, pg.rows_t, px.rows_t, plan, 2 * H, D, dW1, H * D, dW3, H * D, split=H)
        aw1, aw3 = torch.full_like(dW1, float("nan")), torch.full_like(dW3, float("nan"))
        _gemm_k(k, pg.rows_t, px.rows_t, plan, 2 * H, D, aw1, H * D, aw3, H * D, split=H, a_cold=True)
        assert torch.equal(aw1, dW1) and torch.equal(aw3, dW3)
        offs = plan.offsets.cpu().numpy()
        av = _deq_cols(pg.rows_t, kind, offs[-1])  # [2H, R]
        bv = _deq_cols(px.rows_t, kind, offs[-1])  # [D, R]
        d1 = dW1.float().cpu().numpy().reshape(E, H, D)
        d3 = dW3.float().cpu().numpy().reshape(E, H, D)
        tol = 1e-3 if out_dtype == torch.float32 else 8e-3
        for e in range(E):
            r0, r1 = offs[e], offs[e + 1]
            ref = av[:, r0:r1] @ bv[:, r0:r1].T
            if r1 == r0:
                assert np.all(d1[e] == 0) and np.all(d3[e] == 0)
                continue
            assert max_rel_err(d1[e], ref[:H]) < tol, (kind, e)
            assert max_rel_err(d3[e], ref[H:]) < tol, (kind, e)


def test_expert_mask_skips_tiles(dev):
    E, T, K, D, H = 4, 1024, 1, 256, 256
    x = randn_bf16((T, D), seed=1)
    _, idx = zipf_routing(T, E, K, 0.0, seed=1)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=s, std=0.02) for s in (2, 3, 4))
    ew = ExpertWeights(_lib.QUANT_BF16).refresh(w1.to(dev), w2.to(dev), w3.to(dev), E)
    pt = fm.fused_permute_pad(x.to(dev), idx.to(dev), E, granularity=None)
    mask = torch.tensor([1, 0, 1, 0], dtype=torch.int32, device=dev)
    out = torch.full((pt.plan.rows_max, 2 * H), 7.0, dtype=torch.float32, device=dev)
    fm.fp8_grouped_gemm(pt.rows, ew.w13, pt.plan, expert_mask=mask, mask_want=1, out=out)
    offs = pt.plan.offsets.cpu().numpy()
    o = out.cpu().numpy()
    assert np.all(o[offs[1]:offs[2]] == 7.0) and np.all(o[offs[3]:offs[4]] == 7.0)
    assert not np.all(o[offs[0]:offs[1]] == 7.0)


def _kmajor(w: "ExpertWeightOperand", E):
    """The [E][K, N] rows operand ``w`` (N = w.K columns) read as [N, K] weights."""
    from nanopysche_amd.flow_moe import ExpertWeightOperand
    K, N = w.N, w.K
    return ExpertWeightOperand(w.data, w.scale, ld=N, gs=K * N, s_row=1, s_kb=N // 128,
                               s_gs=(K // 128) * (N // 128), shift=7, N=N, K=K, kmajor=True)


@pytest.mark.parametrize("E,T,K,zeros,D,H", [(8, 3000, 2, (2, 5), 512, 384), (5, 2500, 3, (0,), 768, 256),
                                             (64, 6000, 4, (7, 63), 256, 256)])
def test_ragged_m_kmajor_weights_match(dev, E, T, K, zeros, D, H):
    """FM_GEMM_W_KMAJOR: the down (w2 rows [H, D]) and dgrad dX (w13 rows
    [2H, D]) GEMMs reading the row-quantised weights transposed in LDS give the
    bits of the same GEMMs on the separately quantised transposed copies (the
    same 128 x 128 blocks, so the same codes and scales)."""
    x = randn_bf16((T, D), seed=1)
    _, idx = zipf_routing(T, E, K, 1.1, seed=E, zero_experts=zeros)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=s, std=0.02) for s in (2, 3, 4))
    ew = ExpertWeights(_lib.QUANT_POW2).refresh(w1.to(dev), w2.to(dev), w3.to(dev), E)
    pt = fm.fused_permute_pad(x.to(dev), idx.to(dev), E, granularity="1x128", pow2_scale=True)
    plan = pt.plan
    for kk, w_nt, w_rows in ((H, ew.w2t, ew.w2), (2 * H, ew.w13t, ew.w13)):
        a = randn_bf16((plan.rows_max, kk), seed=kk).to(dev)
        aq = fm.quantize_to_fp8(a, "1x128", pow2_scale=True)
        nn = _kmajor(w_rows, E)
        assert (nn.N, nn.K) == (w_nt.N, w_nt.K) == (D, kk)
        for dt in (torch.float32, torch.bfloat16):
            ref = fm.fp8_grouped_gemm(aq, w_nt, plan, out_dtype=dt)
            got = fm.fp8_grouped_gemm(aq, nn, plan, out_dtype=dt)
            offs = plan.offsets.cpu().numpy()
            for e in range(E):
                r0, r1 = offs[e], offs[e + 1]
                assert torch.equal(got[r0:r1], ref[r0:r1]), (kk, dt, e)
    if H % 256:   # w2t's rows read as [K = D][N = H] weights: N not a multiple of 256 is refused
        aq = fm.quantize_to_fp8(randn_bf16((plan.rows_max, D), seed=9).to(dev), "1x128", pow2_scale=True)
        with pytest.raises(RuntimeError, match=r"\[K\]\[N\] weights need"):
            fm.fp8_grouped_gemm(aq, _kmajor(ew.w2t, E), plan)


@pytest.mark.parametrize("kind", ["bf16", "pow2", "mx"])
@pytest.mark.parametrize("E,T,K,zeros,D,H,masked", [(8, 3000, 2, (2, 5), 512, 384, False),
                                                    (6, 2500, 2, (4,), 256, 256, True),
                                                    (80, 3000, 2, (3, 70), 256, 256, False)])
def test_ragged_m_k_one_grid_matches_two_launches(dev, kind, E, T, K, zeros, D, H, masked):
    """fm_grouped_gemm_ragged_m_k (dH = dY w2 and dW2 = h^T dY in one grid
    for BF16 and pow2; MX runs the two launches) writes the bits of
    fm_grouped_gemm_ragged_m then fm_grouped_gemm_ragged_k, zero-token experts
    (dW2 zeros), masked experts (untouched) and more than 64 experts
    included."""
    from nanopysche_amd.flow_moe import _gemm_m, _gemm_mk
    k = KINDS[kind]
    gran = {"bf16": None, "pow2": "1x128", "mx": "1x32"}[kind]
    dy = randn_bf16((T, D), seed=11)
    hh = randn_bf16((T, H), seed=12)
    _, idx = zipf_routing(T, E, K, 1.1, seed=E + 1, zero_experts=zeros)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=s, std=0.02) for s in (2, 3, 4))
    ew = ExpertWeights(k).refresh(w1.to(dev), w2.to(dev), w3.to(dev), E)
    pd = fm.fused_permute_pad(dy.to(dev), idx.to(dev), E, granularity=gran, pow2_scale=kind == "pow2",
                              return_transpose=True, kmajor_scales=True)
    ph = fm.fused_permute_pad(hh.to(dev), pd.plan, E, granularity=gran, pow2_scale=kind == "pow2",
                              return_transpose=True)
    plan = pd.plan
    mask = None
    if masked:
        mask = torch.tensor([e % 2 for e in range(E)], dtype=torch.int32, device=dev)
    R = plan.rows_max
    outs = []
    for one_grid in (False, True):
        dH = torch.full((R, H), 7.0, dtype=torch.bfloat16, device=dev)
        dW2 = torch.full((E * H, D), 7.0, dtype=torch.float32, device=dev)
        if one_grid:
            _gemm_mk(k, pd.rows, ew.w2, plan, dH, ph.rows_t, pd.rows_t, H, D, dW2, H * D, mask, 1, a_cold=True)
        else:
            _gemm_m(k, pd.rows, ew.w2, plan, dH, mask, 1)
            _gemm_k(k, ph.rows_t, pd.rows_t, plan, H, D, dW2, H * D, mask=mask, want=1, may_split=False,
                    a_cold=True)
        outs.append((dH, dW2))
    (h0, w0), (h1, w1_) = outs
    used = int(plan.offsets[-1].item())
    assert torch.equal(h0[:used], h1[:used]) and torch.equal(w0, w1_)
    offs = plan.offsets.cpu().numpy()
    for e in range(E):
        if mask is not None and e % 2 == 0:   # left to the other precision's launch
            assert torch.all(w1_[e * H:(e + 1) * H] == 7.0) and torch.all(h1[offs[e]:offs[e + 1]] == 7.0)
        elif offs[e + 1] == offs[e]:
            assert torch.all(w1_[e * H:(e + 1) * H] == 0)


@pytest.mark.parametrize("kind", ["bf16", "pow2"])
def test_ragged_k_short_and_long_experts(dev, kind):
    """Experts of 0, 100, 128, 129, 256, 300 and 1000 tokens (0, 1, 1, 2, 2, 3
    and 8 FP8 K steps of 128 rows): the persistent weight-gradient kernel
    pipelines the tiles of two or more K steps and does the others one at a
    time afterwards (zeros for the empty expert); every expert against the
    dequantised fp32 product."""
    counts = [0, 100, 128, 129, 256, 300, 1000]
    E, D, H = len(counts), 256, 256
    T = sum(counts)
    k = KINDS[kind]
    idx = torch.cat([torch.full((n,), e, dtype=torch.int64) for e, n in enumerate(counts)])
    idx = idx[torch.randperm(T, generator=torch.Generator().manual_seed(3))].view(T, 1)
    x = randn_bf16((T, D), seed=21)
    g = randn_bf16((T, 2 * H), seed=22)
    gran = None if kind == "bf16" else "1x128"
    px = fm.fused_permute_pad(x.to(dev), idx.to(dev), E, granularity=gran, pow2_scale=kind == "pow2",
                              return_transpose=True)
    pg = fm.fused_permute_pad(g.to(dev), px.plan, E, granularity=gran, pow2_scale=kind == "pow2",
                              return_transpose=True)
    plan = px.plan
    dW1 = torch.full((E * H, D), float("nan"), dtype=torch.float32, device=dev)
    dW3 = torch.full_like(dW1, float("nan"))
    _gemm_k(k, pg.rows_t, px.rows_t, plan, 2 * H, D, dW1, H * D, dW3, H * D, split=H, may_split=False)
    offs = plan.offsets.cpu().numpy()
    av, bv = _deq_cols(pg.rows_t, kind, offs[-1]), _deq_cols(px.rows_t, kind, offs[-1])
    assert [int(offs[e + 1] - offs[e]) for e in range(E)] == [0, 128, 128, 256, 256, 384, 1024]
    d1 = dW1.cpu().numpy().reshape(E, H, D)
    d3 = dW3.cpu().numpy().reshape(E, H, D)
    for e in range(E):
        r0, r1 = offs[e], offs[e + 1]
        if r1 == r0:
            assert np.all(d1[e] == 0) and np.all(d3[e] == 0)
            continue
        ref = av[:, r0:r1] @ bv[:, r0:r1].T
        assert max_rel_err(d1[e], ref[:H]) < 1e-3, (kind, e)
        assert max_rel_err(d3[e], ref[H:]) < 1e-3, (kind, e)


@pytest.mark.parametrize("E,T,K,zeros,masked", [(8, 3000, 2, (2, 5), False), (6, 2500, 2, (4,), True)])
def test_bf16_split_weights_match_stacked(dev, E, T, K, zeros, masked):
    """BF16 gate|up with w1 and w3 read as stored (a split operand, rows from H
    on from w3) gives the bits of the same GEMM on the stacked [E, 2H, D] copy,
    in a single launch and as the dgrad of the dH + dW2 pair (persistent, or
    as two launches when an expert mask is given)."""
    from nanopysche_amd.flow_moe import ExpertWeightOperand, _gemm_m, _gemm_mk
    D, H = 256, 512
    x = randn_bf16((T, D), seed=1)
    _, idx = zipf_routing(T, E, K, 1.1, seed=E, zero_experts=zeros)
    w1, w3 = (randn_bf16((E * H, D), seed=s, std=0.02).to(dev) for s in (2, 4))
    pt = fm.fused_permute_pad(x.to(dev), idx.to(dev), E, granularity=None, return_transpose=True)
    plan = pt.plan
    split = ExpertWeightOperand(w1, None, D, H * D, N=2 * H, K=D, data2=w3, split=H)
    W13 = torch.cat([w1.view(E, H, D), w3.view(E, H, D)], 1).contiguous()
    stacked = ExpertWeightOperand(W13, None, D, 2 * H * D, N=2 * H, K=D)
    mask = torch.tensor([e % 2 for e in range(E)], dtype=torch.int32, device=dev) if masked else None
    used = int(plan.offsets[-1].item())
    outs = []
    for w in (stacked, split):
        out = torch.zeros(plan.rows_max, 2 * H, dtype=torch.float32, device=dev)
        _gemm_m(_lib.QUANT_BF16, pt.rows, w, plan, out, mask, 1)
        outs.append(out[:used])
    assert torch.equal(outs[0], outs[1])
    # the same operand as the dgrad of the pair (the weight gradient: x^T x)
    pair = []
    for w in (stacked, split):
        o1 = torch.zeros(plan.rows_max, 2 * H, dtype=torch.float32, device=dev)
        o2 = torch.zeros(E * D, D, dtype=torch.float32, device=dev)
        _gemm_mk(_lib.QUANT_BF16, pt.rows, w, plan, o1, pt.rows_t, pt.rows_t, D, D, o2, D * D, mask, 1)
        pair.append((o1[:used], o2))
    assert torch.equal(pair[0][0], pair[1][0]) and torch.equal(pair[0][1], pair[1][1])
    assert torch.equal(pair[1][0], outs[1])


@pytest.mark.parametrize("E,T,K,zeros,D,H", [(8, 3000, 2, (2, 5), 512, 384), (4, 2500, 1, (1,), 256, 512),
                                             (64, 6000, 4, (7, 63), 256, 128)])
def test_bf16_kmajor_weights_match(dev, E, T, K, zeros, D, H):
    """FM_GEMM_W_KMAJOR with BF16: the down GEMM reading w2 [E][K = H][N = D]
    transposed in LDS (ds_read_b64_tr_b16) gives the bits of the same GEMM on
    the transposed copy [E][D][H], fp32 and bf16 outputs."""
    from nanopysche_amd.flow_moe import ExpertWeightOperand, _gemm_m
    x = randn_bf16((T, H), seed=1)
    _, idx = zipf_routing(T, E, K, 1.1, seed=E, zero_experts=zeros)
    w2 = randn_bf16((E * H, D), seed=3, std=0.02).to(dev)
    pt = fm.fused_permute_pad(x.to(dev), idx.to(dev), E, granularity=None)
    plan = pt.plan
    nn = ExpertWeightOperand(w2, None, D, H * D, N=D, K=H, kmajor=True)
    nt = ExpertWeightOperand(w2.view(E, H, D).transpose(1, 2).contiguous(), None, H, D * H, N=D, K=H)
    used = int(plan.offsets[-1].item())
    for dt in (torch.float32, torch.bfloat16):
        outs = []
        for w in (nt, nn):
            out = torch.zeros(plan.rows_max, D, dtype=dt, device=dev)
            _gemm_m(_lib.QUANT_BF16, pt.rows, w, plan, out)
            outs.append(out[:used])
        assert torch.equal(outs[0], outs[1]), dt


@pytest.mark.parametrize("E,T,K,zeros,D,H", [(8, 3000, 2, (2, 5), 512, 384), (64, 6000, 4, (7, 63), 256, 128)])
def test_bf16_kmajor_split_weights_match(dev, E, T, K, zeros, D, H):
    """BF16 dX reading w1 then w3 as one [K = 2H][N = D] operand split along K
    (rows k >= H from w3) gives the bits of the same GEMM on the stacked
    transposed copy [E][D][2H]."""
    from nanopysche_amd.flow_moe import ExpertWeightOperand, _gemm_m
    g = randn_bf16((T, 2 * H), seed=1)
    _, idx = zipf_routing(T, E, K, 1.1, seed=E, zero_experts=zeros)
    w1, w3 = (randn_bf16((E * H, D), seed=s, std=0.02).to(dev) for s in (2, 4))
    pt = fm.fused_permute_pad(g.to(dev), idx.to(dev), E, granularity=None)
    plan = pt.plan
    nn = ExpertWeightOperand(w1, None, D, H * D, N=D, K=2 * H, kmajor=True, data2=w3, split=H)
    W13t = torch.cat([w1.view(E, H, D), w3.view(E, H, D)], 1).transpose(1, 2).contiguous()
    nt = ExpertWeightOperand(W13t, None, 2 * H, D * 2 * H, N=D, K=2 * H)
    used = int(plan.offsets[-1].item())
    outs = []
    for w in (nt, nn):
        out = torch.zeros(plan.rows_max, D, dtype=torch.bfloat16, device=dev)
        _gemm_m(_lib.QUANT_BF16, pt.rows, w, plan, out)
        outs.append(out[:used])
    assert torch.equal(outs[0], outs[1])
