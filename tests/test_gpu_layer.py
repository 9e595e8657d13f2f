"""Expert block forward + backward on the GPU against the CPU oracles:
FP8 recipes within 2e-2 (max|err| / max|ref|) of the dequantise-then-fp32
flow, BF16 within 1e-2 of the reference's per-expert loop
(model/moe.py:1542-1596)."""

import numpy as np
import pytest
import torch

import nanopysche_amd as fm
from oracle import layer as olayer
from oracle import routing as orouting
from tests.helpers import randn_bf16, zipf_routing

pytestmark = pytest.mark.gpu

FP8_TOL = 2e-2
BF16_TOL = 1e-2


def _run(dev, x, w, idx, w1, w2, w3, go, E, recipe, threshold, param_dtype=torch.bfloat16,
         taps=None):
    H = w1.shape[0] // E
    D = x.shape[1]
    rt = fm.FP8RecipeType(recipe)
    cfg = fm.FP8FlowMoEConfig(enabled=True, fp8_recipe=fm.FP8RecipeConfig(True, rt))
    blk = fm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=threshold)
    blk.capture_intermediates = taps
    p = [t.to(dev).to(param_dtype).requires_grad_(True) for t in (w1, w2, w3)]
    blk.set_weights(*p)
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    out = blk(xd, wd, idx.to(dev), 0, E)
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    grads = dict(x=xd.grad, weights=wd.grad, w1=p[0].grad, w2=p[1].grad, w3=p[2].grad)
    return out, grads


def _case(T, D, H, E, K, seed, skew=0.0, zeros=()):
    x = randn_bf16((T, D), seed=seed)
    w, idx = zipf_routing(T, E, K, skew, seed=seed + 1, zero_experts=zeros)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=seed + s, std=0.02) for s in (2, 3, 4))
    go = randn_bf16((T, D), seed=seed + 5, std=1e-2)
    return x, w, idx, w1, w2, w3, go


def _check(out, grads, ref_out, ref_grads, tol, label):
    e = olayer.max_rel_err(out.detach().float().cpu().numpy(), ref_out)
    assert e <= tol, f"{label}: forward {e}"
    for name in ("x", "weights", "w1", "w2", "w3"):
        r = ref_grads[name]
        r = r.numpy() if torch.is_tensor(r) else r
        e = olayer.max_rel_err(grads[name].float().cpu().numpy(), r)
        assert e <= tol, f"{label}: grad {name} {e}"


@pytest.mark.parametrize("recipe", ["blockwise", "flow_moe", "mxfp8"])
@pytest.mark.parametrize("shape", [(512, 256, 256, 4, 2, 0.0, ()), (700, 384, 256, 8, 2, 1.2, (1, 6))])
def test_fp8_block_matches_flow_oracle(dev, recipe, shape):
    """Stage-synchronised: the oracle takes the device's bf16 gate|up and dH
    GEMM outputs, so every quantiser sees identical inputs; what remains is the
    FP8 MFMA's own summation error (~1e-5 relative)."""
    T, D, H, E, K, skew, zeros = shape
    x, w, idx, w1, w2, w3, go = _case(T, D, H, E, K, seed=T, skew=skew, zeros=zeros)
    taps = {}
    out, grads = _run(dev, x, w, idx, w1, w2, w3, go, E, recipe, threshold=0, taps=taps)
    taps = {k: v.float().cpu().numpy() for k, v in taps.items()}
    ref_out, ref_grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=recipe, taps=taps)
    _check(out, grads, ref_out, ref_grads, FP8_TOL, recipe)


@pytest.mark.parametrize("recipe", ["blockwise", "flow_moe", "mxfp8"])
def test_fp8_block_free_running(dev, recipe):
    """End-to-end against the independent oracle with no shared intermediates,
    at >= 1024 assignments per expert: max-rel within 2e-2 and mean relative
    error within 5e-3 for the output and every gradient."""
    T, D, H, E, K = 2048, 512, 256, 4, 2
    x, w, idx, w1, w2, w3, go = _case(T, D, H, E, K, seed=17)
    out, grads = _run(dev, x, w, idx, w1, w2, w3, go, E, recipe, threshold=0)
    ref_out, ref_grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=recipe)
    _check(out, grads, ref_out, ref_grads, FP8_TOL, recipe)
    pairs = [(out.detach(), ref_out)] + [(grads[k], ref_grads[k]) for k in ("x", "weights", "w1", "w2", "w3")]
    for got, ref in pairs:
        g = got.float().cpu().numpy()
        assert abs(g - ref).mean() <= 5e-3 * abs(ref).mean()


@pytest.mark.parametrize("param_dtype", [torch.bfloat16, torch.float32])
def test_bf16_block_matches_reference_loop(dev, param_dtype):
    T, D, H, E, K = 600, 256, 384, 4, 2
    x, w, idx, w1, w2, w3, go = _case(T, D, H, E, K, seed=3, skew=1.0, zeros=(2,))
    out, grads = _run(dev, x, w, idx, w1, w2, w3, go, E, "none", threshold=0, param_dtype=param_dtype)
    ref_out, ref_grads = olayer.moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
    _check(out, grads, ref_out.numpy(), ref_grads, BF16_TOL, "bf16")
    assert grads["w1"].dtype == param_dtype


@pytest.mark.parametrize("splits", [None, "2"])
def test_threshold_mixed_fp8_and_bf16(dev, splits, monkeypatch):
    """Experts with >= threshold assignments take FP8, the rest BF16 (with
    splits = 2 the weight gradients take the split-K form, whose reduction
    must leave the other precision's experts alone)."""
    if splits is not None:
        monkeypatch.setenv("FM_RK_SPLITS", splits)
    T, D, H, E, K = 1024, 256, 256, 4, 1
    x, w, idx, w1, w2, w3, go = _case(T, D, H, E, K, seed=9)
    idx = torch.tensor([0] * 600 + [1] * 300 + [2] * 124, dtype=torch.int64).reshape(T, 1)
    out, grads = _run(dev, x, w, idx, w1, w2, w3, go, E, "flow_moe", threshold=400)
    f_out, f_grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe="flow_moe")
    b_out, b_grads = olayer.moe_flow_reference(x, w, idx, w1, w2, w3, E, go, recipe=None)
    o = out.detach().float().cpu().numpy()
    fp8_rows = (idx[:, 0] == 0).numpy()
    assert olayer.max_rel_err(o[fp8_rows], f_out[fp8_rows]) <= FP8_TOL
    assert olayer.max_rel_err(o[~fp8_rows], b_out[~fp8_rows]) <= BF16_TOL
    # expert 0 weight grads follow the FP8 flow, expert 1-2 the BF16 flow, expert 3 is zero
    g1 = grads["w1"].float().cpu().numpy().reshape(E, H, D)
    assert olayer.max_rel_err(g1[0], f_grads["w1"].reshape(E, H, D)[0]) <= FP8_TOL
    assert olayer.max_rel_err(g1[1], b_grads["w1"].reshape(E, H, D)[1]) <= BF16_TOL
    assert (g1[3] == 0).all()


@pytest.mark.parametrize("recipe", ["flow_moe", "mxfp8"])
def test_threshold_mixed_top2_tokens_span_both_precisions(dev, recipe, monkeypatch):
    """Top-2 with the threshold splitting the experts (the split is by each
    expert's assignment count: 0, 1, 2, 3 hold 700, 324, 512, 512; threshold
    500 puts 0, 2, 3 on FP8 and 1 on BF16), so the tokens of expert 1 combine
    a BF16 and an FP8 expert row, and each precision's producers write only
    their own experts' tiles.  Reference:
    the FP8 oracle with the BF16 experts' slots dropped plus the BF16 oracle
    with the FP8 experts' slots dropped (an expert's rows, and so its
    quantisation blocks, are the same in both); weight gradients per expert
    from its precision's oracle.  Also: exactly the producer launches of each
    precision ran with that precision's tile list."""
    from nanopysche_amd import _lib

    T, D, H, E, K = 1024, 256, 256, 4, 2
    x, w, _, w1, w2, w3, go = _case(T, D, H, E, K, seed=13)
    t = torch.arange(T)
    idx = torch.stack([(t >= 700).long(), 2 + (t % 2)], 1)
    counts = torch.bincount(idx.reshape(-1), minlength=E)
    assert counts.tolist() == [700, 324, 512, 512]
    fp8 = (counts >= 500)[idx]                                   # slots on FP8 experts (expert 0, 2, 3)
    calls = []
    real = _lib.call

    def spy(name, *args):
        calls.append((name, args))
        return real(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    taps = {}
    out, grads = _run(dev, x, w, idx, w1, w2, w3, go, E, recipe, threshold=500, taps=taps)
    monkeypatch.setattr(_lib, "call", real)
    drop = torch.full_like(idx, 99)
    f_idx, b_idx = torch.where(fp8, idx, drop), torch.where(fp8, drop, idx)
    # stage-synchronised: each oracle takes the device's gate|up and dH rows of
    # its own experts, moved from the device's padded layout to its own
    dev_offs = orouting.sort_assignments(idx.numpy(), E)["offsets"]

    def sub_taps(sub_idx):
        offs = orouting.sort_assignments(sub_idx.numpy(), E, drop_out_of_range=True)["offsets"]
        out_t = {}
        for k, v in taps.items():
            a = v.float().cpu().numpy()
            b = np.zeros((int(offs[-1]), a.shape[1]), np.float32)
            for e in range(E):
                n = int(offs[e + 1] - offs[e])
                b[offs[e]:offs[e] + n] = a[dev_offs[e]:dev_offs[e] + n]
            out_t[k] = b
        return out_t

    f_out, f_g = olayer.moe_flow_reference(x, w, f_idx, w1, w2, w3, E, go, recipe=recipe, taps=sub_taps(f_idx))
    b_out, b_g = olayer.moe_flow_reference(x, w, b_idx, w1, w2, w3, E, go, recipe=None, taps=sub_taps(b_idx))
    o = out.detach().float().cpu().numpy()
    assert olayer.max_rel_err(o, f_out + b_out) <= FP8_TOL
    assert olayer.max_rel_err(grads["x"].float().cpu().numpy(), f_g["x"] + b_g["x"]) <= FP8_TOL
    dw = grads["weights"].float().cpu().numpy()
    assert olayer.max_rel_err(dw[fp8.numpy()], f_g["weights"][fp8.numpy()]) <= FP8_TOL
    assert olayer.max_rel_err(dw[~fp8.numpy()], b_g["weights"][~fp8.numpy()]) <= BF16_TOL
    fe = [0, 2, 3]
    for name in ("w1", "w2", "w3"):
        g = grads[name].float().cpu().numpy().reshape(E, H, D)
        assert olayer.max_rel_err(g[fe], f_g[name].reshape(E, H, D)[fe]) <= FP8_TOL, name
        assert olayer.max_rel_err(g[1], b_g[name].reshape(E, H, D)[1]) <= BF16_TOL, name
    # the producers of the two precisions ran on the two tile lists
    tl = {}
    for name, args in calls:
        if name in ("fm_permute", "fm_swiglu_quantize", "fm_swiglu_backward"):
            kind = args[8] if name == "fm_permute" else args[6] if name == "fm_swiglu_quantize" else args[8]
            tl.setdefault(name, set()).add((int(kind) & 0xff, args[-2].value))
    assert "fm_route_tile_masks" in [n for n, _ in calls]
    for name in ("fm_permute", "fm_swiglu_quantize", "fm_swiglu_backward"):
        kinds = {k for k, _ in tl[name]}
        lists = {v for _, v in tl[name]}
        assert len(kinds) == 2 and len(lists) == 2, (name, tl[name])


def test_drop_in_call_convention(dev):
    """The reference call: compute(x, weights, indices, 0, E) with [B, S, *] shapes."""
    B, S, D, H, E, K = 2, 64, 256, 256, 4, 2
    x = randn_bf16((B, S, D), seed=4)
    logits = torch.randn(B, S, E, generator=torch.Generator().manual_seed(0))
    w, idx = orouting.softmax_topk(logits.reshape(-1, E).numpy(), K)
    w = torch.from_numpy(w).reshape(B, S, K)
    idx = torch.from_numpy(idx).reshape(B, S, K)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=s, std=0.02) for s in (2, 3, 4))
    from fp8_flow_moe import FP8FlowMoECompute, FP8FlowMoEConfig, FP8RecipeConfig, FP8RecipeType

    cfg = FP8FlowMoEConfig(enabled=True, fp8_recipe=FP8RecipeConfig(enabled=True, recipe_type=FP8RecipeType("flow_moe")))
    blk = FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=0)
    blk.set_weights(w1.to(dev), w2.to(dev), w3.to(dev))
    out = blk(x.to(dev), w.to(dev), idx.to(dev), 0, E)
    assert out.shape == (B, S, D) and out.dtype == torch.bfloat16
    ref, _ = olayer.moe_flow_reference(x.reshape(-1, D), w.reshape(-1, K), idx.reshape(-1, K), w1, w2, w3, E,
                                       recipe="flow_moe")
    assert olayer.max_rel_err(out.detach().reshape(-1, D).float().cpu().numpy(), ref) <= FP8_TOL


def test_weight_cache_tracks_parameter_updates(dev):
    T, D, H, E, K = 256, 256, 256, 2, 1
    x, w, idx, w1, w2, w3, go = _case(T, D, H, E, K, seed=1)
    cfg = fm.FP8FlowMoEConfig(True, fm.FP8RecipeConfig(True, fm.FP8RecipeType.FLOW_MOE))
    blk = fm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=0)
    p = [t.to(dev) for t in (w1, w2, w3)]
    blk.set_weights(*p)
    a = blk(x.to(dev), w.to(dev), idx.to(dev), 0, E)
    with torch.no_grad():
        p[1].mul_(2.0)  # in-place update bumps _version
    b = blk(x.to(dev), w.to(dev), idx.to(dev), 0, E)
    assert torch.allclose(b.float(), 2 * a.float(), rtol=2e-2, atol=1e-3)


@pytest.mark.parametrize("param_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind,D", [("block", 384), ("pow2", 384), ("pow2", 512), ("mx", 384)])
def test_weight_cache_quantises_parameter_values(dev, kind, D, param_dtype):
    """The cached gate|up and down operands are the parameters' own values
    quantised (fp32 master weights are not rounded to bf16 first): bytes and
    scales equal the oracle quantiser applied to the [E, 2H, D] stack of w1|w3
    (128x128 blocks, or 1x32 for MX) and to w2.  pow2 with D a multiple of 256
    keeps no transposed copies: w2t / w13t read the row operands as [K][N]."""
    import numpy as np

    from nanopysche_amd import _lib
    from nanopysche_amd.flow_moe import ExpertWeights
    from oracle import fp8 as ofp8

    E, H = 3, 256
    g = torch.Generator().manual_seed(5)
    w1, w2, w3 = ((torch.randn(E * H, D, generator=g) * 0.02).to(param_dtype) for _ in range(3))
    k = {"block": _lib.QUANT_BLOCK, "pow2": _lib.QUANT_POW2, "mx": _lib.QUANT_MX}[kind]
    ew = ExpertWeights(k).refresh(w1.to(dev), w2.to(dev), w3.to(dev), E)
    f = lambda t: t.float().numpy().reshape(E, H, D)
    W13 = np.concatenate([f(w1), f(w3)], axis=1).reshape(E * 2 * H, D)
    for op, src in ((ew.w13, W13), (ew.w2, f(w2).reshape(E * H, D))):
        data = op.data.reshape(-1, D).cpu().numpy()
        if kind == "mx":
            q, c = ofp8.quant_mx_1x32(src)
            assert np.array_equal(data, q)
            assert np.array_equal(op.scale.reshape(-1, D // 32).cpu().numpy(), c)
        else:
            n = src.shape[0]
            q, s = ofp8.quant_128x128(src, pow2=kind == "pow2")
            assert np.array_equal(data[:n], q)
            assert np.array_equal(op.scale.reshape(-1, D // 128).cpu().numpy()[: n // 128], s)
    # the dgrad operands: w13t [E][D, 2H] and w2t [E][D, H] (128x128 blocks of
    # each expert's transpose; for MX the 32x1 column blocks of the whole
    # [E*2H, D] / [E*H, D] stack, stored transposed)
    assert ew.w2t.kmajor == ew.w13t.kmajor == (kind == "pow2" and D % 256 == 0)
    for op, src, n in ((ew.w13t, W13, 2 * H), (ew.w2t, f(w2).reshape(E * H, D), H)):
        if op.kmajor:
            rows = ew.w13 if n == 2 * H else ew.w2
            assert op.data.data_ptr() == rows.data.data_ptr() and op.scale.data_ptr() == rows.scale.data_ptr()
            assert (op.N, op.K, op.ld, op.gs, op.s_row, op.s_kb, op.s_gs, op.shift) == \
                (D, n, D, n * D, 1, D // 128, (n // 128) * (D // 128), 7)
        elif kind == "mx":
            qt, ct = ofp8.quant_mx_32x1(src)
            assert np.array_equal(op.data.reshape(D, E * n).cpu().numpy(), qt)
            assert np.array_equal(op.scale.reshape(E * n // 32, D).cpu().numpy(), ct)
        else:
            data = op.data.reshape(E, D, n).cpu().numpy()
            scale = op.scale.reshape(E, D // 128, n // 128).cpu().numpy()
            for e in range(E):
                q, s = ofp8.quant_128x128(np.ascontiguousarray(src[e * n:(e + 1) * n].T), pow2=kind == "pow2")
                assert np.array_equal(data[e], q), e
                assert np.array_equal(scale[e], s), e


@pytest.mark.parametrize("kmajor", [True, False])
def test_forward_without_grad_builds_forward_operands_only(dev, kmajor, monkeypatch):
    """A no_grad forward quantises only the forward weight operands (w13,
    w2t) and no column blocks; a later forward that records a backward
    builds the dgrad operands and gives the same output.  With [K][N]
    weights (kmajor) the forward's row operands are the dgrad's too."""
    from nanopysche_amd.flow_moe import ExpertWeights

    monkeypatch.setattr(ExpertWeights, "KMAJOR", kmajor)
    T, D, H, E, K = 512, 256, 256, 4, 2
    x, w, idx, w1, w2, w3, go = _case(T, D, H, E, K, seed=12)
    cfg = fm.FP8FlowMoEConfig(True, fm.FP8RecipeConfig(True, fm.FP8RecipeType.FLOW_MOE))
    blk = fm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=0)
    p = [t.to(dev).requires_grad_(True) for t in (w1, w2, w3)]
    blk.set_weights(*p)
    with torch.no_grad():
        a = blk(x.to(dev), w.to(dev), idx.to(dev), 0, E)
    ew = next(iter(blk._cache.values()))
    assert ew.w2t.kmajor == kmajor
    if kmajor:   # the row operands serve the forward and the dgrad GEMMs alike
        assert ew.has_dgrad and ew.w13t.data is ew.w13.data and ew.w2t.data is ew.w2.data
    else:
        assert ew.w13 is not None and ew.w2t is not None and ew.w13t is None and ew.w2 is None
    b = blk(x.to(dev), w.to(dev), idx.to(dev), 0, E)
    b.backward(go.to(dev))
    assert ew.has_dgrad and ew.w13t is not None and ew.w2 is not None
    assert torch.equal(a, b.detach())
    assert p[0].grad is not None


@pytest.mark.parametrize("param_dtype,H", [(torch.float32, 384), (torch.bfloat16, 384), (torch.bfloat16, 512)])
def test_weight_cache_bf16_operands_are_exact_copies(dev, param_dtype, H):
    """BF16 recipe: w13 is w1 | w3 stacked per expert, w2t each expert's w2
    transposed, w2 and w13t (dgrad) w2 itself and [w1; w3] transposed -- the
    parameters' values rounded to bf16, bit for bit.  bf16 parameters with H a
    multiple of 256 are not copied: w13 reads w1 and w3 as stored (a split
    operand) and w2 is the parameter."""
    from nanopysche_amd import _lib
    from nanopysche_amd.flow_moe import ExpertWeights

    E, D = 3, 256
    g = torch.Generator().manual_seed(9)
    w1, w2, w3 = ((torch.randn(E * H, D, generator=g) * 0.02).to(param_dtype) for _ in range(3))
    p1, p2, p3 = w1.to(dev), w2.to(dev), w3.to(dev)
    ew = ExpertWeights(_lib.QUANT_BF16).refresh(p1, p2, p3, E)
    b = lambda t: t.to(torch.bfloat16).view(E, H, D)
    W13 = torch.cat([b(w1), b(w3)], 1)                      # [E, 2H, D]
    views = param_dtype == torch.bfloat16 and H % 256 == 0
    assert (ew.w13.data2 is not None) == views
    if views:
        same = lambda a, b: a.data_ptr() == b.data_ptr()
        assert same(ew.w13.data, p1) and same(ew.w13.data2, p3) and ew.w13.split == H and same(ew.w2.data, p2)
    else:
        assert torch.equal(ew.w13.data.reshape(E, 2 * H, D).cpu(), W13)
        assert torch.equal(ew.w2.data.reshape(E, H, D).cpu(), b(w2))
    if views and D % 256 == 0:   # the down and dX GEMMs read w2, and w1 then w3, as [K][N] weights
        assert ew.w2t.kmajor and ew.w2t.data.data_ptr() == p2.data_ptr() and (ew.w2t.N, ew.w2t.K) == (D, H)
        assert ew.w13t.kmajor and ew.w13t.data.data_ptr() == p1.data_ptr()
        assert ew.w13t.data2.data_ptr() == p3.data_ptr() and ew.w13t.split == H and (ew.w13t.N, ew.w13t.K) == (D, 2 * H)
    else:
        assert torch.equal(ew.w2t.data.reshape(E, D, H).cpu(), b(w2).transpose(1, 2))
        assert torch.equal(ew.w13t.data.reshape(E, D, 2 * H).cpu(), W13.transpose(1, 2))


@pytest.mark.parametrize("kind,E,H,D,T,K", [("pow2", 8, 256, 512, 3000, 2), ("pow2", 4, 384, 384, 2000, 2),
                                             ("bf16", 4, 256, 384, 2000, 1), ("pow2", 8, 256, 256, 40000, 2)])
def test_weight_batch_with_the_sort_matches(dev, kind, E, H, D, T, K):
    """fm_route_sort_weights: the routing plan and every expert-weight operand
    equal those of fm_route_sort then fm_quantize_weight_batch, bit for bit
    (part of the weight blocks run beside the histograms and the fused scan +
    scatter, the rest on their own; the last case's 80000 assignments take the
    unfused scan and scatter).  Cases: pow2 rows-only, pow2 with transposed
    copies, BF16 transposes of parameters read in place (D = 384: with D a
    multiple of 256 a BF16 layer quantises nothing, checked at the end)."""
    from nanopysche_amd import _lib
    from nanopysche_amd.flow_moe import ExpertWeights
    from nanopysche_amd.routing import route_tokens
    k = {"pow2": _lib.QUANT_POW2, "bf16": _lib.QUANT_BF16}[kind]
    g = torch.Generator().manual_seed(E * H + T)
    w1, w2, w3 = ((torch.randn(E * H, D, generator=g) * 0.02).to(torch.bfloat16).to(dev) for _ in range(3))
    idx = torch.randint(0, E, (T, K), generator=g).to(dev)
    ref_w = ExpertWeights(k).refresh(w1, w2, w3, E)
    ref_p = route_tokens(idx, E, 0)
    pending = []
    ew = ExpertWeights(k).refresh(w1, w2, w3, E, defer=pending)
    assert len(pending) == 1 and ew.w2t is not None
    plan = route_tokens(idx, E, 0, pending[0][:2])
    for f in ("counts", "offsets", "row_of", "assign_of_row", "tile_expert", "use_fp8"):
        assert torch.equal(getattr(plan, f), getattr(ref_p, f)), f
    for name in ("w13", "w2t", "w2", "w13t"):
        a, b = getattr(ew, name), getattr(ref_w, name)
        assert torch.equal(a.data, b.data), name
        assert (a.scale is None) == (b.scale is None) and (a.scale is None or torch.equal(a.scale, b.scale)), name
    if kind == "bf16":
        none = []
        ExpertWeights(k).refresh(*(w[:, :256].contiguous() for w in (w1, w2, w3)), E, defer=none)
        assert none == []
