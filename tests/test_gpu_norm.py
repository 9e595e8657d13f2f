"""GPU parity of the RMSNorm -> quantise kernels (reference RMSNorm.forward,
model/norm.py:32-49, before the MoE at model/transformer.py:261-263) against
the CPU oracle (oracle/norm.py, oracle/fp8.py):

* the bf16 output within one bf16 unit in the last place of the oracle's
  (float32 sums in another order), equal almost everywhere; rsqrt within a few
  float32 ulps;
* the e4m3 row blocks and their scales bit-exact against the oracle's
  quantiser applied to the kernel's own bf16 output, for the fp32-scale,
  power-of-two and MX kinds; the column blocks of the transpose bit-exact too;
* the backward (dx bf16, dw fp32) against the oracle's float64 closed form
  within the BF16 bar (1e-2), and the module under autograd;
* configs[2]'s residual-stream shape [8192, 2048] through the same checks;
* the pre-norm MoE layer against the reference op sequence in float64."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import nanopysche_amd as fm
from oracle import fp8 as ofp8
from oracle import norm as onorm
from oracle.layer import max_rel_err
from tests.helpers import randn_bf16

pytestmark = pytest.mark.gpu
G = fm.BlockScalingGranularity


def _np(t):
    return t.detach().float().cpu().numpy() if t.dtype in (torch.bfloat16,) else t.detach().cpu().numpy()


def _ulps_bf16(a, b):
    ia = torch.from_numpy(np.asarray(a, np.float32)).bfloat16().view(torch.int16).int()
    ib = torch.from_numpy(np.asarray(b, np.float32)).bfloat16().view(torch.int16).int()
    ia = torch.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    return (ia - ib).abs().numpy()


def _inputs(T, D, seed, spread=True, w_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = randn_bf16((T, D), seed=seed).float()
    if spread:   # rows spanning 20 octaves, a few below eps's reach
        x = x * torch.exp2(torch.randint(-14, 6, (T, 1), generator=g).float())
    w = (1.0 + 0.2 * torch.randn(D, generator=g)).to(w_dtype)
    return x.bfloat16(), w


def _check_values(out, x, w):
    y_ref, r_ref = onorm.rmsnorm(x.float().numpy(), w.float().numpy())
    d = _ulps_bf16(_np(out.y), y_ref)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3, (d.max(), (d > 0).mean())
    assert np.abs(_np(out.rstd) / r_ref - 1).max() < 8 * 2.0 ** -24


@pytest.mark.parametrize("D", [512, 2048, 3072, 7168])
@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16])
def test_values_match_oracle(dev, D, w_dtype):
    x, w = _inputs(1001, D, seed=D, w_dtype=w_dtype)
    out = fm.rmsnorm_quantize(x.to(dev), w.to(dev))
    _check_values(out, x, w)
    assert out.rows is None and out.cols is None


@pytest.mark.parametrize("kind", ["block", "pow2", "mx"])
def test_row_blocks_bitexact_on_own_values(dev, kind):
    x, w = _inputs(640, 2048, seed=7)
    x[5, :128] = 0                      # a zero block
    x[6, 128:256] *= 1e15               # one block far above the rest of its row
    gran = G.MX_1x32 if kind == "mx" else G.ROW_1x128
    out = fm.rmsnorm_quantize(x.to(dev), w.to(dev), granularity=gran, pow2_scale=kind == "pow2",
                              return_transpose=True)
    _check_values(out, x, w)
    y = _np(out.y)
    if kind == "mx":
        rq, rs = ofp8.quant_mx_1x32(y)
        cq, cs = ofp8.quant_mx_32x1(y)
    else:
        rq, rs = ofp8.quant_1x128(y, pow2=kind == "pow2")
        cq, cs = ofp8.scaling_aware_transpose(rq, rs) if kind == "pow2" else ofp8.quant_128x1(y)
    assert np.array_equal(_np(out.rows.scale), rs) and np.array_equal(_np(out.rows.data), rq)
    assert np.array_equal(_np(out.cols.scale), cs) and np.array_equal(_np(out.cols.data), cq)


def test_config2_shape_and_fp32_input_and_pitch(dev):
    x, w = _inputs(8192, 2048, seed=2, spread=False)
    out = fm.rmsnorm_quantize(x.to(dev), w.to(dev), granularity=G.ROW_1x128, pow2_scale=True)
    _check_values(out, x, w)
    rq, rs = ofp8.quant_1x128(_np(out.y), pow2=True)
    assert np.array_equal(_np(out.rows.scale), rs) and np.array_equal(_np(out.rows.data), rq)
    # fp32 input and a pitched view give the same bf16 output as the bf16 input
    wide = torch.zeros(256, 2048 + 64, dtype=torch.bfloat16, device=dev)
    wide[:, :2048] = x[:256].to(dev)
    a = fm.rmsnorm_quantize(wide[:, :2048], w.to(dev))
    b = fm.rmsnorm_quantize(x[:256].to(dev).float(), w.to(dev))
    assert torch.equal(a.y, out.y[:256]) and torch.equal(b.y, out.y[:256])


def test_empty_and_single_row(dev):
    w = torch.ones(512, device=dev)
    out = fm.rmsnorm_quantize(torch.empty(0, 512, dtype=torch.bfloat16, device=dev), w, granularity=G.ROW_1x128)
    assert out.y.shape == (0, 512) and out.rows.data.shape == (0, 512)
    x, w1 = _inputs(1, 512, seed=3)
    _check_values(fm.rmsnorm_quantize(x.to(dev), w1.to(dev)), x, w1)
    with pytest.raises(ValueError):
        fm.rmsnorm_quantize(torch.zeros(4, 640, dtype=torch.bfloat16, device=dev), torch.ones(640, device=dev))


@pytest.mark.parametrize("T,D", [(1000, 2048), (37, 7168), (8192, 2048)])
def test_backward_matches_oracle(dev, T, D):
    x, w = _inputs(T, D, seed=T + D, spread=T < 8192)
    dy = randn_bf16((T, D), seed=T + D + 1, std=1e-2)
    out = fm.rmsnorm_quantize(x.to(dev), w.to(dev))
    dx, dw = fm.rmsnorm_backward(dy.to(dev), x.to(dev), w.to(dev), out.rstd)
    rdx, rdw = onorm.rmsnorm_backward(dy.float().numpy(), x.float().numpy(), w.numpy())
    assert dx.dtype == torch.bfloat16 and dw.dtype == torch.float32
    # per row: each row's dx is O(r |dy|), rows span 20 octaves
    e = np.abs(_np(dx) - rdx).max(axis=1) / np.abs(rdx).max(axis=1)
    assert e.max() < 1e-2
    assert max_rel_err(_np(dw), rdw) < 1e-4
    # without dw: same dx
    dx2, none = fm.rmsnorm_backward(dy.to(dev), x.to(dev), w.to(dev), out.rstd, need_dw=False)
    assert none is None and torch.equal(dx2, dx)


def test_module_autograd(dev):
    T, D = 300, 1024
    x, w = _inputs(T, D, seed=9)
    dy = randn_bf16((T, D), seed=10, std=1e-2)
    norm = fm.RMSNorm(D).to(dev)
    with torch.no_grad():
        norm.weight.copy_(w)
    xd = x.to(dev).requires_grad_(True)
    y = norm(xd)
    y.backward(dy.to(dev))
    rdx, rdw = onorm.rmsnorm_backward(dy.float().numpy(), x.float().numpy(), w.numpy())
    y_ref, _ = onorm.rmsnorm(x.float().numpy(), w.numpy())
    assert y.dtype == torch.bfloat16 and _ulps_bf16(_np(y), y_ref).max() <= 1
    e = np.abs(_np(xd.grad) - rdx).max(axis=1) / np.abs(rdx).max(axis=1)
    assert e.max() < 1e-2
    assert norm.weight.grad.dtype == torch.float32 and max_rel_err(_np(norm.weight.grad), rdw) < 1e-4


def test_prenorm_layer_matches_reference_ops(dev):
    """RMSNorm -> router -> BF16 experts (MoEHybridTransformerBlock's
    moe.route(moe_norm(h)) then MoEBase) against the reference op sequence in
    float64, gradients into h, the norm weight, the gate and the experts."""
    T, D, H, E, K = 512, 512, 256, 8, 2
    h, nw = _inputs(T, D, seed=31, spread=False)
    gw = randn_bf16((E, D), seed=32, std=0.05)
    gb = randn_bf16((E,), seed=33, std=0.1)
    w1, w2, w3 = (randn_bf16((E * H, D), seed=34 + s, std=0.02) for s in range(3))
    R = torch.randn(T, D, generator=torch.Generator().manual_seed(40)) * 1e-2

    leaves = [t.double().requires_grad_(True) for t in (h, nw, gw, gb, w1, w2, w3)]
    hd, nwd, gwd, gbd, a, b, c = leaves
    xn = hd * torch.rsqrt(hd.pow(2).mean(-1, keepdim=True) + 1e-6) * nwd     # model/norm.py:40-45
    xd = xn + (xn.bfloat16().double() - xn).detach()    # out.to(x.dtype), :47-48 (identity backward)
    logits = F.linear(xd, gwd, gbd)
    vals, idx = logits.topk(K, dim=-1)
    wts = F.softmax(vals, dim=-1)
    out = torch.zeros_like(xd)
    for e in range(E):
        tok = (idx == e).any(dim=-1).nonzero(as_tuple=True)[0]
        if tok.numel() == 0:
            continue
        pw = (wts[tok] * (idx[tok] == e).double()).sum(-1)
        sl = slice(e * H, (e + 1) * H)
        hh = F.silu(xd[tok] @ a[sl].T) * (xd[tok] @ c[sl].T)
        out = out.index_add(0, tok, pw[:, None] * (hh @ b[sl]))
    (out * R.double()).sum().backward()

    g = [t.to(dev).requires_grad_(True) for t in (h, nw, gw, gb, w1, w2, w3)]
    cfg = fm.FP8FlowMoEConfig(enabled=False, fp8_recipe=fm.FP8RecipeConfig(False, fm.FP8RecipeType("none")))
    layer = fm.FP8FlowMoELayer(cfg, D, H, E, K, fp8_gemm_threshold=0, pre_norm=True)
    layer.set_weights(g[2], g[3], g[4], g[5], g[6], norm_weight=g[1])
    o, _ = layer(g[0])
    (o.float() * R.to(dev)).sum().backward()
    torch.cuda.synchronize()
    assert max_rel_err(_np(o), out.detach().numpy()) < 1e-2
    for name, got, ref in zip(("h", "norm_w", "gate_w", "gate_b", "w1", "w2", "w3"), g, leaves):
        assert max_rel_err(_np(got.grad), ref.grad.numpy()) < 1e-2, name
