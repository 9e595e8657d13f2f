"""Capacity dropping and router jitter on the GPU.

* ``fm_capacity_select`` (``routing.capacity_select``) against the oracle's
  restatement of ``MoEBase._apply_capacity`` (reference
  ``model/moe.py:1395-1448``, pinned in tests/test_oracle_routing.py), bit
  for bit: positions, kept tokens, per-expert drops -- int32 and int64
  indices, out-of-range slots, no token, 2^20 tokens.
* ``fm_gather_rows`` against torch indexing, with -1 and out-of-range rows.
* The layer with a capacity factor (and a shared expert) against float64
  autograd of the reference's op sequence with the drop applied
  (``:1338-1393``: route all tokens, drop, experts and shared expert on the
  kept tokens, zeros elsewhere); adaptive capacity and the drop statistics
  against the oracle's update (``:1450-1498``) over three calls.
* Jitter (``:145-148``): a seeded training-mode layer draws the same noise
  as torch does for the reference; the router sees x + noise, the experts
  x; eval mode adds none.
* FP8 recipes (flow_moe, mxfp8) with a capacity factor: bit for bit the
  expert block run by hand on the kept tokens.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import nanopysche_amd as fm
from nanopysche_amd import routing as R
from oracle import routing as orouting
from oracle.layer import max_rel_err
from tests.helpers import randn_bf16, zipf_routing

pytestmark = pytest.mark.gpu


def _indices(T, E, K, seed):
    if T == 0:
        return np.zeros((0, K), np.int64)
    idx = zipf_routing(T, E, K, 1.1, seed=seed)[1].numpy().copy()
    idx[::101, K - 1] = -1                 # slots outside [0, E): no constraint, as the
    idx[50::211, 0] = E + 3                # reference's (indices == e) never matches them
    return idx


@pytest.mark.parametrize("T,E,K", [(0, 8, 2), (1, 4, 1), (3000, 8, 2), (5000, 16, 4), (1 << 20, 8, 2)])
@pytest.mark.parametrize("i64", [True, False])
def test_capacity_select_matches_oracle(dev, T, E, K, i64):
    print(f"capacity_select T={T} E={E} K={K} i64={i64}", flush=True)
    idx = _indices(T, E, K, seed=T + E + K)
    d = torch.from_numpy(idx).to(dev, torch.int64 if i64 else torch.int32)
    plan = fm.route_tokens(d, E)
    counts = np.bincount(idx[(idx >= 0) & (idx < E)], minlength=E)
    mean = T * K // E
    for cap in sorted({0, 1, int(mean * 0.9), int(counts.max()) - 1, int(counts.max()), T}):
        if cap < 0:
            continue
        sel = R.capacity_select(d, plan, cap)
        keep, drops, dropped = orouting.capacity_keep(idx, E, cap)
        assert sel.drops == drops.tolist() and sel.dropped == dropped, cap
        assert sel.n_kept == int(keep.sum()), cap
        want_pos = np.where(keep, np.cumsum(keep) - 1, -1)
        assert np.array_equal(sel.pos_of.cpu().numpy(), want_pos), cap
        assert np.array_equal(sel.kept_index.cpu().numpy(), np.nonzero(keep)[0]), cap


@pytest.mark.parametrize("shape,dtype", [((700, 2048), torch.bfloat16), ((333, 3), torch.float32),
                                         ((129, 4), torch.int64), ((50, 24), torch.bfloat16)])
def test_gather_rows_matches_indexing(dev, shape, dtype):
    g = torch.Generator().manual_seed(shape[0])
    src = (torch.randn(*shape, generator=g) * 100).to(dtype)
    n = shape[0] + 17
    index = torch.randint(-3, shape[0] + 3, (n,), generator=g, dtype=torch.int32)
    got = R.gather_rows(src.to(dev), index.to(dev)).cpu()
    ok = (index >= 0) & (index < shape[0])
    want = torch.zeros(n, *shape[1:], dtype=dtype)
    want[ok] = src[index[ok].long()]
    assert torch.equal(got, want)


def test_gather_rows_rejects_odd_rows(dev):
    with pytest.raises(Exception, match="multiple of 4"):
        R.gather_rows(torch.zeros(4, 3, dtype=torch.bfloat16, device=dev), torch.zeros(2, dtype=torch.int32,
                                                                                      device=dev))


def _params(T, D, H, E, Hs, seed):
    x = randn_bf16((T, D), seed=seed)
    gw = randn_bf16((E, D), seed=seed + 1, std=0.05)
    gb = randn_bf16((E,), seed=seed + 2, std=0.1)
    w = [randn_bf16((E * H, D), seed=seed + s, std=0.02) for s in (3, 4, 5)]
    ws = [randn_bf16((Hs, D), seed=seed + s, std=0.02) for s in (6, 7, 8)] if Hs else []
    g = torch.Generator().manual_seed(seed + 9)
    Rm = torch.randn(T, D, generator=g) * 1e-2
    return x, gw, gb, w, ws, Rm


def _reference(x, gw, gb, w, ws, Rm, E, K, c_aux, capacity=None, noise=None, replay=None):
    """float64 autograd of model/moe.py:1338-1393 with the router of
    :133-184 (softmax top-k, load-balancing loss), jitter noise on the
    router's input (:145-148, the noise given), capacity dropping via the
    oracle's keep mask (:1395-1448), experts (:1565-1594) and the shared
    ExpertMLP (:1181-1183) on the kept tokens, zeros for dropped ones."""
    leaves = [t.double().requires_grad_(True) for t in (x, gw, gb, *w, *ws)]
    xd, gwd, gbd, a, b, c = leaves[:6]
    xr = xd if noise is None else (x + noise).double() + (xd - xd.detach())
    logits = F.linear(xr, gwd, gbd)
    if replay is None:
        vals, idx = logits.topk(K, dim=-1)
        wts = F.softmax(vals, dim=-1)
    else:
        mask = torch.zeros_like(logits).scatter_(1, replay, 1.0)
        masked = F.softmax(logits, dim=-1) * mask
        wts, idx = (masked / masked.sum(dim=-1, keepdim=True).clamp(min=1e-8)).topk(K, dim=-1)
    T = xd.shape[0]
    f = F.one_hot(idx, E).sum(dim=1).double().sum(dim=0) / T
    aux = E * (f * F.softmax(logits, dim=-1).mean(dim=0)).sum()
    keep = torch.ones(T, dtype=torch.bool)
    if capacity is not None:
        keep = torch.from_numpy(orouting.capacity_keep(idx.numpy(), E, capacity)[0])
    H = a.shape[0] // E
    out = torch.zeros_like(xd)
    for e in range(E):
        tok = ((idx == e).any(dim=-1) & keep).nonzero(as_tuple=True)[0]
        if tok.numel() == 0:
            continue
        pw = (wts[tok] * (idx[tok] == e).double()).sum(-1)
        sl = slice(e * H, (e + 1) * H)
        h = F.silu(xd[tok] @ a[sl].T) * (xd[tok] @ c[sl].T)
        out = out.index_add(0, tok, pw[:, None] * (h @ b[sl]))
    if ws:
        s1, s2, s3 = leaves[6:]
        sh = (F.silu(xd @ s1.T) * (xd @ s3.T)) @ s2
        out = out + sh * keep[:, None].double()
    ((out * Rm.double()).sum() + c_aux * aux).backward()
    return out.detach(), aux.detach(), [t.grad for t in leaves], keep


def _layer(D, H, E, K, Hs=None, **kw):
    cfg = fm.FP8FlowMoEConfig(enabled=False, fp8_recipe=fm.FP8RecipeConfig(False, fm.FP8RecipeType("none")))
    return fm.FP8FlowMoELayer(cfg, D, H, E, K, fp8_gemm_threshold=0, shared_hidden_size=Hs, **kw)


def _run(dev, layer, x, gw, gb, w, ws, Rm, c_aux, replay=None):
    leaves = [t.to(dev).requires_grad_(True) for t in (x, gw, gb, *w, *ws)]
    layer.set_weights(leaves[1], leaves[2], *leaves[3:6], shared=tuple(leaves[6:]) if ws else None)
    out, aux = layer(leaves[0], replay_indices=replay)
    ((out.float() * Rm.to(dev)).sum() + c_aux * aux).backward()
    torch.cuda.synchronize()
    return out, aux, leaves


NAMES = ("x", "gate_w", "gate_b", "w1", "w2", "w3", "s1", "s2", "s3")


def _check(out, aux, leaves, ref_out, ref_aux, ref_grads, tol=1e-2):
    assert max_rel_err(out.detach().float().cpu().numpy(), ref_out.numpy()) < tol
    assert abs(float(aux.detach()) - float(ref_aux)) < 1e-5 * float(ref_aux)
    for name, got, ref in zip(NAMES, leaves, ref_grads):
        err = max_rel_err(got.grad.float().cpu().numpy(), ref.numpy())
        assert err < tol, (name, err)


@pytest.mark.parametrize("cf,Hs", [(2.0, None), (1.25, 256), (8.0, None)])
def test_layer_with_capacity_matches_reference_ops(dev, cf, Hs):
    print(f"capacity layer cf={cf} shared={Hs}", flush=True)
    T, D, H, E, K = 600, 256, 256, 8, 2
    x, gw, gb, w, ws, Rm = _params(T, D, H, E, Hs, seed=31)
    capacity = int(cf * T / E)
    ref_out, ref_aux, ref_grads, keep = _reference(x, gw, gb, w, ws, Rm, E, K, 0.5, capacity=capacity)
    layer = _layer(D, H, E, K, Hs, capacity_factor=cf)
    out, aux, leaves = _run(dev, layer, x, gw, gb, w, ws, Rm, 0.5)
    _check(out, aux, leaves, ref_out, ref_aux, ref_grads)
    dropped_rows = (~keep).nonzero(as_tuple=True)[0]
    assert torch.count_nonzero(out.detach().cpu()[dropped_rows]) == 0
    st = layer.get_drop_stats()
    assert st["total_tokens_routed"] == T and st["last_dropped"] == st["total_dropped"]
    assert (st["last_dropped"] > 0) == (cf < 8.0) and st["capacity_factor"] == cf
    assert sum(st["per_expert_drops"]) == st["last_dropped"]
    assert st["drop_rate"] == st["total_dropped"] / T


def test_adaptive_capacity_follows_the_oracle(dev):
    """Three calls with replayed routing (the experts of each token fixed, so
    the oracle sees the same sets): capacity factor, EMA, step and the drop
    counts after each call."""
    T, D, H, E, K = 512, 256, 256, 8, 2
    x, gw, gb, w, ws, Rm = _params(T, D, H, E, None, seed=41)
    layer = _layer(D, H, E, K, capacity_factor=1.0, adaptive_capacity=True, adaptive_capacity_target=0.01)
    leaves = [t.to(dev) for t in (x, gw, gb, *w)]
    layer.set_weights(leaves[1], leaves[2], *leaves[3:6])
    cf, ema, step, total = 1.0, 0.0, 0, 0
    for call in range(3):
        rep = zipf_routing(T, E, K, 1.3, seed=50 + call)[1]
        with torch.no_grad():
            layer(leaves[0], replay_indices=rep.to(dev))
        cf, ema, step = orouting.adaptive_capacity_update(cf, ema, step, rep.numpy(), E, 0.01, 0.3)
        _, drops, dropped = orouting.capacity_keep(rep.numpy(), E, int(cf * T / E))
        total += dropped
        st = layer.get_drop_stats()
        assert st["capacity_factor"] == cf and st["adaptive_capacity_step"] == step
        assert abs(st["adaptive_drop_rate_ema"] - ema) < 1e-12
        assert st["per_expert_drops"] == drops.tolist() and st["total_dropped"] == total
    layer.reset_drop_stats()
    assert layer.get_drop_stats()["total_dropped"] == 0 and layer.per_expert_drops is None


@pytest.mark.parametrize("capacity", [False, True])
def test_jitter_draws_torch_noise_for_the_router(dev, capacity):
    print(f"jitter capacity={capacity}", flush=True)
    T, D, H, E, K, eps = 600, 256, 256, 8, 2, 0.05
    x, gw, gb, w, ws, Rm = _params(T, D, H, E, None, seed=61)
    kw = dict(capacity_factor=2.0) if capacity else {}
    layer = _layer(D, H, E, K, jitter_eps=eps, **kw)
    torch.cuda.manual_seed(1234)
    out, aux, leaves = _run(dev, layer, x, gw, gb, w, ws, Rm, 0.5)
    torch.cuda.manual_seed(1234)
    noise = (torch.randn_like(x.to(dev)) * eps).cpu()      # MoERouter.forward's draw, :146
    cap = int(2.0 * T / E) if capacity else None
    ref_out, ref_aux, ref_grads, _ = _reference(x, gw, gb, w, ws, Rm, E, K, 0.5, capacity=cap, noise=noise)
    _check(out, aux, leaves, ref_out, ref_aux, ref_grads)
    # eval mode: no noise
    layer.eval()
    out_e, aux_e, leaves_e = _run(dev, layer, x, gw, gb, w, ws, Rm, 0.5)
    ref_out, ref_aux, ref_grads, _ = _reference(x, gw, gb, w, ws, Rm, E, K, 0.5, capacity=cap)
    _check(out_e, aux_e, leaves_e, ref_out, ref_aux, ref_grads)


@pytest.mark.parametrize("recipe", ["flow_moe", "mxfp8"])
def test_fp8_layer_with_capacity_is_the_block_on_kept_tokens(dev, recipe):
    """With an FP8 recipe the capacity path is route() on every token, the
    oracle's keep mask on the routed experts, and FP8FlowMoECompute on the
    kept tokens' rows, weights and experts with zeros elsewhere (reference
    model/moe.py:1351-1356, :1386-1391): the same kernels on the same inputs,
    so the output and the expert-weight gradients match bit for bit."""
    T, D, H, E, K = 1024, 512, 256, 8, 2
    x, gw, gb, w, _, Rm = _params(T, D, H, E, None, seed=71)
    cfg = fm.FP8FlowMoEConfig(enabled=True, fp8_recipe=fm.FP8RecipeConfig(True, fm.FP8RecipeType(recipe)))
    layer = fm.FP8FlowMoELayer(cfg, D, H, E, K, fp8_gemm_threshold=0, capacity_factor=1.25)
    out, aux, leaves = _run(dev, layer, x, gw, gb, w, [], Rm, 0.5)
    assert layer.get_drop_stats()["last_dropped"] > 0

    ref = [t.to(dev).requires_grad_(True) for t in (x, gw, gb, *w)]
    wts, idx, aux_r = fm.route(ref[0], ref[1], ref[2], top_k=K)
    keep = torch.from_numpy(orouting.capacity_keep(idx.cpu().numpy(), E, int(1.25 * T / E))[0]).to(dev)
    block = fm.FP8FlowMoECompute(cfg, D, H, E, 0)
    block.set_weights(*ref[3:6])
    out_k = block(ref[0][keep], wts[keep], idx[keep])
    out_r = torch.zeros(T, D, dtype=out_k.dtype, device=dev).index_put((keep.nonzero(as_tuple=True)[0],), out_k)
    ((out_r.float() * Rm.to(dev)).sum() + 0.5 * aux_r).backward()
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), out_r.detach()) and torch.equal(aux.detach(), aux_r.detach())
    for name, a, b in zip(("x", "gate_w", "gate_b", "w1", "w2", "w3"), leaves, ref):
        assert torch.allclose(a.grad.float(), b.grad.float(), rtol=1e-6, atol=0), name
