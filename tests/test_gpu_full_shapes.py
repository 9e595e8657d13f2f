"""Expert-block parity at configs[3] and configs[4]'s own dimensions:

* configs[3] (D=4096, E=8, top-2, H=14336, Zipf(1.1) Gumbel-top-2 routing)
  at 512 tokens per expert on average, FP8 flow_moe (threshold 0) and BF16:
  the whole forward and every gradient against the CPU oracles (FP8:
  ``oracle.layer.moe_flow_reference``, stage-synchronised, within 2e-2;
  BF16: the reference's per-expert loop ``model/moe.py:1542-1596`` within
  1e-2), and the [K][N] / split weight operands against the transposed
  weight copies bit for bit;
* configs[3] at 4096 tokens per expert (T=16384, 32,768 assignments; buffers
  of several GiB, the 112-step K loops of the down and dX GEMMs at full
  depth) and configs[4] (D=7168, H=2048, 32 local experts of 256, sigmoid
  top-8 with a Zipf(1.2) bias, 65,536 local assignments, one expert holding
  most of them, two with none, MXFP8): sampled checks free-running against
  ``oracle.layer.moe_flow_sampled`` -- the output, input gradient and
  router-weight gradient of sampled tokens and 128 x 128 blocks of dW1, dW2,
  dW3 of the most loaded, the least loaded and a middle expert -- within
  2e-2 (FP8) / 1e-2 (BF16, against the BF16 grouped dataflow), exact zeros for
  the experts without tokens and for other ranks' slots.

Reference: model/moe.py:153-162, :257-265 (sigmoid routing with score bias),
:1542-1596 (the expert loop), :1560-1565 (local experts only); README.md:71-85
(the configs[3] crossover).  Inputs are drawn on the device from seeded
generators; each case runs the oracle once on the host (tens of seconds)."""

import numpy as np
import pytest
import torch

import nanopysche_amd as fm
from bench import C5_SHAPE, c5_routing, device_normal, zipf_gumbel_topk
from nanopysche_amd.flow_moe import ExpertWeights
from oracle import layer as olayer
from oracle import routing as orouting

pytestmark = pytest.mark.gpu

FP8_TOL = 2e-2
BF16_TOL = 1e-2
GRADS = ("x", "weights", "w1", "w2", "w3")
C4 = dict(D=4096, E=8, K=2, H=14336)


def _flush(msg):
    print(msg, flush=True)


def _run(x, w, idx, w1, w2, w3, go, E, recipe, taps=None, expert_offset=0):
    """Forward + backward of the expert block on device tensors; fresh leaves
    share the callers' storage.  Returns the device results."""
    D = x.shape[1]
    H = w1.shape[0] // E
    on = recipe != "none"
    cfg = fm.FP8FlowMoEConfig(enabled=on, fp8_recipe=fm.FP8RecipeConfig(on, fm.FP8RecipeType(recipe)))
    blk = fm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=0)
    blk.capture_intermediates = taps
    p = [t.detach().requires_grad_(True) for t in (w1, w2, w3)]
    blk.set_weights(*p)
    xd = x.detach().requires_grad_(True)
    wd = w.detach().requires_grad_(True)
    out = blk(xd, wd, idx, expert_offset, E)
    out.backward(go)
    torch.cuda.synchronize()
    got = {"out": out.detach()}
    for name, t in zip(GRADS, (xd, wd, *p)):
        got[name] = t.grad
    return got


def _host(t):
    return t.detach().float().cpu().numpy()


# ------------------------------------------------------------ configs[3] ----
@pytest.fixture(scope="module")
def c4_weights(dev):
    D, E, H = C4["D"], C4["E"], C4["H"]
    gen = torch.Generator(device=dev).manual_seed(3)
    return [device_normal((E * H, D), 0.02, gen, dev, torch.bfloat16) for _ in range(3)]


def _c4_tokens(t_per_expert, dev, seed):
    D, E, K = C4["D"], C4["E"], C4["K"]
    T = 4 * t_per_expert
    w, idx = zipf_gumbel_topk(T, E, K, 1.1, seed=3)
    gen = torch.Generator(device=dev).manual_seed(seed)
    x = device_normal((T, D), 1.0, gen, dev, torch.bfloat16)
    go = device_normal((T, D), 1e-2, gen, dev, torch.bfloat16)
    return x, w.to(dev), idx.to(dev), go


@pytest.mark.timeout(900)
@pytest.mark.parametrize("recipe", ["flow_moe", "none"])
def test_c4_full_dims_against_oracle(dev, c4_weights, recipe):
    """512 tokens per expert on average (T=2048); experts hold ~100 to ~1300 rows."""
    E = C4["E"]
    x, w, idx, go = _c4_tokens(512, dev, seed=30)
    w1, w2, w3 = c4_weights
    _flush(f"configs[3] D=4096 H=14336 T=2048 recipe={recipe}: device")
    taps = {} if recipe == "flow_moe" else None
    got = _run(x, w, idx, w1, w2, w3, go, E, recipe, taps=taps)
    # the [K][N] and split weight operands give the transposed copies' bits
    ExpertWeights.KMAJOR = False
    try:
        alt = _run(x, w, idx, w1, w2, w3, go, E, recipe)
    finally:
        ExpertWeights.KMAJOR = True
    for k in got:
        assert torch.equal(got[k], alt[k]), k
    del alt
    _flush("oracle")
    host = [t.cpu() for t in (x, w, idx, w1, w2, w3, go)]
    if recipe == "flow_moe":
        taps = {k: _host(v) for k, v in taps.items()}
        ref_out, ref_grads = olayer.moe_flow_reference(*host[:6], E, host[6], recipe="flow_moe", taps=taps)
        tol = FP8_TOL
    else:
        ref_out, ref_grads = olayer.moe_bf16_loop(*host[:6], E, host[6])
        ref_out = ref_out.numpy()
        ref_grads = {k: v.numpy() for k, v in ref_grads.items()}
        tol = BF16_TOL
    errs = {"out": olayer.max_rel_err(_host(got["out"]), ref_out)}
    for k in GRADS:
        errs[k] = olayer.max_rel_err(_host(got[k]), ref_grads[k])
    _flush(f"errors {errs}")
    assert max(errs.values()) <= tol, errs


def _sample_experts(counts):
    """The most loaded, the least loaded non-empty and a middle expert."""
    order = [int(e) for e in np.argsort(counts, kind="stable") if counts[e] > 0]
    return sorted({order[-1], order[0], order[len(order) // 2]})


def _sample_tokens(idx_local, E, experts, n, seed):
    """Up to n tokens whose local slots all lie in ``experts`` (and at least one does)."""
    inside = np.isin(idx_local, experts)
    local = (idx_local >= 0) & (idx_local < E)
    ok = np.nonzero(np.all(inside | ~local, axis=1) & inside.any(axis=1))[0]
    rng = np.random.default_rng(seed)
    pick = rng.choice(ok, size=min(n, ok.size), replace=False)
    return np.sort(pick)


def _sample_blocks(experts, H, D):
    """Per expert: first, last and a middle hidden block against first, last
    and a middle model block, for each of w1, w2, w3."""
    nh, nd = H // 128, D // 128
    out = []
    for i, e in enumerate(experts):
        for name, (bi, bj) in zip(("w1", "w2", "w3"), ((0, nd - 1), (nh - 1, 0), (nh // 2 + i, nd // 2 - i))):
            out.append((name, e, bi, bj))
    return out


def _check_sampled(got, host, E, recipe, tokens, blocks, tol, expert_offset=0):
    x, w, idx, w1, w2, w3, go = host
    idx_l = idx - expert_offset
    s_out, s_g = olayer.moe_flow_sampled(x, w, idx_l, w1, w2, w3, E, go,
                                         None if recipe == "none" else recipe, tokens, blocks)
    ti = torch.from_numpy(tokens)
    H = w1.shape[0] // E
    errs = {"out": olayer.max_rel_err(_host(got["out"].index_select(0, ti.to(got["out"].device))), s_out),
            "x": olayer.max_rel_err(_host(got["x"].index_select(0, ti.to(got["x"].device))), s_g["x"]),
            "weights": olayer.max_rel_err(_host(got["weights"].index_select(0, ti.to(got["x"].device))),
                                          s_g["weights"])}
    for name in ("w1", "w2", "w3"):
        sel = [i for i, b in enumerate(blocks) if b[0] == name]
        dev_blocks = np.stack([_host(got[name][e * H + bi * 128:e * H + bi * 128 + 128, bj * 128:bj * 128 + 128])
                               for _, e, bi, bj in (blocks[i] for i in sel)])
        errs[name] = olayer.max_rel_err(dev_blocks, s_g["blocks"][sel])
    _flush(f"sampled errors {errs}")
    assert max(errs.values()) <= tol, errs


@pytest.mark.timeout(900)
@pytest.mark.parametrize("recipe", ["flow_moe", "none"])
def test_c4_full_size_sampled(dev, c4_weights, recipe):
    """4096 tokens per expert on average (T=16384, A=32768)."""
    D, E, H = C4["D"], C4["E"], C4["H"]
    x, w, idx, go = _c4_tokens(4096, dev, seed=31)
    w1, w2, w3 = c4_weights
    _flush(f"configs[3] T=16384 recipe={recipe}: device")
    got = _run(x, w, idx, w1, w2, w3, go, E, recipe)
    _flush("oracle (sampled)")
    host = [t.cpu() for t in (x, w, idx, w1, w2, w3, go)]
    counts = np.bincount(host[2].numpy().reshape(-1), minlength=E)
    experts = _sample_experts(counts)
    tokens = _sample_tokens(host[2].numpy(), E, experts, 48, seed=5)
    assert tokens.size >= 16
    blocks = _sample_blocks(experts, H, D)
    _check_sampled(got, host, E, recipe, tokens, blocks, FP8_TOL if recipe != "none" else BF16_TOL)


# ------------------------------------------------------------ configs[4] ----
@pytest.mark.timeout(900)
def test_c5_full_size_sampled(dev):
    D, E, K, H = (C5_SHAPE[k] for k in ("D", "E_local", "K", "H"))
    gen = torch.Generator(device=dev).manual_seed(4)
    w, idx, A = c5_routing(dev, gen)
    T = idx.shape[0]
    x = device_normal((T, D), 1.0, gen, dev, torch.bfloat16)
    go = device_normal((T, D), 1e-2, gen, dev, torch.bfloat16)
    w1, w2, w3 = [device_normal((E * H, D), 0.02, gen, dev, torch.bfloat16) for _ in range(3)]
    assert A == C5_SHAPE["A_target"]
    _flush(f"configs[4] T={T} A={A} MXFP8: device")
    got = _run(x, w, idx, w1, w2, w3, go, E, "mxfp8")
    idx_h = idx.cpu().numpy()
    local = idx_h < E
    counts = np.bincount(idx_h[local], minlength=E)
    assert counts.sum() == A and counts[5] == 0 and counts[17] == 0 and counts.max() > A // 2
    # other ranks' slots: exactly zero router-weight gradient; experts without
    # tokens: exactly zero weight gradients
    dwt = got["weights"].cpu().numpy()
    assert np.all(dwt[~local] == 0)
    for name in ("w1", "w2", "w3"):
        g = got[name].view(E, H, D)
        assert int(torch.count_nonzero(g[[5, 17]])) == 0, name
    _flush("oracle (sampled)")
    host = [t.cpu() for t in (x, w, idx, w1, w2, w3, go)]
    experts = _sample_experts(counts)
    tokens = _sample_tokens(idx_h, E, experts, 32, seed=6)
    assert tokens.size >= 8
    blocks = _sample_blocks(experts, H, D) + [("w1", 5, 3, 7), ("w2", 17, 0, 55)]
    _check_sampled(got, host, E, "mxfp8", tokens, blocks, FP8_TOL)
