"""Benchmark of the fp8_flow_moe expert block on one MI355X.

Default workload (the metric's configuration): T=8192
tokens, d_model=2048, 8 experts, top-2, SwiGLU ffn_hidden=1408, exactly
balanced routing (2048 assignments per expert, router weights = softmax of
seeded logits at those indices), FP8 GEMMs forced (threshold 0), recipe
flow_moe (1x128 / 128x128 power-of-two scales).  One step = expert-block
forward + backward, including the routing sort, all quantisation and the
re-quantisation of the expert weights (their cache is dropped every step, as
after an optimizer update).  Inputs are resident in HBM before timing starts.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--recipe flow_moe]
    python bench.py --workload c1|c2|c4|c5    # the other configs, one JSON line each
    python bench.py --workload shared         # shared expert / dense SwiGLU FFN at configs[2]'s shapes

Prints one JSON line.  --gpus > 1 is refused: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
PEAK_TFLOPS = {"fp8": 5000.0, "bf16": 2500.0}


def synthetic_inputs(T, D, H, E, K, seed, dev):
    """configs[2] inputs: balanced routing, weights N(0, 0.02), upstream grad N(0, 1e-2)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g).bfloat16()
    logits = torch.randn(T, E, generator=g)
    # exactly balanced: token t -> experts (t mod E, (t + E/2) mod E)
    t = torch.arange(T)
    idx = torch.stack([(t % E), ((t + E // 2) % E)], dim=1)[:, :K].contiguous()
    w = torch.softmax(torch.gather(logits, 1, idx), dim=-1)
    w1, w2, w3 = [(torch.randn(E * H, D, generator=g) * 0.02).bfloat16() for _ in range(3)]
    go = (torch.randn(T, D, generator=g) * 1e-2).bfloat16()
    return [a.to(dev) for a in (x, w, idx, w1, w2, w3, go)]


def router_params(D, E, seed, dev):
    """Router gate of configs[2]: nn.Linear(D, E, bias=True) weight and bias
    N(0, 0.02) (bf16 parameters, as the reference's model under bf16)."""
    import torch

    g = torch.Generator().manual_seed(seed + 1000)
    gw = (torch.randn(E, D, generator=g) * 0.02).bfloat16()
    gb = (torch.randn(E, generator=g) * 0.02).bfloat16()
    return gw.to(dev), gb.to(dev)


def device_normal(shape, std, gen, dev, dtype):
    import torch

    return (torch.randn(*shape, generator=gen, device=dev) * std).to(dtype)


class GemmTimer:
    """Records HIP events around every grouped-GEMM launch on the launch stream."""

    def __init__(self):
        self.records = []

    def __call__(self, name, flops, fn):
        import torch

        s = torch.cuda.current_stream()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        fn()
        b.record(s)
        self.records.append((name, flops, a, b))

    def summary(self):
        import torch

        torch.cuda.synchronize()
        out = {}
        for name, flops, a, b in self.records:
            ms = a.elapsed_time(b)
            d = out.setdefault(name, {"launches": 0, "ms": 0.0, "flops": 0.0})
            d["launches"] += 1
            d["ms"] += ms
            d["flops"] += flops
        return out


GRAPH_ERRORS = []


def time_graphed(step, leaves, steps, warmup):
    """ms per replay of `step` captured as a HIP graph (GraphedStep), or None
    (with the reason kept in GRAPH_ERRORS) if the capture raised."""
    import torch

    import nanopysche_amd as fm

    try:
        gstep = fm.GraphedStep(step, leaves, warmup=2)
    except RuntimeError as e:
        GRAPH_ERRORS.append(str(e).splitlines()[0][:200])
        torch.cuda.synchronize()
        return None
    for _ in range(warmup):
        gstep.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        gstep.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def launch_note(args):
    if args.eager:
        return "eager"
    if GRAPH_ERRORS:
        return "eager (HIP graph capture failed: " + GRAPH_ERRORS[-1] + ")"
    return "hip_graph: the step captured once, replayed per step"


def time_layer(x, w, idx, w1, w2, w3, go, E, recipe, threshold, steps, warmup, backward=True,
               gemm_timer=True, pre_step=None, overlap=True, router=None, graph=False):
    """Times `steps` calls of the expert block (forward, + backward when
    `backward`), weight cache dropped every step, with nothing recorded between
    the launches.  With `router` = (gate weight, gate bias, top_k, gating[,
    replay]) the step is the MoE layer (FP8FlowMoELayer): the router (gate
    GEMM, gating -- with `idx` replayed as an R3 routing mask unless replay is
    False --, expert counts, load-balancing loss) and the expert block, and the
    backward takes out * go + aux loss through both (the Trainer's
    `loss + aux_loss`, reference train/trainer.py:320-339).  With `gemm_timer`,
    a second pass of `steps` identical steps then records HIP events around
    every grouped-GEMM launch, on one stream so that no other kernel runs
    beside the one timed (each event record leaves a few-microsecond bubble in
    the stream, so this pass is not the one the step time comes from).
    With `graph` the step is then captured once as a HIP graph
    (nanopysche_amd.GraphedStep: every kernel of the step, weight
    re-quantisation included, with no host work between launches) and `steps`
    replays are timed; the eager step time is returned beside it.
    Returns (ms per step, GEMM event summary or None, eager ms per step)."""
    if pre_step is not None and graph:
        raise ValueError("a graphed step takes no per-step host input")
    import torch

    import nanopysche_amd as fm
    from nanopysche_amd import flow_moe as fmm

    D = x.shape[1]
    H = w1.shape[0] // E
    cfg = fm.FP8FlowMoEConfig(enabled=True, fp8_recipe=fm.FP8RecipeConfig(True, fm.FP8RecipeType(recipe)))
    blk = fm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=threshold)
    blk.overlap_streams = overlap
    params = [t.detach().clone().requires_grad_(backward) for t in (w1, w2, w3)]
    blk.set_weights(*params)
    xr = x.detach().clone().requires_grad_(backward)
    wr = w.detach().clone().requires_grad_(backward)
    gparams = []
    layer = None
    if router is not None:
        # the MoE layer: router + expert block under one autograd node
        gparams = [t.detach().clone().requires_grad_(backward) for t in router[:2]]
        layer = fm.FP8FlowMoELayer(cfg, D, H, E, router[2], gating=router[3], fp8_gemm_threshold=threshold)
        layer.set_weights(*gparams, *params)
        layer.block.overlap_streams = overlap
        blk = layer.block
    one = torch.ones((), device=x.device)
    replay = idx if (router is None or len(router) <= 4 or router[4]) else None

    def step():
        blk._cache.clear()  # weights change every training step: re-quantise them
        if backward:
            for p in params + gparams:
                p.grad = None
            xr.grad = None
            wr.grad = None
            if layer is not None:
                out, aux = layer(xr, replay_indices=replay)
                torch.autograd.backward([out, aux], [go, one])
            else:
                r_w, r_idx = (wr, idx) if pre_step is None else pre_step()
                blk(xr, r_w, r_idx, 0, E).backward(go)
        else:
            with torch.no_grad():
                if layer is not None:
                    layer(xr, replay_indices=replay)
                else:
                    r_w, r_idx = (wr, idx) if pre_step is None else pre_step()
                    blk(xr, r_w, r_idx, 0, E)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    eager_ms = elapsed * 1e3 / steps
    if graph:
        leaves = (params + gparams + [xr] + ([] if layer is not None else [wr])) if backward else []
        graph_ms = time_graphed(step, leaves, steps, warmup)
        if graph_ms is not None:
            elapsed = graph_ms * steps / 1e3
    summary = None
    if gemm_timer:
        timer = GemmTimer()
        fmm.GEMM_TIMER = timer
        blk.overlap_streams = False
        try:
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
        finally:
            fmm.GEMM_TIMER = None
            blk.overlap_streams = overlap
        summary = timer.summary()
    return elapsed * 1e3 / steps, summary, eager_ms


def gemm_report(summ, steps, flops_scale=1.0):
    """GEMM event totals per step.  The timer counts 2*T*K*N*K' FLOPs per launch
    (every routing slot); `flops_scale` = valid assignments / (T*K) corrects
    that when some slots point outside the local experts."""
    gemm_ms = sum(v["ms"] for v in summ.values()) / steps
    kernels = {k: {"avg_us": round(v["ms"] * 1e3 / v["launches"], 2),
                   "tflops": round(v["flops"] * flops_scale / (v["ms"] * 1e-3) / 1e12, 1),
                   "launches_per_step": v["launches"] // steps} for k, v in summ.items()}
    flops = sum(v["flops"] for v in summ.values()) * flops_scale / steps
    return {"tflops_all_gemms": round(flops / (gemm_ms * 1e-3) / 1e12, 1),
            "gemm_ms_per_step": round(gemm_ms, 4), "kernels": kernels}


def recorded_traffic(kernel, recipe):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, calibrated against a plain copy), or
    None when no summary for this kernel and recipe is committed."""
    path = ROOT / "profiles" / "c3_hbm_traffic.json"
    try:
        rec = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    ent = rec.get("kernels", {}).get(kernel)
    if ent is None or rec.get("recipe") != recipe:
        return None
    return {"bytes_per_launch": ent["hbm_bytes_per_launch"], "source": "profiles/c3_hbm_traffic.json"}


def hbm_kernels_c3(x, w, idx, w1, w2, w3, go, E, H, reps=20):
    """The HBM-bound kernels of one flow_moe step at configs[2]'s shapes, each
    timed alone: `reps` launches back to back between two HIP events (C ABI
    called directly with preallocated outputs, so host overhead stays below
    the kernel time).  Algorithmic bytes: every input tensor read once at its
    size (the gathered x counted once per token, not per assignment), every
    output written once."""
    import torch

    import nanopysche_amd as fm
    from nanopysche_amd import _lib
    from nanopysche_amd.flow_moe import ExpertWeights, _alloc_quant, _tile_args

    dev = x.device
    T, D = x.shape
    K = idx.shape[1]
    P2 = _lib.QUANT_POW2
    plan = fm.route_tokens(idx, E, 0)
    R = plan.rows_max
    gen = torch.Generator(device=dev).manual_seed(5)
    GU = device_normal((R, 2 * H), 1.0, gen, dev, torch.bfloat16)
    dH = device_normal((R, H), 0.01, gen, dev, torch.bfloat16)
    Y = device_normal((R, D), 1.0, gen, dev, torch.bfloat16)
    wts = w.reshape(-1).to(torch.float32).contiguous()
    st = _lib.stream_of(x)

    def nb(*ts):
        return sum(t.numel() * t.element_size() for t in ts if t is not None)

    # buffers of the padded expert layout hold R = rows_max rows, of which the
    # producers write (and the consumers read) only the offsets[E] rows of
    # the expert groups: count those
    R_used = int(plan.offsets[-1].item())

    def nbq(*ts):
        return nb(*ts) * R_used // R

    pq = _alloc_quant(R, D, P2, True, True, dev, True)
    sq = _alloc_quant(R, H, P2, True, True, dev, True)
    gq = _alloc_quant(R, 2 * H, P2, True, True, dev, True)
    out = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    ew = ExpertWeights(P2)
    ew._build(w1, w2, w3, E)
    wouts = {o.data.data_ptr(): o for o in (ew.w13, ew.w13t, ew.w2, ew.w2t)}   # [K][N] operands alias the rows
    wbytes = nb(w1, w2, w3) + sum(nb(o.data, o.scale) for o in wouts.values())

    # RMSNorm ahead of the MoE on the residual stream (x stands in for it)
    nw = torch.ones(D, dtype=torch.float32, device=dev)
    ny = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    nq = torch.empty(T, D, dtype=torch.uint8, device=dev)
    ns = torch.empty(T, D // 128, dtype=torch.float32, device=dev)
    nr = torch.empty(T, dtype=torch.float32, device=dev)
    ndx = torch.empty_like(ny)
    ndw = torch.empty(D, dtype=torch.float32, device=dev)
    nws = torch.empty(int(_lib.load().fm_rmsnorm_backward_workspace_bytes(T, D)) // 4, dtype=torch.float32,
                      device=dev)
    _lib.call("fm_rmsnorm_quantize", _lib.ptr(x), _lib.DTYPE_BF16, x.stride(0), T, D, _lib.ptr(nw), _lib.DTYPE_F32,
              1e-6, None, 0, -1, None, 0, None, 0, _lib.ptr(nr), st)

    ops = [
        ("RMSNorm + quantise (residual stream -> bf16 y + e4m3 row blocks, pow2, + rsqrt)",
         lambda: _lib.call("fm_rmsnorm_quantize", _lib.ptr(x), _lib.DTYPE_BF16, x.stride(0), T, D, _lib.ptr(nw),
                           _lib.DTYPE_F32, 1e-6, _lib.ptr(ny), D, P2, _lib.ptr(nq), D, _lib.ptr(ns), D // 128,
                           _lib.ptr(nr), st), nb(x, nw, ny, nq, ns, nr)),
        ("RMSNorm backward (dx + dw)",
         lambda: _lib.call("fm_rmsnorm_backward", _lib.ptr(go), go.stride(0), _lib.ptr(x), _lib.DTYPE_BF16,
                           x.stride(0), T, D, _lib.ptr(nw), _lib.DTYPE_F32, _lib.ptr(nr), _lib.ptr(ndx), D,
                           _lib.ptr(ndw), _lib.DTYPE_F32, _lib.ptr(nws), nws.numel() * 4, st),
         nb(go, x, nw, nr, ndx, ndw)),
        ("permute + quantise (x rows, row + transposed, pow2)",
         lambda: _lib.call("fm_permute", _lib.ptr(x), T, D, x.stride(0), _lib.ptr(plan.assign_of_row), R, K, None,
                           *_tile_args(P2, *pq), _lib.ptr(plan.tile_expert), st), nb(x) + nbq(*pq)),
        ("permute + quantise (dY rows x router weight)",
         lambda: _lib.call("fm_permute", _lib.ptr(go), T, D, go.stride(0), _lib.ptr(plan.assign_of_row), R, K,
                           _lib.ptr(wts), *_tile_args(P2, *pq), _lib.ptr(plan.tile_expert), st),
         nb(go, wts) + nbq(*pq)),
        ("SwiGLU + quantise (row + transposed)",
         lambda: _lib.call("fm_swiglu_quantize", _lib.ptr(GU), GU.stride(0), _lib.ptr(GU[:, H:]), GU.stride(0), R, H,
                           *_tile_args(P2, *sq), _lib.ptr(plan.tile_expert), st), nbq(GU, *sq)),
        ("SwiGLU backward + quantise (dg|du row + transposed)",
         lambda: _lib.call("fm_swiglu_backward", _lib.ptr(GU), GU.stride(0), _lib.ptr(GU[:, H:]), GU.stride(0),
                           _lib.ptr(dH), dH.stride(0), R, H, *_tile_args(P2, *gq), _lib.ptr(plan.tile_expert), st),
         nbq(GU, dH, *gq)),
        ("unpermute (weighted sum over top-k)",
         lambda: _lib.call("fm_unpermute", _lib.ptr(Y), Y.stride(0), _lib.ptr(plan.row_of), _lib.ptr(wts), T, K, D,
                           _lib.ptr(out), _lib.DTYPE_BF16, out.stride(0), None, 0, st), nbq(Y) + nb(wts, out)),
        ("expert weight re-quantisation (w1, w3, w2 in one launch, 128x128 pow2 "
         + ("rows; the down and dX GEMMs read them as [K][N])" if ew.w2t.kmajor else "+ transposed)"),
         lambda: ew._build(w1, w2, w3, E), wbytes),
    ]
    return time_hbm_ops(ops, reps)


def time_hbm_ops(ops, reps):
    """(name, launch, algorithmic bytes) -> one dict per op: `reps` launches
    back to back between two events on the current stream, after 3 untimed."""
    import torch

    results = []
    for name, fn, nbytes in ops:
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps
        gbs = nbytes / (us * 1e-6) / 1e9
        results.append({"op": name, "us": round(us, 2), "bytes": int(nbytes), "GB_s": round(gbs, 1),
                        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
    return results


def hbm_kernels_c5(x, w, idx, w1, w2, w3, go, E, H, reps=5):
    """The HBM-bound kernels of one MXFP8 expert-block step at configs[4]'s
    shapes, each timed alone as in hbm_kernels_c3 (C ABI, preallocated
    outputs, paired-row operands as the block writes them).  Slots of other
    ranks' experts (index E_global) move no bytes: the gathered rows are the
    local assignments' rows."""
    import torch

    import nanopysche_amd as fm
    from nanopysche_amd import _lib
    from nanopysche_amd.flow_moe import ExpertWeights, _alloc_quant, _tile_args

    dev = x.device
    T, D = x.shape
    K = idx.shape[1]
    MX = _lib.QUANT_MX
    plan = fm.route_tokens(idx, E, 0)
    R = plan.rows_max
    R_used = int(plan.offsets[-1].item())
    A = int(plan.counts.sum().item())
    gen = torch.Generator(device=dev).manual_seed(5)
    GU = device_normal((R, 2 * H), 1.0, gen, dev, torch.bfloat16)
    dH = device_normal((R, H), 0.01, gen, dev, torch.bfloat16)
    Y = device_normal((R, D), 1.0, gen, dev, torch.bfloat16)
    wts = w.reshape(-1).to(torch.float32).contiguous()
    st = _lib.stream_of(x)

    def nb(*ts):
        return sum(t.numel() * t.element_size() for t in ts if t is not None)

    def nbq(*ts):   # padded-layout buffers: the rows of the expert groups
        return nb(*ts) * R_used // R

    row_bytes = D * 2
    pq = _alloc_quant(R, D, MX, True, True, dev, True)
    sq = _alloc_quant(R, H, MX, True, True, dev, True)
    gq = _alloc_quant(R, 2 * H, MX, True, True, dev, True)
    out = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    dw = torch.empty(T * K, dtype=torch.float32, device=dev)
    ew = ExpertWeights(MX, paired=True)
    ew._build(w1, w2, w3, E)
    wouts = {o.data.data_ptr(): o for o in (ew.w13, ew.w13t, ew.w2, ew.w2t)}
    wbytes = nb(w1, w2, w3) + sum(nb(o.data, o.scale) for o in wouts.values())
    tiles = plan.tile_expert
    ops = [
        ("permute + quantise (x rows, MX row + transposed)",
         lambda: _lib.call("fm_permute", _lib.ptr(x), T, D, x.stride(0), _lib.ptr(plan.assign_of_row), R, K, None,
                           *_tile_args(MX, *pq, True, True), _lib.ptr(tiles), st), nb(x) + nbq(*pq)),
        ("permute + quantise (dY rows x router weight)",
         lambda: _lib.call("fm_permute", _lib.ptr(go), T, D, go.stride(0), _lib.ptr(plan.assign_of_row), R, K,
                           _lib.ptr(wts), *_tile_args(MX, *pq, True, True), _lib.ptr(tiles), st),
         nb(go, wts) + nbq(*pq)),
        ("SwiGLU + quantise (MX row + transposed)",
         lambda: _lib.call("fm_swiglu_quantize", _lib.ptr(GU), GU.stride(0), _lib.ptr(GU[:, H:]), GU.stride(0), R, H,
                           *_tile_args(MX, *sq, True, True), _lib.ptr(tiles), st), nbq(GU, *sq)),
        ("SwiGLU backward + quantise (dg|du MX row + transposed)",
         lambda: _lib.call("fm_swiglu_backward", _lib.ptr(GU), GU.stride(0), _lib.ptr(GU[:, H:]), GU.stride(0),
                           _lib.ptr(dH), dH.stride(0), R, H, *_tile_args(MX, *gq, True, True), _lib.ptr(tiles), st),
         nbq(GU, dH, *gq)),
        ("unpermute (weighted sum over the local slots)",
         lambda: _lib.call("fm_unpermute", _lib.ptr(Y), Y.stride(0), _lib.ptr(plan.row_of), _lib.ptr(wts), T, K, D,
                           _lib.ptr(out), _lib.DTYPE_BF16, out.stride(0), None, 0, st),
         A * row_bytes + nb(wts, out)),
        ("router-weight gradient (dw = <dY row, expert output row>)",
         lambda: _lib.call("fm_router_weight_grad", _lib.ptr(go), go.stride(0), _lib.ptr(Y), Y.stride(0),
                           _lib.ptr(plan.row_of), T, K, D, _lib.ptr(dw), st),
         nb(go, dw) + A * row_bytes),
        ("expert weight re-quantisation (w1|w3 pair, w2; MX rows + transposed, two launches)",
         lambda: ew._build(w1, w2, w3, E), wbytes),
    ]
    return time_hbm_ops(ops, reps)


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(T, D, H, E, K, runs=2):
    """configs[2]'s layer step on the host cores, all T tokens: the router
    (fp32 gate, softmax of the replayed balanced experts, load-balancing loss;
    reference model/moe.py:151-281) and the expert block as the FP8 flow's
    dequantise-then-fp32-matmul restatement, forward + backward (the oracle's
    moe_flow_reference: numpy quantisers, torch CPU matmuls).  1 warmup, then
    the median of `runs` timed runs."""
    import numpy as np
    import torch

    from oracle import layer as olayer
    from oracle import routing as orouting

    torch.set_num_threads(os.cpu_count() or 1)
    x, w, idx, w1, w2, w3, go = synthetic_inputs(T, D, H, E, K, seed=2, dev="cpu")
    gw, gb = router_params(D, E, 2, "cpu")

    def once():
        logits = orouting.router_logits(x.float().numpy(), gw.float().numpy(), gb.float().numpy())
        wts, ridx = orouting.replay_gating(logits, idx.numpy(), K)
        orouting.load_balancing_loss(logits, ridx, E)
        olayer.moe_flow_reference(x, torch.from_numpy(wts), torch.from_numpy(ridx), w1, w2, w3, E, go,
                                  recipe="flow_moe")

    once()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": round(T / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"all {T} tokens of configs[2] (D={D}, H={H}, E={E}, top-{K}): router + FP8 flow_moe expert "
                      f"block as dequantise-then-fp32-matmul, fwd+bwd (torch CPU matmuls on "
                      f"{torch.get_num_threads()} threads, numpy quantisers on one), median of {runs} runs, "
                      f"{med:.2f} s per step; cpu: {cpu_model_name()}"}


# ============================================================== configs[2] ====
def workload_c3(args, dev):
    import torch

    T, D, E, K, H = 8192, 2048, 8, 2, 1408
    A = T * K
    x, w, idx, w1, w2, w3, go = synthetic_inputs(T, D, H, E, K, seed=2, dev=dev)
    if args.copy_probe:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b
    gw, gb = router_params(D, E, 2, dev)
    ms, summ, eager_ms = time_layer(x, w, idx, w1, w2, w3, go, E, args.recipe, 0, args.steps, args.warmup,
                                    overlap=not args.no_overlap, router=(gw, gb, K, "softmax"),
                                    graph=not args.eager)
    dom = max(summ, key=lambda k: summ[k]["ms"])
    d = summ[dom]
    achieved = d["flops"] / (d["ms"] * 1e-3) / 1e12
    peak = PEAK_TFLOPS["bf16" if args.recipe == "none" else "fp8"]
    traffic = recorded_traffic(dom, args.recipe)
    cpu = None if args.no_cpu_baseline else cpu_baseline(T, D, H, E, K)
    hbm = hbm_kernels_c3(x, w, idx, w1, w2, w3, go, E, H) if args.recipe == "flow_moe" else None
    probe = None
    if hbm is not None:   # the same kernels against what a plain copy reaches on this board
        probe = bw_probe(dev, reps=5)
        for h in hbm:
            h["frac_of_copy_probe"] = round(h["GB_s"] / 1e3 / probe["copy"]["TB_s"], 3)
    return {
        "metric": "MoE layer fwd+bwd tokens/s on 1 MI355X",
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.recipe == "none" else "fp8-e4m3",
        "data": "synthetic",
        "config": {"workload": "configs[2]: router + FP8-Flow-MoE expert block, fwd+bwd of out*grad + aux loss, "
                               "FP8 forced",
                   "tokens": T, "d_model": D, "experts": E, "top_k": K, "ffn_hidden": H,
                   "routing": "top-2 softmax router (fp32 gate, load-balancing loss) with the exactly balanced "
                              "assignment (2048 per expert) replayed as its R3 routing mask",
                   "recipe": args.recipe, "assignments": A,
                   "launch": launch_note(args)},
        "eager_ms_per_step": round(eager_ms, 4),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4),
                     "traffic": None if traffic is None else traffic["bytes_per_launch"],
                     "kernel": dom,
                     "traffic_source": None if traffic is None else traffic["source"]},
        "gemm": gemm_report(summ, args.steps),
        "hbm_kernels": hbm,
        "hbm_probe": probe,
        "cpu_baseline": cpu,
    }


# ======================================================= shared expert ====
def workload_shared(args, dev):
    """Shared expert / dense SwiGLU FFN (FP8SharedExpertCompute: one group on
    the grouped-GEMM path) at configs[2]'s shapes: every one of T = 8192
    tokens through one SwiGLU FFN, D = 2048, H = 1408, fwd + bwd, weights
    re-quantised every step."""
    import torch

    import nanopysche_amd as fm
    from nanopysche_amd import flow_moe as fmm

    T, D, H = 8192, 2048, 1408
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(T, D, device=dev, generator=g).bfloat16().requires_grad_(True)
    params = [(torch.randn(H, D, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True)
              for _ in range(3)]
    go = (torch.randn(T, D, device=dev, generator=g) * 1e-2).bfloat16()
    cfg = fm.FP8FlowMoEConfig(enabled=args.recipe != "none",
                              fp8_recipe=fm.FP8RecipeConfig(args.recipe != "none", fm.FP8RecipeType(args.recipe)))
    blk = fm.FP8SharedExpertCompute(cfg, D, H)
    blk.set_weights(*params)

    def step():
        blk.block._cache.clear()
        for p in params + [x]:
            p.grad = None
        blk(x).backward(go)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    if not args.eager:
        graph_ms = time_graphed(step, params + [x], args.steps, args.warmup)
        ms = eager_ms if graph_ms is None else graph_ms
    timer = GemmTimer()
    fmm.GEMM_TIMER = timer
    blk.block.overlap_streams = False
    try:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    finally:
        fmm.GEMM_TIMER = None
    summ = timer.summary()
    dom = max(summ, key=lambda k: summ[k]["ms"])
    d = summ[dom]
    achieved = d["flops"] / (d["ms"] * 1e-3) / 1e12
    peak = PEAK_TFLOPS["bf16" if args.recipe == "none" else "fp8"]
    return {
        "metric": "Shared-expert SwiGLU FFN fwd+bwd tokens/s on 1 MI355X",
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.recipe == "none" else "fp8-e4m3",
        "data": "synthetic",
        "config": {"workload": "shared expert at configs[2]'s shapes (one group on the grouped-GEMM path)",
                   "tokens": T, "d_model": D, "ffn_hidden": H, "recipe": args.recipe,
                   "launch": launch_note(args)},
        "eager_ms_per_step": round(eager_ms, 4),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4), "traffic": None, "kernel": dom},
        "gemm": gemm_report(summ, args.steps),
        "cpu_baseline": None,
    }


# ============================================================== configs[1] ====
def workload_c2(args, dev):
    """Quantisation primitives on configs[1]'s inputs: x [8192, 4096] bf16
    N(0,1) with 0.1% of entries x100, W [14336, 4096] bf16 N(0,0.02).  Each
    primitive runs `steps` times back to back between two HIP events (outputs
    preallocated, C ABI called directly); GB/s = algorithmic bytes (every input
    byte read once, every output byte written once) / time per launch."""
    import torch

    from nanopysche_amd import _lib
    from nanopysche_amd.flow_moe import _alloc_quant, _tile_args

    R, C = 8192, 4096
    WR = 14336
    gen = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(R, C, generator=gen, device=dev)
    n_out = round(0.001 * R * C)
    pos = torch.randperm(R * C, generator=gen, device=dev)[:n_out]
    x.view(-1)[pos] *= 100.0
    x = x.bfloat16()
    w = device_normal((WR, C), 0.02, gen, dev, torch.bfloat16)
    st = _lib.stream_of(x)
    n = R * C
    BLK, P2, MX = _lib.QUANT_BLOCK, _lib.QUANT_POW2, _lib.QUANT_MX

    def quant_args(kind, row, col):
        bufs = _alloc_quant(R, C, kind, row, col, dev)
        return bufs, _tile_args(kind, *bufs)

    rowb, rowb_a = quant_args(BLK, True, False)
    rowp, rowp_a = quant_args(P2, True, False)
    fused, fused_a = quant_args(BLK, True, True)
    fusedp, fusedp_a = quant_args(P2, True, True)
    mxb, mx_a = quant_args(MX, True, False)
    q, s = rowb[0], rowb[1]
    qt = torch.empty(C, R, dtype=torch.uint8, device=dev)
    sct = torch.empty(R // 128, C, dtype=torch.float32, device=dev)
    deq = torch.empty(R, C, dtype=torch.bfloat16, device=dev)
    wq = torch.empty(WR, C, dtype=torch.uint8, device=dev)
    ws = torch.empty(WR // 128, C // 128, dtype=torch.float32, device=dev)

    def fm_quantize(a):
        return lambda: _lib.call("fm_quantize", _lib.ptr(x), _lib.DTYPE_BF16, R, C, C, *a, st)

    ops = [
        ("quantize 1x128 (fp32 scale)", fm_quantize(rowb_a), n * 2 + n + n // 128 * 4),
        ("quantize 1x128 (pow2 scale)", fm_quantize(rowp_a), n * 2 + n + n // 128 * 4),
        ("quantize 1x128 + 128x1 transpose (fp32 scale)", fm_quantize(fused_a), n * 2 + 2 * n + 2 * (n // 128) * 4),
        ("quantize 1x128 + scaling-aware transpose (pow2)", fm_quantize(fusedp_a),
         n * 2 + 2 * n + 2 * (n // 128) * 4),
        ("quantize MX 1x32 (e8m0)", fm_quantize(mx_a), n * 2 + n + n // 32),
        ("scaling-aware transpose (from e4m3)",
         lambda: _lib.call("fm_scaling_aware_transpose", _lib.ptr(q), R, C, C, _lib.ptr(s), C // 128,
                           _lib.ptr(qt), R, _lib.ptr(sct), C, st), 2 * n + 2 * (n // 128) * 4),
        ("dequantize 1x128 -> bf16",
         lambda: _lib.call("fm_dequantize", _lib.ptr(q), R, C, C, _lib.ptr(s), 0, 0, 7, C // 128, 1,
                           _lib.ptr(deq), _lib.DTYPE_BF16, C, st), n + n // 128 * 4 + 2 * n),
        ("quantize weight 128x128", lambda: _lib.call(
            "fm_quantize_weight", _lib.ptr(w), _lib.DTYPE_BF16, 1, WR, C, C, 0, BLK, _lib.ptr(wq), C, 0, 0, _lib.ptr(ws),
            C // 128, 0, None, 0, 0, 0, None, 0, 0, st), WR * C * 3 + (WR // 128) * (C // 128) * 4),
    ]
    fm_quantize(rowb_a)()  # inputs of the transpose / dequantise
    results = []
    for name, fn, nbytes in ops:
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / args.steps
        results.append({"op": name, "us": round(us, 2), "bytes": nbytes,
                        "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "frac_of_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    # headline: configs[1]'s own chain -- 1x128 quantise with fp32 scales, the
    # scaling-aware transpose of its output, dequantise, 128x128 weight quantise
    chain = [results[i] for i in (0, 5, 6, 7)]
    chain_us = sum(r["us"] for r in chain)
    chain_gbs = sum(r["bytes"] for r in chain) / (chain_us * 1e-6) / 1e9
    # the roofline reports the op furthest from the HBM peak (of all ops timed)
    dom = min(results, key=lambda r: r["frac_of_hbm_peak"])
    # each op against what a plain copy reaches on this board
    probe = bw_probe(dev, reps=5)
    for r in results:
        r["frac_of_copy_probe"] = round(r["GB_s"] / 1e3 / probe["copy"]["TB_s"], 3)
    cpu = None if args.no_cpu_baseline else cpu_baseline_quant(C)
    return {
        "metric": "HBM GB/s of the FP8 quantisation primitives on 1 MI355X (configs[1])",
        "value": round(chain_gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": 3,
        "ms_per_step": round(chain_us / 1e3, 5), "higher_is_better": True, "vs_baseline": None,
        "dtype": "bf16 -> e4m3", "data": "synthetic",
        "config": {"workload": "configs[1]: x [8192, 4096] bf16 N(0,1), 0.1% outliers x100; W [14336, 4096] "
                               "bf16 N(0,0.02)",
                   "chain": [r["op"] for r in chain]},
        "roofline": {"bound": "hbm", "achieved": dom["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["frac_of_hbm_peak"], "traffic": None, "kernel": dom["op"],
                     "note": "the slowest op by fraction of the HBM peak; every op's fraction in 'per_op'"},
        "per_op": {r["op"]: r["frac_of_hbm_peak"] for r in results},
        "cpu_baseline": cpu,
        "ops": results,
        "hbm_probe": probe,
    }


def cpu_baseline_quant(C, budget_s=10.0):
    """The oracle's 1x128 fp32-scale quantiser (numpy, one host thread) on a
    bounded row sample of configs[1]'s activation, in the same algorithmic
    GB/s as the GPU ops (bf16 read, e4m3 + scales written)."""
    import numpy as np

    from oracle import fp8 as ofp8

    Rs = 2048
    rng = np.random.default_rng(1)
    x = rng.standard_normal((Rs, C)).astype(np.float32)
    x = ofp8.bf16_round(x)
    nbytes = Rs * C * 3 + Rs * C // 128 * 4
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 2 or (time.perf_counter() < t_end and len(times) < 5):
        t0 = time.perf_counter()
        ofp8.quant_1x128(x)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(nbytes / med / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{Rs} x {C} rows of N(0,1) bf16 values, oracle quant_1x128 (numpy, fp32 scales), "
                      f"median of {len(times)} runs"}


# ============================================================== configs[0] ====
def workload_c1(args, dev):
    """BF16 MoE layer forward, top-1 softmax router over 4 experts (gate GEMM,
    top-1 gating, counts and load-balancing loss run inside the step)."""
    import torch

    T, D, E, K, H = 4096, 2048, 4, 1, 5632
    gen = torch.Generator(device=dev).manual_seed(0)
    x = device_normal((T, D), 1.0, gen, dev, torch.bfloat16)
    wg = device_normal((E, D), 0.02, gen, dev, torch.bfloat16)
    bg = device_normal((E,), 0.02, gen, dev, torch.bfloat16)
    w1, w2, w3 = [device_normal((E * H, D), 0.02, gen, dev, torch.bfloat16) for _ in range(3)]
    import nanopysche_amd as fm

    with torch.no_grad():
        w0, i0, _ = fm.route(x, wg, bg, top_k=K, gating="softmax")
    ms, summ, eager_ms = time_layer(x, w0, i0, w1, w2, w3, None, E, "none", 1 << 40, args.steps, args.warmup,
                                    backward=False, router=(wg, bg, K, "softmax", False), graph=not args.eager)
    counts = torch.bincount(i0.reshape(-1), minlength=E).tolist()
    flops = 6.0 * T * K * D * H
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_c1(x.cpu(), wg.cpu(), bg.cpu(), w1.cpu(), w2.cpu(), w3.cpu(), E, K)
    return {
        "metric": "MoE layer fwd tokens/s on 1 MI355X (configs[0], BF16)",
        "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "configs[0]: router + BF16 expert block forward, top-1 softmax", "tokens": T,
                   "d_model": D, "experts": E, "top_k": K, "ffn_hidden": H, "tokens_per_expert": counts,
                   "launch": launch_note(args)},
        "eager_ms_per_step": round(eager_ms, 4),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "frac_of_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_TFLOPS["bf16"], 4),
        "roofline": gemm_roofline(summ, "bf16"),
        "gemm": gemm_report(summ, args.steps),
        "cpu_baseline": cpu,
    }


def gemm_roofline(summ, arith, flops_scale=1.0):
    """`roofline` of the dominant grouped-GEMM kernel of an event summary: its
    algorithmic FLOPs per launch / its HIP-event time against the dense peak."""
    dom = max(summ, key=lambda k: summ[k]["ms"])
    d = summ[dom]
    achieved = d["flops"] * flops_scale / (d["ms"] * 1e-3) / 1e12
    peak = PEAK_TFLOPS[arith]
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": None, "kernel": dom}


def _median_time(fn, runs, warmup=1):
    import numpy as np

    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def cpu_baseline_c1(x, wg, bg, w1, w2, w3, E, K, runs=2):
    """configs[0]'s layer forward on the host cores, all tokens: the router
    (fp32 gate, top-1 softmax; reference model/moe.py:151-255) and the
    reference's BF16 per-expert loop (model/moe.py:1542-1596) restated in
    torch CPU fp32 (oracle.layer.moe_bf16_loop)."""
    import torch

    from oracle import layer as olayer
    from oracle import routing as orouting

    torch.set_num_threads(os.cpu_count() or 1)

    def once():
        logits = orouting.router_logits(x.float().numpy(), wg.float().numpy(), bg.float().numpy())
        w, idx = orouting.softmax_topk(logits, K)
        olayer.moe_bf16_loop(x, torch.from_numpy(w), torch.from_numpy(idx), w1, w2, w3, E)

    med = _median_time(once, runs)
    T = x.shape[0]
    return {"value": round(T / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"all {T} tokens of configs[0]: router + BF16 per-expert loop forward in torch CPU fp32 "
                      f"({torch.get_num_threads()} threads), 1 warmup + median of {runs} runs, {med:.2f} s per "
                      f"forward; cpu: {cpu_model_name()}"}


# ============================================================== configs[3] ====
def zipf_gumbel_topk(T, E, K, s, seed):
    """Per-token K distinct experts by Gumbel-top-K on log p_e, p_e proportional
    to rank^-s over a seeded permutation; router weights softmax of the
    perturbed scores at the chosen experts."""
    import numpy as np
    import torch

    rng = np.random.default_rng(seed)
    ranks = rng.permutation(E) + 1
    logp = -s * np.log(ranks.astype(np.float64))
    score = logp[None, :] + rng.gumbel(size=(T, E))
    idx = np.argsort(-score, axis=1, kind="stable")[:, :K]
    sel = np.take_along_axis(score, idx, axis=1)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    w = w / w.sum(axis=1, keepdims=True)
    return torch.from_numpy(w.astype(np.float32)), torch.from_numpy(idx.astype(np.int64))


def workload_c4(args, dev):
    """FP8 (flow_moe) vs BF16 grouped GEMM crossover, fwd+bwd, Zipf(1.1) routing."""
    import torch

    D, E, K, H = 4096, 8, 2, 14336
    gen = torch.Generator(device=dev).manual_seed(3)
    w1, w2, w3 = [device_normal((E * H, D), 0.02, gen, dev, torch.bfloat16) for _ in range(3)]
    points = [int(v) for v in args.c4_points.split(",")]
    sweep = []
    for t in points:
        T = 4 * t
        w, idx = zipf_gumbel_topk(T, E, K, 1.1, seed=3)
        w, idx = w.to(dev), idx.to(dev)
        x = device_normal((T, D), 1.0, gen, dev, torch.bfloat16)
        go = device_normal((T, D), 1e-2, gen, dev, torch.bfloat16)
        flops = 18.0 * T * K * D * H
        steps = max(2, min(args.steps, int(2e15 / flops) + 1))
        row = {"tokens_per_expert": t, "tokens": T,
               "max_tokens_per_expert": int(torch.bincount(idx.reshape(-1), minlength=E).max())}
        for name, recipe in (("bf16", "none"), ("fp8", "flow_moe")):
            ms, summ, _ = time_layer(x, w, idx, w1, w2, w3, go, E, recipe, 0, steps, 1,
                                     overlap=not args.no_overlap)
            row[f"{name}_ms"] = round(ms, 3)
            row[f"{name}_tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
            row[f"{name}_gemm"] = gemm_report(summ, steps)
            row[f"{name}_roofline"] = gemm_roofline(summ, "bf16" if recipe == "none" else "fp8")
        row["fp8_speedup"] = round(row["bf16_ms"] / row["fp8_ms"], 3)
        # the threshold split (model/moe.py:1215-1216): experts with at least the
        # mean count (t assignments) take FP8, the others BF16
        ms, summ, _ = time_layer(x, w, idx, w1, w2, w3, go, E, "flow_moe", t, steps, 1,
                                 overlap=not args.no_overlap)
        counts = torch.bincount(idx.reshape(-1), minlength=E)
        row["mixed"] = {"threshold": t, "fp8_experts": int((counts >= t).sum()), "ms": round(ms, 3),
                        "gemm": gemm_report(summ, steps)}
        sweep.append(row)
        print(json.dumps({"progress": row}), file=sys.stderr, flush=True)
        del x, go
        torch.cuda.empty_cache()
    faster = [r["tokens_per_expert"] for r in sweep if r["fp8_speedup"] > 1.0]
    # the roofline of the point the >= 60 % target is stated at (>= 4096 tokens/expert)
    big = [r for r in sweep if r["tokens_per_expert"] >= 4096] or sweep
    cpu = None if args.no_cpu_baseline else cpu_baseline_c4(w1, w2, w3, E, K, points)
    return {
        "metric": "FP8 vs BF16 expert block fwd+bwd crossover on 1 MI355X (configs[3])",
        "n_gpus": 1, "data": "synthetic", "dtype": "fp8-e4m3 vs bf16",
        "config": {"workload": "configs[3]: D=4096, E=8, top-2, H=14336, Zipf(1.1) Gumbel-top-2 routing",
                   "fp8_recipe": "flow_moe", "threshold": 0},
        "roofline": dict(big[0]["fp8_roofline"], tokens_per_expert=big[0]["tokens_per_expert"]),
        "sweep": sweep,
        "fp8_faster_from_tokens_per_expert": min(faster) if faster else None,
        "cpu_baseline": cpu,
    }


def cpu_baseline_c4(w1, w2, w3, E, K, points, cap_s=60.0):
    """configs[3]'s expert block fwd+bwd on the host cores: the BF16 arm as the
    reference's per-expert loop (model/moe.py:1542-1596, torch CPU fp32
    autograd) and the FP8 arm as the flow's dequantise-then-fp32-matmul
    (oracle.layer.moe_flow_reference), each point timed once on all its
    tokens, smallest first, while the CPU time spent stays under `cap_s`;
    later points are reported as not timed (cap), never extrapolated."""
    import torch

    from oracle import layer as olayer

    torch.set_num_threads(os.cpu_count() or 1)
    D = w1.shape[1]
    W = [t.cpu() for t in (w1, w2, w3)]
    g = torch.Generator().manual_seed(33)
    spent, rows = 0.0, []
    for t in sorted(points):
        T = 4 * t
        row = {"tokens_per_expert": t}
        for name, fn in (("bf16", lambda *a: olayer.moe_bf16_loop(*a)),
                         ("fp8", lambda *a: olayer.moe_flow_reference(*a, recipe="flow_moe"))):
            if spent >= cap_s:
                row[f"{name}_tokens_per_s"] = "CPU not timed (cap)"
                continue
            w, idx = zipf_gumbel_topk(T, E, K, 1.1, seed=3)
            x = torch.randn(T, D, generator=g).bfloat16()
            go = (torch.randn(T, D, generator=g) * 1e-2).bfloat16()
            t0 = time.perf_counter()
            fn(x, w, idx, *W, E, go)
            dt = time.perf_counter() - t0
            spent += dt
            row[f"{name}_tokens_per_s"] = round(T / dt, 1)
            row[f"{name}_s"] = round(dt, 2)
        rows.append(row)
    first = rows[0]
    return {"value": first["bf16_tokens_per_s"], "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"BF16 per-expert loop fwd+bwd (torch CPU fp32) on all {4 * first['tokens_per_expert']} "
                      f"tokens of the {first['tokens_per_expert']} tokens/expert point, one run; the per-point "
                      f"figures (FP8 arm as dequantise-then-fp32-matmul) are in 'points', points past "
                      f"{cap_s:.0f} s of CPU time not timed; cpu: {cpu_model_name()}",
            "points": rows}


# ============================================================== configs[4] ====
C5_SHAPE = dict(D=7168, E_local=32, E_global=256, K=8, H=2048, A_target=65536)


def c5_routing(dev, gen):
    """configs[4]'s routing on the device: sigmoid top-8 over 256 experts with a
    Zipf(1.2) per-expert bias added before the sigmoid (model/moe.py:153-162,
    :257-265), two local experts (5 and 17) that never receive tokens; this
    rank (experts 0-31) keeps the tokens with at least one local slot, in
    order, until 65,536 local assignments; other slots carry the out-of-range
    index 256.  Returns (weights [T, 8] fp32, indices [T, 8] int64, A)."""
    import torch

    import nanopysche_amd as fm

    E_local, E_global, K, A_target = (C5_SHAPE[k] for k in ("E_local", "E_global", "K", "A_target"))
    # per-expert bias from Zipf(1.2) popularity (added before the sigmoid, model/moe.py:153-162);
    # two local experts never receive tokens
    g = torch.Generator().manual_seed(4)
    ranks = torch.randperm(E_global, generator=g).float() + 1
    bias = (-1.2 * torch.log(ranks)).to(dev)
    bias[[5, 17]] = -1e9
    # this rank receives the tokens with at least one assignment to its 32
    # experts (ids 0-31), in order, until A_target local assignments
    ws, ids, total = [], [], 0
    while total < A_target:
        logits = device_normal((65536, E_global), 1.0, gen, dev, torch.float32) + bias
        w_, i_ = fm.topk_gating(logits.contiguous(), K, "sigmoid")
        has = (i_ < E_local).any(dim=1)
        ws.append(w_[has])
        ids.append(i_[has])
        total += int((i_[has] < E_local).sum())
    wts, idx = torch.cat(ws), torch.cat(ids)
    local = idx < E_local
    csum = torch.cumsum(local.reshape(-1).int(), 0).reshape(idx.shape)
    keep = local & (csum <= A_target)
    n_tok = int((csum[:, 0] - local[:, 0].int() < A_target).sum())   # tokens holding a kept slot
    # assignments outside this rank's experts carry an out-of-range index, which routing ignores
    idx = torch.where(keep, idx, torch.full_like(idx, E_global))[:n_tok].contiguous()
    wts = wts[:n_tok].contiguous()
    return wts, idx, int(keep[:n_tok].sum())


def workload_c5(args, dev):
    """One GPU's 32-expert share of a 256-expert layer, MXFP8, fwd+bwd."""
    import torch

    D, E_local, K, H = (C5_SHAPE[k] for k in ("D", "E_local", "K", "H"))
    gen = torch.Generator(device=dev).manual_seed(4)
    wts, idx, A = c5_routing(dev, gen)
    n_tok = idx.shape[0]
    counts = torch.bincount(idx[idx < E_local], minlength=E_local)
    x = device_normal((n_tok, D), 1.0, gen, dev, torch.bfloat16)
    go = device_normal((n_tok, D), 1e-2, gen, dev, torch.bfloat16)
    w1, w2, w3 = [device_normal((E_local * H, D), 0.02, gen, dev, torch.bfloat16) for _ in range(3)]
    ms, summ, _ = time_layer(x, wts, idx, w1, w2, w3, go, E_local, "mxfp8", 0, args.steps, args.warmup,
                          overlap=not args.no_overlap)
    flops = 18.0 * A * D * H
    gemm = gemm_report(summ, args.steps, flops_scale=A / (n_tok * K))
    # the step's HBM-bound kernels alone, against a plain copy's rate: the
    # time outside the GEMMs and the least it could be at that rate
    hbm = hbm_kernels_c5(x, wts, idx, w1, w2, w3, go, E_local, H)
    probe = bw_probe(dev, reps=5)
    copy = probe["copy"]["TB_s"] * 1e12
    per_step = {"unpermute (weighted sum over the local slots)": 2}   # forward combine and the dx sum
    floor_ms = 0.0
    for h in hbm:
        h["frac_of_copy_probe"] = round(h["GB_s"] / 1e3 / probe["copy"]["TB_s"], 3)
        h["per_step"] = per_step.get(h["op"], 1)
        floor_ms += h["per_step"] * h["bytes"] / copy * 1e3
    outside = ms - gemm["gemm_ms_per_step"]
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_c5(x, wts, idx, w1, w2, w3, go, E_local)
    return {
        "metric": "MoE expert block fwd+bwd assignments/s on 1 MI355X (configs[4], MXFP8)",
        "value": round(A / (ms * 1e-3), 1), "unit": "assignments/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "dtype": "fp8-e4m3 (MX e8m0 1x32)", "data": "synthetic",
        "config": {"workload": "configs[4]: 32 local experts of 256, sigmoid top-8 with Zipf(1.2) bias",
                   "tokens": n_tok, "assignments": A, "d_model": D, "local_experts": E_local,
                   "ffn_hidden": H, "zero_token_experts": int((counts == 0).sum()),
                   "max_tokens_per_expert": int(counts.max())},
        "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "frac_of_fp8_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_TFLOPS["fp8"], 4),
        "roofline": gemm_roofline(summ, "fp8", flops_scale=A / (n_tok * K)),
        "gemm": gemm,
        "outside_gemms": {"ms": round(outside, 4), "share": round(outside / ms, 4),
                          "floor_ms_at_copy_rate": round(floor_ms, 4),
                          "floor_share": round(floor_ms / (floor_ms + gemm["gemm_ms_per_step"]), 4),
                          "note": "floor: the algorithmic bytes of the step's HBM-bound kernels (each op below "
                                  "times its launches per step) at the copy probe's rate; floor_share: their "
                                  "share of a step whose GEMMs keep their measured time"},
        "hbm_kernels": hbm,
        "hbm_probe": probe,
        "cpu_baseline": cpu,
    }


def cpu_baseline_c5(x, wts, idx, w1, w2, w3, go, E, n_experts=4, a_sample=8192):
    """configs[4]'s MXFP8 expert block fwd+bwd on the host cores as the flow's
    dequantise-then-fp32-matmul (oracle.layer.moe_flow_reference, recipe
    mxfp8) on a bounded sample of the same workload: the slots of the
    `n_experts` most loaded local experts (the others' slots treated as
    another GPU's), on the first tokens holding `a_sample` of them, with
    those experts' weights quantised as the GPU step quantises every
    expert's (an eighth of the experts: weight and token work in about the
    layer's proportion); one run."""
    import torch

    from oracle import layer as olayer

    torch.set_num_threads(os.cpu_count() or 1)
    idx_h = idx.cpu()
    counts = torch.bincount(idx_h[idx_h < E], minlength=E)
    keep_e = torch.argsort(counts, descending=True, stable=True)[:n_experts]
    keep = torch.isin(idx_h, keep_e)
    csum = torch.cumsum(keep.sum(dim=1), 0)
    n = min(int((csum < a_sample).sum()) + 1, idx_h.shape[0])
    idx_s = torch.where(keep[:n], idx_h[:n], torch.full_like(idx_h[:n], 1 << 20))
    A = int(keep[:n].sum())
    host = [t.cpu() for t in (x[:n], wts[:n])] + [idx_s] + [t.cpu() for t in (w1, w2, w3, go[:n])]
    t0 = time.perf_counter()
    olayer.moe_flow_reference(*host[:6], E, host[6], recipe="mxfp8")
    dt = time.perf_counter() - t0
    return {"value": round(A / dt, 1), "unit": "assignments/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{A} assignments of configs[4] (the first {n} tokens' slots on the {n_experts} most loaded "
                      f"of the 32 local experts), MXFP8 flow as dequantise-then-fp32-matmul fwd+bwd incl. those "
                      f"experts' weight quantisation (torch CPU), one run, {dt:.1f} s; cpu: {cpu_model_name()}"}


def bw_probe(dev, gib=1, reps=10):
    """HBM rates of plain kernels (fm_hbm_probe): a copy with one 4 KiB chunk
    per workgroup (the tile producers' launch shape), a read-only and a
    write-only pass, `gib` GiB each, `reps` back-to-back launches between two
    HIP events after three warm-up launches.  The HBM-bound kernels' fractions
    are quoted against 8 TB/s; these say what a kernel with nothing but the
    memory traffic reaches on the same board."""
    import torch

    from nanopysche_amd import _lib

    n = gib << 30
    a = torch.ones(n, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    st = _lib.stream_of(a)
    out = {}
    for kind, name, moved in ((0, "copy", 2 * n), (1, "read", n), (2, "write", n)):
        def launch():
            _lib.call("fm_hbm_probe", kind, _lib.ptr(a), _lib.ptr(b), n, st)
        for _ in range(3):
            launch()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            launch()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        out[name] = {"us": round(us, 1), "TB_s": round(moved / us / 1e6, 3), "frac_of_8TBps": round(moved / us / 8e6, 3)}
    return {"probe": "HBM bandwidth (fm_hbm_probe)", "bytes_per_buffer": n, **out}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c3", choices=["c3", "c1", "c2", "c4", "c5", "shared"])
    ap.add_argument("--recipe", default="flow_moe", choices=["flow_moe", "blockwise", "mxfp8", "none"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="time eagerly issued steps instead of replays of the step captured as a HIP graph "
                         "(configs[2], configs[0], shared expert)")
    ap.add_argument("--no-overlap", action="store_true",
                    help="keep every launch on one stream (the router's backward not beside the dY "
                         "permute and dH + dW2; MX: no dW2 / dH overlap)")
    ap.add_argument("--c4-points", default="512,1024,2048,4096,8192,16384",
                    help="configs[3] tokens/expert points (comma list)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run one plain 256 MiB device copy (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against known bytes)")
    ap.add_argument("--bw-probe", action="store_true",
                    help="print the HBM rates of a plain copy, read and write (fm_hbm_probe) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    if args.bw_probe:
        print(json.dumps(bw_probe(dev)))
        return
    run = {"c3": workload_c3, "c1": workload_c1, "c2": workload_c2, "c4": workload_c4,
           "c5": workload_c5, "shared": workload_shared}[args.workload]
    print(json.dumps(run(args, dev)))


if __name__ == "__main__":
    main()
