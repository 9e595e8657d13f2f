"""Benchmark of the fp8_flow_moe expert block on one MI355X.

Workload: T=8192 tokens, d_model=2048, 8 experts,
top-2, SwiGLU ffn_hidden=1408, exactly balanced routing (2048 assignments per
expert, router weights = softmax of seeded logits at those indices), FP8 GEMMs
forced (threshold 0), recipe flow_moe (1x128 / 128x128 power-of-two scales).
One step = expert-block forward + backward, including the routing sort, all
quantisation and the re-quantisation of the expert weights (their cache is
dropped every step, as after an optimizer update).  Inputs are resident in HBM
before timing starts.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--recipe flow_moe]

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


def cpu_baseline(T, D, H, E, K, budget_s=12.0):
    """The reference's BF16 per-expert loop (model/moe.py:1542-1596) restated in
    fp32 torch on the host cores, forward + backward, on a bounded token sample."""
    import torch

    from oracle.layer import moe_bf16_loop

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    Ts = 1024
    x, w, idx, w1, w2, w3, go = synthetic_inputs(Ts, D, H, E, K, seed=2, dev="cpu")
    moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)  # warmup
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 2 or (time.perf_counter() < t_end and len(times) < 5):
        t0 = time.perf_counter()
        moe_bf16_loop(x, w, idx, w1, w2, w3, E, go)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(Ts / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{Ts} tokens of the same layer (D={D}, H={H}, E={E}, top-{K}), fp32 torch CPU "
                      f"per-expert loop fwd+bwd, median of {len(times)} runs; cpu: {model}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--recipe", default="flow_moe", choices=["flow_moe", "blockwise", "mxfp8", "none"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run one plain 256 MiB device copy (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against known bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)

    import torch

    import nanopysche_amd as fm
    from nanopysche_amd import flow_moe as fmm

    dev = torch.device("cuda:0")
    T, D, E, K, H = 8192, 2048, 8, 2, 1408
    A = T * K
    x, w, idx, w1, w2, w3, go = synthetic_inputs(T, D, H, E, K, seed=2, dev=dev)
    rt = fm.FP8RecipeType(args.recipe)
    cfg = fm.FP8FlowMoEConfig(enabled=True, fp8_recipe=fm.FP8RecipeConfig(True, rt))
    blk = fm.FP8FlowMoECompute(cfg, D, H, E, fp8_gemm_threshold=0)
    params = [t.clone().requires_grad_(True) for t in (w1, w2, w3)]
    blk.set_weights(*params)
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)

    def step():
        blk._cache.clear()  # weights change every training step: re-quantise them
        for p in params:
            p.grad = None
        xr.grad = None
        wr.grad = None
        out = blk(xr, wr, idx, 0, E)
        out.backward(go)

    if args.copy_probe:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # timed region: HIP events around every grouped GEMM on its launch stream
    timer = GemmTimer()
    fmm.GEMM_TIMER = timer
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    fmm.GEMM_TIMER = None
    ms = elapsed * 1e3 / args.steps

    summ = timer.summary()
    dom = max(summ, key=lambda k: summ[k]["ms"])
    d = summ[dom]
    achieved = d["flops"] / (d["ms"] * 1e-3) / 1e12
    peak = PEAK_TFLOPS["bf16" if args.recipe == "none" else "fp8"]
    gemm_ms = sum(v["ms"] for v in summ.values()) / args.steps
    kernels = {k: {"avg_us": round(v["ms"] * 1e3 / v["launches"], 2),
                   "tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 1),
                   "launches_per_step": v["launches"] // args.steps} for k, v in summ.items()}
    traffic = recorded_traffic(dom, args.recipe)

    cpu = None if args.no_cpu_baseline else cpu_baseline(T, D, H, E, K)
    res = {
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
        "config": {"workload": "configs[2]: FP8-Flow-MoE expert block fwd+bwd, FP8 forced",
                   "tokens": T, "d_model": D, "experts": E, "top_k": K, "ffn_hidden": H,
                   "routing": "exactly balanced (2048 assignments per expert)",
                   "recipe": args.recipe, "assignments": A},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4),
                     "traffic": None if traffic is None else traffic["bytes_per_launch"],
                     "kernel": dom,
                     "traffic_source": None if traffic is None else traffic["source"]},
        "gemm": {"tflops_all_gemms": round(18 * A * D * H / (gemm_ms * 1e-3) / 1e12, 1),
                 "gemm_ms_per_step": round(gemm_ms, 4), "kernels": kernels},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
