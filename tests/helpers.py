"""Shared input generators for the tests (seeded, CPU tensors)."""

from __future__ import annotations

import numpy as np
import torch


def randn_bf16(shape, seed, std=1.0, outlier_frac=0.0, outlier_scale=100.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * std
    if outlier_frac:
        n = int(round(outlier_frac * x.numel()))
        pos = torch.randperm(x.numel(), generator=g)[:n]
        x.view(-1)[pos] *= outlier_scale
    return x.bfloat16()


def zipf_routing(T, E, K, s, seed, zero_experts=()):
    """Per-token K distinct experts drawn by Gumbel-top-K on log p_e with
    p_e proportional to rank^-s over a seeded permutation of the experts."""
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(E) + 1
    logp = -s * np.log(ranks.astype(np.float64))
    for z in zero_experts:
        logp[z] = -np.inf
    g = rng.gumbel(size=(T, E))
    idx = np.argsort(-(logp[None, :] + g), axis=1, kind="stable")[:, :K]
    w = rng.random((T, K)).astype(np.float32) + 0.1
    w = w / w.sum(axis=1, keepdims=True)
    return torch.from_numpy(w.astype(np.float32)), torch.from_numpy(idx.astype(np.int64))


def c3_inputs():
    """BASELINE configs[2] (seed 2): T=8192, D=2048, E=8, top-2, H=1408,
    exactly balanced routing (token t -> experts t mod 8 and (t + 4) mod 8,
    2048 assignments per expert), router weights = softmax of seeded logits at
    those experts, weights N(0, 0.02), upstream grad N(0, 1e-2); the inputs
    bench.py times."""
    T, D, H, E, K = 8192, 2048, 1408, 8, 2
    g = torch.Generator().manual_seed(2)
    x = torch.randn(T, D, generator=g).bfloat16()
    logits = torch.randn(T, E, generator=g)
    t = torch.arange(T)
    idx = torch.stack([(t % E), ((t + E // 2) % E)], dim=1)[:, :K].contiguous()
    w = torch.softmax(torch.gather(logits, 1, idx), dim=-1)
    w1, w2, w3 = [(torch.randn(E * H, D, generator=g) * 0.02).bfloat16() for _ in range(3)]
    go = (torch.randn(T, D, generator=g) * 1e-2).bfloat16()
    return x, w, idx, w1, w2, w3, go


def expert_share_routing(T, E_global, E_local, K, s, seed, local_start=0, zero_local=(), min_local=0):
    """One GPU's share of sigmoid top-K routing over E_global experts with a
    per-expert score bias from Zipf(s) popularity added before the sigmoid
    (reference model/moe.py:153-162, :257-265).  Tokens are drawn in batches
    of T until at least ``min_local`` slots land on the local experts
    [local_start, local_start + E_local); tokens with no local slot are
    dropped and the other slots keep their global expert ids.  ``zero_local``
    lists local experts (0-based) whose bias is -100, so they receive no token.

    Returns (weights [T', K] fp32, global indices [T', K] int64)."""
    from oracle import routing as orouting

    rng = np.random.default_rng(seed)
    ranks = rng.permutation(E_global) + 1
    bias = (-s * np.log(ranks.astype(np.float64))).astype(np.float32)
    for z in zero_local:
        bias[local_start + z] = -100.0
    ws, ids, n_local = [], [], 0
    while True:
        logits = rng.standard_normal((T, E_global)).astype(np.float32) + bias[None, :]
        w, idx = orouting.sigmoid_topk(logits, K)
        local = (idx >= local_start) & (idx < local_start + E_local)
        keep = local.any(axis=1)
        ws.append(w[keep])
        ids.append(idx[keep])
        n_local += int(local.sum())
        if n_local >= min_local:
            break
    return torch.from_numpy(np.concatenate(ws)), torch.from_numpy(np.concatenate(ids))
