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
