"""Numpy restatement of the routing half of the path (test oracle only).

Follows:
  ``model/moe.py:249-255``  softmax gating: top-k of the logits, softmax over
                            the K selected logits only.
  ``model/moe.py:257-265``  sigmoid gating: top-k of sigmoid(logits),
                            weights / (sum + 1e-8).
  ``model/moe.py:267-281``  load-balancing loss E * sum_i f_i * P_i.
  ``model/moe.py:1565-1567`` per-expert token lists in ascending token order
                            (``nonzero``), which is the stable sort of the
                            flat (token, slot) assignments by expert.
  ``model/moe.py:1395-1448`` capacity dropping (``_apply_capacity``): expert
                            e keeps the first ``capacity`` of its tokens in
                            token order; per-expert drop counts.
  ``model/moe.py:1450-1498`` adaptive capacity factor update.

Spec choices the absent ``fp8_flow_moe`` package would have fixed:
  * ties in top-k go to the lower expert index;
  * each expert's group in the permuted buffer is padded to a multiple of
    128 rows (``PAD``) so no 128-row quantisation block straddles experts;
    pad rows hold zeros and map to assignment -1.

Pinning (tests/test_oracle_routing.py): brute-force Python loops over
tokens/experts on small cases; invariants (counts sum to T*K, every
assignment appears once, rows ascending within an expert, offsets multiples
of 128); top-1 softmax weights are exactly 1.0 (``model/moe.py:253-254``).
Capacity: a token-by-token running count per expert (a different algorithm
from the per-expert token lists restated here), the closed cases (capacity
>= T keeps all, capacity 0 drops every routed token), hand-worked cases and
the invariant that no expert keeps more than ``capacity`` tokens.  Adaptive
capacity: hand-computed EMA steps and the clamp to [1, 4].
"""

from __future__ import annotations

import numpy as np

PAD = 128


def topk_lower_index(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest per row, descending, ties -> lower index;
    NaN ranks above every number (torch.topk's order), lower index first."""
    scores = np.asarray(scores)
    nan = np.isnan(scores)
    key = np.where(nan, 0.0, -scores.astype(np.float64))
    cols = np.broadcast_to(np.arange(scores.shape[-1]), scores.shape)
    order = np.lexsort((cols, key, ~nan), axis=-1)
    return order[:, :k].astype(np.int64)


def softmax_topk(logits: np.ndarray, k: int):
    """model/moe.py:249-255."""
    logits = np.asarray(logits, dtype=np.float32)
    idx = topk_lower_index(logits, k)
    sel = np.take_along_axis(logits, idx, axis=-1).astype(np.float64)
    e = np.exp(sel - sel.max(axis=-1, keepdims=True))
    w = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32, copy=False)
    return w, idx


def sigmoid_topk(logits: np.ndarray, k: int):
    """model/moe.py:257-265 (score bias, if any, is already inside ``logits``)."""
    logits = np.asarray(logits, dtype=np.float32)
    s = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32, copy=False)
    idx = topk_lower_index(s, k)
    sel = np.take_along_axis(s, idx, axis=-1).astype(np.float64)
    w = (sel / (sel.sum(axis=-1, keepdims=True) + 1e-8)).astype(np.float32, copy=False)
    return w, idx


def replay_gating(logits: np.ndarray, replay_idx: np.ndarray, k: int):
    """model/moe.py:187-247 (R3 routing replay): p = softmax(logits) over all
    E; weights = p on the replayed experts renormalised by their sum (clamped
    to >= 1e-8); the k largest of that masked distribution, descending (ties
    to the lower index).  Softmax in float64, rounded to fp32 at the end."""
    logits = np.asarray(logits, dtype=np.float64)
    p = np.exp(logits - logits.max(axis=-1, keepdims=True))
    p = p / p.sum(axis=-1, keepdims=True)
    mask = np.zeros_like(p)
    np.put_along_axis(mask, np.asarray(replay_idx, dtype=np.int64), 1.0, axis=-1)
    mp = p * mask
    mp = mp / np.maximum(mp.sum(axis=-1, keepdims=True), 1e-8)
    mp32 = mp.astype(np.float32)
    idx = topk_lower_index(mp32, k)
    return np.take_along_axis(mp32, idx, axis=-1), idx


def l2_normalize(w: np.ndarray) -> np.ndarray:
    """model/moe.py:167-170: w / (||w||_2 + 1e-8) over the K weights (float64 inside)."""
    w64 = np.asarray(w, dtype=np.float64)
    return (w64 / (np.sqrt((w64 * w64).sum(axis=-1, keepdims=True)) + 1e-8)).astype(np.float32)


def z_loss(logits: np.ndarray) -> float:
    """model/moe.py:176-178: mean over tokens of logsumexp(logits)^2 (float64)."""
    lg = np.asarray(logits, dtype=np.float64)
    m = lg.max(axis=-1, keepdims=True)
    lse = (m + np.log(np.exp(lg - m).sum(axis=-1, keepdims=True)))[..., 0]
    return float((lse * lse).mean())


def score_bias_update(score_bias: np.ndarray, tokens_per_expert: np.ndarray, total_tokens: int, gamma: float):
    """model/moe.py:294-321 on one GPU, in fp32 as the reference's tensors are:
    score_bias + gamma * (tokens_per_expert / total - 1 / E); unchanged when
    total is 0.  ``total`` counts tokens (B * S), so the actual fractions sum
    to K (``_update_expert_counts``, :284-292)."""
    sb = np.asarray(score_bias, dtype=np.float32)
    if total_tokens == 0:
        return sb.copy()
    E = sb.size
    actual = np.asarray(tokens_per_expert).astype(np.float32) / np.float32(total_tokens)
    ideal = np.float32(1.0) / np.float32(E)
    return (sb + np.float32(gamma) * (actual - ideal)).astype(np.float32)


def load_balancing_loss(logits: np.ndarray, idx: np.ndarray, num_experts: int) -> float:
    """model/moe.py:267-281: f_i counts every one of the K slots, divided by
    the number of tokens; P_i is the mean softmax over all E experts."""
    logits = np.asarray(logits, dtype=np.float64).reshape(-1, num_experts)
    T = logits.shape[0]
    counts = np.bincount(np.asarray(idx).reshape(-1), minlength=num_experts).astype(np.float64)
    f = counts / T
    p = np.exp(logits - logits.max(axis=-1, keepdims=True))
    p = p / p.sum(axis=-1, keepdims=True)
    P = p.mean(axis=0)
    return float(num_experts * (f * P).sum())


def sort_assignments(idx: np.ndarray, num_experts: int, pad: int = PAD, drop_out_of_range: bool = False):
    """Stable counting sort of the flat assignments a = t*K + k by expert.

    With ``drop_out_of_range`` an index outside [0, E) -- a slot routed to an
    expert this GPU does not hold -- takes no row (``row_of`` = -1) and is not
    counted, as the reference loop never selects it (``model/moe.py:1560-1567``
    walks only the local experts); otherwise such an index raises.

    Returns a dict:
      counts      [E] int32       assignments per expert
      offsets     [E+1] int32     padded group starts (multiples of ``pad``)
      row_of      [T*K] int32     padded row of each assignment (-1: dropped)
      assign_of_row [offsets[E]] int32  assignment in each row, -1 for pad
      perm        [A'] int64      kept assignments in sorted order (unpadded)
    """
    flat = np.asarray(idx, dtype=np.int64).reshape(-1)
    valid = (flat >= 0) & (flat < num_experts)
    if not drop_out_of_range and not valid.all():
        raise ValueError("expert index out of range")
    key = np.where(valid, flat, num_experts)
    counts = np.bincount(key, minlength=num_experts + 1)[:num_experts].astype(np.int64)
    perm = np.argsort(key, kind="stable")[: int(counts.sum())]
    padded = (counts + pad - 1) // pad * pad
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(padded)
    starts = np.zeros(num_experts + 1, dtype=np.int64)
    starts[1:] = np.cumsum(counts)
    row_of = np.full(flat.size, -1, dtype=np.int64)
    pos = np.arange(perm.size)
    e_sorted = flat[perm]
    row_of[perm] = offsets[e_sorted] + (pos - starts[e_sorted])
    assign_of_row = np.full(int(offsets[-1]), -1, dtype=np.int64)
    assign_of_row[row_of[perm]] = perm
    return dict(
        counts=counts.astype(np.int32),
        offsets=offsets.astype(np.int32),
        row_of=row_of.astype(np.int32),
        assign_of_row=assign_of_row.astype(np.int32),
        perm=perm,
    )


def permute_pad(x: np.ndarray, assign_of_row: np.ndarray, top_k: int) -> np.ndarray:
    """Row r of the output is x[assign_of_row[r] // K], zeros for pad rows."""
    import torch

    xt = torch.from_numpy(np.ascontiguousarray(x))
    a = torch.from_numpy(np.asarray(assign_of_row).astype(np.int64))
    valid = (a >= 0)[:, None]
    out = xt.index_select(0, a.clamp(min=0) // top_k)
    return torch.where(valid, out, torch.zeros((), dtype=out.dtype)).numpy()


def unpermute_unpad(y: np.ndarray, row_of: np.ndarray, weights, num_tokens: int, top_k: int):
    """out[t] = sum_k w[t,k] * y[row_of[t*K+k]], summed in fp32 in k order
    (each product and sum rounded to fp32); slots with row_of = -1 (dropped)
    add nothing.  Torch CPU ops on the numpy buffers."""
    import torch

    yt = torch.from_numpy(np.ascontiguousarray(y, dtype=np.float32))
    ro = torch.from_numpy(np.asarray(row_of).reshape(num_tokens, top_k).astype(np.int64))
    if weights is None:
        w = torch.ones(num_tokens, top_k, dtype=torch.float32)
    else:
        w = torch.from_numpy(np.ascontiguousarray(weights, dtype=np.float32).reshape(num_tokens, top_k))
    acc = torch.zeros(num_tokens, yt.shape[1], dtype=torch.float32)
    for k in range(top_k):
        keep = (ro[:, k] >= 0)[:, None]
        term = w[:, k : k + 1] * yt.index_select(0, ro[:, k].clamp(min=0))
        acc = acc + torch.where(keep, term, torch.zeros((), dtype=torch.float32))
    return acc.numpy()


def router_logits(x: np.ndarray, w: np.ndarray, b=None, score_bias=None) -> np.ndarray:
    """model/moe.py:151-154: gate(x.float()) (nn.Linear, fp32) + score_bias.
    Computed in float64 and rounded to fp32 once."""
    out = np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T
    if b is not None:
        out = out + np.asarray(b, dtype=np.float64)
    if score_bias is not None:
        out = out + np.asarray(score_bias, dtype=np.float64)
    return out.astype(np.float32, copy=False)


def capacity_keep(idx: np.ndarray, num_experts: int, capacity: int):
    """``MoEBase._apply_capacity`` (reference model/moe.py:1421-1437): for each
    expert, its tokens in ascending order (``(indices == e).any(-1)
    .nonzero()``); those past the first ``capacity`` are dropped.  Returns
    (keep [T] bool, drops [E] int64, dropped = drops.sum())."""
    idx = np.asarray(idx)
    T = idx.shape[0]
    keep = np.ones(T, dtype=bool)
    drops = np.zeros(num_experts, dtype=np.int64)
    for e in range(num_experts):
        tok = np.nonzero((idx == e).any(axis=-1))[0]
        if tok.shape[0] > capacity:
            keep[tok[capacity:]] = False
            drops[e] = tok.shape[0] - capacity
    return keep, drops, int(drops.sum())


def adaptive_capacity_update(cf: float, ema: float, step: int, idx: np.ndarray, num_experts: int, target: float,
                             ema_coef: float):
    """``_update_adaptive_capacity`` (reference model/moe.py:1450-1498): the
    drop rate the current factor would give, EMA-smoothed; the factor grows
    10% above 1.5x the target, shrinks 5% below 0.5x, clamped to [1, 4].
    Returns (cf, ema, step)."""
    idx = np.asarray(idx)
    T = idx.shape[0]
    capacity = int(cf * T / num_experts)
    est = 0.0
    for e in range(num_experts):
        n = float((idx == e).any(axis=-1).sum())
        if n > capacity:
            est += n - capacity
    rate = est / max(1, T)
    ema = ema_coef * rate + (1 - ema_coef) * ema
    if ema > target * 1.5:
        cf *= 1.1
    elif ema < target * 0.5:
        cf *= 0.95
    return max(1.0, min(4.0, cf)), ema, step + 1
