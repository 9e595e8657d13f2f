"""Token routing on the GPU: top-k gating, load-balancing loss and the
stable counting sort that orders (token, slot) assignments by expert.

Reference behaviour restated by these kernels:
  ``model/moe.py:249-255``   softmax gating (top-k of logits, softmax over the
                             K selected logits)
  ``model/moe.py:257-265``   sigmoid gating (top-k of sigmoid, /(sum + 1e-8))
  ``model/moe.py:267-281``   load-balancing loss E * sum f_i P_i
  ``model/moe.py:1565-1567`` per-expert token lists in ascending token order
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib

PAD_ROWS = 128  # every expert group is padded to a multiple of this many rows


@dataclass
class RoutingPlan:
    """Device-resident result of the counting sort (no host synchronisation).

    counts        [E] int32       assignments per expert
    offsets       [E+1] int32     padded group starts (multiples of 128)
    row_of        [T*K] int32     padded row of assignment a = t*K + k (-1 if its
                                  expert index is outside [0, E))
    assign_of_row [rows_max] int32  assignment held by each row, -1 on padding
    tile_expert   [rows_max/128] int32  expert of each 128-row tile, -1 past the end
    use_fp8       [E] int32       counts[e] >= fp8_gemm_threshold
    """

    num_tokens: int
    top_k: int
    num_experts: int
    rows_max: int
    counts: torch.Tensor
    offsets: torch.Tensor
    row_of: torch.Tensor
    assign_of_row: torch.Tensor
    tile_expert: torch.Tensor
    use_fp8: torch.Tensor

    @property
    def m_tiles(self) -> int:
        return self.rows_max // PAD_ROWS

    def precision_tiles(self):
        """(tiles_fp8, tiles_bf16) [rows_max/128] int32: ``tile_expert`` split
        by the experts' ``use_fp8`` flags (-1 elsewhere), the tile lists of
        the two precisions' producers when the threshold splits the experts
        (``fm_route_tile_masks``; made once per plan, on the device)."""
        tm = getattr(self, "_precision_tiles", None)
        if tm is None:
            n = self.m_tiles
            tf = torch.empty(n, dtype=torch.int32, device=self.tile_expert.device)
            tb = torch.empty_like(tf)
            _lib.call("fm_route_tile_masks", _lib.ptr(self.tile_expert), n, _lib.ptr(self.use_fp8), _lib.ptr(tf),
                      _lib.ptr(tb), _lib.stream_of(tf))
            tm = self._precision_tiles = (tf, tb)
        return tm


def rows_max(num_assignments: int, num_experts: int) -> int:
    """Upper bound of the padded buffer's rows, known without reading counts."""
    return int(_lib.load().fm_route_rows_max(num_assignments, num_experts))


def route_tokens(indices: torch.Tensor, num_experts: int, fp8_gemm_threshold: int = 0,
                 weight_jobs=None) -> RoutingPlan:
    """Stable counting sort of ``indices`` [T, K] (int64 or int32) by expert.

    ``weight_jobs`` = (ctypes FmWeightJob array, count): an expert-weight
    batch run with the sort (``fm_route_sort_weights``: part of its blocks as
    extra workgroups of the sort's launches), as if ``fm_quantize_weight_batch``
    had been called after it on the same stream."""
    _lib.require_device(indices, "indices")
    if indices.dim() != 2:
        indices = indices.reshape(-1, indices.shape[-1])
    if indices.dtype not in (torch.int64, torch.int32):
        raise TypeError(f"indices must be int64 or int32, got {indices.dtype}")
    indices = indices.contiguous()
    T, K = indices.shape
    A = T * K
    lib = _lib.load()
    rmax = int(lib.fm_route_rows_max(A, num_experts))
    dev = indices.device
    i32 = dict(dtype=torch.int32, device=dev)
    counts = torch.empty(num_experts, **i32)
    offsets = torch.empty(num_experts + 1, **i32)
    row_of = torch.empty(max(A, 1), **i32)
    assign_of_row = torch.empty(rmax, **i32)
    tile_expert = torch.empty(rmax // PAD_ROWS, **i32)
    use_fp8 = torch.empty(num_experts, **i32)
    ws_bytes = int(lib.fm_route_workspace_bytes(A, num_experts))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    args = (_lib.ptr(indices), int(indices.dtype == torch.int64), T, K, num_experts, int(fp8_gemm_threshold),
            _lib.ptr(counts), _lib.ptr(offsets), _lib.ptr(row_of), _lib.ptr(assign_of_row), rmax,
            _lib.ptr(tile_expert), _lib.ptr(use_fp8), _lib.ptr(ws), ws_bytes)
    if weight_jobs is None:
        _lib.call("fm_route_sort", *args, _lib.stream_of(indices))
    else:
        _lib.call("fm_route_sort_weights", *args, weight_jobs[0], weight_jobs[1], _lib.stream_of(indices))
    return RoutingPlan(T, K, num_experts, rmax, counts, offsets, row_of[:A], assign_of_row,
                       tile_expert, use_fp8)


@dataclass
class CapacitySelection:
    """Tokens kept by expert capacity (``fm_capacity_select``).

    pos_of      [T] int32       position of each token among the kept ones, -1 if dropped
    kept_index  [n_kept] int32  the kept tokens in token order
    drops       list[int] [E]   tokens beyond each expert's capacity
    dropped     int             sum of drops (a token over two experts' capacity counts twice)
    """

    capacity: int
    n_kept: int
    pos_of: torch.Tensor
    kept_index: torch.Tensor
    drops: list
    dropped: int


def capacity_select(indices: torch.Tensor, plan: RoutingPlan, capacity: int) -> CapacitySelection:
    """The token dropping of ``MoEBase._apply_capacity`` (reference
    ``model/moe.py:1395-1448``): expert e keeps the first ``capacity`` of its
    tokens in token order; a token over the capacity of any of its experts is
    dropped.  ``plan`` is ``route_tokens`` of the same ``indices`` [T, K].
    Reads n_kept and the drop counts back to the host (one synchronisation,
    as the reference's ``nonzero`` and ``dropped`` are host values)."""
    _lib.require_device(indices, "indices")
    indices = indices.reshape(-1, indices.shape[-1]).contiguous()
    if indices.dtype not in (torch.int64, torch.int32):
        raise TypeError(f"indices must be int64 or int32, got {indices.dtype}")
    T, K = indices.shape
    if T != plan.num_tokens or K != plan.top_k:
        raise ValueError("indices do not match the routing plan")
    if capacity < 0:
        raise ValueError("capacity must be >= 0")
    E = plan.num_experts
    dev = indices.device
    pos_of = torch.empty(max(T, 1), dtype=torch.int32, device=dev)
    kept = torch.empty(max(T, 1), dtype=torch.int32, device=dev)
    tally = torch.empty(1 + E, dtype=torch.int32, device=dev)      # n_kept, drops[E]
    ws_bytes = int(_lib.load().fm_capacity_workspace_bytes(T))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _lib.call("fm_capacity_select", _lib.ptr(indices), int(indices.dtype == torch.int64), T, K, E,
              _lib.ptr(plan.counts), _lib.ptr(plan.offsets), _lib.ptr(plan.row_of), int(capacity), _lib.ptr(pos_of),
              _lib.ptr(kept), _lib.ptr(tally), _lib.ptr(tally[1:]), _lib.ptr(ws), ws_bytes, _lib.stream_of(indices))
    host = tally.cpu().tolist()
    n_kept, drops = int(host[0]), [int(v) for v in host[1:]]
    return CapacitySelection(int(capacity), n_kept, pos_of[:T], kept[:n_kept], drops, sum(drops))


def gather_rows(src: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """``out[i] = src[index[i]]`` over the first dimension, zeros where
    ``index[i]`` is outside [0, src.shape[0]) (``fm_gather_rows``; index
    int32).  Not differentiable by itself: ``select_rows`` is."""
    _lib.require_device(src, "src")
    if index.dtype != torch.int32:
        raise TypeError("index must be int32")
    src = src.contiguous()
    n_src = src.shape[0]
    row = int(torch.Size(src.shape[1:]).numel()) * src.element_size()
    out = torch.empty((index.shape[0], *src.shape[1:]), dtype=src.dtype, device=src.device)
    if row % 4:
        raise ValueError("fm_gather_rows moves rows of a multiple of 4 bytes")
    _lib.call("fm_gather_rows", _lib.ptr(src), n_src, row, _lib.ptr(index.contiguous()), index.shape[0], row,
              _lib.ptr(out), row, _lib.stream_of(src))
    return out


class _SelectRows(torch.autograd.Function):
    @staticmethod
    def forward(ctx, src, index, inverse):
        ctx.save_for_backward(inverse)
        return gather_rows(src, index)

    @staticmethod
    def backward(ctx, g):
        (inverse,) = ctx.saved_tensors
        return gather_rows(g, inverse), None, None


def select_rows(src: torch.Tensor, index: torch.Tensor, inverse: torch.Tensor) -> torch.Tensor:
    """Differentiable ``gather_rows``: ``inverse`` maps each row of ``src`` to
    the output row that holds it, or -1 (index must be injective), so the
    gradient is ``gather_rows(grad, inverse)``: zeros for rows not selected."""
    return _SelectRows.apply(src, index, inverse)


def _gating_code(gating) -> int:
    return {"softmax": _lib.GATING_SOFTMAX, "sigmoid": _lib.GATING_SIGMOID}[str(gating).lower().split(".")[-1]]


def _norm_flags(normalize) -> int:
    if normalize is None:
        return 0
    if str(normalize).lower() == "l2":
        return _lib.GATING_L2_NORMALIZE
    raise ValueError(f"normalize_expert_weights must be None or 'l2', got {normalize!r}")


N_WAVES = 1024   # waves of the gating kernel = rows of its per-wave partials


def topk_gating(logits: torch.Tensor, top_k: int, gating: str = "softmax",
                return_prob_partial: bool = False, *, replay_indices=None, normalize=None,
                return_z_partial: bool = False):
    """Top-k gating over the last dimension of fp32 ``logits`` [..., E].

    ``replay_indices`` [..., K] (R3 routing replay, reference
    ``model/moe.py:187-247``): the weights are softmax(logits) restricted to
    those experts and renormalised, the K largest in order, for either gating.
    ``normalize="l2"`` divides the K weights by their l2 norm + 1e-8
    (``:167-170``).  Selection: NaN above every number, then larger, then the
    lower expert index; no expert twice.

    Returns (weights [..., K] fp32, indices [..., K] int64[, prob_partial][, z_partial])."""
    _lib.require_device(logits, "logits")
    if logits.dtype != torch.float32:
        raise TypeError("logits must be float32 (the router runs the gate in fp32)")
    E = logits.shape[-1]
    lead = logits.shape[:-1]
    lg = logits.reshape(-1, E).contiguous()
    T = lg.shape[0]
    w = torch.empty(T, top_k, dtype=torch.float32, device=lg.device)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=lg.device)
    part = torch.empty(N_WAVES, E, dtype=torch.float32, device=lg.device) if return_prob_partial else None
    zpart = torch.empty(N_WAVES, dtype=torch.float32, device=lg.device) if return_z_partial else None
    rep = None
    if replay_indices is not None:
        rep = replay_indices.reshape(T, top_k)
        if rep.dtype not in (torch.int64, torch.int32):
            raise TypeError("replay_indices must be int64 or int32")
        rep = rep.contiguous()
    _lib.call("fm_topk_gating", _lib.ptr(lg), T, E, E, top_k, _gating_code(gating), _norm_flags(normalize),
              _lib.ptr(rep), int(rep is not None and rep.dtype == torch.int64), _lib.ptr(w), _lib.ptr(idx), 1,
              _lib.ptr(part), _lib.ptr(zpart), N_WAVES, _lib.stream_of(lg))
    w = w.reshape(*lead, top_k)
    idx = idx.reshape(*lead, top_k)
    out = (w, idx)
    if return_prob_partial:
        out += (part,)
    if return_z_partial:
        out += (zpart,)
    return out


def load_balancing_loss(prob_partial: torch.Tensor, counts: torch.Tensor, num_tokens: int,
                        z_partial: torch.Tensor = None, z_loss_multiplier: float = 0.0) -> torch.Tensor:
    """E * sum_e (counts[e]/T) * mean_t softmax(logits)[t, e] (+ z_loss_multiplier
    * mean_t logsumexp(logits[t])^2 with ``z_partial``) as a 0-d fp32 tensor."""
    E = counts.numel()
    loss = torch.empty((), dtype=torch.float32, device=counts.device)
    _lib.call("fm_aux_loss", _lib.ptr(prob_partial), prob_partial.shape[0], _lib.ptr(counts), E,
              num_tokens, _lib.ptr(z_partial), float(z_loss_multiplier), _lib.ptr(loss), _lib.stream_of(counts))
    return loss


# ================================================================== router ====
def _x_dtype(x: torch.Tensor) -> int:
    if x.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if x.dtype == torch.float32:
        return _lib.DTYPE_F32
    raise TypeError(f"router input must be bfloat16 or float32, got {x.dtype}")


def _gate_params(gate_weight: torch.Tensor, gate_bias, score_bias):
    """The gate weight and bias as stored (fp32 or bf16; the bias in the
    weight's dtype, as nn.Linear keeps them) and the fp32 score bias."""
    w = gate_weight.detach()
    if w.dtype not in (torch.float32, torch.bfloat16):
        w = w.float()
    if w.stride(-1) != 1 or w.stride(0) % 4:
        w = w.contiguous()
    b = None if gate_bias is None else gate_bias.detach().to(w.dtype).contiguous()
    sb = None if score_bias is None else score_bias.detach().float().contiguous()
    return w, b, sb


def _dt_code(t: torch.Tensor) -> int:
    return _lib.DTYPE_BF16 if t.dtype == torch.bfloat16 else _lib.DTYPE_F32


def router_logits(x: torch.Tensor, gate_weight: torch.Tensor, gate_bias=None, score_bias=None) -> torch.Tensor:
    """fp32 logits [T, E] = x.float() @ gate_weight.T + gate_bias (+ score_bias),
    the gate of MoERouter.forward (reference model/moe.py:151-154); a bf16 gate
    is read as stored (its values widened exactly)."""
    _lib.require_device(x, "x")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w, b, sb = _gate_params(gate_weight, gate_bias, score_bias)
    E, D = w.shape
    T = x2.shape[0]
    logits = torch.empty(T, E, dtype=torch.float32, device=x2.device)
    _lib.call("fm_router_logits", _lib.ptr(x2), _x_dtype(x2), x2.stride(0), T, D, _lib.ptr(w), _dt_code(w),
              w.stride(0), _lib.ptr(b), _lib.ptr(sb), E, _lib.ptr(logits), logits.stride(0), _lib.stream_of(x2))
    return logits


def expert_counts(indices: torch.Tensor, num_experts: int, load_tracker=None) -> torch.Tensor:
    """[E] int32 number of routed slots per expert (indices outside [0, E) ignored);
    with ``load_tracker`` also added to its running totals (with the number of
    tokens, indices.numel() / K)."""
    idx = indices.contiguous()
    counts = torch.empty(num_experts, dtype=torch.int32, device=idx.device)
    acc = tot = None
    tokens = 0
    if load_tracker is not None:
        acc, tot = load_tracker.tokens_per_expert, load_tracker.total_tokens
        tokens = idx.numel() // idx.shape[-1]
    _lib.call("fm_expert_counts", _lib.ptr(idx), int(idx.dtype == torch.int64), idx.numel(), num_experts,
              _lib.ptr(counts), _lib.ptr(acc), _lib.ptr(tot), tokens, _lib.stream_of(idx))
    return counts


class ExpertLoadTracker:
    """Device-resident per-expert token counts of the DeepSeek-V3 score-bias
    update (reference ``MoERouter._update_expert_counts`` / ``post_batch``,
    ``model/moe.py:284-321``), with every tensor on the GPU (the reference adds
    ``counts.cpu()`` into a buffer that lives on the model's device).

    ``route(..., load_tracker=t)`` adds each forward's counts; ``t.post_batch(
    score_bias, gamma)`` applies ``score_bias += gamma * (counts / tokens - 1 /
    E)`` (the reference's sign) and clears the totals, no host sync.  With
    expert parallelism all-reduce ``tokens_per_expert`` and ``total_tokens``
    before ``post_batch``, as the reference does."""

    def __init__(self, num_experts: int, device):
        self.num_experts = num_experts
        self.tokens_per_expert = torch.zeros(num_experts, dtype=torch.int64, device=device)
        self.total_tokens = torch.zeros(1, dtype=torch.int64, device=device)

    @torch.no_grad()
    def post_batch(self, score_bias: torch.Tensor, gamma: float) -> None:
        if score_bias.dtype != torch.float32 or not score_bias.is_contiguous() or score_bias.numel() != self.num_experts:
            raise ValueError("score_bias must be a contiguous float32 tensor of num_experts values")
        _lib.require_device(score_bias, "score_bias")
        _lib.call("fm_score_bias_update", _lib.ptr(self.tokens_per_expert), _lib.ptr(self.total_tokens),
                  self.num_experts, float(gamma), _lib.ptr(score_bias), _lib.stream_of(score_bias))


@dataclass
class RouterState:
    """What the router's backward needs from its forward."""

    logits: torch.Tensor     # [T, E] fp32, score bias included
    indices: torch.Tensor    # [T, K]
    counts: torch.Tensor     # [E] int32
    gating: int
    flags: int
    replay: bool
    z_mult: float


def router_forward(x2, gate_weight, gate_bias, score_bias, top_k, gating, replay=None, normalize=None,
                   z_mult=0.0, tracker=None):
    """Gate, gating, counts and aux loss of MoERouter.forward (reference
    model/moe.py:133-184) on x2 [T, D]: (weights [T, K], indices [T, K], aux, state).
    One library call (fm_router_forward): for E <= 8 and D = 512 n <= 2048 a
    single pass over x forms the logits, the gating, the loss partials and the
    expert histograms, and one small kernel the counts and the loss."""
    T, D = x2.shape
    if T == 0:
        raise ValueError("the router needs at least one token")
    w_, b, sb = _gate_params(gate_weight, gate_bias, score_bias)
    E = w_.shape[0]
    if w_.shape[1] != D:
        raise ValueError(f"gate_weight must be [E, {D}], got {tuple(w_.shape)}")
    K = int(top_k)
    dev = x2.device
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    w = torch.empty(T, K, dtype=torch.float32, device=dev)
    idx = torch.empty(T, K, dtype=torch.int64, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    aux = torch.empty((), dtype=torch.float32, device=dev)
    ws = torch.empty(int(_lib.load().fm_router_forward_workspace_bytes(T, E)), dtype=torch.uint8, device=dev)
    rep = None
    if replay is not None:
        rep = replay.reshape(T, K)
        if rep.dtype not in (torch.int64, torch.int32):
            raise TypeError("replay_indices must be int64 or int32")
        rep = rep.contiguous()
    acc = tot = None
    if tracker is not None:
        acc, tot = tracker.tokens_per_expert, tracker.total_tokens
    _lib.call("fm_router_forward", _lib.ptr(x2), _x_dtype(x2), x2.stride(0), T, D, _lib.ptr(w_), _dt_code(w_),
              w_.stride(0), _lib.ptr(b), _lib.ptr(sb), E, K, _gating_code(gating), _norm_flags(normalize),
              _lib.ptr(rep), int(rep is not None and rep.dtype == torch.int64), _lib.ptr(logits), logits.stride(0),
              _lib.ptr(w), _lib.ptr(idx), 1, _lib.ptr(counts), _lib.ptr(acc), _lib.ptr(tot), float(z_mult),
              _lib.ptr(aux), _lib.ptr(ws), ws.numel(), _lib.stream_of(x2))
    state = RouterState(logits, idx, counts, _gating_code(gating), _norm_flags(normalize), replay is not None,
                        float(z_mult))
    return w, idx, aux, state


@dataclass
class RouterDotInputs:
    """What the router-weight gradient is formed from when the gating backward
    forms it itself: dw[t, k] = <dout[t], y[row_of[t K + k]]> (the expert
    block's upstream gradient and its saved expert outputs, both bf16)."""

    dout: torch.Tensor      # [T, D]
    y: torch.Tensor         # [rows, D]
    row_of: torch.Tensor    # [T * K] int32


def router_backward(state: RouterState, x2, gate_weight, dweights, daux, need_x=True, need_w=True, need_b=True,
                    bias_dtype=None, dot: RouterDotInputs = None):
    """Gradients of the router (dx [T, D] in x2's dtype, dW [E, D] in the gate
    weight's dtype, db [E] in ``bias_dtype`` (default fp32); None where not
    needed) from those of its weights [T, K] (or ``dot``: formed in the gating
    backward from the expert outputs, K <= 8) and aux loss, and the logits'
    gradient dlogits [T, E] fp32 they come from."""
    logits, idx = state.logits, state.indices
    T, D = x2.shape
    E = logits.shape[1]
    K = idx.shape[1]
    dev = x2.device
    st = _lib.stream_of(x2)
    dwts = None if dweights is None else dweights.reshape(T, K).float().contiguous()
    da = None if daux is None else daux.reshape(1).float().contiguous()
    dlogits = torch.empty(T, E, dtype=torch.float32, device=dev)
    if dot is not None:
        _lib.call("fm_gating_grad_dot", _lib.ptr(logits), T, E, logits.stride(0), K, state.gating, state.flags,
                  int(state.replay), _lib.ptr(idx), int(idx.dtype == torch.int64), None, _lib.ptr(dot.dout),
                  dot.dout.stride(0), _lib.ptr(dot.y), dot.y.stride(0), _lib.ptr(dot.row_of), D, None, _lib.ptr(da),
                  _lib.ptr(state.counts), state.z_mult, _lib.ptr(dlogits), dlogits.stride(0), st)
    elif dwts is None and da is None:
        dlogits.zero_()
    else:
        _lib.call("fm_gating_grad", _lib.ptr(logits), T, E, logits.stride(0), K, state.gating, state.flags,
                  int(state.replay), _lib.ptr(idx), int(idx.dtype == torch.int64), _lib.ptr(dwts), _lib.ptr(da),
                  _lib.ptr(state.counts), state.z_mult, _lib.ptr(dlogits), dlogits.stride(0), st)
    w, _, _ = _gate_params(gate_weight, None, None)
    dx = torch.empty_like(x2) if need_x else None
    dW = torch.empty(E, D, dtype=w.dtype, device=dev) if need_w else None
    db = torch.empty(E, dtype=bias_dtype or torch.float32, device=dev) if need_b else None
    ws = None
    if dW is not None or db is not None:
        ws = torch.empty(int(_lib.load().fm_router_workspace_bytes(T, D, E)), dtype=torch.uint8, device=dev)
    if dx is not None or dW is not None or db is not None:
        _lib.call("fm_router_backward", _lib.ptr(dlogits), dlogits.stride(0), _lib.ptr(x2), _x_dtype(x2),
                  x2.stride(0), T, D, _lib.ptr(w), _dt_code(w), w.stride(0), E, _lib.ptr(dx),
                  0 if dx is None else dx.stride(0), _lib.ptr(dW), _lib.DTYPE_F32 if dW is None else _dt_code(dW),
                  0 if dW is None else dW.stride(0), _lib.ptr(db), _lib.DTYPE_F32 if db is None else _dt_code(db),
                  _lib.ptr(ws), 0 if ws is None else ws.numel(), st)
    return dx, dW, db, dlogits


class _RouterFunction(torch.autograd.Function):
    """Gate + gating (top-k or replay, optional l2) + load-balancing loss (+ z-loss),
    forward and backward on the GPU."""

    @staticmethod
    def forward(ctx, x, gate_weight, gate_bias, score_bias, top_k, gating, replay, normalize, z_mult, tracker):
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        w, idx, aux, state = router_forward(x2, gate_weight, gate_bias, score_bias, top_k, gating, replay,
                                            normalize, z_mult, tracker)
        ctx.save_for_backward(x2, gate_weight)
        ctx.state = state
        ctx.has_bias = gate_bias is not None
        ctx.bias_dtype = None if gate_bias is None else gate_bias.dtype
        ctx.lead = lead
        ctx.mark_non_differentiable(idx)
        ctx.set_materialize_grads(False)   # no zero gradient for the indices
        return w.reshape(*lead, top_k), idx.reshape(*lead, top_k), aux

    @staticmethod
    def backward(ctx, dweights, _dindices, daux):
        x2, gate_weight = ctx.saved_tensors
        need_x, need_w, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        dx, dW, db, _ = router_backward(ctx.state, x2, gate_weight, dweights, daux, need_x, need_w,
                                        need_b and ctx.has_bias, bias_dtype=ctx.bias_dtype)
        if dx is not None:
            dx = dx.reshape(*ctx.lead, x2.shape[1])
        if dW is not None:
            dW = dW.to(gate_weight.dtype)
        return dx, dW, db, None, None, None, None, None, None, None


def route(x: torch.Tensor, gate_weight: torch.Tensor, gate_bias=None, *, top_k: int, gating: str = "softmax",
          score_bias=None, replay_indices=None, normalize_expert_weights=None, z_loss_multiplier=None,
          load_tracker: ExpertLoadTracker = None, jitter_eps=None, training: bool = True):
    """MoERouter.forward on the GPU (reference model/moe.py:133-184): with
    ``jitter_eps`` and ``training``, x + randn_like(x) * jitter_eps first
    (:145-148, torch's generator, so a seeded run draws the reference's
    noise), then fp32 gate logits x.float() @ W.T + b (+ score_bias) -> gating
    (softmax over the K selected logits, sigmoid / (sum + 1e-8), or R3 replay
    of ``replay_indices``) -> optional l2 normalisation of the weights ->
    (weights [..., K] fp32, indices [..., K] int64, aux loss = E * sum_i f_i P_i
    (+ z_loss_multiplier * mean logsumexp(logits)^2)).  ``load_tracker``
    accumulates the per-expert counts for ``ExpertLoadTracker.post_batch``
    (``_update_expert_counts``, :284-292; the reference does this whenever it
    has a score bias).  Differentiable in x, gate_weight and gate_bias through
    the weights and the loss."""
    _lib.require_device(x, "x")
    if jitter_eps is not None and training:
        x = x + torch.randn_like(x) * jitter_eps
    z = 0.0 if z_loss_multiplier is None else float(z_loss_multiplier)
    return _RouterFunction.apply(x, gate_weight, gate_bias, score_bias, int(top_k), gating, replay_indices,
                                 normalize_expert_weights, z, load_tracker)
