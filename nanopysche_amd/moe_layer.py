"""The MoE layer on the MI355X path: router, FP8-Flow-MoE expert block and an
optional shared expert as one differentiable call -- the composition of
``MoEBase.forward`` (reference ``model/moe.py:1338-1393``: route ->
expert compute -> combine -> shared expert) at expert-parallel size 1, with
the router of ``MoERouter.forward`` (``:133-184``).

Beyond calling ``route`` and ``FP8FlowMoECompute`` one after the other, the
layer runs both under one autograd node, so the input gradient -- which
autograd would otherwise form as the sum of the router's and the experts'
shares in a separate pass -- is summed inside the expert block's unpermute,
and the router's gating gradient is formed as soon as the experts' backward
has the router-weight gradient.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .flow_moe import FP8FlowMoECompute, FP8FlowMoEConfig, FP8SharedExpertCompute
from .norm import DEFAULT_EPS, rmsnorm
from .routing import (ExpertLoadTracker, capacity_select, gather_rows, route, route_tokens, router_backward,
                      router_forward, select_rows)


class _BlockCtx:
    """The part of an autograd ctx FP8FlowMoECompute's forward and backward use,
    so they can run inside the layer's own autograd Function."""

    def __init__(self, needs_input_grad):
        self.needs_input_grad = needs_input_grad
        self.saved_tensors = ()

    def save_for_backward(self, *tensors):
        self.saved_tensors = tensors


class _MoELayerFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gate_weight, gate_bias, w1, w2, w3, layer, replay, tracker, noise):
        lead = x.shape[:-1]
        D = x.shape[-1]
        x2 = _bf16_rows(x)
        # the router's input: x, or x + noise (jitter) in x's dtype
        xr = x2 if noise is None else _bf16_rows(x + noise)
        w, idx, aux, state = router_forward(xr, gate_weight, gate_bias, layer.score_bias, layer.top_k, layer.gating,
                                            replay, layer.normalize_expert_weights, layer.z_loss_multiplier, tracker)
        need_x, need_gw, need_gb = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        bctx = _BlockCtx((need_x, need_x or need_gw or need_gb, *ctx.needs_input_grad[3:6], False, False))
        out = layer.block._forward(bctx, x2, w, w1, w2, w3, idx)
        ctx.save_for_backward(xr, gate_weight)
        ctx.state = state
        ctx.bctx = bctx
        ctx.layer = layer
        ctx.lead = lead
        ctx.x_dtype = x.dtype
        ctx.has_bias = gate_bias is not None
        ctx.bias_dtype = None if gate_bias is None else gate_bias.dtype
        ctx.set_materialize_grads(False)
        return out.to(x.dtype).reshape(*lead, D), aux

    @staticmethod
    def backward(ctx, dout, daux):
        x2, gate_weight = ctx.saved_tensors
        T, D = x2.shape
        need_x, need_gw, need_gb = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        if dout is None:
            dout = torch.zeros(T, D, dtype=torch.bfloat16, device=x2.device)
        grads = {}

        def on_router_grad(dw, can_fold, dot=None):
            # E <= 8: the unpermute forms the router's share of dx from dlogits and
            # the gate weight itself; otherwise the router's own kernel writes it.
            # With `dot` the gating backward forms the router-weight gradient from
            # the expert outputs in its own pass.
            fold = need_x and can_fold and ctx.state.logits.shape[1] <= 8
            dx_r, dW, db, dlogits = router_backward(ctx.state, x2, gate_weight, dw, daux, need_x and not fold,
                                                    need_gw, need_gb and ctx.has_bias, bias_dtype=ctx.bias_dtype,
                                                    dot=dot)
            grads["gw"], grads["gb"] = dW, db
            if fold:
                return {"dlogits": dlogits, "gate_w": gate_weight}
            return {} if dx_r is None else {"addend": dx_r}

        on_router_grad.fused_dot = True
        dx, _, dW1, dW2, dW3, _, _ = ctx.layer.block._backward(ctx.bctx, dout.reshape(T, D), on_router_grad)
        ctx.bctx = None
        dx = None if not need_x else dx.to(ctx.x_dtype).reshape(*ctx.lead, D)
        dgw = grads.get("gw")
        if dgw is not None:
            dgw = dgw.to(gate_weight.dtype)
        return dx, dgw, grads.get("gb"), dW1, dW2, dW3, None, None, None, None


def _bf16_rows(x):
    """x as contiguous bf16 rows [-1, D] (differentiable)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    return x2.contiguous()


class FP8FlowMoELayer:
    """``MoEBase.forward`` at expert-parallel size 1 on the MI355X path:
    ``(out, aux_loss) = layer(x)`` with x [..., D].

    Router (``MoERouter``, reference ``model/moe.py:133-184``): fp32 gate
    ``x.float() @ gate_weight.T + gate_bias (+ score_bias)``, softmax or
    sigmoid top-k gating (or R3 replay of ``replay_indices``), optional l2
    weight normalisation, load-balancing loss plus optional z-loss.  Experts:
    ``FP8FlowMoECompute`` with the given FP8 recipe and threshold.  Shared
    expert (``shared_hidden_size``): ``FP8SharedExpertCompute``, added out of
    place as ``:1383-1384`` does.  Pre-norm (``pre_norm=True``): the layer
    takes the residual stream h and applies RMSNorm with ``norm_weight``
    first, as ``MoEHybridTransformerBlock`` feeds ``self.moe_norm(h)`` to the
    MoE (``model/transformer.py:261-263``); the residual add stays with the
    caller.  Differentiable in x, the gate weight and bias, w1, w2, w3, the
    norm weight and the shared expert's weights; the object owns no
    parameters (``set_weights`` borrows them).

    Training-time options of the reference, both off by default: router
    jitter (``jitter_eps``: the router sees x + randn_like(x) * jitter_eps
    while ``training``, ``:145-148``) and capacity dropping
    (``capacity_factor``, optionally ``adaptive_capacity``: a token beyond
    the capacity int(capacity_factor * T / E) of any of its experts is
    dropped, its output is zero and the shared expert skips it too,
    ``:1351-1356``, ``:1386-1391``, ``:1395-1498``; drop statistics as
    ``:1787-1825`` keeps them).  With a capacity factor the layer runs the
    router, the expert block and the shared expert as separate autograd
    nodes on the kept tokens."""

    def __init__(self, config: FP8FlowMoEConfig, d_model: int, hidden_size: int, num_experts: int, top_k: int,
                 gating: str = "softmax", fp8_gemm_threshold: int = 0,
                 normalize_expert_weights: Optional[str] = None, z_loss_multiplier: Optional[float] = None,
                 shared_hidden_size: Optional[int] = None, pre_norm: bool = False, norm_eps: float = DEFAULT_EPS,
                 jitter_eps: Optional[float] = None, capacity_factor: Optional[float] = None,
                 adaptive_capacity: bool = False, adaptive_capacity_target: float = 0.01,
                 adaptive_capacity_ema: float = 0.3):
        self.block = FP8FlowMoECompute(config, d_model, hidden_size, num_experts, fp8_gemm_threshold)
        self.num_experts = num_experts
        self.top_k = int(top_k)
        self.gating = gating
        self.normalize_expert_weights = normalize_expert_weights
        self.z_loss_multiplier = 0.0 if z_loss_multiplier is None else float(z_loss_multiplier)
        self.shared = (FP8SharedExpertCompute(config, d_model, shared_hidden_size, fp8_gemm_threshold)
                       if shared_hidden_size else None)
        self.gate_weight = self.gate_bias = self.score_bias = None
        self.pre_norm = bool(pre_norm)
        self.norm_eps = float(norm_eps)
        self.norm_weight = None
        self.jitter_eps = jitter_eps
        self.training = True
        self.capacity_factor = capacity_factor
        self.adaptive_capacity = bool(adaptive_capacity)
        self.adaptive_capacity_target = float(adaptive_capacity_target)
        self.adaptive_capacity_ema = float(adaptive_capacity_ema)
        self.reset_drop_stats()

    def train(self, mode: bool = True) -> "FP8FlowMoELayer":
        """Training mode (jitter on when ``jitter_eps`` is set), as nn.Module.train."""
        self.training = bool(mode)
        return self

    def eval(self) -> "FP8FlowMoELayer":
        return self.train(False)

    # ------------------------------------------------------ drop statistics --
    @property
    def drop_rate(self) -> float:
        """total dropped / total tokens routed (reference ``model/moe.py:1787-1791``)."""
        return 0.0 if self._total_tokens_routed == 0 else self._total_dropped / self._total_tokens_routed

    @property
    def per_expert_drops(self) -> Optional[torch.Tensor]:
        """Per-expert drop counts of the last forward (int64, on the device)."""
        return self._per_expert_drop_counts

    @property
    def adaptive_drop_rate_ema(self) -> float:
        return self._adaptive_capacity_ema_drop_rate

    def reset_drop_stats(self) -> None:
        self._last_dropped = 0
        self._total_dropped = 0
        self._total_tokens_routed = 0
        self._per_expert_drop_counts = None
        self._adaptive_capacity_ema_drop_rate = 0.0
        self._adaptive_capacity_step = 0

    def get_drop_stats(self) -> dict:
        """Snapshot of the drop statistics, keyed as reference ``:1808-1825``."""
        pe = self._per_expert_drop_counts
        return {
            "last_dropped": self._last_dropped,
            "total_dropped": self._total_dropped,
            "total_tokens_routed": self._total_tokens_routed,
            "drop_rate": self.drop_rate,
            "per_expert_drops": None if pe is None else pe.tolist(),
            "capacity_factor": self.capacity_factor,
            "adaptive_capacity_enabled": self.adaptive_capacity,
            "adaptive_drop_rate_ema": self._adaptive_capacity_ema_drop_rate,
            "adaptive_capacity_step": self._adaptive_capacity_step,
        }

    def _update_adaptive_capacity(self, num_tokens: int, counts) -> None:
        """``_update_adaptive_capacity`` (reference ``model/moe.py:1450-1498``)
        from the routing sort's per-expert counts (a token's K experts are
        distinct, so counts[e] is its number of tokens)."""
        cf = self.capacity_factor
        capacity = int(cf * num_tokens / self.num_experts)
        estimated = sum(float(c - capacity) for c in counts if c > capacity)
        rate = estimated / max(1, num_tokens)
        a = self.adaptive_capacity_ema
        self._adaptive_capacity_ema_drop_rate = a * rate + (1 - a) * self._adaptive_capacity_ema_drop_rate
        self._adaptive_capacity_step += 1
        if self._adaptive_capacity_ema_drop_rate > self.adaptive_capacity_target * 1.5:
            cf *= 1.1
        elif self._adaptive_capacity_ema_drop_rate < self.adaptive_capacity_target * 0.5:
            cf *= 0.95
        self.capacity_factor = max(1.0, min(4.0, cf))

    def set_weights(self, gate_weight: torch.Tensor, gate_bias: Optional[torch.Tensor], w1: torch.Tensor,
                    w2: torch.Tensor, w3: torch.Tensor, score_bias: Optional[torch.Tensor] = None,
                    shared: Optional[tuple] = None, norm_weight: Optional[torch.Tensor] = None) -> None:
        """gate_weight [E, D] (+ gate_bias [E]) of the router's nn.Linear, the
        experts' w1, w2, w3 [E*H, D], the DeepSeek-V3 score bias [E] (optional),
        the shared expert's (w1, w2, w3) [H_s, D] each when it has one, and the
        RMSNorm weight [D] exactly when the layer is pre-norm."""
        if tuple(gate_weight.shape) != (self.num_experts, self.block.d_model):
            raise ValueError(f"gate_weight must be [E, D] = [{self.num_experts}, {self.block.d_model}]")
        self.gate_weight, self.gate_bias, self.score_bias = gate_weight, gate_bias, score_bias
        self.block.set_weights(w1, w2, w3)
        if (shared is None) != (self.shared is None):
            raise ValueError("shared expert weights must be given exactly when the layer has a shared expert")
        if shared is not None:
            self.shared.set_weights(*shared)
        if (norm_weight is None) == self.pre_norm:
            raise ValueError("norm_weight must be given exactly when the layer is pre-norm")
        if norm_weight is not None and tuple(norm_weight.shape) != (self.block.d_model,):
            raise ValueError(f"norm_weight must be [D] = [{self.block.d_model}]")
        self.norm_weight = norm_weight

    def __call__(self, x: torch.Tensor, replay_indices: Optional[torch.Tensor] = None,
                 load_tracker: Optional[ExpertLoadTracker] = None):
        if self.gate_weight is None:
            raise RuntimeError("set_weights() must be called before the layer runs")
        _lib.require_device(x, "x")
        if self.pre_norm:
            x = rmsnorm(x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16), self.norm_weight, self.norm_eps)
        noise = None
        if self.jitter_eps is not None and self.training:
            noise = torch.randn_like(x) * self.jitter_eps
        if self.capacity_factor is not None:
            return self._forward_with_capacity(x, noise, replay_indices, load_tracker)
        w1, w2, w3 = self.block._w
        self.block._record = torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (x, self.gate_weight, self.gate_bias, w1, w2, w3))
        out, aux = _MoELayerFunction.apply(x, self.gate_weight, self.gate_bias, w1, w2, w3, self, replay_indices,
                                           load_tracker, noise)
        if self.shared is not None:
            out = out + self.shared(x)
        return out, aux

    def _forward_with_capacity(self, x, noise, replay_indices, load_tracker):
        """MoEBase.forward with ``capacity_factor`` (reference ``model/moe.py:1338-1393``):
        route all tokens, drop those over capacity (``_apply_capacity``), run
        the experts and the shared expert on the kept tokens and scatter
        their outputs into zeros."""
        lead, D = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, D)
        xr = x2 if noise is None else x2 + noise.reshape(-1, D)
        w, idx, aux = route(_bf16_rows(xr), self.gate_weight, self.gate_bias, top_k=self.top_k,
                            gating=self.gating, score_bias=self.score_bias, replay_indices=replay_indices,
                            normalize_expert_weights=self.normalize_expert_weights,
                            z_loss_multiplier=self.z_loss_multiplier, load_tracker=load_tracker)
        T, E = x2.shape[0], self.num_experts
        plan = route_tokens(idx, E)
        if self.adaptive_capacity:
            self._update_adaptive_capacity(T, plan.counts.cpu().tolist())
        sel = capacity_select(idx, plan, int(self.capacity_factor * T / E))
        self._per_expert_drop_counts = torch.tensor(sel.drops, dtype=torch.int64, device=x.device)
        self._last_dropped = sel.dropped
        self._total_dropped += sel.dropped
        self._total_tokens_routed += T
        xb = _bf16_rows(x2)
        if sel.dropped > 0:
            if sel.n_kept == 0:
                return torch.zeros_like(x), aux
            xb = select_rows(xb, sel.kept_index, sel.pos_of)
            w = select_rows(w, sel.kept_index, sel.pos_of)
            idx = gather_rows(idx, sel.kept_index)
        out = self.block(xb, w, idx)
        if self.shared is not None:
            out = out + self.shared(xb)
        if sel.dropped > 0:
            out = select_rows(out, sel.pos_of, sel.kept_index)
        return out.to(x.dtype).reshape(*lead, D), aux
