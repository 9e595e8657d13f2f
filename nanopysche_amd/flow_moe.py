"""fp8_flow_moe operator path on MI355X: the functions and the expert-block
object that nanopsyche imports from ``fp8_flow_moe`` (reference
``fp8/__init__.py:8-24``, ``fp8/flow_moe.py:3-15``) and calls from
``MoEBase`` (reference ``model/moe.py:1313-1332`` construction,
``:1516-1517`` / ``:1557-1558`` call, ``:1716-1754`` post-hoc install).

Every function here enqueues hand-written HIP kernels from libfm_hip.so on the
current stream.  Nothing falls back to torch math: tensors must live on a
ROCm device and the library must be built.

The absent reference package's free-function signatures are not recoverable
(only their names are), so the signatures below are this build's own; the
object API (``FP8FlowMoECompute(cfg, d_model, hidden, E,
fp8_gemm_threshold=...)``, ``set_weights``, ``__call__(x, weights, indices,
expert_offset, num_local_experts)``) is the reference's.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _lib
from .recipes import BlockScalingGranularity, FP8RecipeConfig, FP8RecipeType
from .routing import PAD_ROWS, RouterDotInputs, RoutingPlan, route_tokens

FP8_BLOCK_SIZE = 128
MX_BLOCK_SIZE = 32

G = BlockScalingGranularity


# ======================================================================= tensors ====
@dataclass
class FP8Tensor:
    """e4m3 payload with its block scales.

    granularity ROW_1x128 / MX_1x32:  data [R, C], scale [R, C/128] fp32 / [R, C/32] e8m0
    granularity COL_128x1 / MX_32x1:  data [C, R] holds the transpose of a source
                                      [R, C]; scale [R/128, C] fp32 / [R/32, C] e8m0
    granularity BLOCK_128x128:        data [R, C], scale [R/128, C/128] fp32
    """

    data: torch.Tensor
    scale: torch.Tensor
    granularity: BlockScalingGranularity
    pow2: bool = False
    # row blocks stored in the paired-row layout (rows 2p and 2p + 1
    # interleaved in 64-byte pieces): a grouped-GEMM operand of the expert
    # block, not a row-major payload
    paired: bool = False

    @property
    def shape(self):
        return self.data.shape

    def dequantize(self, out_dtype=torch.bfloat16) -> torch.Tensor:
        return dequantize_from_fp8(self, out_dtype=out_dtype)


def _as_2d(x: torch.Tensor) -> torch.Tensor:
    if x.dim() < 2:
        raise ValueError("expected a tensor with at least 2 dimensions")
    x = x.reshape(-1, x.shape[-1])
    return x if x.stride(-1) == 1 and x.stride(0) % 8 == 0 else x.contiguous()


def _src_dtype(x: torch.Tensor) -> int:
    if x.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if x.dtype == torch.float32:
        return _lib.DTYPE_F32
    raise TypeError(f"expected bfloat16 or float32 input, got {x.dtype}")


def _alloc_quant(rows: int, cols: int, kind: int, row: bool, col: bool, dev, kmajor: bool = False):
    """Payload / scale buffers for a [rows, cols] source quantised as `kind`.
    With ``kmajor`` the row scales [rows, blocks] are a transposed view of a
    block-major [blocks, rows] buffer (the grouped GEMM reads one block of 256
    rows from a contiguous span)."""
    u8, f32, bf = torch.uint8, torch.float32, torch.bfloat16
    q = s = qt = st = None
    pay = bf if kind == _lib.QUANT_BF16 else u8
    if row:
        q = torch.empty(rows, cols, dtype=pay, device=dev)
        if kind != _lib.QUANT_BF16:
            blk, dt = (MX_BLOCK_SIZE, u8) if kind == _lib.QUANT_MX else (FP8_BLOCK_SIZE, f32)
            if kmajor:
                s = torch.empty(cols // blk, rows, dtype=dt, device=dev).t()
            else:
                s = torch.empty(rows, cols // blk, dtype=dt, device=dev)
    if col:
        qt = torch.empty(cols, rows, dtype=pay, device=dev)
        if kind in (_lib.QUANT_BLOCK, _lib.QUANT_POW2):
            st = torch.empty(rows // FP8_BLOCK_SIZE, cols, dtype=f32, device=dev)
        elif kind == _lib.QUANT_MX:
            st = torch.empty(rows // MX_BLOCK_SIZE, cols, dtype=u8, device=dev)
    return q, s, qt, st


def _ld(t):
    return 0 if t is None else t.stride(0)


def _tile_args(kind, q, s, qt, st, paired=False, col_paired=False):
    """(kind, q, ld_q, s, ld_s, qt, ld_qt, st, ld_st) for the tile producers;
    block-major row scales (a transposed view) add SCALES_KMAJOR to the kind,
    ``paired`` / ``col_paired`` (e4m3 row / transposed output in the
    paired-row layout) ROWS_PAIRED / COLS_PAIRED."""
    ld_s = _ld(s)
    if s is not None and s.stride(1) != 1:
        kind |= _lib.SCALES_KMAJOR
        ld_s = s.stride(1)
    if paired:
        kind |= _lib.ROWS_PAIRED
    if col_paired:
        kind |= _lib.COLS_PAIRED
    return (kind, _lib.ptr(q), _ld(q), _lib.ptr(s), ld_s, _lib.ptr(qt), _ld(qt), _lib.ptr(st), _ld(st))


def _wrap(q, s, qt, st, kind, paired=False, col_paired=False):
    if kind == _lib.QUANT_BF16:
        return q, qt
    pow2 = kind == _lib.QUANT_POW2
    row_g = G.MX_1x32 if kind == _lib.QUANT_MX else G.ROW_1x128
    col_g = G.MX_32x1 if kind == _lib.QUANT_MX else G.COL_128x1
    row = FP8Tensor(q, s, row_g, pow2, paired) if q is not None else None
    col = FP8Tensor(qt, st, col_g, pow2, col_paired) if qt is not None else None
    return row, col


# ================================================================== quantisation ====
def quantize_to_fp8(x: torch.Tensor,
                    granularity: BlockScalingGranularity = G.ROW_1x128,
                    *, pow2_scale: bool = False, return_transpose: bool = False):
    """Blockwise e4m3 quantisation of a bf16 / fp32 tensor (last dim = columns).

    ROW_1x128 / MX_1x32:  row blocks; with ``return_transpose`` also the
        column-block (128x1 / 32x1) quantisation of the transpose from the
        same read, returned as a second FP8Tensor (no double quantisation;
        with ``pow2_scale`` the transposed output is the scaling-aware
        transpose of the row output).
    COL_128x1 / MX_32x1:  only the column-block quantisation of the transpose.
    BLOCK_128x128:        weight blocks.
    """
    granularity = BlockScalingGranularity(granularity)
    _lib.require_device(x, "x")
    x2 = _as_2d(x)
    R, C = x2.shape
    if granularity == G.BLOCK_128x128:
        if R % 128 or C % 128:
            raise ValueError(f"128x128 quantisation needs both dims % 128 == 0, got {tuple(x2.shape)}")
        kind = _lib.QUANT_POW2 if pow2_scale else _lib.QUANT_BLOCK
        q = torch.empty(R, C, dtype=torch.uint8, device=x.device)
        s = torch.empty(R // 128, C // 128, dtype=torch.float32, device=x.device)
        _lib.call("fm_quantize_weight", _lib.ptr(x2), _src_dtype(x2), 1, R, C, x2.stride(0), 0, kind,
                  _lib.ptr(q), C, 0, 0, _lib.ptr(s), C // 128, 0, None, 0, 0, 0, None, 0, 0,
                  _lib.stream_of(x2))
        return FP8Tensor(q, s, G.BLOCK_128x128, pow2_scale)
    mx = granularity in (G.MX_1x32, G.MX_32x1)
    kind = _lib.QUANT_MX if mx else (_lib.QUANT_POW2 if pow2_scale else _lib.QUANT_BLOCK)
    want_row = granularity in (G.ROW_1x128, G.MX_1x32)
    want_col = return_transpose or not want_row
    if C % 128:
        raise ValueError(f"columns must be a multiple of 128, got {C}")
    if want_col and R % 128:
        raise ValueError(f"column-block quantisation needs rows % 128 == 0, got {R}")
    q, s, qt, st = _alloc_quant(R, C, kind, want_row, want_col, x.device)
    _lib.call("fm_quantize", _lib.ptr(x2), _src_dtype(x2), R, C, x2.stride(0),
              *_tile_args(kind, q, s, qt, st), _lib.stream_of(x2))
    row, col = _wrap(q, s, qt, st, kind)
    if want_row and return_transpose:
        return row, col
    return row if want_row else col


def dequantize_from_fp8(t: FP8Tensor, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """decode(q) * scale, rounded once to ``out_dtype`` (bf16 or fp32)."""
    if t.paired:
        raise ValueError("a paired-row payload is a grouped-GEMM operand, not a row-major tensor")
    q, s = t.data, t.scale
    _lib.require_device(q, "data")
    R, C = q.shape
    g = BlockScalingGranularity(t.granularity)
    e8m0 = g in (G.MX_1x32, G.MX_32x1)
    if g == G.ROW_1x128:
        shifts = (0, 7, s.stride(0), s.stride(1))
    elif g == G.MX_1x32:
        shifts = (0, 5, s.stride(0), s.stride(1))
    elif g == G.BLOCK_128x128:
        shifts = (7, 7, s.stride(0), s.stride(1))
    elif g in (G.COL_128x1, G.MX_32x1):
        shifts = (0, 7 if g == G.COL_128x1 else 5, s.stride(1), s.stride(0))
    else:
        raise ValueError(g)
    out = torch.empty(R, C, dtype=out_dtype, device=q.device)
    od = _lib.DTYPE_F32 if out_dtype == torch.float32 else _lib.DTYPE_BF16
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("out_dtype must be bfloat16 or float32")
    _lib.call("fm_dequantize", _lib.ptr(q), R, C, q.stride(0), _lib.ptr(s), int(e8m0), shifts[0],
              shifts[1], shifts[2], shifts[3], _lib.ptr(out), od, out.stride(0), _lib.stream_of(q))
    return out


def scaling_aware_transpose(t: FP8Tensor) -> FP8Tensor:
    """Row-quantised (1x128) e4m3 -> column-quantised (128x1) e4m3 of the
    transpose, computed from the e4m3 payload alone: each 128x128 tile's
    column scale is the largest of its row scales and every element is
    re-expressed as e4m3(decode(q) * s_row / s_col).  Exact for power-of-two
    scales (an exponent shift) unless the result is an e4m3 subnormal."""
    if t.paired:
        raise ValueError("a paired-row payload is a grouped-GEMM operand, not a row-major tensor")
    if BlockScalingGranularity(t.granularity) != G.ROW_1x128:
        raise ValueError("scaling_aware_transpose expects a ROW_1x128 tensor")
    q, s = t.data, t.scale
    _lib.require_device(q, "data")
    R, C = q.shape
    if R % 128 or C % 128:
        raise ValueError(f"scaling_aware_transpose needs both dims % 128 == 0, got {tuple(q.shape)}")
    if s.stride(1) != 1:
        s = s.contiguous()   # the kernel reads row-major scales
    qt = torch.empty(C, R, dtype=torch.uint8, device=q.device)
    st = torch.empty(R // 128, C, dtype=torch.float32, device=q.device)
    _lib.call("fm_scaling_aware_transpose", _lib.ptr(q), R, C, q.stride(0), _lib.ptr(s), s.stride(0),
              _lib.ptr(qt), qt.stride(0), _lib.ptr(st), st.stride(0), _lib.stream_of(q))
    return FP8Tensor(qt, st, G.COL_128x1, t.pow2)


# ======================================================================= SwiGLU ====
def _swiglu(g, u, rows, H, kind, row, col, dev, tile_valid=None, kmajor=False, paired=False, col_paired=False):
    q, s, qt, st = _alloc_quant(rows, H, kind, row, col, dev, kmajor)
    _lib.call("fm_swiglu_quantize", _lib.ptr(g), g.stride(0), _lib.ptr(u), u.stride(0), rows, H,
              *_tile_args(kind, q, s, qt, st, paired, col_paired and col), _lib.ptr(tile_valid),
              _lib.stream_of(g))
    return q, s, qt, st


def _act_kind(granularity, pow2_scale):
    if granularity is None:
        return _lib.QUANT_BF16
    granularity = BlockScalingGranularity(granularity)
    if granularity in (G.MX_1x32, G.MX_32x1):
        return _lib.QUANT_MX
    return _lib.QUANT_POW2 if pow2_scale else _lib.QUANT_BLOCK


def fused_silu_multiply_quantize(gate: torch.Tensor, up: torch.Tensor,
                                 granularity: Optional[BlockScalingGranularity] = G.ROW_1x128,
                                 *, pow2_scale: bool = False, return_transpose: bool = False):
    """h = silu(gate) * up in fp32 from bf16 inputs [M, H], quantised like
    ``quantize_to_fp8`` (granularity None -> bf16 output)."""
    _lib.require_device(gate, "gate")
    if gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise TypeError("gate and up must be bfloat16")
    if gate.shape != up.shape or gate.dim() != 2:
        raise ValueError("gate and up must be 2-D tensors of one shape")
    if gate.stride(1) != 1 or up.stride(1) != 1:
        raise ValueError("gate and up must have unit column stride")
    M, H = gate.shape
    kind = _act_kind(granularity, pow2_scale)
    want_col = return_transpose
    q, s, qt, st = _swiglu(gate, up, M, H, kind, True, want_col, gate.device)
    row, col = _wrap(q, s, qt, st, kind)
    return (row, col) if return_transpose else row


def fused_swiglu_quantize(gate_up: torch.Tensor,
                          granularity: Optional[BlockScalingGranularity] = G.ROW_1x128,
                          *, pow2_scale: bool = False, return_transpose: bool = False):
    """Same as ``fused_silu_multiply_quantize`` for a packed [M, 2H] input
    whose first H columns are the gate and last H the up projection."""
    H = gate_up.shape[-1] // 2
    return fused_silu_multiply_quantize(gate_up[:, :H], gate_up[:, H:], granularity,
                                        pow2_scale=pow2_scale, return_transpose=return_transpose)


# ======================================================== permute / unpermute ====
@dataclass
class PermutedTokens:
    """Expert-contiguous, per-expert padded copy of the tokens plus its plan."""

    plan: RoutingPlan
    rows: object            # FP8Tensor (row blocks) or bf16 tensor [rows_max, D]
    rows_t: object = None   # FP8Tensor (column blocks) or bf16 tensor [D, rows_max]


def fused_permute_pad(x: torch.Tensor, indices, num_experts: int, *,
                      granularity: Optional[BlockScalingGranularity] = G.ROW_1x128,
                      pow2_scale: bool = False, return_transpose: bool = False,
                      weights: Optional[torch.Tensor] = None,
                      fp8_gemm_threshold: int = 0, kmajor_scales: bool = False,
                      tile_valid: Optional[torch.Tensor] = None, paired_rows: bool = False,
                      paired_cols: bool = False) -> PermutedTokens:
    """Gather the rows of ``x`` [T, D] (bf16) into expert order, each expert's
    group padded to 128 rows (zeros), and quantise them in the same pass.
    Rows past the last group (``plan.offsets[-1]`` up to ``plan.rows_max``)
    are left unwritten.

    ``indices`` is the router's [T, K] expert indices or a RoutingPlan from an
    earlier call.  ``weights`` [T, K] (optional) scales each gathered row by
    its router weight.  granularity None keeps bf16.  ``kmajor_scales``
    stores the row scales block-major (``rows.scale`` is then a transposed
    view), the layout the grouped GEMM streams fastest.  ``tile_valid``
    [rows_max/128] int32 (default ``plan.tile_expert``): 128-row tiles with a
    negative entry are not written (``RoutingPlan.precision_tiles`` gives
    each precision's tiles under the threshold split).  ``paired_rows``
    (e4m3 kinds) writes the row blocks in the paired-row layout that the
    grouped GEMM streams in 64-deep half steps (``rows.paired``; a GEMM
    operand only), ``paired_cols`` the transposed output likewise."""
    _lib.require_device(x, "x")
    if x.dtype != torch.bfloat16:
        raise TypeError("x must be bfloat16")
    x2 = _as_2d(x)
    T, D = x2.shape
    plan = indices if isinstance(indices, RoutingPlan) else route_tokens(indices, num_experts,
                                                                         fp8_gemm_threshold)
    if plan.num_tokens != T:
        raise ValueError(f"plan is for {plan.num_tokens} tokens, x has {T}")
    kind = _act_kind(granularity, pow2_scale)
    q, s, qt, st = _alloc_quant(plan.rows_max, D, kind, True, return_transpose, x.device, kmajor_scales)
    w = None
    if weights is not None:
        w = weights.reshape(-1).to(torch.float32).contiguous()
    _lib.call("fm_permute", _lib.ptr(x2), T, D, x2.stride(0), _lib.ptr(plan.assign_of_row),
              plan.rows_max, plan.top_k, _lib.ptr(w),
              *_tile_args(kind, q, s, qt, st, paired_rows, paired_cols and return_transpose),
              _lib.ptr(plan.tile_expert if tile_valid is None else tile_valid), _lib.stream_of(x2))
    row, col = _wrap(q, s, qt, st, kind, paired_rows, paired_cols)
    return PermutedTokens(plan, row, col)


def fused_unpermute_unpad(y: torch.Tensor, plan: RoutingPlan,
                          weights: Optional[torch.Tensor] = None,
                          out_dtype: torch.dtype = torch.bfloat16,
                          addend: Optional[torch.Tensor] = None,
                          router_terms: Optional[tuple] = None) -> torch.Tensor:
    """out[t] = addend[t] + sum_k weights[t, k] * y[row(t, k)] (weights None ->
    1, addend None -> 0), summed in fp32 in slot order and rounded once.  y
    and addend are bf16 ([rows_max, D] and [T, D]).  ``router_terms`` =
    (dlogits [T, E] fp32, gate_weight [E, D] bf16 / fp32), E <= 8, adds
    sum_e dlogits[t, e] gate_weight[e] in the same pass (a MoE layer's input
    gradient: the router's share)."""
    _lib.require_device(y, "y")
    if y.dtype != torch.bfloat16:
        raise TypeError("y must be bfloat16")
    D = y.shape[1]
    T, K = plan.num_tokens, plan.top_k
    if addend is not None and (addend.dtype != torch.bfloat16 or tuple(addend.shape) != (T, D)
                               or addend.stride(1) != 1):
        raise ValueError("addend must be a bf16 [T, D] tensor with unit column stride")
    out = torch.empty(T, D, dtype=out_dtype, device=y.device)
    w = None if weights is None else weights.reshape(-1).to(torch.float32).contiguous()
    od = _lib.DTYPE_F32 if out_dtype == torch.float32 else _lib.DTYPE_BF16
    if router_terms is not None:
        dl, gw = router_terms
        gw = gw.detach()
        if gw.dtype not in (torch.float32, torch.bfloat16) or gw.stride(1) != 1:
            gw = gw.float().contiguous()
        _lib.call("fm_unpermute_router", _lib.ptr(y), y.stride(0), _lib.ptr(plan.row_of), _lib.ptr(w), T, K, D,
                  _lib.ptr(out), od, out.stride(0), _lib.ptr(addend), 0 if addend is None else addend.stride(0),
                  _lib.ptr(dl), dl.stride(0), _lib.ptr(gw), _dt(gw), gw.stride(0), gw.shape[0], _lib.stream_of(y))
        return out
    _lib.call("fm_unpermute", _lib.ptr(y), y.stride(0), _lib.ptr(plan.row_of), _lib.ptr(w), T, K, D,
              _lib.ptr(out), od, out.stride(0), _lib.ptr(addend), 0 if addend is None else addend.stride(0),
              _lib.stream_of(y))
    return out


# ================================================================ grouped GEMM ====
def _operand(data, scale=None, *, ld=None, gs=0, s_row=0, s_kb=0, s_gs=0, shift=0, data2=None, split=0):
    o = _lib.FmGemmOperand()
    o.data = data.data_ptr()
    o.data2 = None if data2 is None else data2.data_ptr()
    o.split_rows = split if data2 is not None else 0
    o.ld = data.stride(0) if ld is None else ld
    o.group_stride = gs
    o.scale = None if scale is None else scale.data_ptr()
    o.scale_row_stride = s_row
    o.scale_kb_stride = s_kb
    o.scale_group_stride = s_gs
    o.scale_row_shift = shift
    return o


def _token_operand(t, kind):
    """Row-major activations [rows, K] (FP8Tensor or bf16 tensor)."""
    if kind == _lib.QUANT_BF16:
        return _operand(t)
    return _operand(t.data, t.scale, s_row=t.scale.stride(0), s_kb=t.scale.stride(1))


def _col_operand(t, kind):
    """Column-quantised transposed activations [C, rows] with scales [rows/blk, C]."""
    if kind == _lib.QUANT_BF16:
        return _operand(t)
    return _operand(t.data, t.scale, s_row=1, s_kb=t.scale.stride(0))


@dataclass
class ExpertWeightOperand:
    """One expert-weight GEMM operand: E matrices [N, K] (K contiguous), or,
    with ``kmajor``, E matrices stored [K, N] (N contiguous) that the FP8 pow2
    GEMM reads transposed.  With ``data2`` (BF16) each expert's rows from
    ``split`` on come from ``data2``: w1 and w3 read as stored."""

    data: torch.Tensor
    scale: Optional[torch.Tensor]
    ld: int
    gs: int
    s_row: int = 0
    s_kb: int = 0
    s_gs: int = 0
    shift: int = 0
    N: int = 0
    K: int = 0
    kmajor: bool = False
    data2: Optional[torch.Tensor] = None
    split: int = 0
    paired: bool = False   # rows (K rows with kmajor) in the paired-row layout

    def operand(self):
        return _operand(self.data, self.scale, ld=self.ld, gs=self.gs, s_row=self.s_row,
                        s_kb=self.s_kb, s_gs=self.s_gs, shift=self.shift, data2=self.data2, split=self.split)


def _gemm_kind(kind):
    return {_lib.QUANT_BF16: _lib.GEMM_BF16, _lib.QUANT_BLOCK: _lib.GEMM_FP8_F32,
            _lib.QUANT_POW2: _lib.GEMM_FP8_POW2, _lib.QUANT_MX: _lib.GEMM_FP8_MX}[kind]


# Optional per-launch timer (bench.py sets it): called as
# GEMM_TIMER(name, algorithmic_flops, launch_fn) around each grouped GEMM.
GEMM_TIMER = None
_KIND_NAME = {_lib.QUANT_BF16: "bf16", _lib.QUANT_BLOCK: "fp8_f32", _lib.QUANT_POW2: "fp8_pow2",
              _lib.QUANT_MX: "fp8_mx"}


def _timed(name, flops, fn):
    if GEMM_TIMER is None:
        fn()
    else:
        GEMM_TIMER(name, flops, fn)


def _assignments(plan: RoutingPlan, mask, want) -> float:
    """Assignments a launch computes: all of them, or with an expert mask those
    of the experts it selects (read back from the device: only when a GEMM
    timer asks for the launch's FLOPs)."""
    if mask is None or GEMM_TIMER is None:
        return float(plan.num_tokens * plan.top_k)
    sel = (mask == want).to(torch.int64)
    return float((plan.counts.to(torch.int64) * sel).sum().item())


def _gemm_m(kind, tokens, w: ExpertWeightOperand, plan: RoutingPlan, out, mask=None, want=1):
    t_paired = getattr(tokens, "paired", False)
    if (w.paired and not w.kmajor) and not t_paired:
        raise ValueError("paired-row weights need paired-row tokens")

    def launch():
        gk = _gemm_kind(kind) | (_lib.GEMM_W_KMAJOR if w.kmajor else 0)
        if t_paired:
            gk |= _lib.GEMM_PAIRED | (_lib.GEMM_W_PAIRED if w.kmajor and w.paired else 0)
        elif w.paired:
            raise ValueError("paired-row weights need paired-row tokens")
        _lib.call("fm_grouped_gemm_ragged_m", gk, _token_operand(tokens, kind),
                  w.operand(), plan.m_tiles, _lib.ptr(plan.tile_expert), _lib.ptr(plan.offsets),
                  plan.num_experts, w.N, w.K,
                  _lib.ptr(mask), want, _lib.ptr(out), _dt(out), out.stride(0), _lib.stream_of(out))

    _timed(f"grouped_gemm_ragged_m/{_KIND_NAME[kind]}", 2.0 * _assignments(plan, mask, want) * w.N * w.K, launch)


# Model of a ragged-K launch for choosing its K split: ~1.3 us per 128-deep K
# step of a 256 x 256 tile, and the partials' HBM round trip at ~5 TB/s.
_K_STEP_US = 1.3
_HBM_BYTES_PER_US = 5.0e6
_CUS = {}


def _cus(dev) -> int:
    n = _CUS.get(dev)
    if n is None:
        n = _CUS[dev] = torch.cuda.get_device_properties(dev).multi_processor_count
    return n


def _k_splits(kind, plan: RoutingPlan, M, N, dev) -> int:
    """K slices per weight-gradient tile: more than one only when the launch
    has fewer 256 x 256 output tiles than the GPU has CUs (one group, as for a
    shared expert, or few small experts).  Chosen on the host from the shapes
    and the padded row bound alone (no read of the device counts), minimising
    rounds x slice length + the fp32 partials' write and re-read.
    FM_RK_SPLITS=<n> fixes it (1 = never split)."""
    forced = os.environ.get("FM_RK_SPLITS")
    if kind == _lib.QUANT_BLOCK:
        return 1   # the fp32-scale kernel takes no split
    if forced is not None:
        return max(1, min(16, int(forced)))
    E = plan.num_experts
    tiles = E * -(-M // 256) * -(-N // 256)
    cus = _cus(dev)
    if tiles >= cus:
        return 1
    steps = plan.rows_max / E / 128
    part_us = E * M * N * 4 / _HBM_BYTES_PER_US
    best, best_us = 1, -(-tiles // cus) * steps * _K_STEP_US
    for S in range(2, 9):
        if steps / S < 4:
            break
        us = -(-tiles * S // cus) * steps / S * _K_STEP_US + (S + 0.5) * part_us
        if us < best_us:
            best, best_us = S, us
    return best


def _gemm_k(kind, a_t, b_t, plan: RoutingPlan, M, N, out, out_gs, out2=None, out2_gs=0, split=None,
            mask=None, want=1, may_split=True, a_cold=False):
    """Weight-gradient grouped GEMM.  ``a_cold``: a_t was written long before
    this launch (saved by the forward) and b_t just now, so a_t's tiles are
    walked fastest (GEMM_A_FAST: fetched from memory once); by default b_t's."""
    S = _k_splits(kind, plan, M, N, out.device) if may_split else 1
    gk = _gemm_kind(kind) | (_lib.GEMM_A_FAST if a_cold else 0)
    pa, pb = getattr(a_t, "paired", False), getattr(b_t, "paired", False)
    if pa != pb or (pa and (S > 1 or mask is not None)):
        raise ValueError("paired-row weight-gradient operands: both paired, unsplit and unmasked")
    if pa:
        gk |= _lib.GEMM_PAIRED
    ws = None
    if S > 1:
        nbytes = int(_lib.load().fm_grouped_gemm_ragged_k_split_workspace_bytes(plan.num_experts, M, N, S))
        ws = torch.empty(nbytes // 4, dtype=torch.float32, device=out.device)

    def launch():
        if ws is None:
            _lib.call("fm_grouped_gemm_ragged_k", gk, _col_operand(a_t, kind),
                      _col_operand(b_t, kind), _lib.ptr(plan.offsets), plan.num_experts, M, N,
                      _lib.ptr(mask), want, _lib.ptr(out), out_gs, _lib.ptr(out2), out2_gs,
                      M if split is None else split, _dt(out), N, _lib.stream_of(out))
        else:
            _lib.call("fm_grouped_gemm_ragged_k_split", gk, _col_operand(a_t, kind),
                      _col_operand(b_t, kind), _lib.ptr(plan.offsets), plan.num_experts, M, N,
                      _lib.ptr(mask), want, _lib.ptr(out), out_gs, _lib.ptr(out2), out2_gs,
                      M if split is None else split, _dt(out), N, S, _lib.ptr(ws), ws.numel() * 4,
                      _lib.stream_of(out))

    _timed(f"grouped_gemm_ragged_k/{_KIND_NAME[kind]}", 2.0 * _assignments(plan, mask, want) * M * N, launch)


# Kinds whose dgrad and weight-gradient launches can share one grid
# (fm_grouped_gemm_ragged_m_k); the others run them on two streams.
_MK_KINDS = (_lib.QUANT_BF16, _lib.QUANT_POW2)


def _gemm_mk(kind, tokens, w: ExpertWeightOperand, plan: RoutingPlan, out, a_t, b_t, M2, N2, out2, out2_gs,
             mask=None, want=1, a_cold=False):
    """_gemm_m(kind, tokens, w, plan, out) and the unsplit _gemm_k(kind, a_t,
    b_t, plan, M2, N2, out2, out2_gs) as one grid: the weight-gradient tiles
    fill the last round of the dgrad's."""
    gk = (_gemm_kind(kind) | (_lib.GEMM_W_KMAJOR if w.kmajor else 0) | (_lib.GEMM_A_FAST if a_cold else 0))
    flags = {getattr(tokens, "paired", False), w.paired, getattr(a_t, "paired", False), getattr(b_t, "paired", False)}
    if len(flags) != 1:
        raise ValueError("fm_grouped_gemm_ragged_m_k: every operand paired or none")
    if w.paired:
        gk |= _lib.GEMM_PAIRED

    def launch():
        _lib.call("fm_grouped_gemm_ragged_m_k", gk, _token_operand(tokens, kind), w.operand(), plan.m_tiles,
                  _lib.ptr(plan.tile_expert), w.N, w.K, _lib.ptr(out), _dt(out), out.stride(0),
                  _col_operand(a_t, kind), _col_operand(b_t, kind), M2, N2, _lib.ptr(out2), out2_gs, None, 0, M2,
                  _dt(out2), N2, _lib.ptr(plan.offsets), plan.num_experts, _lib.ptr(mask), want,
                  _lib.stream_of(out))

    _timed(f"grouped_gemm_ragged_m_k/{_KIND_NAME[kind]}",
           2.0 * _assignments(plan, mask, want) * (w.N * w.K + M2 * N2), launch)


def _dt(t):
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    raise TypeError(f"unsupported output dtype {t.dtype}")


def fp8_grouped_gemm(tokens, weights: ExpertWeightOperand, plan: RoutingPlan,
                     out_dtype: torch.dtype = torch.bfloat16,
                     expert_mask: Optional[torch.Tensor] = None, mask_want: int = 1,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-expert out[r] = tokens[r] @ W_e^T over the padded expert buffer.

    ``tokens`` is a row-quantised FP8Tensor (or a bf16 tensor for the BF16
    path) of [plan.rows_max, K]; ``weights`` an ExpertWeightOperand from
    ``ExpertWeights``.  Tiles of experts with ``expert_mask[e] != mask_want``
    are skipped (the fp8_gemm_threshold switch)."""
    if isinstance(tokens, FP8Tensor):
        g = BlockScalingGranularity(tokens.granularity)
        kind = _lib.QUANT_MX if g == G.MX_1x32 else (_lib.QUANT_POW2 if tokens.pow2 else _lib.QUANT_BLOCK)
        rows = tokens.data.shape[0]
        dev = tokens.data.device
    else:
        kind = _lib.QUANT_BF16
        rows = tokens.shape[0]
        dev = tokens.device
    if out is None:
        out = torch.empty(rows, weights.N, dtype=out_dtype, device=dev)
    _gemm_m(kind, tokens, weights, plan, out, expert_mask, mask_want)
    return out


# ============================================================== expert weights ====
class ExpertWeights:
    """GEMM operands of the expert weights for one recipe, rebuilt only when
    the parameters change (their ``_version`` counters or storage move).

    w13   [E][2H, D]  forward gate|up          (rows of w1 then w3 per expert)
    w2t   [E][D, H]   forward down             (w2_e transposed)
    w2    [E][H, D]   dgrad dH = dY w2_e^T
    w13t  [E][D, 2H]  dgrad dX = [dg|du] [w1_e; w3_e]

    The forward pair is always built; the dgrad pair only when ``need_dgrad``
    (a forward that records a backward), from the same read of the weights
    (the transposed outputs of one launch).

    FP8 pow2 with at most 64 experts, D a multiple of 256 and H >= 256
    (``kmajor_ok``): only the row operands w13 and w2 are quantised, and w2t /
    w13t are those same bytes read as [K][N] weights (``kmajor``) -- the
    128 x 128 blocks of a transpose are the transposed blocks, so the GEMMs
    give the bits of the transposed copies, and the weight pass writes half
    the bytes."""

    KMAJOR = True   # class switch: build the transposed copies instead (for comparisons)
    PAIRED = True   # class switch: the expert block's pow2 operands in row-major layout (for comparisons)

    @staticmethod
    def kmajor_ok(kind: int, E: int, H: int, D: int) -> bool:
        return (ExpertWeights.KMAJOR and kind == _lib.QUANT_POW2 and E <= 64 and D % 256 == 0 and H >= 256)

    @staticmethod
    def paired_ok(kind: int, E: int, H: int, D: int) -> bool:
        """Paired-row weights and token operands: the pow2 [K][N] build or the
        MX build (at most 64 experts, D and H multiples of 64), with every
        ragged-M GEMM of the block at least 384 deep (the paired kernel's ring
        of half steps)."""
        if not ExpertWeights.PAIRED or D < 384 or H < 384:
            return False
        if kind == _lib.QUANT_MX:
            return E <= 64 and D % 64 == 0 and H % 64 == 0
        return ExpertWeights.kmajor_ok(kind, E, H, D)

    def __init__(self, kind: int, paired: bool = False):
        """``paired``: in the [K][N] (kmajor) build, w13 and w2 (and w13t,
        w2t, the same bytes) are written in the paired-row layout; the expert
        block pairs its token operands to match (``paired_ok``)."""
        self.kind = kind
        self.paired = paired
        self.key = None
        self.has_dgrad = False
        self._defer = None
        self.w13 = self.w2t = self.w2 = self.w13t = None

    def refresh(self, w1, w2, w3, E: int, need_dgrad: bool = True, defer: Optional[list] = None) -> "ExpertWeights":
        """Rebuild the operands if a parameter changed.  With ``defer`` (a list)
        the batched quantisation launch is not made but appended as (FmWeightJob
        array, count, sources): the caller runs it (``route_tokens(weight_jobs=
        (array, count))`` or ``fm_quantize_weight_batch``) before the operands are
        read, holding ``sources`` (the tensors the jobs read) until then, and
        calls ``invalidate()`` if it cannot.

        Inside a stream capture the operands are always rebuilt: the graph's
        replays then re-quantise the parameters' storage as it is at each
        replay (an optimizer step between replays changes it in place), and
        the buffers, which every replay rewrites, are not kept as the cache of
        later eager calls."""
        key = tuple((w.data_ptr(), w._version, w.dtype) for w in (w1, w2, w3))
        capturing = torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
        if capturing or key != self.key or (need_dgrad and not self.has_dgrad):
            self.key = None
            self.w13 = self.w2t = self.w2 = self.w13t = None
            self.has_dgrad = need_dgrad
            self._defer = defer
            try:
                self._build(w1.detach(), w2.detach(), w3.detach(), E, need_dgrad)
            finally:
                self._defer = None
            self.key = None if capturing else key
        return self

    def invalidate(self) -> None:
        """Forget the cache key, so the next refresh rebuilds (a deferred
        quantisation that was never launched leaves the operands unwritten)."""
        self.key = None

    def _launch(self, jobs, n: int, like: torch.Tensor, sources) -> None:
        """Run (or defer) a weight-quantisation batch on ``like``'s current stream."""
        if self._defer is not None:
            self._defer.append((jobs, n, sources))
        else:
            _lib.call("fm_quantize_weight_batch", jobs, n, _lib.stream_of(like))

    def _build(self, w1, w2, w3, E, dgrad=True):
        EH, D = w1.shape
        H = EH // E
        dev = w1.device
        kind = self.kind
        if kind == _lib.QUANT_MX:
            self._build_mx(w1, w2, w3, E, H, D, dgrad, self.paired and self.paired_ok(kind, E, H, D))
            return
        if self.kmajor_ok(kind, E, H, D):
            self._build_kmajor(w1, w2, w3, E, H, D, self.paired and self.paired_ok(kind, E, H, D))
            return
        if self.views_ok(kind, E, H, D, (w1, w2, w3)):
            self._build_bf16_views(w1, w2, w3, E, H, D, dgrad)
            return
        pay = torch.bfloat16 if kind == _lib.QUANT_BF16 else torch.uint8
        f32 = torch.float32
        fp8 = kind != _lib.QUANT_BF16
        W13 = torch.empty(E, 2 * H, D, dtype=pay, device=dev)
        W2t = torch.empty(E, D, H, dtype=pay, device=dev)
        S13 = torch.empty(E, 2 * H // 128, D // 128, dtype=f32, device=dev) if fp8 else None
        S2t = torch.empty(E, D // 128, H // 128, dtype=f32, device=dev) if fp8 else None
        W13t = W2 = S13t = S2 = None
        if dgrad:
            W13t = torch.empty(E, D, 2 * H, dtype=pay, device=dev)
            W2 = torch.empty(E, H, D, dtype=pay, device=dev)
            S13t = torch.empty(E, D // 128, 2 * H // 128, dtype=f32, device=dev) if fp8 else None
            S2 = torch.empty(E, H // 128, D // 128, dtype=f32, device=dev) if fp8 else None

        srcs = [w.contiguous() for w in (w1, w3, w2)]
        if len({w.dtype for w in srcs}) != 1:
            srcs = [w.float() for w in srcs]

        def job(src, dst, s, dst_t, s_t, row_off, col_off, rows_out):
            return _lib.FmWeightJob(
                _lib.ptr(src), _src_dtype(src), E, H, D, D, H * D, kind,
                _lib.ptr(dst), D, rows_out * D, row_off, _lib.ptr(s), D // 128, (rows_out // 128) * (D // 128),
                _lib.ptr(dst_t), rows_out, D * rows_out, col_off,
                _lib.ptr(s_t), rows_out // 128, (D // 128) * (rows_out // 128))

        # w1 and w3 into the rows (and transposed columns) of the [E, 2H, D] gate|up
        # operand, w2 into its transpose (and its own rows): one launch
        jobs = (_lib.FmWeightJob * 3)(job(srcs[0], W13, S13, W13t, S13t, 0, 0, 2 * H),
                                      job(srcs[1], W13, S13, W13t, S13t, H, H, 2 * H),
                                      job(srcs[2], W2, S2, W2t, S2t, 0, 0, H))
        self._launch(jobs, 3, w1, srcs)
        sh = 7
        self.w13 = ExpertWeightOperand(W13, S13, D, 2 * H * D, D // 128, 1, (2 * H // 128) * (D // 128), sh, 2 * H, D)
        self.w2t = ExpertWeightOperand(W2t, S2t, H, D * H, H // 128, 1, (D // 128) * (H // 128), sh, D, H)
        if dgrad:
            self.w13t = ExpertWeightOperand(W13t, S13t, 2 * H, D * 2 * H, 2 * H // 128, 1,
                                            (D // 128) * (2 * H // 128), sh, D, 2 * H)
            self.w2 = ExpertWeightOperand(W2, S2, D, H * D, D // 128, 1, (H // 128) * (D // 128), sh, H, D)

    def _build_kmajor(self, w1, w2, w3, E, H, D, paired=False):
        """Row operands only (one launch over w1, w3, w2); the down and dX GEMMs
        read them as [K][N] weights.  Forward and dgrad operands together.
        ``paired``: w13 and w2 in the paired-row layout (the down and dX
        GEMMs read them as paired [K][N] weights)."""
        dev = w1.device
        W13 = torch.empty(E, 2 * H, D, dtype=torch.uint8, device=dev)
        W2 = torch.empty(E, H, D, dtype=torch.uint8, device=dev)
        S13 = torch.empty(E, 2 * H // 128, D // 128, dtype=torch.float32, device=dev)
        S2 = torch.empty(E, H // 128, D // 128, dtype=torch.float32, device=dev)
        srcs = [w.contiguous() for w in (w1, w3, w2)]
        if len({w.dtype for w in srcs}) != 1:
            srcs = [w.float() for w in srcs]
        kind = self.kind

        def job(src, dst, s, row_off, rows_out, pair=False):
            return _lib.FmWeightJob(
                _lib.ptr(src), _src_dtype(src), E, H, D, D, H * D, kind | (_lib.ROWS_PAIRED if pair else 0),
                _lib.ptr(dst), D, rows_out * D, row_off, _lib.ptr(s), D // 128, (rows_out // 128) * (D // 128),
                None, 0, 0, 0, None, 0, 0)

        jobs = (_lib.FmWeightJob * 3)(job(srcs[0], W13, S13, 0, 2 * H, paired),
                                      job(srcs[1], W13, S13, H, 2 * H, paired),
                                      job(srcs[2], W2, S2, 0, H, paired))
        self._launch(jobs, 3, w1, srcs)
        sh = 7
        g13, g2 = (2 * H // 128) * (D // 128), (H // 128) * (D // 128)
        self.w13 = ExpertWeightOperand(W13, S13, D, 2 * H * D, D // 128, 1, g13, sh, 2 * H, D, paired=paired)
        self.w2 = ExpertWeightOperand(W2, S2, D, H * D, D // 128, 1, g2, sh, H, D, paired=paired)
        # element (n = d, k) of the [K][N] reading: rows k, column d; scale
        # block (d >> 7, k >> 7) at s[(k >> 7) * D/128 + (d >> 7)]
        self.w2t = ExpertWeightOperand(W2, S2, D, H * D, 1, D // 128, g2, sh, D, H, kmajor=True, paired=paired)
        self.w13t = ExpertWeightOperand(W13, S13, D, 2 * H * D, 1, D // 128, g13, sh, D, 2 * H, kmajor=True,
                                        paired=paired)
        self.has_dgrad = True

    @staticmethod
    def views_ok(kind: int, E: int, H: int, D: int, ws) -> bool:
        """BF16 recipe on contiguous bf16 parameters, at most 64 experts, H a
        multiple of 256: the row operands are the parameters themselves."""
        return (ExpertWeights.KMAJOR and kind == _lib.QUANT_BF16 and E <= 64 and H % 256 == 0
                and all(w.dtype == torch.bfloat16 and w.is_contiguous() for w in ws))

    def _build_bf16_views(self, w1, w2, w3, E, H, D, dgrad):
        """w13: w1 and w3 read as stored (a split operand), w2: the parameter
        itself, and for D a multiple of 256 w2t and w13t too (the down and dX
        GEMMs read w2's [K = H][N = D] rows, and w1's then w3's as one K = 2H
        operand split along K, transposed in LDS): no weight is written then;
        otherwise w2t and w13t (for a backward) are written, in one launch."""
        dev = w1.device
        nn = D % 256 == 0
        W2t = None if nn else torch.empty(E, D, H, dtype=torch.bfloat16, device=dev)
        W13t = torch.empty(E, D, 2 * H, dtype=torch.bfloat16, device=dev) if dgrad and not nn else None
        BF = _lib.QUANT_BF16

        def job(src, dst_t, col_off, cols_out):
            return _lib.FmWeightJob(_lib.ptr(src), _lib.DTYPE_BF16, E, H, D, D, H * D, BF,
                                    None, 0, 0, 0, None, 0, 0,
                                    _lib.ptr(dst_t), cols_out, D * cols_out, col_off, None, 0, 0)

        jobs = [] if nn else [job(w2, W2t, 0, H)]
        if dgrad and not nn:
            jobs += [job(w1, W13t, 0, 2 * H), job(w3, W13t, H, 2 * H)]
        if jobs:
            arr = (_lib.FmWeightJob * len(jobs))(*jobs)
            self._launch(arr, len(jobs), w1, (w1, w2, w3))
        self.w13 = ExpertWeightOperand(w1, None, D, H * D, N=2 * H, K=D, data2=w3, split=H)
        self.w2 = ExpertWeightOperand(w2, None, D, H * D, N=H, K=D)
        if nn:
            self.w2t = ExpertWeightOperand(w2, None, D, H * D, N=D, K=H, kmajor=True)
        else:
            self.w2t = ExpertWeightOperand(W2t, None, H, D * H, N=D, K=H)
        if dgrad:
            self.w13t = (ExpertWeightOperand(w1, None, D, H * D, N=D, K=2 * H, kmajor=True, data2=w3, split=H)
                         if nn else ExpertWeightOperand(W13t, None, 2 * H, D * 2 * H, N=D, K=2 * H))

    def _build_mx(self, w1, w2, w3, E, H, D, dgrad, paired=False):
        """``paired``: every operand (rows and transposed outputs) in the
        paired-row layout; a transposed operand's experts then sit 2x their
        column offset apart in each pair row (a 64-column piece takes 128
        bytes there)."""
        dev = w1.device
        w1, w2, w3 = (w.contiguous() for w in (w1, w2, w3))
        stream = _lib.stream_of(w1)
        MX = _lib.QUANT_MX
        # gate|up: w1 and w3 read in place as the [E, 2H, D] stack
        W13, S13, W13t, S13t = _alloc_quant(E * 2 * H, D, MX, True, dgrad, dev)
        _lib.call("fm_quantize_pair", _lib.ptr(w1), _lib.ptr(w3), _src_dtype(w1), E, H, D, D,
                  *_tile_args(MX, W13, S13, W13t, S13t, paired, paired and dgrad), stream)
        W2, S2, W2t, S2t = _alloc_quant(E * H, D, MX, dgrad, True, dev)
        _lib.call("fm_quantize", _lib.ptr(w2), _src_dtype(w2), E * H, D, D,
                  *_tile_args(MX, W2, S2, W2t, S2t, paired and dgrad, paired), stream)
        cs = 2 if paired else 1   # column-offset group strides in a paired buffer
        self.w13 = ExpertWeightOperand(W13, S13, D, 2 * H * D, D // 32, 1, 2 * H * D // 32, 0, 2 * H, D,
                                       paired=paired)
        self.w2t = ExpertWeightOperand(W2t, S2t, E * H, cs * H, 1, D, (H // 32) * D, 0, D, H, paired=paired)
        if dgrad:
            self.w13t = ExpertWeightOperand(W13t, S13t, E * 2 * H, cs * 2 * H, 1, D, (2 * H // 32) * D, 0, D, 2 * H,
                                            paired=paired)
            self.w2 = ExpertWeightOperand(W2, S2, D, H * D, D // 32, 1, H * D // 32, 0, H, D, paired=paired)


# ================================================================= streams ====
_SIDE = {}


def _side_stream(dev) -> torch.cuda.Stream:
    """One extra stream per device, at the default priority."""
    idx = torch.device(dev).index
    if idx is None:
        idx = torch.cuda.current_device()
    s = _SIDE.get(idx)
    if s is None:
        s = _SIDE[idx] = torch.cuda.Stream(device=idx)
    return s


# ================================================================ expert block ====
@dataclass
class FP8FlowMoEConfig:
    enabled: bool = False
    fp8_recipe: FP8RecipeConfig = field(default_factory=FP8RecipeConfig)


class _FlowMoEFunction(torch.autograd.Function):
    """Forward + backward of the expert block; see FP8FlowMoECompute."""

    @staticmethod
    def forward(ctx, x, weights, w1, w2, w3, indices, compute):
        return compute._forward(ctx, x, weights, w1, w2, w3, indices)

    @staticmethod
    def backward(ctx, grad_out):
        return ctx.compute._backward(ctx, grad_out)


class FP8FlowMoECompute:
    """The expert block behind ``MoEBase._fp8_flow_moe`` (reference
    ``model/moe.py:1313-1332``).

    ``__call__(x [N, D], weights [N, K] fp32, indices [N, K] int, expert_offset,
    num_local_experts) -> [N, D]`` returns sum_k weights[n, k] *
    expert_{indices[n, k]}(x[n]) with SwiGLU experts
    ``(silu(x w1_e^T) * (x w3_e^T)) w2_e`` (reference ``model/moe.py:1164-1183``),
    differentiable with respect to x, weights, w1, w2, w3.

    Dataflow (all on the GPU, no host synchronisation):
      route (stable counting sort, groups padded to 128 rows)
      -> permute + quantise x (row blocks; column blocks kept for dW13)
      -> grouped GEMM gate|up -> SwiGLU + quantise -> grouped GEMM down
      -> weighted unpermute.
    ``fp8_gemm_threshold``: experts with at least that many assignments use
    the FP8 GEMMs, the others BF16 (0 forces FP8 for all).  The object owns no
    parameters and adds no state_dict keys; weights are borrowed via
    ``set_weights``.
    """

    def __init__(self, config: FP8FlowMoEConfig, d_model: int, hidden_size: int,
                 num_experts: int, fp8_gemm_threshold: int = 1000000):
        if d_model % 128 or hidden_size % 128:
            raise ValueError(f"d_model ({d_model}) and hidden_size ({hidden_size}) must be "
                             "multiples of 128")
        self.config = config
        self.d_model = d_model
        self.hidden_size = hidden_size
        self.num_experts = num_experts
        self.fp8_gemm_threshold = int(fp8_gemm_threshold)
        recipe = config.fp8_recipe if config.enabled else FP8RecipeConfig()
        self.recipe = recipe
        self.fp8_kind = recipe.act_kind
        if self.fp8_kind == _lib.QUANT_BF16:
            self.fp8_gemm_threshold = 1 << 62  # no FP8 recipe: every expert on BF16
        self._w = None
        self._cache = {}
        # When set to a dict, forward stores the bf16 gate|up GEMM output
        # ("gate_up") and backward the bf16 dH GEMM output ("dh"), [rows_max, *];
        # used by parity tests to feed a CPU oracle the device's own GEMM results.
        self.capture_intermediates = None
        # Run the router's backward (and dW2 where it does not share dH's
        # grid) on a second stream beside the main stream's work (False keeps
        # every launch on the caller's stream).
        self.overlap_streams = True
        # One group, every token in it with weight 1 (set by
        # FP8SharedExpertCompute): the routing plan is the identity, built once
        # per token count, and the outputs are the padded buffers' first rows
        # (no unpermute copies).
        self._dense = False
        self._dense_plans = {}
        self._record = True

    def set_weights(self, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor) -> None:
        for w in (w1, w2, w3):
            if tuple(w.shape) != (self.num_experts * self.hidden_size, self.d_model):
                raise ValueError(f"expert weights must be [E*H, D] = "
                                 f"[{self.num_experts * self.hidden_size}, {self.d_model}], got {tuple(w.shape)}")
        self._w = (w1, w2, w3)

    def _weights(self, kind: int, need_dgrad: bool = True, defer: Optional[list] = None) -> ExpertWeights:
        ew = self._cache.get(kind)
        if ew is None:
            ew = self._cache[kind] = ExpertWeights(kind, paired=True)
        return ew.refresh(*self._w, self.num_experts, need_dgrad, defer)

    def _paired(self, kind) -> bool:
        """The block's pow2 row operands (tokens, weights) in the paired-row
        layout: every ragged-M GEMM takes the ring kernel."""
        return ExpertWeights.paired_ok(kind, self.num_experts, self.hidden_size, self.d_model)

    def _paired_cols(self, kind, plan, mask) -> bool:
        """The column operands of the weight gradients paired too: the ring
        kernel's ragged-K walk takes no expert mask and no K split."""
        if not self._paired(kind) or mask is not None:
            return False
        H, D = self.hidden_size, self.d_model
        dev = plan.offsets.device
        return _k_splits(kind, plan, 2 * H, D, dev) == 1 and _k_splits(kind, plan, H, D, dev) == 1

    def modes(self, num_assignments: int):
        """Which GEMM families run: (fp8_kind or None, bf16 bool), decided on
        the host from the threshold alone (no read of the device counts)."""
        if self.fp8_kind == _lib.QUANT_BF16:
            return None, True
        if self.fp8_gemm_threshold <= 0:
            return self.fp8_kind, False
        if self.fp8_gemm_threshold > num_assignments:
            return None, True
        return self.fp8_kind, True

    def __call__(self, x, weights, indices, expert_offset: int = 0,
                 num_local_experts: Optional[int] = None):
        if self._w is None:
            raise RuntimeError("set_weights() must be called before the expert block runs")
        E = self.num_experts if num_local_experts is None else int(num_local_experts)
        if E != self.num_experts:
            raise ValueError(f"num_local_experts={E} but the block holds {self.num_experts} experts")
        _lib.require_device(x, "x")
        if expert_offset:
            indices = indices - int(expert_offset)
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        K = indices.shape[-1]
        # the dgrad weight operands are built only for a forward that records a backward
        self._record = torch.is_grad_enabled() and any(
            t.requires_grad for t in (x, weights, *self._w))
        out = _FlowMoEFunction.apply(x2, weights.reshape(-1, K), *self._w,
                                     indices.reshape(-1, K), self)
        return out.reshape(shape)

    # ------------------------------------------------------------------ forward ----
    def _forward(self, ctx, x, weights, w1, w2, w3, indices):
        ctx.x_dtype = x.dtype
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        x = x.contiguous()
        T, D = x.shape
        E, H = self.num_experts, self.hidden_size
        K = indices.shape[1]
        fp8_kind, use_bf16 = self.modes(T * K)
        dev = x.device
        thr = self.fp8_gemm_threshold if fp8_kind is not None else 1 << 62
        # expert-weight refreshes are deferred so the first batch runs with the
        # routing sort (its blocks fill the CUs the sort leaves idle)
        kinds = [k for k in (fp8_kind, _lib.QUANT_BF16 if use_bf16 else None) if k is not None]
        batches = []
        ews = {}
        try:
            for k in kinds:
                ews[k] = self._weights(k, self._record, batches)
            side = batches.pop(0) if batches else None
            if self._dense:
                plan = self._dense_plans.get((T, dev))
                if plan is None:
                    plan = self._dense_plans[(T, dev)] = route_tokens(indices, E, thr, side and side[:2])
                    side = None
            else:
                plan = route_tokens(indices, E, thr, side and side[:2])
                side = None
            for jobs, n, _sources in ([side] if side is not None else []) + batches:
                _lib.call("fm_quantize_weight_batch", jobs, n, _lib.stream_of(x))
        except BaseException:
            # a deferred weight quantisation may not have been launched: the
            # next call must rebuild rather than read unwritten operands
            for ew in ews.values():
                ew.invalidate()
            raise
        del side, batches   # the launches are enqueued: their sources may go
        wts = weights.to(torch.float32).contiguous()
        R = plan.rows_max
        GU = torch.empty(R, 2 * H, dtype=torch.bfloat16, device=dev)
        Y = torch.empty(R, D, dtype=torch.bfloat16, device=dev)
        mask = plan.use_fp8 if (fp8_kind is not None and use_bf16) else None
        # with the threshold splitting the experts, each precision's producers
        # write only its own experts' tiles (the other GEMMs never read them)
        tiles = {}
        if mask is not None:
            tiles[fp8_kind], tiles[_lib.QUANT_BF16] = plan.precision_tiles()
        saved = {}
        pcols = {k: self._paired_cols(k, plan, mask) for k in kinds}
        for kind, want in ((fp8_kind, 1), (_lib.QUANT_BF16 if use_bf16 else None, 0)):
            if kind is None:
                continue
            ew = ews[kind]
            pt = fused_permute_pad(x, plan, E, granularity=_gran(kind), pow2_scale=kind == _lib.QUANT_POW2,
                                   return_transpose=self._record, kmajor_scales=True,
                                   tile_valid=tiles.get(kind, plan.tile_expert), paired_rows=self._paired(kind),
                                   paired_cols=pcols.get(kind, False))
            _gemm_m(kind, pt.rows, ew.w13, plan, GU, mask, want)
            saved[kind] = (pt.rows_t, ew)
        h_cols = {}
        for kind, want in ((fp8_kind, 1), (_lib.QUANT_BF16 if use_bf16 else None, 0)):
            if kind is None:
                continue
            # row blocks feed the down GEMM; the column blocks are kept for dW2
            pr = self._paired(kind)
            pc = pcols[kind]
            q, s, qt, st = _swiglu(GU[:, :H], GU[:, H:], R, H, kind, True, self._record, dev,
                                   tiles.get(kind, plan.tile_expert), kmajor=True, paired=pr, col_paired=pc)
            hrow, hcol = _wrap(q, s, qt, st, kind, pr, pc)
            h_cols[kind] = hcol
            _gemm_m(kind, hrow, saved[kind][1].w2t, plan, Y, mask, want)
        if self._dense:
            # the output must not be a view made inside this Function (callers
            # combine it in place): the padded buffer itself when T fills it
            out = Y if R == T else Y[:T].clone()
        else:
            out = fused_unpermute_unpad(Y, plan, wts)
        if self.capture_intermediates is not None:
            self.capture_intermediates["gate_up"] = GU.detach().clone()
        ctx.compute = self
        ctx.plan = plan
        ctx.tiles = tiles
        ctx.pcols = pcols
        ctx.kinds = (fp8_kind, use_bf16)
        ctx.saved_cols = {k: v[0] for k, v in saved.items()}
        # the dgrad weight operands of this forward's weights (a later forward
        # may rebuild the cache before this backward runs)
        ctx.dgrad_ops = {k: (ew.w2, ew.w13t) for k, ew in ews.items()} if self._record else None
        ctx.saved_hcols = h_cols
        ctx.wdtypes = (w1.dtype, w2.dtype, w3.dtype)
        # Y only feeds the router-weight gradient (the dense path's outputs are
        # views of Y: not saving it leaves them free for in-place use)
        ctx.save_for_backward(wts, GU, Y if ctx.needs_input_grad[1] else None)
        return out if ctx.x_dtype == torch.bfloat16 else out.to(ctx.x_dtype)

    # ----------------------------------------------------------------- backward ----
    def _backward(self, ctx, grad_out, on_router_grad=None):
        """Gradients of the expert block.  ``on_router_grad(dw, can_fold, dot)``
        (a MoE layer whose router feeds this block) is called with the
        router-weight gradient as soon as it exists -- or, when the hook has
        ``fused_dot`` set and K <= 8, with ``dot`` (RouterDotInputs: the
        upstream gradient, the saved expert outputs and the row map) for the
        router's gating backward to form it in its own pass -- and returns the
        router's share of the input gradient, summed in the unpermute:
        {"addend": bf16 [T, D]}, or with ``can_fold`` {"dlogits": [T, E],
        "gate_w": [E, D]} (E <= 8) for the unpermute to form it itself."""
        wts, GU, Y = ctx.saved_tensors
        plan = ctx.plan
        fp8_kind, use_bf16 = ctx.kinds
        E, H, D = self.num_experts, self.hidden_size, self.d_model
        T, K = plan.num_tokens, plan.top_k
        R = plan.rows_max
        dev = GU.device
        dO = grad_out.reshape(T, D).to(torch.bfloat16).contiguous()
        mask = plan.use_fp8 if (fp8_kind is not None and use_bf16) else None
        # router-weight gradient from the saved expert outputs (skipped when
        # the weights need none, e.g. the constant weights of a shared expert)
        dw = dot = None
        if ctx.needs_input_grad[1] and getattr(on_router_grad, "fused_dot", False) and K <= 8 and not self._dense:
            dot = RouterDotInputs(dO, Y, plan.row_of)
        elif ctx.needs_input_grad[1]:
            dw = torch.empty(T * K, dtype=torch.float32, device=dev)
            _lib.call("fm_router_weight_grad", _lib.ptr(dO), dO.stride(0), _lib.ptr(Y), Y.stride(0),
                      _lib.ptr(plan.row_of), T, K, D, _lib.ptr(dw), _lib.stream_of(dO))
        main = torch.cuda.current_stream(dev)
        side = _side_stream(dev) if self.overlap_streams else main
        # the router's share of the input gradient: a [T, D] addend, or its
        # (dlogits, gate weight) terms folded into the unpermute.  Its backward
        # reads only dO, the saved expert outputs and x, so it runs on the second
        # stream beside the dY permute and dH; the unpermute waits for it.
        rshare = {}
        if on_router_grad is not None:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                rshare = on_router_grad(None if dw is None else dw.reshape(T, K), not self._dense, dot)
        dH = torch.empty(R, H, dtype=torch.bfloat16, device=dev)
        dXp = torch.empty(R, D, dtype=torch.bfloat16, device=dev)
        w1dt, w2dt, w3dt = ctx.wdtypes
        dW1 = torch.empty(E * H, D, dtype=w1dt, device=dev)
        dW2 = torch.empty(E * H, D, dtype=w2dt, device=dev)
        dW3 = torch.empty(E * H, D, dtype=w3dt, device=dev)
        if not (w1dt == w3dt and w1dt in (torch.float32, torch.bfloat16) and w2dt in (torch.float32, torch.bfloat16)):
            raise TypeError("expert weights must be float32 or bfloat16 (w1 and w3 alike)")
        runs = [(k, w) for k, w in ((fp8_kind, 1), (_lib.QUANT_BF16 if use_bf16 else None, 0)) if k is not None]
        tiles = ctx.tiles
        pcols = ctx.pcols
        dy = {kind: fused_permute_pad(dO, plan, E, granularity=_gran(kind), pow2_scale=kind == _lib.QUANT_POW2,
                                      return_transpose=True, weights=None if self._dense else wts,
                                      kmajor_scales=True, tile_valid=tiles.get(kind, plan.tile_expert),
                                      paired_rows=self._paired(kind), paired_cols=pcols.get(kind, False))
              for kind, _ in runs}
        # dH and dW2 (contraction over each expert's tokens) both read the
        # permuted dY: each alone leaves its last round of workgroups
        # part-empty when the hidden size is not a multiple of the 256-wide
        # tile.  One grid holds both (BF16, pow2) when dW2's tiles fill at
        # least a round of the GPU's CUs; otherwise (a few long tiles, as for
        # a shared expert's one group) and for the other kinds dW2 runs on the
        # second stream beside dH and what follows it, with no K split (the
        # CUs it leaves idle run the main stream).  The forward's saved SwiGLU
        # columns are dW2's operand not in cache.
        fill = E * -(-H // 256) * -(-D // 256) >= _cus(dev)
        # (paired row operands share a grid only with paired column operands)
        one_grid = [(k, w) for k, w in runs
                    if k in _MK_KINDS and fill and (not self._paired(k) or pcols.get(k, False))]
        two_streams = [(k, w) for k, w in runs if (k, w) not in one_grid]
        if two_streams:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                for kind, want in two_streams:
                    _gemm_k(kind, ctx.saved_hcols[kind], dy[kind].rows_t, plan, H, D, dW2, H * D, mask=mask,
                            want=want, may_split=side is main, a_cold=True)
        if ctx.dgrad_ops is None:
            raise RuntimeError("the expert block's forward did not record a backward")
        for kind, want in one_grid:
            _gemm_mk(kind, dy[kind].rows, ctx.dgrad_ops[kind][0], plan, dH, ctx.saved_hcols[kind],
                     dy[kind].rows_t, H, D, dW2, H * D, mask, want, a_cold=True)
        for kind, want in two_streams:
            _gemm_m(kind, dy[kind].rows, ctx.dgrad_ops[kind][0], plan, dH, mask, want)
        if self.capture_intermediates is not None:
            self.capture_intermediates["dh"] = dH.detach().clone()
        for kind, want in runs:
            pr = self._paired(kind)
            pc = pcols.get(kind, False)
            gq, gs, gqt, gst = _alloc_quant(R, 2 * H, kind, True, True, dev, kmajor=True)
            _lib.call("fm_swiglu_backward", _lib.ptr(GU), GU.stride(0), _lib.ptr(GU[:, H:]), GU.stride(0),
                      _lib.ptr(dH), dH.stride(0), R, H, *_tile_args(kind, gq, gs, gqt, gst, pr, pc),
                      _lib.ptr(tiles.get(kind, plan.tile_expert)), _lib.stream_of(GU))
            dgu_row, dgu_col = _wrap(gq, gs, gqt, gst, kind, pr, pc)
            # dW1 | dW3: contraction over each expert's tokens
            _gemm_k(kind, dgu_col, ctx.saved_cols[kind], plan, 2 * H, D, dW1, H * D, dW3, H * D, split=H,
                    mask=mask, want=want)
            # input gradient
            _gemm_m(kind, dgu_row, ctx.dgrad_ops[kind][1], plan, dXp, mask, want)
        # the router's backward and dW2 (and the buffers they read, referenced
        # until here) are done before the router's dx share is summed
        main.wait_stream(side)
        dx_addend = rshare.get("addend")
        if self._dense:
            dx = dXp[:T] if dx_addend is None else dXp[:T] + dx_addend
        else:
            terms = (rshare["dlogits"], rshare["gate_w"]) if "dlogits" in rshare else None
            dx = fused_unpermute_unpad(dXp, plan, None, addend=dx_addend, router_terms=terms)
        ctx.saved_cols = None
        ctx.saved_hcols = None
        ctx.dgrad_ops = None
        return (dx.to(ctx.x_dtype), None if dw is None else dw.reshape(T, K), dW1, dW2, dW3, None, None)


class FP8SharedExpertCompute:
    """A dense SwiGLU FFN ``(silu(x w1^T) * (x w3^T)) w2^T`` on the expert
    block's path as a single group: the shared expert of a DeepSeek-V2 style
    MoE (reference ``model/moe.py:1299-1301``, added to the routed output at
    ``:1383-1384`` and ``:1686-1687``; ``ExpertMLP`` ``:1164-1183``) or the
    bias-free dense FFN (``model/feed_forward.py:74-80`` with silu).

    Every token goes to the one group with weight 1, so routing reduces to
    padding the rows to a multiple of 128 (the identity plan is built once
    per token count and the output and input gradient are the first rows of
    the padded buffers: no sort and no unpermute copies per step), and the
    same fused quantisers, grouped GEMMs and SwiGLU kernels run as for the
    routed experts (FP8 per the recipe; ``fp8_gemm_threshold`` > number of
    tokens selects BF16).
    ``set_weights(w1 [H, D], w2 [H, D], w3 [H, D])`` borrows the weights
    (``w2`` stored as ``[H, D]``, i.e. the transpose of ``nn.Linear(H, D)``'s
    weight, like the expert block's); ``__call__(x [..., D]) -> [..., D]`` is
    differentiable with respect to x, w1, w2 and w3.
    """

    def __init__(self, config: FP8FlowMoEConfig, d_model: int, hidden_size: int,
                 fp8_gemm_threshold: int = 0):
        self._block = FP8FlowMoECompute(config, d_model, hidden_size, 1, fp8_gemm_threshold)
        self._block._dense = True
        self._route = {}

    @property
    def block(self) -> FP8FlowMoECompute:
        return self._block

    def set_weights(self, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor) -> None:
        self._block.set_weights(w1, w2, w3)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        _lib.require_device(x, "x")
        T = x.numel() // x.shape[-1]
        key = (T, x.device)
        r = self._route.get(key)
        if r is None:
            r = self._route[key] = (torch.ones(T, 1, dtype=torch.float32, device=x.device),
                                    torch.zeros(T, 1, dtype=torch.int64, device=x.device))
        return self._block(x, r[0], r[1])


def _gran(kind):
    if kind == _lib.QUANT_BF16:
        return None
    if kind == _lib.QUANT_MX:
        return G.MX_1x32
    return G.ROW_1x128
