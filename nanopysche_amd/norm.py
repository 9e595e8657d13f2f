"""RMSNorm ahead of the MoE on the MI355X path, fused with the activation
quantisation: ``RMSNorm`` (reference ``model/norm.py:18-49``, the
``moe_norm`` of ``MoEHybridTransformerBlock``, ``model/transformer.py:233``,
applied at ``:261-263``) and ``rmsnorm_quantize``, which emits the norm's
bf16 output, its e4m3 row blocks and their scales from one read of the
residual stream.

The 128-token column blocks of the transpose (the weight-gradient operand of a
dense consumer such as the shared expert) need every row's rsqrt before any
block's amax is known, so they are formed from the kernel's outputs: the
scaling-aware transpose of the power-of-two row blocks (``flow_moe``
recipe), or the column quantiser over the bf16 output (fp32-scale and MX
recipes).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .flow_moe import FP8Tensor, G, quantize_to_fp8, scaling_aware_transpose
from .recipes import BlockScalingGranularity

DEFAULT_EPS = 1e-6   # RMSNorm.__init__ default, model/norm.py:27


@dataclass
class NormOutput:
    """What ``rmsnorm_quantize`` produced: the bf16 output y [T, D], its e4m3
    row blocks, the column blocks of its transpose, and rsqrt [T] (fp32)."""

    y: Optional[torch.Tensor]
    rows: Optional[FP8Tensor]
    cols: Optional[FP8Tensor]
    rstd: torch.Tensor


def _dtype_code(t: torch.Tensor, what: str) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    raise TypeError(f"{what} must be bfloat16 or float32, got {t.dtype}")


def _check_d(D: int) -> None:
    n, rem = divmod(D, 512)
    if rem or n not in (1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16):
        raise ValueError(f"RMSNorm on this path needs D = 512 n with n in 1..8, 10, 12, 14 or 16, got {D}")


def _rows2d(x: torch.Tensor) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1])
    return x2 if x2.stride(-1) == 1 and x2.stride(0) % 8 == 0 else x2.contiguous()


def rmsnorm_quantize(x: torch.Tensor, weight: torch.Tensor, eps: float = DEFAULT_EPS,
                     granularity: Optional[BlockScalingGranularity] = None, *, pow2_scale: bool = False,
                     return_transpose: bool = False, return_normed: bool = True) -> NormOutput:
    """RMSNorm of x [..., D] (bf16 or fp32) with weight [D], in fp32 as the
    reference's full-precision module computes it, emitted as the bf16 output
    (``return_normed``), the e4m3 row blocks of that output (``granularity``
    ROW_1x128 with fp32 or ``pow2_scale`` scales, or MX_1x32 with e8m0) and,
    with ``return_transpose``, the column blocks of its transpose (128x1 /
    32x1; for ``pow2_scale`` the scaling-aware transpose of the row blocks).
    rstd is always returned."""
    _lib.require_device(x, "x")
    _lib.require_device(weight, "weight")
    x2 = _rows2d(x)
    T, D = x2.shape
    _check_d(D)
    if tuple(weight.shape) != (D,):
        raise ValueError(f"weight must be [{D}], got {tuple(weight.shape)}")
    w = weight if weight.is_contiguous() else weight.contiguous()
    dev = x.device
    kind = -1
    q = s = None
    if granularity is not None:
        granularity = BlockScalingGranularity(granularity)
        if granularity == G.MX_1x32:
            kind = _lib.QUANT_MX
            q = torch.empty(T, D, dtype=torch.uint8, device=dev)
            s = torch.empty(T, D // 32, dtype=torch.uint8, device=dev)
        elif granularity == G.ROW_1x128:
            kind = _lib.QUANT_POW2 if pow2_scale else _lib.QUANT_BLOCK
            q = torch.empty(T, D, dtype=torch.uint8, device=dev)
            s = torch.empty(T, D // 128, dtype=torch.float32, device=dev)
        else:
            raise ValueError("granularity must be ROW_1x128 or MX_1x32 (row blocks)")
    elif return_transpose:
        raise ValueError("return_transpose needs a row granularity")
    # the column quantiser of the fp32-scale and MX recipes reads y
    need_y = return_normed or (return_transpose and kind != _lib.QUANT_POW2)
    y = torch.empty(T, D, dtype=torch.bfloat16, device=dev) if need_y else None
    rstd = torch.empty(T, dtype=torch.float32, device=dev)
    _lib.call("fm_rmsnorm_quantize", _lib.ptr(x2), _dtype_code(x2, "x"), x2.stride(0), T, D, _lib.ptr(w),
              _dtype_code(w, "weight"), float(eps), _lib.ptr(y), 0 if y is None else y.stride(0), kind,
              _lib.ptr(q), 0 if q is None else q.stride(0), _lib.ptr(s), 0 if s is None else s.stride(0),
              _lib.ptr(rstd), _lib.stream_of(x2))
    rows = cols = None
    if kind != -1:
        rows = FP8Tensor(q, s, granularity, kind == _lib.QUANT_POW2)
        if return_transpose:
            if T % 128:
                raise ValueError(f"column blocks of the transpose need T % 128 == 0, got {T}")
            if kind == _lib.QUANT_POW2:
                cols = scaling_aware_transpose(rows)
            else:
                cols = quantize_to_fp8(y, G.MX_32x1 if kind == _lib.QUANT_MX else G.COL_128x1)
    if not return_normed:
        y = None
    elif y is not None:
        y = y.reshape(*x.shape[:-1], D)
    return NormOutput(y, rows, cols, rstd)


def rmsnorm_backward(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, rstd: torch.Tensor,
                     need_dw: bool = True):
    """(dx in x's dtype, dw in weight's dtype or None) of y = x r w."""
    x2 = _rows2d(x)
    T, D = x2.shape
    dy2 = _rows2d(dy.to(x2.dtype))
    dx = torch.empty_like(x2)
    dw = ws = None
    nbytes = 0
    if need_dw:
        dw = torch.empty(D, dtype=weight.dtype, device=x.device)
        if T == 0:
            return dx.reshape(x.shape), dw.zero_()
        nbytes = int(_lib.load().fm_rmsnorm_backward_workspace_bytes(T, D))
        ws = torch.empty(nbytes // 4, dtype=torch.float32, device=x.device)
    w = weight if weight.is_contiguous() else weight.contiguous()
    _lib.call("fm_rmsnorm_backward", _lib.ptr(dy2), dy2.stride(0), _lib.ptr(x2), _dtype_code(x2, "x"), x2.stride(0),
              T, D, _lib.ptr(w), _dtype_code(w, "weight"), _lib.ptr(rstd), _lib.ptr(dx), dx.stride(0),
              _lib.ptr(dw), 0 if dw is None else _dtype_code(dw, "weight"), _lib.ptr(ws), nbytes,
              _lib.stream_of(x2))
    return dx.reshape(x.shape), dw


class _RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        out = rmsnorm_quantize(x, weight, eps)
        ctx.save_for_backward(x, weight, out.rstd)
        return out.y

    @staticmethod
    def backward(ctx, dy):
        x, weight, rstd = ctx.saved_tensors
        dx, dw = rmsnorm_backward(dy, x, weight, rstd, need_dw=ctx.needs_input_grad[1])
        return (dx if ctx.needs_input_grad[0] else None), dw, None


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = DEFAULT_EPS) -> torch.Tensor:
    """Differentiable RMSNorm of bf16 x [..., D] -> bf16 (model/norm.py:32-49)."""
    if x.dtype != torch.bfloat16:
        raise TypeError(f"rmsnorm takes the bf16 residual stream, got {x.dtype}")
    return _RMSNormFunction.apply(x, weight, float(eps))


class RMSNorm(torch.nn.Module):
    """``RMSNorm(size, eps=1e-6, full_precision=True)`` of the reference
    (``model/norm.py:18-49``) on the HIP kernels: fp32 weight initialised to
    ones, fp32 arithmetic, bf16 in and out.  ``full_precision=False`` (bf16
    arithmetic) is not offered."""

    def __init__(self, size: int, *, eps: float = DEFAULT_EPS, full_precision: bool = True):
        super().__init__()
        if not full_precision:
            raise NotImplementedError("the MI355X RMSNorm computes in fp32 (full_precision=True)")
        _check_d(size)
        self.eps = eps
        self.full_precision = True
        self.weight = torch.nn.Parameter(torch.ones(size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rmsnorm(x, self.weight, self.eps)
