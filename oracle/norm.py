"""Numpy restatement of the reference's RMSNorm (test oracle only).

Follows ``RMSNorm.forward`` (reference ``model/norm.py:32-49``) with
``full_precision=True`` (its default): the input is widened to float32, the
variance is ``mean(x^2)`` over the last dimension in float32, the row is
multiplied by ``rsqrt(variance + eps)`` and then by the weight (float32,
``weight.type_as(x_normed)``), and the result is narrowed to the input dtype.
``MoEHybridTransformerBlock`` applies it to the residual stream before the MoE
(``model/transformer.py:261-263``).

The backward is the closed form of that map's gradient, in float64:
with ``r = (mean(x^2) + eps)^(-1/2)`` and ``g = dy * w``,
``dx = r g - (r^3 / D) (sum_j g_j x_j) x`` and ``dw = sum_t dy x r``.

Pinning (tests/test_oracle_norm.py): the forward against torch's float64
evaluation of the reference's op sequence (the float32 result within float32
rounding of it, the bf16 output off by at most one unit in the last place
where the float64 value sits on a rounding boundary); the backward against
torch.autograd of that float64 op sequence; invariants that a dropped or
misplaced term breaks (scale invariance, unit mean square with unit weight,
eps dominating tiny rows); planted mistakes in the oracle (eps outside the
square root, sum in place of mean, the r^3 term dropped) fail those checks.
"""

from __future__ import annotations

import numpy as np

from .fp8 import bf16_round

DEFAULT_EPS = 1e-6   # RMSNorm.__init__ default, model/norm.py:27


def rmsnorm_f32(x: np.ndarray, w: np.ndarray, eps: float = DEFAULT_EPS):
    """(out fp32 [T, D], r fp32 [T]): the reference's float32 arithmetic,
    model/norm.py:40-45 (variance -> rsqrt -> x * r -> * weight)."""
    xf = np.asarray(x, np.float32)
    wf = np.asarray(w, np.float32)
    var = np.mean(np.square(xf), axis=-1, dtype=np.float32)
    r = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    out = (xf * r[..., None]).astype(np.float32) * wf
    return out.astype(np.float32), r


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = DEFAULT_EPS):
    """(y, r): the module's output for bf16 input -- the float32 result
    narrowed to bf16 (:47-48), returned as float32 values -- and rsqrt."""
    out, r = rmsnorm_f32(x, w, eps)
    return bf16_round(out), r


def rmsnorm_backward(dy: np.ndarray, x: np.ndarray, w: np.ndarray, eps: float = DEFAULT_EPS):
    """(dx, dw) in float64 for y = x r w, r = (mean(x^2) + eps)^(-1/2)."""
    x64 = np.asarray(x, np.float64)
    dy64 = np.asarray(dy, np.float64)
    w64 = np.asarray(w, np.float64)
    D = x64.shape[-1]
    r = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    g = dy64 * w64
    dot = np.sum(g * x64, axis=-1, keepdims=True)
    dx = r * g - (r ** 3 / D) * dot * x64
    dw = np.sum(dy64 * x64 * r, axis=tuple(range(x64.ndim - 1)))
    return dx, dw
