"""Numpy restatement of the blockwise FP8 quantisation spec (test oracle only).

The reference package ``fp8_flow_moe`` that owns these functions is not in
the reference tree: only its exported names are (``fp8/__init__.py:8-24``,
``fp8/flow_moe.py:3-15``).  The spec restated here is therefore the closed
form fixed by the benchmark configuration (1x128 row blocks, 128x128 weight
blocks, ``scale = amax / 448`` in fp32, OCP e4m3fn payload) plus the OCP MX
v1.0 rule for the 1x32 / e8m0 variant.  Choices the absent package would
have pinned are stated as constants below.

Algorithmic independence: the e4m3 encoder here is a nearest-value search
over the 127 finite positive codes with ties broken to the even code; the
HIP kernels use an integer bit-rounding routine.  Both are checked against
``torch.Tensor.to(torch.float8_e4m3fn)`` in the tests.

Pinning (tests/test_oracle_fp8.py):
  e4m3_encode / e4m3_decode  -- exhaustive code table vs OCP e4m3fn formula,
                                vs torch cast on ~1M floats incl. ties.
  quant_1x128 / quant_128x128 / quant_128x1 -- hand-built blocks with
                                known answers (exact powers of two, ties,
                                zero blocks, saturation), torch-cast
                                cross-check of the whole pipeline.
  pow2 scales                -- closed form 2**ceil(log2(r)) in float64.
  quant_mx_1x32              -- closed form floor(log2(amax)) via frexp.
  scaling_aware_transpose    -- exactness invariant for pow2 scales:
                                dequant(out) == dequant(in).T outside the
                                e4m3 subnormal range; brute-force loop on a
                                tiny case.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
AMAX_FLOOR = np.float32(1e-12)  # all-zero block => scale = 1e-12/448, payload 0
BLOCK = 128
MX_BLOCK = 32
MX_EMAX_E4M3 = 8  # exponent of the largest e4m3fn normal (448 = 1.75 * 2**8)


# ---------------------------------------------------------------- e4m3fn ----
def _e4m3_positive_table() -> np.ndarray:
    """Values of codes 0x00..0x7E (0x7F is NaN), from the OCP FP8 formula."""
    vals = np.empty(127, dtype=np.float64)
    for code in range(127):
        e = code >> 3
        m = code & 7
        if e == 0:
            vals[code] = m * 2.0 ** -9
        else:
            vals[code] = (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


_POS = _e4m3_positive_table()


_LUT = np.empty(256, dtype=np.float32)
_LUT[:127] = _POS
_LUT[127] = np.nan
_LUT[128:] = -_LUT[:128]


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 (0x7F/0xFF -> NaN), by a 256-entry table
    built from the OCP formula above."""
    return _LUT[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x: np.ndarray, saturate: bool = False) -> np.ndarray:
    """float32 -> uint8 e4m3fn, round-to-nearest-even.

    Non-saturating (torch semantics): |x| > 464 (the midpoint between 448 and
    the NaN code's would-be value 480) encodes to NaN (0x7F with sign); the
    tie 464 goes to the even code 0x7E (448).
    Saturating: |x| > 448 clamps to 448.  NaN input -> 0x7F.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = np.signbit(x)
    a = np.abs(x.astype(np.float64))
    nan_in = np.isnan(a)
    a = np.where(nan_in, 0.0, a)
    if saturate:
        a = np.minimum(a, E4M3_MAX)
    hi = np.searchsorted(_POS, a, side="left")  # _POS[hi-1] < a <= _POS[hi]
    hi_c = np.minimum(hi, 126)
    lo_c = np.maximum(hi - 1, 0)
    d_hi = _POS[hi_c] - a
    d_lo = a - _POS[lo_c]
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi_c % 2 == 0))
    code = np.where(pick_hi, hi_c, lo_c)
    code = np.where(a == _POS[hi_c], hi_c, code)
    # above the top code: 448 < a <= 464 rounds to 448, a > 464 is NaN
    over = a > E4M3_MAX
    code = np.where(over, np.where(a > 464.0, 0x7F, 126), code)
    code = np.where(nan_in, 0x7F, code)
    code = code.astype(np.uint8) | (sign.astype(np.uint8) << 7)
    return code


def e4m3_encode_fast(x: np.ndarray, saturate: bool = False) -> np.ndarray:
    """``e4m3_encode`` through torch's CPU cast to float8_e4m3fn (RNE,
    non-saturating), for the large arrays of the layer oracle: the search
    encoder above costs ~1 s per million values.  Same results bit for bit
    (tests/test_oracle_fp8.py pins the two on every float32 bit pattern class
    that matters: ~1M random values, all e4m3 midpoints, the overflow edges and
    NaN); NaN inputs are mapped to 0x7F with their sign as the spec does."""
    import torch

    x = np.asarray(x, dtype=np.float32)
    nan_in = np.isnan(x)
    y = np.clip(x, -E4M3_MAX, E4M3_MAX) if saturate else x
    code = torch.from_numpy(np.ascontiguousarray(y)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    if nan_in.any():
        code = np.where(nan_in, np.uint8(0x7F) | (np.signbit(x).astype(np.uint8) << 7), code)
    return code.astype(np.uint8)


# arrays at least this large take the torch-cast encoder
_FAST_ENCODE_MIN = 1 << 16


def _encode(x: np.ndarray, saturate: bool = False) -> np.ndarray:
    if np.size(x) >= _FAST_ENCODE_MIN:
        return e4m3_encode_fast(x, saturate)
    return e4m3_encode(x, saturate)


# ------------------------------------------------------------------ e8m0 ----
def f32_biased_exponent(x: np.ndarray) -> np.ndarray:
    return ((np.asarray(x, dtype=np.float32).view(np.uint32) >> 23) & 0xFF).astype(np.int32)


def e8m0_decode(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.int32)
    return np.ldexp(np.float32(1.0), c - 127).astype(np.float32, copy=False)


def pow2_ceil(r: np.ndarray) -> np.ndarray:
    """Smallest power of two >= r, for positive normal float32 r."""
    r = np.asarray(r, dtype=np.float32)
    bits = r.view(np.uint32)
    e = (bits >> 23) & 0xFF
    e = e + ((bits & 0x7FFFFF) != 0)
    return (e.astype(np.uint32) << 23).view(np.float32)


# ----------------------------------------------------------- quantisers ----
def block_scale(amax: np.ndarray, pow2: bool) -> np.ndarray:
    """scale = max(amax, 1e-12) / 448 (fp32 IEEE division); pow2 rounds up."""
    amax = np.maximum(np.asarray(amax, dtype=np.float32), AMAX_FLOOR)
    s = (amax / np.float32(E4M3_MAX)).astype(np.float32, copy=False)
    return pow2_ceil(s) if pow2 else s


# Arrays of at least _FAST_ENCODE_MIN elements take torch CPU ops (threaded)
# for the elementwise steps below; each step is the same IEEE fp32 operation
# as the numpy one (division, max of absolute values, product with a scale),
# and tests/test_oracle_fp8.py pins both paths equal bit for bit.
def _tt(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def _amax(xb: np.ndarray, axis) -> np.ndarray:
    if np.size(xb) >= _FAST_ENCODE_MIN:
        return _tt(xb).abs().amax(dim=axis).numpy()
    return np.abs(xb).max(axis=axis)


def _quant_with_scale(x: np.ndarray, s: np.ndarray) -> np.ndarray:
    if np.size(x) >= _FAST_ENCODE_MIN:
        y = (_tt(x) / _tt(s)).clamp_(-E4M3_MAX, E4M3_MAX).numpy()
        return _encode(y)
    y = (x.astype(np.float32, copy=False) / s.astype(np.float32, copy=False)).astype(np.float32, copy=False)
    y = np.clip(y, -E4M3_MAX, E4M3_MAX)
    return _encode(y)


def _scaled_decode(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """decode(q) * s with s broadcast against q's shape."""
    if np.size(q) >= _FAST_ENCODE_MIN:
        import torch

        v = torch.from_numpy(np.ascontiguousarray(q, dtype=np.uint8)).view(torch.float8_e4m3fn).float()
        return (v * _tt(s)).numpy()
    return e4m3_decode(q) * np.asarray(s, dtype=np.float32)


def quant_1x128(x: np.ndarray, pow2: bool = False):
    """Row blocks: x [R, C] (C % 128 == 0) -> (q uint8 [R, C], scale f32 [R, C/128])."""
    x = np.asarray(x, dtype=np.float32)
    R, C = x.shape
    assert C % BLOCK == 0
    xb = x.reshape(R, C // BLOCK, BLOCK)
    s = block_scale(_amax(xb, -1), pow2)
    q = _quant_with_scale(xb, s[..., None]).reshape(R, C)
    return q, s


def quant_128x1(x: np.ndarray, pow2: bool = False):
    """Column blocks, transposed output: x [R, C] (R % 128 == 0) ->
    (qt uint8 [C, R], scale_t f32 [R/128, C])."""
    qt, st = quant_1x128(np.asarray(x, dtype=np.float32).T, pow2)
    return qt, np.ascontiguousarray(st.T)


def quant_128x128(w: np.ndarray, pow2: bool = False):
    """Square blocks: w [R, C] -> (q uint8 [R, C], scale f32 [R/128, C/128])."""
    w = np.asarray(w, dtype=np.float32)
    R, C = w.shape
    assert R % BLOCK == 0 and C % BLOCK == 0
    wb = w.reshape(R // BLOCK, BLOCK, C // BLOCK, BLOCK)
    s = block_scale(_amax(wb, (1, 3)), pow2)
    q = _quant_with_scale(wb, s[:, None, :, None]).reshape(R, C)
    return q, s


def mx_scale_code(amax: np.ndarray) -> np.ndarray:
    """OCP MX: X = floor(log2(amax)) - emax_elem, as a biased e8m0 code.

    Taken from the fp32 exponent field; amax == 0 or subnormal -> code 0."""
    e = f32_biased_exponent(amax)
    return np.clip(e - MX_EMAX_E4M3, 0, 254).astype(np.uint8)


def quant_mx_1x32(x: np.ndarray):
    """MXFP8 row blocks of 32: x [R, C] -> (q uint8 [R, C], e8m0 uint8 [R, C/32]).

    q = saturate_e4m3(x * 2**(127 - code)); the multiply is by an exact power
    of two, identical to dividing by the block scale 2**(code - 127)."""
    x = np.asarray(x, dtype=np.float32)
    R, C = x.shape
    assert C % MX_BLOCK == 0
    xb = x.reshape(R, C // MX_BLOCK, MX_BLOCK)
    code = mx_scale_code(_amax(xb, -1))
    inv = np.ldexp(np.float32(1.0), 127 - code.astype(np.int32)).astype(np.float32, copy=False)
    y = (xb * inv[..., None]).astype(np.float32, copy=False)
    q = _encode(y, saturate=True).reshape(R, C)
    return q, code


def quant_mx_32x1(x: np.ndarray):
    """MXFP8 column blocks of 32, transposed: x [R, C] -> (qt [C, R], e8m0 [R/32, C])."""
    qt, ct = quant_mx_1x32(np.asarray(x, dtype=np.float32).T)
    return qt, np.ascontiguousarray(ct.T)


# ------------------------------------------------------------- dequant ----
def dequant_1x128(q, s):
    R, C = q.shape
    v = _scaled_decode(q.reshape(R, C // BLOCK, BLOCK), np.asarray(s, dtype=np.float32)[..., None])
    return v.reshape(R, C)


def dequant_128x128(q, s):
    R, C = q.shape
    v = _scaled_decode(q.reshape(R // BLOCK, BLOCK, C // BLOCK, BLOCK),
                       np.asarray(s, dtype=np.float32)[:, None, :, None])
    return v.reshape(R, C)


def dequant_mx_1x32(q, code):
    R, C = q.shape
    v = _scaled_decode(q.reshape(R, C // MX_BLOCK, MX_BLOCK), e8m0_decode(code)[..., None])
    return v.reshape(R, C)


# ---------------------------------------------------- scaling-aware transpose ----
def scaling_aware_transpose(q: np.ndarray, s: np.ndarray):
    """Row-quantised (1x128) FP8 -> column-quantised (128x1) FP8 of the transpose.

    No return to the high-precision source.  Column-block scale is the largest
    of the 128 row scales it covers, so no element can overflow; each element is
    re-expressed as e4m3(fp32(fp32(decode(q) * s_row) / s_col)).  With
    power-of-two scales this is an exponent shift and is exact unless the
    result falls below the e4m3 normal range.

    q [R, C] uint8, s [R, C/128] -> (qt [C, R] uint8, st [R/128, C] f32)."""
    R, C = q.shape
    assert R % BLOCK == 0 and C % BLOCK == 0
    s = np.asarray(s, dtype=np.float32)
    # per-element row scale s[r, c // 128], as a broadcast over [R, C/128, 128]
    v = _scaled_decode(q.reshape(R, C // BLOCK, BLOCK), s[..., None])
    st = s.reshape(R // BLOCK, BLOCK, C // BLOCK).max(axis=1)  # [R/128, C/128]
    # column block j of row block b takes the largest row scale of the tile
    y = _quant_with_scale(v.reshape(R // BLOCK, BLOCK, C // BLOCK, BLOCK), st[:, None, :, None])
    qt = np.ascontiguousarray(y.reshape(R, C).T)
    return qt, np.repeat(st, BLOCK, axis=1)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (RNE) -> float32, written with integer ops (torch's
    bf16 cast for large arrays, NaN canonicalised the same way; pinned equal)."""
    x = np.asarray(x, dtype=np.float32)
    if x.size >= _FAST_ENCODE_MIN:
        import torch

        r = torch.from_numpy(np.ascontiguousarray(x)).bfloat16().float().numpy()
        nan = np.isnan(x)
        return np.where(nan, np.float32(np.nan), r).astype(np.float32, copy=False) if nan.any() else r
    b = x.view(np.uint32)
    nan = (b & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = b + (np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1)))   # no wrap for non-NaN b
    r &= np.uint32(0xFFFF0000)
    r = np.where(nan, np.uint32(0x7FC00000), r)
    return r.view(np.float32)
