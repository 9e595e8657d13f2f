"""GPU parity of the quantisation kernels against the CPU oracle: payload
bytes and scales bit-exact (BASELINE config 2 shapes and edge cases)."""

import numpy as np
import pytest
import torch

import nanopysche_amd as fm
from oracle import fp8 as ofp8
from tests.helpers import randn_bf16

pytestmark = pytest.mark.gpu
G = fm.BlockScalingGranularity


def _np(t):
    return t.detach().cpu().numpy()


def _edge_matrix():
    """256 x 512 bf16 with zero blocks, ties, saturation-adjacent values, subnormals."""
    x = randn_bf16((256, 512), seed=11).float()
    x[0:2, 0:128] = 0.0                      # all-zero 1x128 blocks
    x[2, 0:128] = 0.0
    x[2, 5] = 448.0                          # amax exactly 448 -> scale 1
    x[2, 6] = 464.0 * (448.0 / 448.0) / 2    # an exact half-way value after scaling
    x[3, 0:128] = 2.0 ** -20                 # tiny block (amax below the 1e-12 floor? no: 9.5e-7)
    x[4, 0:128] = 1e-13                      # below the amax floor -> payload rounds to 0
    x[5, 128:256] = torch.linspace(-3, 3, 128)
    x[6, 256:384] = -7.0                     # constant block
    x[7, 384:512] = torch.arange(128).float() * 2 ** -12  # e4m3-subnormal range after scaling
    x[8:128, 0:128] = 0.0                    # a whole 128x128 tile of zeros
    x[9, 128:256] = -0.0                     # a negative-zero block (code 0x80)
    x[10, 256:384:2] = -0.0                  # signed zeros beside regular values
    x[10, 257:384:2] = 1.5
    x[11, 384:512] = -1e-30                  # negative values that quantise to -0
    x[11, 400] = 2.0
    return x.bfloat16()


@pytest.mark.parametrize("pow2", [False, True])
def test_quant_1x128_config2_bitexact(dev, pow2):
    x = randn_bf16((8192, 4096), seed=1, outlier_frac=0.001)
    q = fm.quantize_to_fp8(x.to(dev), G.ROW_1x128, pow2_scale=pow2)
    rq, rs = ofp8.quant_1x128(x.float().numpy(), pow2=pow2)
    assert np.array_equal(_np(q.scale), rs)
    assert np.array_equal(_np(q.data), rq)


@pytest.mark.parametrize("pow2", [False, True])
def test_fused_row_col_bitexact(dev, pow2):
    x = randn_bf16((2048, 1024), seed=1, outlier_frac=0.001)
    row, col = fm.quantize_to_fp8(x.to(dev), G.ROW_1x128, pow2_scale=pow2, return_transpose=True)
    rq, rs = ofp8.quant_1x128(x.float().numpy(), pow2=pow2)
    assert np.array_equal(_np(row.data), rq) and np.array_equal(_np(row.scale), rs)
    if pow2:
        cq, cs = ofp8.scaling_aware_transpose(rq, rs)
    else:
        cq, cs = ofp8.quant_128x1(x.float().numpy())
    assert np.array_equal(_np(col.scale), cs)
    assert np.array_equal(_np(col.data), cq)


def test_edge_blocks_bitexact(dev):
    x = _edge_matrix()
    for pow2 in (False, True):
        row, col = fm.quantize_to_fp8(x.to(dev), pow2_scale=pow2, return_transpose=True)
        rq, rs = ofp8.quant_1x128(x.float().numpy(), pow2=pow2)
        assert np.array_equal(_np(row.data), rq) and np.array_equal(_np(row.scale), rs)
        cq, cs = (ofp8.scaling_aware_transpose(rq, rs) if pow2 else ofp8.quant_128x1(x.float().numpy()))
        assert np.array_equal(_np(col.data), cq) and np.array_equal(_np(col.scale), cs)
    mq = fm.quantize_to_fp8(x.to(dev), G.MX_1x32)
    oq, oc = ofp8.quant_mx_1x32(x.float().numpy())
    assert np.array_equal(_np(mq.data), oq) and np.array_equal(_np(mq.scale), oc)


def test_edge_blocks_transpose_and_weights_bitexact(dev):
    """fp32-scale paths on the edge matrix (signed zeros, tiny and saturating
    values): the scaling-aware transpose of the row output and the 128x128
    weight quantiser, bit-exact against the oracle."""
    x = _edge_matrix()
    xf = x.float().numpy()
    row = fm.quantize_to_fp8(x.to(dev))
    t = fm.scaling_aware_transpose(row)
    cq, cs = ofp8.scaling_aware_transpose(_np(row.data), _np(row.scale))
    assert np.array_equal(_np(t.scale), cs) and np.array_equal(_np(t.data), cq)
    w = fm.quantize_to_fp8(x.to(dev), G.BLOCK_128x128)
    wq, ws = ofp8.quant_128x128(xf)
    assert np.array_equal(_np(w.scale), ws) and np.array_equal(_np(w.data), wq)
    assert (_np(row.data)[9, 128:256] == 0x80).all()


def test_fp32_input_and_ragged_rows(dev):
    x = randn_bf16((333, 256), seed=5).float() * 3.7  # rows not a multiple of 128
    q = fm.quantize_to_fp8(x.to(dev))
    rq, rs = ofp8.quant_1x128(x.numpy())
    assert np.array_equal(_np(q.data), rq) and np.array_equal(_np(q.scale), rs)
    mq = fm.quantize_to_fp8(x.to(dev), G.MX_1x32)
    oq, oc = ofp8.quant_mx_1x32(x.numpy())
    assert np.array_equal(_np(mq.data), oq) and np.array_equal(_np(mq.scale), oc)


def test_mx_1x32_and_32x1_bitexact(dev):
    x = randn_bf16((1024, 2048), seed=4, outlier_frac=0.001)
    row, col = fm.quantize_to_fp8(x.to(dev), G.MX_1x32, return_transpose=True)
    oq, oc = ofp8.quant_mx_1x32(x.float().numpy())
    tq, tc = ofp8.quant_mx_32x1(x.float().numpy())
    assert np.array_equal(_np(row.data), oq) and np.array_equal(_np(row.scale), oc)
    assert np.array_equal(_np(col.data), tq) and np.array_equal(_np(col.scale), tc)


@pytest.mark.parametrize("pow2", [False, True])
def test_weight_128x128_config2_bitexact(dev, pow2):
    w = randn_bf16((14336, 4096), seed=1, std=0.02)
    q = fm.quantize_to_fp8(w.to(dev), G.BLOCK_128x128, pow2_scale=pow2)
    rq, rs = ofp8.quant_128x128(w.float().numpy(), pow2=pow2)
    assert np.array_equal(_np(q.scale), rs)
    assert np.array_equal(_np(q.data), rq)


def test_dequantize_bitexact(dev):
    x = randn_bf16((1024, 1024), seed=3, outlier_frac=0.001)
    xd = x.to(dev)
    row, col = fm.quantize_to_fp8(xd, return_transpose=True)
    for out_dtype in (torch.float32, torch.bfloat16):
        d = fm.dequantize_from_fp8(row, out_dtype)
        ref = ofp8.dequant_1x128(_np(row.data), _np(row.scale))
        if out_dtype == torch.bfloat16:
            ref = ofp8.bf16_round(ref)
        assert np.array_equal(d.float().cpu().numpy(), ref)
        dc = fm.dequantize_from_fp8(col, out_dtype)
        refc = ofp8.dequant_1x128(_np(col.data), np.ascontiguousarray(_np(col.scale).T))
        if out_dtype == torch.bfloat16:
            refc = ofp8.bf16_round(refc)
        assert np.array_equal(dc.float().cpu().numpy(), refc)
    w = fm.quantize_to_fp8(xd, G.BLOCK_128x128)
    assert np.array_equal(fm.dequantize_from_fp8(w, torch.float32).cpu().numpy(),
                          ofp8.dequant_128x128(_np(w.data), _np(w.scale)))
    m = fm.quantize_to_fp8(xd, G.MX_1x32)
    assert np.array_equal(fm.dequantize_from_fp8(m, torch.float32).cpu().numpy(),
                          ofp8.dequant_mx_1x32(_np(m.data), _np(m.scale)))


@pytest.mark.parametrize("pow2", [False, True])
def test_scaling_aware_transpose_bitexact(dev, pow2):
    x = randn_bf16((8192, 4096), seed=1, outlier_frac=0.001)
    row = fm.quantize_to_fp8(x.to(dev), pow2_scale=pow2)
    t = fm.scaling_aware_transpose(row)
    cq, cs = ofp8.scaling_aware_transpose(_np(row.data), _np(row.scale))
    assert np.array_equal(_np(t.scale), cs)
    assert np.array_equal(_np(t.data), cq)


def test_scaling_aware_transpose_exact_for_pow2(dev):
    """Size-independent property at full size: with power-of-two scales the
    transpose preserves every dequantised value outside the e4m3 subnormal range."""
    x = randn_bf16((8192, 4096), seed=1, outlier_frac=0.001).to(dev)
    row = fm.quantize_to_fp8(x, pow2_scale=True)
    t = fm.scaling_aware_transpose(row)
    a = fm.dequantize_from_fp8(row, torch.float32).T
    b = fm.dequantize_from_fp8(t, torch.float32)
    st = t.scale.T.repeat_interleave(128, dim=1)  # [C, R] column-block scale per element
    normal = a.abs() / st >= 2.0 ** -6  # the exactly shifted value is an e4m3 normal
    assert normal.float().mean() > 0.5
    assert torch.equal(a[normal], b[normal])


def test_rejects_bad_shapes(dev):
    with pytest.raises((RuntimeError, ValueError)):
        fm.quantize_to_fp8(torch.zeros(128, 100, dtype=torch.bfloat16, device=dev))
    with pytest.raises((RuntimeError, ValueError)):
        fm.quantize_to_fp8(torch.zeros(100, 128, dtype=torch.bfloat16, device=dev), return_transpose=True)


def test_hw_convert_matches_software(dev):
    """The kernels encode with gfx950's v_cvt_pk_fp8_f32 / v_cvt_pk_bf16_f32;
    they must agree bit for bit with the integer routines (which the CPU tests
    pin against torch's casts) on every bf16 pattern, e4m3 midpoints and
    random fp32 values around them."""
    from nanopysche_amd import _lib

    rng = np.random.default_rng(0)
    pos = ofp8._POS.astype(np.float32)
    mids = ((ofp8._POS[1:] + ofp8._POS[:-1]) / 2).astype(np.float32)
    x = np.concatenate([
        (np.arange(0, 65536, dtype=np.uint32) << 16).view(np.float32),
        rng.standard_normal(2_000_000).astype(np.float32) * np.float32(100),
        rng.standard_normal(1_000_000).astype(np.float32) * np.float32(2e-3),
        pos, -pos, mids, -mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e4)),
        ((np.arange(0, 1 << 22, dtype=np.uint32) << 9) | 0x00007FFF).view(np.float32),  # bf16 ties +/- 1
        ((np.arange(0, 1 << 22, dtype=np.uint32) << 9) | 0x00008000).view(np.float32),
    ])
    x = x[np.isfinite(x)]
    x = x[: x.size // 4 * 4]
    xd = torch.from_numpy(x).to(dev)
    n = xd.numel()
    e_hw = torch.empty(n, dtype=torch.uint8, device=dev)
    e_sw = torch.empty_like(e_hw)
    b_hw = torch.empty(n, dtype=torch.int16, device=dev)
    b_sw = torch.empty_like(b_hw)
    _lib.call("fm_convert_check", _lib.ptr(xd), n, _lib.ptr(e_hw), _lib.ptr(e_sw), _lib.ptr(b_hw),
              _lib.ptr(b_sw), _lib.stream_of(xd))
    assert torch.equal(e_hw, e_sw)
    assert torch.equal(b_hw, b_sw)
    # and the software path is the oracle's (torch's) cast
    ref = ofp8.e4m3_encode(np.clip(x, -448, 448))
    assert np.array_equal(e_sw.cpu().numpy(), ref)


def test_hw_decode_matches_software(dev):
    """The scaling-aware transpose decodes e4m3 with gfx950's v_cvt_pk_f32_fp8;
    it must equal the integer decode (pinned against torch on the CPU) for all
    256 codes, NaN codes included."""
    from nanopysche_amd import _lib

    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).repeat(4).to(dev)
    hw = torch.empty(codes.numel(), dtype=torch.float32, device=dev)
    sw = torch.empty_like(hw)
    _lib.call("fm_decode_check", _lib.ptr(codes), codes.numel(), _lib.ptr(hw), _lib.ptr(sw),
              _lib.stream_of(codes))
    h, s_ = hw.cpu().numpy(), sw.cpu().numpy()
    nan = np.isnan(s_)
    assert np.array_equal(np.isnan(h), nan) and nan.sum() == 2 * 4
    assert np.array_equal(h[~nan].view(np.uint32), s_[~nan].view(np.uint32))
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ref), nan[:256])
    assert np.array_equal(ref[~nan[:256]].view(np.uint32), s_[:256][~nan[:256]].view(np.uint32))


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kind", ["block", "pow2"])
def test_weight_batch_matches_single_launches(dev, src_dtype, kind):
    """fm_quantize_weight_batch (w1, w3 into one [E, 2H, D] operand, w2 into
    its own, one launch) writes the same bytes and scales as one
    fm_quantize_weight launch per job."""
    from nanopysche_amd import _lib
    E, H, D = 3, 256, 384
    k = {"block": _lib.QUANT_BLOCK, "pow2": _lib.QUANT_POW2}[kind]
    ws = [randn_bf16((E * H, D), seed=s, std=0.02).to(src_dtype).to(dev) for s in (31, 32, 33)]
    dt = _lib.DTYPE_F32 if src_dtype == torch.float32 else _lib.DTYPE_BF16

    def outputs():
        u8, f32 = torch.uint8, torch.float32
        return [torch.full((E, 2 * H, D), 0x55, dtype=u8, device=dev),
                torch.full((E, 2 * H // 128, D // 128), -1.0, dtype=f32, device=dev),
                torch.full((E, D, 2 * H), 0x55, dtype=u8, device=dev),
                torch.full((E, D // 128, 2 * H // 128), -1.0, dtype=f32, device=dev),
                torch.full((E, H, D), 0x55, dtype=u8, device=dev),
                torch.full((E, H // 128, D // 128), -1.0, dtype=f32, device=dev),
                torch.full((E, D, H), 0x55, dtype=u8, device=dev),
                torch.full((E, D // 128, H // 128), -1.0, dtype=f32, device=dev)]

    def args(src, q, s, qt, st, row_off, rows_out):
        return (_lib.ptr(src), dt, E, H, D, D, H * D, k, _lib.ptr(q), D, rows_out * D, row_off,
                _lib.ptr(s), D // 128, (rows_out // 128) * (D // 128), _lib.ptr(qt), rows_out, D * rows_out,
                row_off, _lib.ptr(st), rows_out // 128, (D // 128) * (rows_out // 128))

    st = _lib.stream_of(ws[0])
    single, batch = outputs(), outputs()
    plan = [(ws[0], 0, 0, 2 * H), (ws[1], 0, H, 2 * H), (ws[2], 4, 0, H)]
    for src, o, off, rows_out in plan:
        _lib.call("fm_quantize_weight", *args(src, *single[o:o + 4], off, rows_out), st)
    jobs = (_lib.FmWeightJob * 3)(*[_lib.FmWeightJob(*args(src, *batch[o:o + 4], off, rows_out))
                                    for src, o, off, rows_out in plan])
    _lib.call("fm_quantize_weight_batch", jobs, 3, st)
    torch.cuda.synchronize()
    for a, b in zip(single, batch):
        assert torch.equal(a, b)
    # every byte and scale was written (the fill values are gone)
    assert not (single[1] < 0).any() and not (single[5] < 0).any()
