"""Pins the FP8 oracle (oracle/fp8.py) without trusting its own formulas:
against torch's float8_e4m3fn cast and decode (a library routine), closed
forms computed in float64, hand-built known-answer blocks, and brute-force
loops on tiny inputs."""

import math

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8

GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def torch_cast(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_matches_torch_and_spot_values():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(ofp8.e4m3_decode(codes), ref, equal_nan=True)
    dec = ofp8.e4m3_decode(np.uint8([0x7E, 0x01, 0x08, 0x38, 0x7F, 0x80, 0xFE]))
    assert dec[0] == 448.0 and dec[1] == 2.0 ** -9 and dec[2] == 2.0 ** -6 and dec[3] == 1.0
    assert np.isnan(dec[4]) and dec[5] == 0.0 and np.signbit(dec[5]) and dec[6] == -448.0


def test_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    pos = ofp8._POS.astype(np.float32)
    mids = ((ofp8._POS[1:] + ofp8._POS[:-1]) / 2).astype(np.float32)
    x = np.concatenate([
        (np.arange(0, 65536, dtype=np.uint32) << 16).view(np.float32),
        rng.standard_normal(500_000).astype(np.float32) * np.float32(60),
        rng.standard_normal(100_000).astype(np.float32) * np.float32(1e-3),
        pos, -pos, mids, -mids,
        np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e4)),
        np.float32([464.0, 463.99997, 464.00003, np.inf, -np.inf]),
    ])
    x = x[~np.isnan(x)]
    a, b = ofp8.e4m3_encode(x), torch_cast(x)
    nan_a, nan_b = (a & 0x7F) == 0x7F, (b & 0x7F) == 0x7F
    assert np.array_equal(nan_a, nan_b)
    assert np.array_equal(a[~nan_a], b[~nan_a])


@pytest.mark.parametrize("saturate", [False, True])
def test_fast_encoder_equals_search_encoder(saturate):
    """The torch-cast encoder the layer oracle uses on large arrays gives the
    search encoder's codes bit for bit, NaN codes and their signs included,
    and the quantisers give the same bytes through either encoder."""
    rng = np.random.default_rng(7)
    mids = ((ofp8._POS[1:] + ofp8._POS[:-1]) / 2).astype(np.float32)
    x = np.concatenate([
        (np.arange(0, 65536, dtype=np.uint32) << 16).view(np.float32),
        rng.standard_normal(300_000).astype(np.float32) * np.float32(60),
        mids, -mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e4)),
        np.float32([464.0, -464.0, 463.99997, 464.00003, 1e6, -1e6, np.inf, -np.inf, np.nan, -np.nan]),
    ])
    assert np.array_equal(ofp8.e4m3_encode_fast(x, saturate), ofp8.e4m3_encode(x, saturate))
    a = (rng.standard_normal((512, 256)) * np.exp(rng.standard_normal((512, 1)) * 4)).astype(np.float32)
    old = ofp8._FAST_ENCODE_MIN
    try:
        ofp8._FAST_ENCODE_MIN = 1 << 62
        slow = [ofp8.quant_1x128(a), ofp8.quant_128x128(a, pow2=True), ofp8.quant_mx_1x32(a),
                ofp8.scaling_aware_transpose(*ofp8.quant_1x128(a, pow2=True))]
        slow_deq = [ofp8.dequant_1x128(*slow[0]), ofp8.dequant_128x128(*slow[1]),
                    ofp8.dequant_mx_1x32(*slow[2]), ofp8.bf16_round(x)]
        ofp8._FAST_ENCODE_MIN = 0
        fast = [ofp8.quant_1x128(a), ofp8.quant_128x128(a, pow2=True), ofp8.quant_mx_1x32(a),
                ofp8.scaling_aware_transpose(*ofp8.quant_1x128(a, pow2=True))]
        fast_deq = [ofp8.dequant_1x128(*slow[0]), ofp8.dequant_128x128(*slow[1]),
                    ofp8.dequant_mx_1x32(*slow[2]), ofp8.bf16_round(x)]
    finally:
        ofp8._FAST_ENCODE_MIN = old
    for (qs, ss), (qf, sf) in zip(slow, fast):
        assert np.array_equal(qs, qf) and np.array_equal(ss, sf)
    for vs, vf in zip(slow_deq, fast_deq):
        assert np.array_equal(vs.view(np.uint32), vf.view(np.uint32))


def test_saturating_encode():
    x = np.float32([447.0, 448.0, 460.0, 470.0, 1e6, -1e6, -500.0])
    assert ofp8.e4m3_encode(x, saturate=True).tolist() == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE]


def _torch_rowquant(x, pow2=False):
    """Spec restated with torch ops: amax / 448 via torch division and torch's cast."""
    t = torch.from_numpy(x.astype(np.float32)).reshape(x.shape[0], -1, 128)
    amax = t.abs().amax(-1).clamp(min=torch.tensor(1e-12, dtype=torch.float32))
    s = amax / 448.0
    if pow2:
        s = torch.tensor([[2.0 ** math.ceil(math.log2(float(v))) for v in row] for row in s],
                         dtype=torch.float32)
    q = (t / s[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    return q.reshape(x.shape).numpy(), s.numpy()


def test_known_answer_blocks():
    x = np.zeros((4, 256), np.float32)
    x[0, :128] = 1.0                     # constant block: every element -> 448 (0x7E), scale 1/448
    x[1, :128] = np.linspace(-448, 448, 128)  # amax 448 -> scale exactly 1, payload = cast(x)
    x[2, 128:] = 3.0
    x[2, 200] = -6.0                     # amax 6 -> scale 6/448; 3 -> 224 (0x76), -6 -> -448 (0xFE)
    q, s = ofp8.quant_1x128(x)
    assert np.all(q[0, :128] == 0x7E) and s[0, 0] == np.float32(1.0) / np.float32(448.0)
    assert s[1, 0] == 1.0 and np.array_equal(q[1, :128], torch_cast(x[1, :128]))
    assert s[2, 1] == np.float32(6.0) / np.float32(448.0)
    assert q[2, 200] == 0xFE and np.all(np.delete(q[2, 128:], 200 - 128) == 0x76)
    # all-zero block: scale is the 1e-12 floor / 448, payload zero
    assert q[3].max() == 0 and s[3, 0] == np.float32(1e-12) / np.float32(448.0)


@pytest.mark.parametrize("pow2", [False, True])
def test_rowquant_matches_torch_restatement(pow2):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 100
    x = ofp8.bf16_round(x)
    q, s = ofp8.quant_1x128(x, pow2=pow2)
    tq, ts = _torch_rowquant(x, pow2)
    assert np.array_equal(s, ts) and np.array_equal(q, tq)
    # a scale taken along the wrong axis or a multiply by 448/amax would not round-trip
    d = ofp8.dequant_1x128(q, s)
    assert np.all(np.abs(d - x) <= np.abs(x) * 2.0 ** -4 + s.repeat(128, 1) * 2.0 ** -9)


def test_pow2_scale_closed_form():
    rng = np.random.default_rng(2)
    amax = np.exp(rng.uniform(-30, 10, 20000)).astype(np.float32)
    amax[:5] = np.float32([448.0, 896.0, 1.0, 0.0, 1e-20])
    s = ofp8.block_scale(amax, pow2=True)
    r = np.maximum(amax.astype(np.float32), np.float32(1e-12)) / np.float32(448)
    ref = np.array([2.0 ** math.ceil(math.log2(float(v))) for v in r], dtype=np.float32)
    assert np.array_equal(s, ref)
    assert s[0] == 1.0 and s[1] == 2.0 and s[2] == 2.0 ** -8


def test_mx_scale_closed_form():
    rng = np.random.default_rng(3)
    amax = np.exp(rng.uniform(-40, 40, 20000)).astype(np.float32)
    code = ofp8.mx_scale_code(amax).astype(np.int64)
    m, e = np.frexp(amax.astype(np.float64))  # amax = m * 2**e, m in [0.5, 1)
    ref = np.clip((e - 1) - 8 + 127, 0, 254)
    assert np.array_equal(code, ref)
    normal = (ref > 0) & (ref < 254)
    scaled = amax[normal] * np.exp2(127.0 - code[normal])
    assert np.all((scaled >= 256) & (scaled < 512))


def test_mx_quant_brute_force():
    rng = np.random.default_rng(4)
    x = ofp8.bf16_round(rng.standard_normal((8, 64)).astype(np.float32) * 10)
    x[0, :32] = 0.0
    q, c = ofp8.quant_mx_1x32(x)
    for r in range(8):
        for b in range(2):
            blk = x[r, 32 * b: 32 * b + 32]
            am = float(np.abs(blk).max())
            code = 0 if am == 0 else min(max(math.floor(math.log2(am)) - 8 + 127, 0), 254)
            assert c[r, b] == code
            y = torch.tensor(blk / np.float32(2.0 ** (code - 127))).clamp(-448, 448)
            assert np.array_equal(q[r, 32 * b: 32 * b + 32], y.to(torch.float8_e4m3fn).view(torch.uint8).numpy())


def test_128x128_and_128x1_brute_force():
    rng = np.random.default_rng(5)
    w = ofp8.bf16_round(rng.standard_normal((256, 384)).astype(np.float32) * 0.02)
    q, s = ofp8.quant_128x128(w)
    for bi in range(2):
        for bj in range(3):
            blk = w[128 * bi:128 * bi + 128, 128 * bj:128 * bj + 128]
            sc = np.float32(max(float(np.abs(blk).max()), np.float32(1e-12))) / np.float32(448)
            assert s[bi, bj] == sc
            ref = torch.tensor(blk / sc).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(q[128 * bi:128 * bi + 128, 128 * bj:128 * bj + 128], ref)
    qt, st = ofp8.quant_128x1(w)
    assert qt.shape == (384, 256) and st.shape == (2, 384)
    for c in (0, 77, 383):
        for rb in range(2):
            col = w[128 * rb:128 * rb + 128, c]
            sc = np.float32(max(float(np.abs(col).max()), np.float32(1e-12))) / np.float32(448)
            assert st[rb, c] == sc
            ref = torch.tensor(col / sc).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(qt[c, 128 * rb:128 * rb + 128], ref)


@pytest.mark.parametrize("pow2", [False, True])
def test_scaling_aware_transpose_brute_force(pow2):
    rng = np.random.default_rng(6)
    x = ofp8.bf16_round(rng.standard_normal((256, 256)).astype(np.float32))
    x[:128, :128] *= np.exp(rng.uniform(-6, 6, (128, 1))).astype(np.float32)  # very different rows
    q, s = ofp8.quant_1x128(x, pow2=pow2)
    qt, st = ofp8.scaling_aware_transpose(q, s)
    dec = torch.from_numpy(q).view(torch.float8_e4m3fn).float().numpy()
    for rb in range(2):
        for cb in range(2):
            rows = slice(128 * rb, 128 * rb + 128)
            smax = s[rows, cb].max()
            for c in range(128 * cb, 128 * cb + 128):
                assert st[rb, c] == smax
                v = (dec[rows, c] * s[rows, cb]).astype(np.float32)
                ref = torch.tensor(v / smax).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
                assert np.array_equal(qt[c, rows], ref)
    if pow2:
        # exactness: values survive unless they fall into the e4m3 subnormal range
        a = ofp8.dequant_1x128(q, s).T
        b = ofp8.dequant_1x128(qt, np.ascontiguousarray(st.T))
        normal = np.abs(a) / np.repeat(st.T, 128, axis=1) >= 2.0 ** -6  # exact value is e4m3-normal
        assert normal.mean() > 0.5
        assert np.array_equal(a[normal], b[normal])


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 1e3,
                        (np.arange(0, 1 << 20, 7, dtype=np.uint32) * 4093).view(np.float32)])
    x = x[np.isfinite(x)]
    ref = torch.from_numpy(x).bfloat16().float().numpy()
    assert np.array_equal(ofp8.bf16_round(x), ref)


def test_golden_fixtures():
    """Committed vectors written by tests/golden/make_golden.py from torch's cast."""
    g = np.load(GOLDEN / "e4m3_cases.npz")
    assert np.array_equal(ofp8.e4m3_encode(g["x"]), g["codes"])
    k = np.load(GOLDEN / "quant_kat.npz")
    q, s = ofp8.quant_1x128(k["x"])
    assert np.array_equal(q, k["q"]) and np.array_equal(s, k["s"])
    q2, s2 = ofp8.quant_1x128(k["x"], pow2=True)
    assert np.array_equal(q2, k["q_pow2"]) and np.array_equal(s2, k["s_pow2"])
    qm, cm = ofp8.quant_mx_1x32(k["x"])
    assert np.array_equal(qm, k["q_mx"]) and np.array_equal(cm, k["c_mx"])
