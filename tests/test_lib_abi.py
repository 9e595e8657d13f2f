"""CPU checks of the C ABI: the library loads, exports every function that
include/fm_hip.h declares (and ctypes signatures cover them), rejects bad
arguments before touching the device, and its host e4m3 codec (the same
routine the kernels inline) agrees with torch's cast."""

import ctypes as C
import re
from pathlib import Path

import numpy as np
import torch

from nanopysche_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "fm_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(fm_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_version():
    assert b"gfx950" in _lib.load().fm_version()


def test_host_codec_matches_torch():
    lib = _lib.load()
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (np.arange(0, 65536, dtype=np.uint32) << 16).view(np.float32),
        rng.standard_normal(200_000).astype(np.float32) * np.float32(50),
        np.float32([464.0, 463.99997, 464.00003, 448.0, 2 ** -10, 3 * 2 ** -11, -0.0]),
    ])
    x = x[np.isfinite(x)]
    out = np.empty(x.size, np.uint8)
    lib.fm_host_encode_e4m3(x.ctypes.data, out.ctypes.data, x.size)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    nan_a, nan_b = (out & 0x7F) == 0x7F, (ref & 0x7F) == 0x7F
    assert np.array_equal(nan_a, nan_b)
    assert np.array_equal(out[~nan_a], ref[~nan_a])
    codes = np.arange(256, dtype=np.uint8)
    dec = np.empty(256, np.float32)
    lib.fm_host_decode_e4m3(codes.ctypes.data, dec.ctypes.data, 256)
    tdec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(dec, tdec, equal_nan=True)


def test_argument_validation_without_device():
    lib = _lib.load()
    rc = lib.fm_quantize(None, 0, 128, 128, 128, 1, None, 0, None, 0, None, 0, None, 0, None)
    assert rc != 0 and b"null" in lib.fm_last_error_string()
    rc = lib.fm_quantize(C.c_void_p(16), 0, 128, 100, 128, 1, C.c_void_p(16), 128, C.c_void_p(16), 1,
                         None, 0, None, 0, None)
    assert rc != 0 and b"multiple of 128" in lib.fm_last_error_string()
    rc = lib.fm_topk_gating(C.c_void_p(16), 10, 300, 300, 2, 0, 0, None, 0, C.c_void_p(16), C.c_void_p(16), 1,
                            None, None, 1024, None)
    assert rc != 0 and b"E must be" in lib.fm_last_error_string()
    op = _lib.FmGemmOperand()
    rc = lib.fm_grouped_gemm_ragged_m(0, C.byref(op), C.byref(op), 1, C.c_void_p(16), C.c_void_p(16),
                                      1, 128, 128, None, 1, C.c_void_p(16), 0, 128, None)
    assert rc != 0
    assert lib.fm_route_rows_max(16384, 8) == (16384 + 8 * 127) // 128 * 128
    assert lib.fm_route_rows_max(8192, 1) == 8192 and lib.fm_route_rows_max(1000, 1) == 1024
    assert lib.fm_route_rows_max(0, 1) == 128
    # the bound holds for every split of A over E experts (brute force, small sizes)
    import itertools
    for E in (1, 2, 3):
        for counts in itertools.product(range(0, 300, 37), repeat=E):
            need = sum(-(-c // 128) * 128 for c in counts)
            assert lib.fm_route_rows_max(sum(counts), E) >= need, counts
    try:
        _lib.check(1, "probe")
    except RuntimeError as e:
        assert "probe" in str(e)


def test_library_stamp_matches_sources(monkeypatch):
    """The loader refuses a library built from other sources."""
    from nanopysche_amd import build

    assert _lib.load().fm_source_hash().decode() == build.source_hash()
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(build, "source_hash", lambda: "0000000000000000")
    try:
        _lib.load()
        raise AssertionError("a stale library was accepted")
    except RuntimeError as e:
        assert "rebuild" in str(e)
