"""Tile producers over a capped grid (the walk of row tiles taken when a tile
list is given and the tiles outnumber about 32,768 workgroups).

Each case runs a producer twice on the same inputs: with the tile list, whose
grid is capped so that workgroups take several valid tiles each (and skip the
empty ones among their candidates), and with no list, one workgroup per tile
over every tile.  The tiles the list marks valid must hold identical bytes
(payload and scales, row and transposed outputs, row-major layouts:
the walk does not depend on the paired layouts): both runs compute each
tile with the same code, so any difference is a tile the walk missed,
computed twice over another's LDS, or placed at the wrong row.  The list
has gaps (the tiles of odd experts are dropped, as the split by
``fp8_gemm_threshold`` drops one precision's experts), and a sample of rows
is checked against the oracle's quantisers as well.  Reference:
fp8/__init__.py:15-20 (fused_permute_pad, fused_swiglu_quantize), the
routing sort of model/moe.py:1542-1556."""

import numpy as np
import pytest
import torch

import nanopysche_amd as fm
from nanopysche_amd import _lib
from nanopysche_amd.flow_moe import _alloc_quant, _tile_args
from oracle import fp8 as ofp8
from oracle import routing as orouting

pytestmark = pytest.mark.gpu

KINDS = {"pow2": _lib.QUANT_POW2, "mx": _lib.QUANT_MX}


def _np(t):
    return t.detach().cpu().numpy()


def _plan(T, E, K, dev, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    plan = fm.route_tokens(idx.to(dev), E)
    te = plan.tile_expert
    tiles = torch.where(te % 2 == 1, torch.full_like(te, -1), te).contiguous()
    return idx, plan, tiles


def _valid_rows(tiles):
    return torch.repeat_interleave(tiles >= 0, 128)


def _compare(a_bufs, b_bufs, rows_ok, mx):
    """Row outputs [rows, *] and scales, transposed outputs [*, rows] and
    their scales [rows / block, *], on the valid tiles' rows (on the device)."""
    q, s, qt, st = a_bufs
    rq, rs, rqt, rst = b_bufs
    assert torch.equal(q[rows_ok], rq[rows_ok])
    assert torch.equal(s[rows_ok], rs[rows_ok])
    assert torch.equal(qt[:, rows_ok], rqt[:, rows_ok])
    sb = rows_ok[::32 if mx else 128]
    assert torch.equal(st[sb], rst[sb])


@pytest.mark.parametrize("kind", ["pow2", "mx"])
def test_permute_walk_matches_one_tile_per_workgroup(dev, kind):
    """D = 16384 (128 column tiles: the grid is capped at 256 row tiles);
    T = 40000 tokens, top-2 of 4 experts: 629 row tiles, half of them valid,
    so workgroups of the capped grid take up to two tiles of their three
    candidates."""
    T, E, K, D = 40000, 4, 2, 16384
    idx, plan, tiles = _plan(T, E, K, dev, seed=31)
    R = plan.rows_max
    assert R // 128 > 32768 // (D // 128)   # the walk is taken
    g = torch.Generator(device=dev).manual_seed(32)
    x = torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16)
    qk = KINDS[kind]
    st = _lib.stream_of(x)
    outs = []
    for tl in (tiles, None):
        bufs = _alloc_quant(R, D, qk, True, True, dev, True)
        for b in bufs:
            b.zero_()
        _lib.call("fm_permute", _lib.ptr(x), T, D, x.stride(0), _lib.ptr(plan.assign_of_row), R, K, None,
                  *_tile_args(qk, *bufs), _lib.ptr(tl), st)
        outs.append(bufs)
    torch.cuda.synchronize()
    rows_ok = _valid_rows(tiles)
    assert int(rows_ok.sum()) > 128 * 256   # more valid tiles than grid rows
    _compare(outs[0], outs[1], rows_ok, kind == "mx")

    # a sample of valid rows against the oracle (unpaired layout)
    bufs = _alloc_quant(R, D, qk, True, False, dev, False)
    _lib.call("fm_permute", _lib.ptr(x), T, D, x.stride(0), _lib.ptr(plan.assign_of_row), R, K, None,
              *_tile_args(qk, *bufs), _lib.ptr(tiles), st)
    torch.cuda.synchronize()
    ref = orouting.sort_assignments(idx.numpy(), E)
    aor = np.full(R, -1, np.int64)
    aor[:ref["assign_of_row"].size] = ref["assign_of_row"]
    sample = np.flatnonzero(_np(rows_ok) & (aor >= 0))
    sample = sample[np.linspace(0, sample.size - 1, 64).astype(int)]
    xs = x[torch.from_numpy(aor[sample] // K).to(dev)].float().cpu().numpy()
    if kind == "mx":
        rq, rs = ofp8.quant_mx_1x32(xs)
    else:
        rq, rs = ofp8.quant_1x128(xs, pow2=True)
    assert np.array_equal(_np(bufs[0])[sample], rq)
    assert np.array_equal(_np(bufs[1])[sample], rs)


@pytest.mark.parametrize("kind", ["pow2", "mx"])
def test_swiglu_backward_walk_matches_one_tile_per_workgroup(dev, kind):
    """Two outputs (dg | du), each with its LDS code tile (pow2: the codes of
    the scaling-aware transpose; MX: the column-scaled codes), H = 16384 (the
    grid is capped at 256 row tiles), 629 row tiles, half of them valid."""
    T, E, K, H = 40000, 4, 2, 16384
    _, plan, tiles = _plan(T, E, K, dev, seed=41)
    R = plan.rows_max
    g = torch.Generator(device=dev).manual_seed(42)
    GU = torch.randn(R, 2 * H, generator=g, device=dev).to(torch.bfloat16)
    dH = (torch.randn(R, H, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    qk = KINDS[kind]
    st = _lib.stream_of(GU)
    outs = []
    for tl in (tiles, None):
        bufs = _alloc_quant(R, 2 * H, qk, True, True, dev, True)
        for b in bufs:
            b.zero_()
        _lib.call("fm_swiglu_backward", _lib.ptr(GU), GU.stride(0), _lib.ptr(GU[:, H:]), GU.stride(0),
                  _lib.ptr(dH), dH.stride(0), R, H, *_tile_args(qk, *bufs), _lib.ptr(tl), st)
        outs.append(bufs)
    torch.cuda.synchronize()
    rows_ok = _valid_rows(tiles)
    assert int(rows_ok.sum()) > 128 * 256
    _compare(outs[0], outs[1], rows_ok, kind == "mx")
