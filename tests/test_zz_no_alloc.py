"""fm_route_sort_noalloc (the allocation-free routing sort, whose block
histogram lives in a fixed device array) against fm_route_sort with a caller
workspace: every output bit-exact, on two calls in a row, the second with a
smaller input (the array keeps the first call's contents), called through the
C ABI.  Also: a size beyond the array is rejected before anything runs."""

import numpy as np
import pytest
import torch

from nanopysche_amd import _lib
from tests.helpers import zipf_routing

pytestmark = pytest.mark.gpu


def _outputs(T, K, E, dev):
    A = T * K
    rmax = int(_lib.load().fm_route_rows_max(A, E))
    i32 = dict(dtype=torch.int32, device=dev)
    # filled with a marker so unwritten entries show
    return dict(counts=torch.full((E,), -7, **i32), offsets=torch.full((E + 1,), -7, **i32),
                row_of=torch.full((max(A, 1),), -7, **i32), assign_of_row=torch.full((rmax,), -7, **i32),
                tile_expert=torch.full((rmax // 128,), -7, **i32), use_fp8=torch.full((E,), -7, **i32)), rmax


def _sort(idx, E, threshold, noalloc):
    T, K = idx.shape
    o, rmax = _outputs(T, K, E, idx.device)
    args = (_lib.ptr(idx), int(idx.dtype == torch.int64), T, K, E, threshold, _lib.ptr(o["counts"]),
            _lib.ptr(o["offsets"]), _lib.ptr(o["row_of"]), _lib.ptr(o["assign_of_row"]), rmax,
            _lib.ptr(o["tile_expert"]), _lib.ptr(o["use_fp8"]))
    if noalloc:
        _lib.call("fm_route_sort_noalloc", *args, _lib.stream_of(idx))
    else:
        nbytes = int(_lib.load().fm_route_workspace_bytes(T * K, E))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=idx.device)
        _lib.call("fm_route_sort", *args, _lib.ptr(ws), nbytes, _lib.stream_of(idx))
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in o.items()}


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_noalloc_sort_matches_workspace_sort_twice(dev, dtype):
    # first call: C5-like, 256 experts with skew and zero-token experts;
    # second call: smaller, fewer experts, so the array holds stale entries
    cases = [(9000, 256, 8, 1.2, (0, 5, 17), 64), (3000, 8, 2, 0.5, (3,), 0)]
    for T, E, K, skew, zeros, thr in cases:
        _, idx = zipf_routing(T, E, K, skew, seed=T + E, zero_experts=zeros)
        idx = idx.to(dtype).to(dev)
        ref = _sort(idx, E, thr, noalloc=False)
        got = _sort(idx, E, thr, noalloc=True)
        for name in ref:
            assert np.array_equal(got[name], ref[name]), f"T={T} E={E}: {name} differs"


def test_noalloc_sort_rejects_oversized(dev):
    lib = _lib.load()
    cap = int(lib.fm_route_sort_noalloc_max_workspace_bytes())
    E = 1024
    T = (cap // (4 * E) + 1) * 1024    # one histogram block more than fits
    assert int(lib.fm_route_workspace_bytes(T, E)) > cap
    idx = torch.zeros(1, 1, dtype=torch.int64, device=dev)   # never read: rejected on the host
    o, _ = _outputs(1, 1, E, dev)
    rc = lib.fm_route_sort_noalloc(_lib.ptr(idx), 1, T, 1, E, 0, _lib.ptr(o["counts"]), _lib.ptr(o["offsets"]),
                                   _lib.ptr(o["row_of"]), _lib.ptr(o["assign_of_row"]),
                                   int(lib.fm_route_rows_max(T, E)), _lib.ptr(o["tile_expert"]),
                                   _lib.ptr(o["use_fp8"]), _lib.stream_of(idx))
    assert rc != 0 and b"scratch" in lib.fm_last_error_string()
