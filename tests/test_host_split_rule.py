"""Host rule that picks the K split of a weight-gradient launch
(nanopysche_amd.flow_moe._k_splits): no GPU needed, the CU count is fixed."""

from types import SimpleNamespace

import pytest

from nanopysche_amd import _lib
from nanopysche_amd import flow_moe as fmm


@pytest.fixture(autouse=True)
def _cus_256(monkeypatch):
    monkeypatch.setattr(fmm, "_cus", lambda dev: 256)
    monkeypatch.delenv("FM_RK_SPLITS", raising=False)


def _plan(E, rows):
    return SimpleNamespace(num_experts=E, rows_max=rows)


def test_configs2_shapes_take_no_split():
    # dW1|dW3 (2H = 2816 x D = 2048) and dW2 (H x D) over 8 experts: 704 and 384 tiles >= 256 CUs
    p = _plan(8, 16384 + 8 * 127)
    assert fmm._k_splits(_lib.QUANT_POW2, p, 2816, 2048, None) == 1
    assert fmm._k_splits(_lib.QUANT_POW2, p, 1408, 2048, None) == 1


def test_shared_expert_shapes_split():
    # one group of 8192 rows: 88 and 48 tiles on 256 CUs
    p = _plan(1, 8192 + 127)
    s13 = fmm._k_splits(_lib.QUANT_POW2, p, 2816, 2048, None)
    s2 = fmm._k_splits(_lib.QUANT_POW2, p, 1408, 2048, None)
    assert 2 <= s13 <= 8 and 2 <= s2 <= 8
    assert 88 * s13 <= 2 * 256 and 48 * s2 <= 256 * 2


def test_short_k_and_blockwise_take_no_split(monkeypatch):
    # fewer than 8 K steps per expert: slices would be shorter than 4 steps
    assert fmm._k_splits(_lib.QUANT_POW2, _plan(1, 896), 2816, 2048, None) == 1
    # the fp32-scale kernel has no split form, even when forced
    monkeypatch.setenv("FM_RK_SPLITS", "4")
    assert fmm._k_splits(_lib.QUANT_BLOCK, _plan(1, 8192), 2816, 2048, None) == 1
    assert fmm._k_splits(_lib.QUANT_POW2, _plan(8, 16384), 2816, 2048, None) == 4
    monkeypatch.setenv("FM_RK_SPLITS", "99")
    assert fmm._k_splits(_lib.QUANT_BF16, _plan(8, 16384), 2816, 2048, None) == 16
