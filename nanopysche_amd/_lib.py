"""ctypes binding of libfm_hip.so (declared in include/fm_hip.h).

The library is built in-tree by ``nanopysche_amd.build``.  There is no CPU
fallback anywhere in the package: if the library is missing, or no ROCm
device is present when a kernel is requested, the call raises.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libfm_hip.so"

DTYPE_BF16 = 0
DTYPE_F32 = 1

QUANT_BF16 = 0
QUANT_BLOCK = 1
QUANT_POW2 = 2
QUANT_MX = 3
SCALES_KMAJOR = 0x100   # OR-ed into a quant kind: row scales stored block-major
ROWS_PAIRED = 0x400     # OR-ed into a quant kind: e4m3 rows in the paired-row layout
COLS_PAIRED = 0x800     # OR-ed into a quant kind: the e4m3 transposed payload paired too

GEMM_BF16 = 0
GEMM_FP8_F32 = 1
GEMM_FP8_POW2 = 2
GEMM_FP8_MX = 3
GEMM_A_FAST = 0x100       # OR-ed into a ragged-K kind: a_t's tiles vary fastest (a_t not in cache)
GEMM_W_KMAJOR = 0x200     # OR-ed into a ragged-M FP8 pow2 kind: weights stored [K][N]
GEMM_PAIRED = 0x400       # OR-ed into a ragged-M FP8 pow2 kind: tokens (and [N][K] weights) paired rows
GEMM_W_PAIRED = 0x800     # with GEMM_W_KMAJOR: the [K][N] weights paired too

GATING_SOFTMAX = 0
GATING_SIGMOID = 1
GATING_L2_NORMALIZE = 1   # fm_topk_gating / fm_gating_grad flag


class FmGemmOperand(C.Structure):
    _fields_ = [
        ("data", C.c_void_p),
        ("ld", C.c_int64),
        ("group_stride", C.c_int64),
        ("scale", C.c_void_p),
        ("scale_row_stride", C.c_int64),
        ("scale_kb_stride", C.c_int64),
        ("scale_group_stride", C.c_int64),
        ("scale_row_shift", C.c_int),
        ("data2", C.c_void_p),
        ("split_rows", C.c_int64),
    ]


class FmWeightJob(C.Structure):
    _fields_ = [
        ("w", C.c_void_p), ("w_dtype", C.c_int),
        ("groups", C.c_int64), ("rows", C.c_int64), ("cols", C.c_int64), ("ld_w", C.c_int64),
        ("gs_w", C.c_int64), ("kind", C.c_int),
        ("q", C.c_void_p), ("ld_q", C.c_int64), ("gs_q", C.c_int64), ("q_row_off", C.c_int64),
        ("s", C.c_void_p), ("ld_s", C.c_int64), ("gs_s", C.c_int64),
        ("qt", C.c_void_p), ("ld_qt", C.c_int64), ("gs_qt", C.c_int64), ("qt_col_off", C.c_int64),
        ("st", C.c_void_p), ("ld_st", C.c_int64), ("gs_st", C.c_int64),
    ]


_vp, _i64, _i32 = C.c_void_p, C.c_int64, C.c_int
_OPND = C.POINTER(FmGemmOperand)

# name -> (restype, argtypes); must match include/fm_hip.h
SIGNATURES = {
    "fm_last_error_string": (C.c_char_p, []),
    "fm_version": (C.c_char_p, []),
    "fm_source_hash": (C.c_char_p, []),
    "fm_host_encode_e4m3": (None, [_vp, _vp, _i64]),
    "fm_host_decode_e4m3": (None, [_vp, _vp, _i64]),
    "fm_hbm_probe": (_i32, [_i32, _vp, _vp, _i64, _vp]),
    "fm_convert_check": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _vp]),
    "fm_decode_check": (_i32, [_vp, _i64, _vp, _vp, _vp]),
    "fm_quantize": (_i32, [_vp, _i32, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _i64,
                           _vp, _i64, _vp]),
    "fm_quantize_pair": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _i64,
                                _vp, _i64, _vp, _i64, _vp]),
    "fm_quantize_weight": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i32, _vp, _i64, _i64,
                                  _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64,
                                  _vp]),
    "fm_quantize_weight_batch": (_i32, [C.POINTER(FmWeightJob), _i32, _vp]),
    "fm_dequantize": (_i32, [_vp, _i64, _i64, _i64, _vp, _i32, _i32, _i32, _i64, _i64, _vp, _i32,
                             _i64, _vp]),
    "fm_scaling_aware_transpose": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64,
                                          _vp]),
    "fm_topk_gating": (_i32, [_vp, _i64, _i32, _i64, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _i32, _vp, _vp,
                               _i64, _vp]),
    "fm_aux_loss": (_i32, [_vp, _i64, _vp, _i32, _i64, _vp, C.c_float, _vp, _vp]),
    "fm_router_logits": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i32, _i64, _vp, _vp, _i32, _vp, _i64, _vp]),
    "fm_router_forward_workspace_bytes": (_i64, [_i64, _i32]),
    "fm_router_forward_fused": (_i32, [_i32, _i64, _i32]),
    "fm_router_forward": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i32, _i64, _vp, _vp, _i32, _i32, _i32, _i32,
                                 _vp, _i32, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _vp, C.c_float, _vp, _vp, _i64,
                                 _vp]),
    "fm_expert_counts": (_i32, [_vp, _i32, _i64, _i32, _vp, _vp, _vp, _i64, _vp]),
    "fm_score_bias_update": (_i32, [_vp, _vp, _i32, C.c_float, _vp, _vp]),
    "fm_gating_grad": (_i32, [_vp, _i64, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _vp, C.c_float,
                              _vp, _i64, _vp]),
    "fm_gating_grad_dot": (_i32, [_vp, _i64, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _i64, _vp,
                                  _i64, _vp, _i64, _vp, _vp, _vp, C.c_float, _vp, _i64, _vp]),
    "fm_router_workspace_bytes": (_i64, [_i64, _i64, _i32]),
    "fm_router_backward": (_i32, [_vp, _i64, _vp, _i32, _i64, _i64, _i64, _vp, _i32, _i64, _i32, _vp, _i64, _vp,
                                  _i32, _i64, _vp, _i32, _vp, _i64, _vp]),
    "fm_rmsnorm_quantize": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i32, C.c_float, _vp, _i64, _i32, _vp, _i64,
                                   _vp, _i64, _vp, _vp]),
    "fm_rmsnorm_backward_workspace_bytes": (_i64, [_i64, _i64]),
    "fm_rmsnorm_backward": (_i32, [_vp, _i64, _vp, _i32, _i64, _i64, _i64, _vp, _i32, _vp, _vp, _i64, _vp, _i32,
                                   _vp, _i64, _vp]),
    "fm_route_rows_max": (_i64, [_i64, _i32]),
    "fm_route_workspace_bytes": (_i64, [_i64, _i32]),
    "fm_route_sort": (_i32, [_vp, _i32, _i64, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp,
                             _vp, _i64, _vp]),
    "fm_route_sort_weights": (_i32, [_vp, _i32, _i64, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp,
                                     _vp, _i64, C.POINTER(FmWeightJob), _i32, _vp]),
    "fm_route_sort_noalloc_max_workspace_bytes": (_i64, []),
    "fm_route_sort_noalloc": (_i32, [_vp, _i32, _i64, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp,
                                     _vp]),
    "fm_capacity_workspace_bytes": (_i64, [_i64]),
    "fm_capacity_select": (_i32, [_vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64,
                                  _vp]),
    "fm_gather_rows": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp]),
    "fm_route_tile_masks": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp]),
    "fm_permute": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _vp, _i32, _vp, _i64, _vp, _i64,
                          _vp, _i64, _vp, _i64, _vp, _vp]),
    "fm_unpermute": (_i32, [_vp, _i64, _vp, _vp, _i64, _i32, _i64, _vp, _i32, _i64, _vp, _i64, _vp]),
    "fm_unpermute_router": (_i32, [_vp, _i64, _vp, _vp, _i64, _i32, _i64, _vp, _i32, _i64, _vp, _i64, _vp, _i64,
                                   _vp, _i32, _i64, _i32, _vp]),
    "fm_router_weight_grad": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _i64, _vp, _vp]),
    "fm_swiglu_quantize": (_i32, [_vp, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _i64, _vp,
                                  _i64, _vp, _i64, _vp, _vp]),
    "fm_swiglu_backward": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _vp,
                                  _i64, _vp, _i64, _vp, _i64, _vp, _vp]),
    "fm_swiglu_values": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    "fm_grouped_gemm_ragged_m": (_i32, [_i32, _OPND, _OPND, _i64, _vp, _vp, _i32, _i64, _i64, _vp,
                                        _i32, _vp, _i32, _i64, _vp]),
    "fm_grouped_gemm_ragged_k": (_i32, [_i32, _OPND, _OPND, _vp, _i32, _i64, _i64, _vp, _i32, _vp,
                                        _i64, _vp, _i64, _i64, _i32, _i64, _vp]),
    "fm_grouped_gemm_ragged_m_k": (_i32, [_i32, _OPND, _OPND, _i64, _vp, _i64, _i64, _vp, _i32, _i64,
                                          _OPND, _OPND, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i64,
                                          _vp, _i32, _vp, _i32, _vp]),
    "fm_grouped_gemm_ragged_k_split_workspace_bytes": (_i64, [_i32, _i64, _i64, _i32]),
    "fm_grouped_gemm_ragged_k_split": (_i32, [_i32, _OPND, _OPND, _vp, _i32, _i64, _i64, _vp, _i32, _vp,
                                              _i64, _vp, _i64, _i64, _i32, _i64, _i32, _vp, _i64, _vp]),
}

_lib = None
_lock = threading.Lock()


def load() -> C.CDLL:
    """Load libfm_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m nanopysche_amd.build` "
                    "(there is no CPU fallback)")
            lib = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            from .build import source_hash

            built, now = lib.fm_source_hash().decode(), source_hash()
            if built != now:
                raise RuntimeError(
                    f"{LIB_PATH} was built from other sources (stamp {built}, sources {now}): rebuild it "
                    "with `python -m nanopysche_amd.build`")
            _lib = lib
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = load().fm_last_error_string().decode(errors="replace")
        raise RuntimeError(f"libfm_hip {what} failed (code {rc}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def require_device(t: torch.Tensor, name: str = "tensor") -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{name} must be on a ROCm device: the fp8_flow_moe kernels run only on the GPU "
            "(there is no CPU fallback)")


def stream_of(t: torch.Tensor) -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t) -> C.c_void_p:
    return C.c_void_p(0 if t is None else t.data_ptr())
