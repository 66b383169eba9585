"""ctypes binding of libpackboost_hip.so (declared in include/packboost_hip.h).

torch is imported before the library is opened so that the library's libamdhip64.so.7
dependency resolves to the HIP runtime torch already loaded (one runtime per process).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("PACKBOOST_HIP_LIB", PKG_DIR / "libpackboost_hip.so"))

PB_OK = 0
PB_ERR_INVALID = -1
PB_ERR_RANGE = -2
PB_ERR_HIP = -3
PB_ERR_UNSUPPORTED = -4
PB_ERR_NOMEM = -5
PB_INACTIVE = 0xFFFF
PB_MAX_DEPTH = 16

EXPORTED_SYMBOLS = (
    "pb_last_error", "pb_version", "pb_device_available",
    "pb_ctx_create", "pb_ctx_destroy", "pb_hist_plane_elems", "pb_max_nodes",
    "pb_era_offsets_dev", "pb_round_begin", "pb_hist_build", "pb_des_score", "pb_decide",
    "pb_partition", "pb_round_end", "pb_grow_round", "pb_profile_enable",
    "pb_profile_read", "pb_frontier_set", "pb_frontier_counts", "pb_predict_pack",
    "pb_predict_forest", "pb_predict_bins", "pb_era_corr", "pb_quantile_edges", "pb_apply_bins",
    "pb_forest_create", "pb_forest_predict", "pb_forest_destroy", "pb_pack_bins4",
    "pb_set_bin_layout", "pb_select_subsets", "pb_rowlist_work_elems", "pb_rowlist_partition",
    "pb_rowlist_gather", "pb_best_thresholds", "pb_pick_sequential", "pb_set_segment_mode", "pb_rowlist_noalloc_max_segments",
    "pb_rowlist_partition_noalloc",
)


class HipBackendError(RuntimeError):
    """Raised for any failing libpackboost_hip call; HIP failures read "HIP error: ..."."""


class PbDims(ctypes.Structure):
    _fields_ = [
        ("num_rows", ctypes.c_int64), ("ld", ctypes.c_int64), ("num_features", ctypes.c_int32),
        ("num_eras", ctypes.c_int32), ("max_bins", ctypes.c_int32), ("max_depth", ctypes.c_int32),
        ("max_feats", ctypes.c_int32), ("min_samples_leaf", ctypes.c_int32),
    ]


class PbSplitParams(ctypes.Structure):
    _fields_ = [
        ("lambda_l2", ctypes.c_double), ("lambda_dro", ctypes.c_double),
        ("direction_weight", ctypes.c_double), ("era_alpha", ctypes.c_double),
        ("min_samples_leaf", ctypes.c_int32), ("k_cuts", ctypes.c_int32),
        ("cut_selection", ctypes.c_int32), ("skip_last_bin", ctypes.c_int32),
    ]


class PbFitBuffers(ctypes.Structure):
    _fields_ = [
        ("bins_dev", ctypes.c_void_p), ("bins4_dev", ctypes.c_void_p),
        ("y_dev", ctypes.c_void_p), ("preds_dev", ctypes.c_void_p),
        ("grad_dev", ctypes.c_void_p), ("nid_dev", ctypes.c_void_p), ("tnode_dev", ctypes.c_void_p),
        ("hist_cnt_dev", ctypes.c_void_p), ("hist_grad_dev", ctypes.c_void_p),
        ("values_dev", ctypes.c_void_p), ("pack_size", ctypes.c_int32),
        ("learning_rate", ctypes.c_float), ("params", PbSplitParams),
    ]


HEADER_DTYPE = np.dtype([("u_active", "<i4", (PB_MAX_DEPTH + 1,)), ("tree_size", "<i4"),
                         ("reserved", "<i4", (6,))])

DECISION_DTYPE = np.dtype([
    ("node_id", "<i4"), ("split", "<i4"), ("feature", "<i4"), ("threshold", "<i4"),
    ("score", "<f4"), ("left_grad", "<f4"), ("left_hess", "<f4"), ("right_grad", "<f4"),
    ("right_hess", "<f4"), ("left_count", "<i4"), ("right_count", "<i4"), ("left_id", "<i4"),
    ("right_id", "<i4"), ("node_grad", "<f4"), ("node_count", "<i4"), ("reserved", "<i4"),
])
CANDIDATE_DTYPE = np.dtype([
    ("score", "<f4"), ("left_total", "<i4"), ("left_grad", "<f4"), ("feature", "<i4"),
    ("threshold", "<i4"), ("valid", "<i4"), ("reserved", "<i4", (2,)),
])
assert DECISION_DTYPE.itemsize == 64 and CANDIDATE_DTYPE.itemsize == 32
assert HEADER_DTYPE.itemsize == 96

_VP = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float

_SIGNATURES = {
    "pb_last_error": (ctypes.c_char_p, []),
    "pb_version": (_I32, []),
    "pb_device_available": (_I32, []),
    "pb_ctx_create": (ctypes.c_int, [ctypes.POINTER(PbDims), _VP, ctypes.POINTER(_VP)]),
    "pb_ctx_destroy": (ctypes.c_int, [_VP]),
    "pb_hist_plane_elems": (_I64, [_VP, _I32]),
    "pb_max_nodes": (_I32, [_VP, _I32]),
    "pb_era_offsets_dev": (_VP, [_VP]),
    "pb_round_begin": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP]),
    "pb_hist_build": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _I32, _I32, _I32, _VP, _VP, _VP]),
    "pb_des_score": (ctypes.c_int, [_VP, _VP, _VP, _VP, _I32, _I32, _I32,
                                    ctypes.POINTER(PbSplitParams), _VP, _VP]),
    "pb_decide": (ctypes.c_int, [_VP, _I32, _I32, ctypes.POINTER(PbSplitParams), _VP, _VP, _VP]),
    "pb_partition": (ctypes.c_int, [_VP, _VP, _I32, _VP, _VP, _VP]),
    "pb_round_end": (ctypes.c_int, [_VP, _VP, _VP, _I32, _F32, _VP, _VP]),
    "pb_grow_round": (ctypes.c_int, [_VP, ctypes.POINTER(PbFitBuffers), _VP, _I32, _VP, _VP, _VP]),
    "pb_profile_enable": (ctypes.c_int, [_VP, _I32]),
    "pb_era_corr": (ctypes.c_int, [_VP, _VP, _VP, _I32, _VP, _VP, _VP]),
    "pb_forest_create": (ctypes.c_int, [_VP] * 7 + [_I32, _I32, _VP]),
    "pb_forest_predict": (ctypes.c_int, [_VP, _VP, _I64, _I64, _I32, _F32, _VP, _VP, _VP]),
    "pb_forest_destroy": (ctypes.c_int, [_VP]),
    "pb_quantile_edges": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _I32, _VP, _I32, _VP]),
    "pb_apply_bins": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _I32, _I32, _I32, _VP, _VP, _I64, _VP]),
    "pb_pack_bins4": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _VP]),
    "pb_set_bin_layout": (ctypes.c_int, [_VP, _I32]),
    "pb_select_subsets": (ctypes.c_int, [_VP, _VP, _I32, _I32, _VP, _VP]),
    "pb_profile_read": (ctypes.c_int, [_VP, _VP, _VP]),
    "pb_frontier_set": (ctypes.c_int, [_VP, _I32, _I32, _VP, _I32, _VP]),
    "pb_frontier_counts": (ctypes.c_int, [_VP, _VP, _VP, _VP]),
    "pb_predict_pack": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                       _I32, _I32, _F32, _VP, _VP, _VP]),
    "pb_predict_forest": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                         _I32, _I32, _F32, _VP, _VP]),
    "pb_predict_bins": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _I32,
                                       _VP, _VP]),
    "pb_rowlist_work_elems": (_I64, [_I32, _I32]),
    "pb_rowlist_partition": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _I64, _VP, _VP, _I32, _I32, _VP,
                                            _VP, _VP, _VP, _I64, _VP, _VP, _VP, _VP]),
    "pb_rowlist_gather": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _I32, _VP, _VP, _I64, _VP, _VP,
                                         _I32, _I32, _I32, _VP, _I64, _VP, _VP, _VP, _VP, _VP]),
    "pb_best_thresholds": (ctypes.c_int, [_VP, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP]),
    "pb_pick_sequential": (ctypes.c_int, [_VP, _I32, _I32, _I32, _VP, _VP, _VP]),
    "pb_set_segment_mode": (ctypes.c_int, [_VP, _I32, _I32]),
    "pb_rowlist_noalloc_max_segments": (ctypes.c_int64, []),
    "pb_rowlist_partition_noalloc": (ctypes.c_int, [_VP, _I64, _I64, _I32, _VP, _I64, _VP, _VP, _I32, _I32,
                                                    _VP, _VP, _VP, _VP, _I64, _VP, _VP, _VP, _VP]),
}

_LIB: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Opens the library once; raises HipBackendError if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise HipBackendError(
            f"{LIB_PATH} is not built: run `python packboost_amd/build.py` "
            "(or __graft_entry__.build()) to compile the gfx950 backend")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def last_error() -> str:
    msg = load().pb_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(rc: int, what: str) -> None:
    if rc != PB_OK:
        raise HipBackendError(f"{what} failed ({rc}): {last_error()}")


def device_available() -> bool:
    try:
        if not torch.cuda.is_available():
            return False
        return bool(load().pb_device_available())
    except (HipBackendError, OSError):
        return False


def ptr(t: "torch.Tensor | None") -> int | None:
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(stream: "torch.cuda.Stream | None" = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)
