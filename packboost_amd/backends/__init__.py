"""Backend shim with the reference's names (packboost/backends/__init__.py:9-163).

The reference resolves these names on its pybind11 module; here they are served by
libpackboost_hip.so through ctypes, and every one of them computes on the HIP device.
`find_best_splits_batched` keeps the host schema of the reference's CPU splitter (numpy
inputs, per-node per-era row lists, decision dicts with left/right row lists;
frontier_cpu.cpp:111-515), so `cpu_available()` reports whether that entry point is served,
i.e. whether a gfx950 device and the library are present. The "cuda" names keep their spelling
for drop-in callers.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _hip

__all__ = [
    "cpu_available",
    "find_best_splits_batched",
    "cuda_available",
    "find_best_splits_batched_cuda",
    "partition_frontier_cuda",
    "predict_bins_cuda",
    "predict_pack_cuda",
]


def cpu_available() -> bool:
    """True when the host-schema split finder can run: a gfx950 device and the library."""
    return _hip.device_available()


def find_best_splits_batched(*args: Any, **kwargs: Any):
    """find_best_splits_batched_cpu's schema on the HIP device (frontier_cpu.cpp:111-515; caller
    booster.py:1080-1093): (decisions, stats)."""
    if not _hip.device_available():
        raise RuntimeError("CPU backend is unavailable in this build.")
    from .rowlist import find_best_splits_batched_host

    return find_best_splits_batched_host(*args, **kwargs)


def cuda_available() -> bool:
    """True when a gfx950 device is visible and libpackboost_hip.so loads."""
    return _hip.device_available()


def _u8_fm(bins: torch.Tensor) -> torch.Tensor:
    """Feature-major [F, N] int8/uint8 -> contiguous uint8 [F, ld] with ld % 16 == 0."""
    if bins.dim() != 2:
        raise ValueError("bins must be 2-D feature-major [F, N]")
    F, N = bins.shape
    ld = (int(N) + 15) // 16 * 16
    if bins.dtype == torch.uint8 and ld == N and bins.is_contiguous():
        return bins
    out = torch.zeros((int(F), ld), dtype=torch.uint8, device=bins.device)
    out[:, :N] = bins.view(torch.uint8) if bins.dtype == torch.int8 else bins.to(torch.uint8)
    return out


def predict_bins_cuda(bins_fm: torch.Tensor, feature: torch.Tensor, threshold: torch.Tensor,
                      left: torch.Tensor, right: torch.Tensor, value: torch.Tensor,
                      is_leaf: torch.Tensor) -> torch.Tensor:
    """One tree over feature-major bins (frontier_cuda.cu:853-920): float32 [N] leaf values."""
    lib = _hip.load()
    F, N = bins_fm.shape
    b = _u8_fm(bins_fm)
    dev = b.device
    cast = lambda t, dt: t.to(device=dev, dtype=dt).contiguous()  # noqa: E731
    f, t, l, r = (cast(x, torch.int32) for x in (feature, threshold, left, right))
    v, lf = cast(value, torch.float32), cast(is_leaf, torch.uint8)
    out = torch.empty(int(N), dtype=torch.float32, device=dev)
    _hip.check(lib.pb_predict_bins(b.data_ptr(), int(N), b.shape[1], int(F), f.data_ptr(),
                                   t.data_ptr(), l.data_ptr(), r.data_ptr(), v.data_ptr(),
                                   lf.data_ptr(), int(f.numel()), out.data_ptr(),
                                   _hip.stream_ptr()), "pb_predict_bins")
    return out


def predict_pack_cuda(bins_fm: torch.Tensor, feature: torch.Tensor, threshold: torch.Tensor,
                      left_abs: torch.Tensor, right_abs: torch.Tensor, value: torch.Tensor,
                      is_leaf: torch.Tensor, offsets: torch.Tensor, tree_weight: float) -> torch.Tensor:
    """tree_weight * sum of leaf values over one packed forest (frontier_cuda.cu:989-1068)."""
    lib = _hip.load()
    F, N = bins_fm.shape
    if int(N) == 0:
        return torch.empty(0, dtype=torch.float32, device=bins_fm.device)
    b = _u8_fm(bins_fm)
    dev = b.device
    cast = lambda t, dt: t.to(device=dev, dtype=dt).contiguous()  # noqa: E731
    f, t, l, r, o = (cast(x, torch.int32) for x in (feature, threshold, left_abs, right_abs, offsets))
    v, lf = cast(value, torch.float32), cast(is_leaf, torch.uint8)
    out = torch.empty(int(N), dtype=torch.float32, device=dev)
    _hip.check(lib.pb_predict_pack(b.data_ptr(), int(N), b.shape[1], int(F), f.data_ptr(),
                                   t.data_ptr(), l.data_ptr(), r.data_ptr(), v.data_ptr(),
                                   lf.data_ptr(), o.data_ptr(), int(o.numel() - 1), int(f.numel()),
                                   float(tree_weight), out.data_ptr(), None, _hip.stream_ptr()),
               "pb_predict_pack")
    return out


def find_best_splits_batched_cuda(*args: Any, **kwargs: Any):
    """Row-list split finder of the reference's CUDA path (frontier_cuda.cu:576-716).

    This backend grows trees from per-row node ids (engine.DeviceFit / pb_hist_build +
    pb_des_score); the row-list entry point is provided by packboost_amd.backends.rowlist.
    """
    from .rowlist import find_best_splits_batched_rowlist

    return find_best_splits_batched_rowlist(*args, **kwargs)


def partition_frontier_cuda(*args: Any, **kwargs: Any):
    """Row-list partition of the reference's CUDA path (frontier_cuda.cu:719-851)."""
    from .rowlist import partition_frontier_rowlist

    return partition_frontier_rowlist(*args, **kwargs)
