"""Data preparation: quantile binning, prebinned detection, era indexing.

Semantics follow the reference's packboost/data.py:
  * detect_prebinned (data.py:31-41): integer dtype, min >= 0, max < max_bins (and <= 127 in
    the reference's int8 storage; up to 254 here, since bins are stored as uint8);
  * quantile_bin (data.py:44-57): interior edges np.quantile(X, linspace(0,1,nb+1)[1:-1],
    method="linear") per column, cast to float32; bin = searchsorted(edges, x, side="left")
    clipped to [0, nb-1];
  * build_era_index (data.py:114-134): per era, ascending row ids.
Bins are returned as uint8 (values identical to the reference's int8 for max_bins <= 128).

quantile_bin_device / apply_bins_device do the same on the HIP device (pb_quantile_edges,
pb_apply_bins) and write the histogram kernel's column-major layout directly; their edges and
bins are bit-identical to the NumPy path.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable, Sequence

import numpy as np

MAX_BINS_LIMIT = 255


@dataclass(slots=True)
class BinningResult:
    bins: np.ndarray            # uint8 [N, F], row-major
    bin_edges: np.ndarray | None  # float32 [max_bins-1, F] or None when prebinned
    prebinned: bool


def ensure_numpy(array) -> np.ndarray:
    try:
        import torch

        if isinstance(array, torch.Tensor):
            return array.detach().cpu().numpy()
    except ImportError:  # pragma: no cover
        pass
    if hasattr(array, "to_numpy"):
        return np.asarray(array.to_numpy())
    return np.asarray(array)


def _check_max_bins(max_bins: int) -> None:
    if not (2 <= int(max_bins) <= MAX_BINS_LIMIT):
        raise ValueError(f"max_bins must be in [2, {MAX_BINS_LIMIT}], got {max_bins}")


def detect_prebinned(X: np.ndarray, max_bins: int) -> bool:
    if not np.issubdtype(X.dtype, np.integer):
        return False
    if X.size == 0:
        return True
    if int(X.min()) < 0:
        return False
    hi = int(X.max())
    return hi < int(max_bins) and hi < MAX_BINS_LIMIT


def _bin_columns(X: np.ndarray, edges: np.ndarray, max_bins: int) -> np.ndarray:
    out = np.empty(X.shape, dtype=np.uint8)
    for j in range(X.shape[1]):
        col = np.searchsorted(edges[:, j], X[:, j], side="left")
        np.clip(col, 0, max_bins - 1, out=col)
        out[:, j] = col.astype(np.uint8)
    return out


def quantile_bin(X: np.ndarray, max_bins: int) -> tuple[np.ndarray, np.ndarray]:
    _check_max_bins(max_bins)
    X = np.asarray(X, dtype=np.float32)
    qs = np.linspace(0.0, 1.0, max_bins + 1, dtype=np.float64)[1:-1]
    edges = np.quantile(X, qs, axis=0, method="linear").astype(np.float32)
    if edges.ndim == 1:
        edges = edges.reshape(-1, X.shape[1])
    return _bin_columns(X, edges, max_bins), edges


def preprocess_features(X, max_bins: int, *, assume_prebinned: bool = False) -> BinningResult:
    _check_max_bins(max_bins)
    X_np = ensure_numpy(X)
    if X_np.ndim != 2:
        raise ValueError("X must be 2-D [rows, features]")
    if assume_prebinned:
        if not detect_prebinned(X_np, max_bins):
            raise ValueError("prebinned=True requires X to contain integer bins within [0, max_bins).")
        return BinningResult(bins=X_np.astype(np.uint8, copy=False), bin_edges=None, prebinned=True)
    if detect_prebinned(X_np, max_bins):
        return BinningResult(bins=X_np.astype(np.uint8, copy=False), bin_edges=None, prebinned=True)
    bins, edges = quantile_bin(X_np, max_bins)
    return BinningResult(bins=bins, bin_edges=edges, prebinned=False)


def apply_bins(X, bin_edges: np.ndarray | None, max_bins: int) -> np.ndarray:
    X_np = ensure_numpy(X)
    if bin_edges is None:
        if not detect_prebinned(X_np, max_bins):
            raise ValueError("Input must already be prebinned when no edges are provided")
        return X_np.astype(np.uint8, copy=False)
    return _bin_columns(np.asarray(X_np, dtype=np.float32), bin_edges, max_bins)


def encode_eras(era, n_rows: int) -> tuple[np.ndarray, np.ndarray]:
    """Era labels -> (codes int32 [N], unique labels). None gives one era (booster.py:396-407)."""
    if era is None:
        return np.zeros(n_rows, dtype=np.int32), np.zeros(1, dtype=np.int16)
    era_np = np.asarray(ensure_numpy(era)).astype(np.int16)
    if era_np.shape[0] != n_rows:
        raise ValueError("era must align with X rows")
    uniq, inv = np.unique(era_np, return_inverse=True)
    return inv.astype(np.int32).reshape(-1), uniq


def build_era_index(era_codes: Iterable[int] | np.ndarray, num_eras: int | None) -> list[np.ndarray]:
    codes = np.asarray(era_codes).astype(np.int64).reshape(-1)
    if num_eras is None:
        num_eras = int(codes.max()) + 1 if codes.size else 1
    order = np.argsort(codes, kind="stable")
    counts = np.bincount(codes, minlength=num_eras)
    splits = np.cumsum(counts)[:-1]
    return [np.ascontiguousarray(p, dtype=np.int64) for p in np.split(order, splits)]


def era_major_order(era_codes: np.ndarray, num_eras: int) -> tuple[np.ndarray | None, np.ndarray]:
    """Stable era-major row permutation and era offsets int32 [E+1].

    Returns (perm, offsets) with perm None when the rows are already era-major. Within an era
    rows keep ascending id order, the order of the reference's era row lists.
    """
    codes = np.asarray(era_codes).reshape(-1)
    counts = np.bincount(codes, minlength=num_eras).astype(np.int64)
    offsets = np.zeros(num_eras + 1, dtype=np.int64)
    np.cumsum(counts, out=offsets[1:])
    if codes.size == 0 or bool(np.all(codes[1:] >= codes[:-1])):
        return None, offsets.astype(np.int32)
    return np.argsort(codes, kind="stable"), offsets.astype(np.int32)


def feature_names_or_default(feature_names: Sequence[str] | None, n_features: int) -> list[str]:
    if feature_names is not None:
        names = list(feature_names)
        if len(names) != n_features:
            raise ValueError("feature_names length must match X columns")
        return names
    return [f"f{i}" for i in range(n_features)]


def _float_matrix_device(X, device):
    import torch

    if isinstance(X, torch.Tensor):
        return X.detach().to(device=device, dtype=torch.float32).contiguous()
    Xn = np.ascontiguousarray(ensure_numpy(X), dtype=np.float32)
    return torch.from_numpy(Xn).to(device)


def _device_bins(X, max_bins: int, device, perm, edges, chunk_features: int):
    import torch

    from .backends import _hip

    lib = _hip.load()
    x = _float_matrix_device(X, device)
    if x.dim() != 2:
        raise ValueError("X must be 2-D [rows, features]")
    N, F = int(x.shape[0]), int(x.shape[1])
    ld = (N + 15) // 16 * 16
    nq = int(max_bins) - 1
    out = torch.zeros((F, ld), dtype=torch.uint8, device=device)
    perm_dev = None
    if perm is not None:
        perm_dev = torch.as_tensor(np.ascontiguousarray(perm, dtype=np.int64)).to(device)
    if edges is None:
        qs = np.linspace(0.0, 1.0, int(max_bins) + 1, dtype=np.float64)[1:-1]
        q_dev = torch.from_numpy(np.ascontiguousarray(qs)).to(device)
        edges_dev = torch.empty((nq, F), dtype=torch.float32, device=device)
    else:
        q_dev = None
        edges_dev = torch.from_numpy(np.ascontiguousarray(edges, dtype=np.float32)).to(device)
        if tuple(edges_dev.shape) != (nq, F):
            raise ValueError(f"bin_edges must be [{nq}, {F}]")
    s = _hip.stream_ptr()
    for f0 in range(0, F, chunk_features):
        f1 = min(F, f0 + chunk_features)
        xt = x[:, f0:f1].t().contiguous()  # [fc, N] column values
        e_ptr = edges_dev.data_ptr() + 4 * f0
        if q_dev is not None:
            srt = torch.sort(xt, dim=1).values  # ascending, NaN last
            _hip.check(lib.pb_quantile_edges(srt.data_ptr(), N, N, f1 - f0, q_dev.data_ptr(), nq,
                                             e_ptr, F, s), "pb_quantile_edges")
            del srt
        _hip.check(lib.pb_apply_bins(xt.data_ptr(), N, N, f1 - f0, e_ptr, nq, F, int(max_bins),
                                     None if perm_dev is None else perm_dev.data_ptr(),
                                     out[f0].data_ptr(), ld, s), "pb_apply_bins")
        del xt
    return out, (edges_dev.cpu().numpy() if edges is None else np.asarray(edges, np.float32))


def quantile_bin_device(X, max_bins: int, device, *, perm: np.ndarray | None = None,
                        chunk_features: int = 256):
    """quantile_bin on the device: (bins uint8 [F, roundup16(N)] on `device` with row r holding
    input row perm[r], edges float32 [max_bins - 1, F] on the host)."""
    _check_max_bins(max_bins)
    return _device_bins(X, max_bins, device, perm, None, chunk_features)


def apply_bins_device(X, bin_edges: np.ndarray, max_bins: int, device, *,
                      perm: np.ndarray | None = None, chunk_features: int = 256):
    """apply_bins on the device with given edges: uint8 [F, roundup16(N)] on `device`."""
    _check_max_bins(max_bins)
    return _device_bins(X, max_bins, device, perm, bin_edges, chunk_features)[0]
