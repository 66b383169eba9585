"""Row-list entry points of the reference's CUDA backend, served by the HIP kernels.

The reference's CUDA path hands its split finder and partition per-node, per-era row lists
(`rows_index` with `node_row_splits` / `node_era_splits`, frontier_cuda.cu:576-716, 719-851;
callers booster.py:1414-1431, 1485-1492, 2027-2034). This backend grows trees from per-row
node ids over era-major rows instead (pb_hist_build / pb_des_score). The adapters orchestrate
HIP entry points only (torch allocates the buffers): pb_rowlist_gather moves the listed rows of
the requested features into that layout, pb_hist_build / pb_des_score score them,
pb_best_thresholds picks per (node, feature), and pb_rowlist_partition splits the lists. They
return the reference's schemas:

  find_best_splits_batched_rowlist -> {scores f32 [M,K] (-inf: no valid threshold),
      thresholds i32 [M,K] (-1), left_grad f32, left_hess f32, left_count i64 [M,K], kernel_ms}
  partition_frontier_rowlist -> {left_index, right_index i32, left_splits, right_splits
      i32 [S,E+1] (absolute offsets into the flat outputs)}

Scores follow the reference's CPU split finder (frontier_cpu.cpp:342-444), which the HIP
scorer reproduces bit-for-bit; the per-(node, feature) choice uses the CUDA path's
tie-break (frontier_cuda.cu:537-560: score within 1e-12, then larger left count, then larger
threshold). Squared loss only: `hess` must be all ones, and `era_weights` must be the
reference's weights for some era_alpha (1 per non-empty era, or count + alpha).
"""

from __future__ import annotations

import ctypes
import math
import time

import numpy as np
import torch

from . import _hip

_NODE_CHUNK = 4096  # nodes per HIP context (frontier depth 12)


def _era_alpha(era_weights: torch.Tensor, counts: torch.Tensor) -> float:
    w = era_weights.detach().to("cpu", torch.float64)
    c = counts.detach().to("cpu", torch.float64)
    has = c > 0
    if bool((w[~has] != 0).any()):
        raise RuntimeError("era_weights must be 0 for eras without rows")
    if not bool(has.any()) or bool((w[has] == 1.0).all()):
        return 0.0
    alpha = (w[has] - c[has]).unique()
    if alpha.numel() != 1 or float(alpha[0]) <= 0.0:
        raise RuntimeError("era_weights are not count + era_alpha for one era_alpha > 0")
    return float(alpha[0])


_STATUS = ("a (node, era) segment lies outside rows_index", "a row id lies outside [0, N)",
           "a feature id lies outside [0, F)", "an output would pass its capacity")


def _check_status(work: torch.Tensor, what: str) -> None:
    st = work[:4].cpu().tolist()
    bad = [msg for flag, msg in zip(st, _STATUS) if flag]
    if bad:
        raise RuntimeError(f"{what}: " + "; ".join(bad))


def _bins_fm(bins: torch.Tensor):
    """Feature-major uint8 bins [F][N] (the reference's int8 [F][N]) and their row stride."""
    if bins.dim() != 2:
        raise ValueError("bins must be a 2-D feature-major [F, N] tensor")
    b = bins.view(torch.uint8) if bins.dtype == torch.int8 else bins
    if b.dtype != torch.uint8:
        raise TypeError("bins must be int8 or uint8")
    if b.stride(1) != 1:
        b = b.contiguous()
    return b, int(b.shape[0]), int(b.shape[1]), int(b.stride(0))


def _i32(t: torch.Tensor, dev) -> torch.Tensor:
    return t.to(device=dev, dtype=torch.int32).contiguous()


def find_best_splits_batched_rowlist(bins, grad, hess, rows_index, node_row_splits, node_era_splits,
                                     era_weights, total_grad, total_hess, total_count, feature_ids,
                                     max_bins, k_cuts, cut_selection, lambda_l2, lambda_dro,
                                     direction_weight, min_samples_leaf, rows_total_compact=None):
    lib = _hip.load()
    M = int(node_row_splits.numel()) - 1
    if M <= 0:
        return {"scores": None, "thresholds": None, "left_grad": None, "left_hess": None,
                "left_count": None, "kernel_ms": 0.0}
    dev = bins.device
    nb = int(max_bins)
    if not 2 <= nb <= 255:
        raise ValueError("max_bins must lie in [2, 255]")
    if bool((hess.to(torch.float32) != 1.0).any()):
        raise RuntimeError("HIP backend supports squared loss only (hess == 1)")
    b_fm, F, N, ld_in = _bins_fm(bins)
    rows = _i32(rows_index, dev)
    nrs = _i32(node_row_splits, dev)
    nes = _i32(node_era_splits, dev)
    E = int(nes.shape[1]) - 1
    if E < 1:
        raise ValueError("node_era_splits must have at least 2 columns")
    counts = nes[:, 1:] - nes[:, :-1]  # [M, E]
    alpha = _era_alpha(era_weights, counts)
    K = int(feature_ids.numel())
    fid = _i32(feature_ids, dev)
    vals = grad.to(device=dev, dtype=torch.float32).contiguous()
    R = int(rows.numel())
    T = k_cuts if 0 < int(k_cuts) < nb - 1 else nb - 1
    out_s = torch.full((M, K), float("-inf"), dtype=torch.float32, device=dev)
    out_t = torch.full((M, K), -1, dtype=torch.int32, device=dev)
    out_g = torch.zeros((M, K), dtype=torch.float32, device=dev)
    out_h = torch.zeros((M, K), dtype=torch.float32, device=dev)
    out_c = torch.zeros((M, K), dtype=torch.int64, device=dev)
    if K == 0:
        return {"scores": out_s, "thresholds": out_t, "left_grad": out_g, "left_hess": out_h,
                "left_count": out_c, "kernel_ms": 0.0}
    p = _hip.PbSplitParams(lambda_l2=float(lambda_l2), lambda_dro=float(lambda_dro),
                           direction_weight=float(direction_weight), era_alpha=alpha,
                           min_samples_leaf=int(min_samples_leaf), k_cuts=int(k_cuts),
                           cut_selection=1 if str(cut_selection) == "mass" else 0, reserved=0)
    # rows listed per node (the gather places exactly these when the segments are consistent)
    node_rows = (nes[:, E] - nes[:, 0]).to(torch.int64).clamp_min(0).cpu()
    s = _hip.stream_ptr()
    t0 = time.perf_counter()
    for m0 in range(0, M, _NODE_CHUNK):
        m1 = min(M, m0 + _NODE_CHUNK)
        U = m1 - m0
        cap = int(node_rows[m0:m1].sum())
        if cap == 0:
            continue
        ld = (cap + 15) // 16 * 16
        b = torch.zeros((K, ld), dtype=torch.uint8, device=dev)
        preds = torch.zeros(ld, dtype=torch.float32, device=dev)
        nid = torch.full((ld,), -1, dtype=torch.int16, device=dev)  # 0xFFFF: rows in no node
        era_off_dev = torch.empty(E + 1, dtype=torch.int32, device=dev)
        work = torch.empty(int(lib.pb_rowlist_work_elems(U, E)), dtype=torch.int32, device=dev)
        _hip.check(lib.pb_rowlist_gather(b_fm.data_ptr(), N, ld_in, F, fid.data_ptr(), K, vals.data_ptr(),
                                         rows.data_ptr(), R, nrs.data_ptr(), nes.data_ptr(), m0, m1, E,
                                         b.data_ptr(), ld, preds.data_ptr(), nid.data_ptr(),
                                         era_off_dev.data_ptr(), work.data_ptr(), s), "pb_rowlist_gather")
        _check_status(work, "find_best_splits_batched_cuda")
        era_off = np.ascontiguousarray(era_off_dev.cpu().numpy())
        Rc = int(era_off[E])
        if Rc == 0:
            continue
        zeros = torch.zeros(ld, dtype=torch.float32, device=dev)
        g = torch.empty(ld, dtype=torch.float32, device=dev)
        nid_root = torch.empty(ld, dtype=torch.int16, device=dev)  # pb_round_begin's root ids, unused
        tnode = torch.empty(ld, dtype=torch.int16, device=dev)
        depth = max(0, math.ceil(math.log2(U)))
        dims = _hip.PbDims(num_rows=Rc, ld=ld, num_features=K, num_eras=E, max_bins=nb,
                           max_depth=depth + 1, max_feats=K, min_samples_leaf=0)
        ctx = ctypes.c_void_p()
        _hip.check(lib.pb_ctx_create(ctypes.byref(dims), era_off.ctypes.data, ctypes.byref(ctx)),
                   "pb_ctx_create")
        try:
            # grad = values - 0 (exact) and max|grad| for the histogram's fixed-point scale
            _hip.check(lib.pb_round_begin(ctx, preds.data_ptr(), zeros.data_ptr(), g.data_ptr(),
                                          nid_root.data_ptr(), tnode.data_ptr(), s), "pb_round_begin")
            _hip.check(lib.pb_frontier_set(ctx, depth, U, None, U, s), "pb_frontier_set")
            mx = int(lib.pb_max_nodes(ctx, depth))
            if mx < U:
                raise RuntimeError("HIP backend: too many nodes for the listed rows")
            plane = int(lib.pb_hist_plane_elems(ctx, mx))
            cnt = torch.empty(plane, dtype=torch.int32, device=dev)
            gp = torch.empty(plane, dtype=torch.float32, device=dev)
            local = torch.arange(K, dtype=torch.int32, device=dev)
            _hip.check(lib.pb_hist_build(ctx, b.data_ptr(), g.data_ptr(), nid.data_ptr(),
                                         local.data_ptr(), K, depth, mx, cnt.data_ptr(), gp.data_ptr(),
                                         s), "pb_hist_build")
            cand = torch.empty(mx * K * T * _hip.CANDIDATE_DTYPE.itemsize, dtype=torch.uint8, device=dev)
            _hip.check(lib.pb_des_score(ctx, cnt.data_ptr(), gp.data_ptr(), fid.data_ptr(), K, depth,
                                        mx, ctypes.byref(p), cand.data_ptr(), s), "pb_des_score")
            _hip.check(lib.pb_best_thresholds(cand.data_ptr(), U, K, T, out_s[m0].data_ptr(),
                                              out_t[m0].data_ptr(), out_g[m0].data_ptr(),
                                              out_h[m0].data_ptr(), out_c[m0].data_ptr(), s),
                       "pb_best_thresholds")
        finally:
            torch.cuda.synchronize(dev)
            lib.pb_ctx_destroy(ctx)
    kernel_ms = (time.perf_counter() - t0) * 1e3
    return {"scores": out_s, "thresholds": out_t, "left_grad": out_g, "left_hess": out_h,
            "left_count": out_c, "kernel_ms": kernel_ms}


def partition_frontier_rowlist(bins, rows_index, node_row_splits, node_era_splits, feat_per_node,
                               thr_per_node):
    lib = _hip.load()
    dev = bins.device
    S = int(node_row_splits.numel()) - 1
    if S <= 0:
        z = torch.empty(0, dtype=torch.int32, device=dev)
        return {"left_index": z, "right_index": z.clone(),
                "left_splits": torch.empty((0, 0), dtype=torch.int32, device=dev),
                "right_splits": torch.empty((0, 0), dtype=torch.int32, device=dev)}
    b_fm, F, N, ld_in = _bins_fm(bins)
    rows = _i32(rows_index, dev)
    nrs = _i32(node_row_splits, dev)
    nes = _i32(node_era_splits, dev)
    E = int(nes.shape[1]) - 1
    R = int(rows.numel())
    feat = _i32(feat_per_node, dev)
    thr = _i32(thr_per_node, dev)
    if feat.numel() < S or thr.numel() < S:
        raise ValueError("feat_per_node and thr_per_node need one entry per node")
    left = torch.empty(R, dtype=torch.int32, device=dev)
    right = torch.empty(R, dtype=torch.int32, device=dev)
    ls = torch.empty((S, E + 1), dtype=torch.int32, device=dev)
    rs = torch.empty((S, E + 1), dtype=torch.int32, device=dev)
    work = torch.empty(int(lib.pb_rowlist_work_elems(S, E)), dtype=torch.int32, device=dev)
    _hip.check(lib.pb_rowlist_partition(b_fm.data_ptr(), N, ld_in, F, rows.data_ptr(), R, nrs.data_ptr(),
                                        nes.data_ptr(), S, E, feat.data_ptr(), thr.data_ptr(),
                                        left.data_ptr(), right.data_ptr(), R, ls.data_ptr(), rs.data_ptr(),
                                        work.data_ptr(), _hip.stream_ptr()), "pb_rowlist_partition")
    _check_status(work, "partition_frontier_cuda")
    nl, nr = int(ls[-1, -1]), int(rs[-1, -1])
    return {"left_index": left[:nl], "right_index": right[:nr], "left_splits": ls, "right_splits": rs}
