"""Row-list entry points of the reference's CUDA backend, served by the HIP kernels.

The reference's CUDA path hands its split finder and partition per-node, per-era row lists
(`rows_index` with `node_row_splits` / `node_era_splits`, frontier_cuda.cu:576-716, 719-851;
callers booster.py:1414-1431, 1485-1492, 2027-2034). This backend grows trees from per-row
node ids over era-major rows instead (pb_hist_build / pb_des_score), so these adapters gather
the listed rows of the requested features into that layout, run the HIP histogram and DES
scorer, and return the reference's schemas:

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


def _segments(node_row_splits: torch.Tensor, node_era_splits: torch.Tensor):
    """Per concatenated row position: its node and era (rows are node-major, era-minor)."""
    counts = (node_era_splits[:, 1:] - node_era_splits[:, :-1]).to(torch.int64)  # [M, E]
    M, E = counts.shape
    seg = torch.repeat_interleave(torch.arange(M * E, device=counts.device), counts.reshape(-1))
    return counts, seg // E, seg % E


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
    counts, node_of, era_of = _segments(node_row_splits.to(dev), node_era_splits.to(dev))
    E = int(counts.shape[1])
    alpha = _era_alpha(era_weights, counts)
    K = int(feature_ids.numel())
    feats_all = feature_ids.to(device=dev, dtype=torch.int64)
    T = k_cuts if 0 < int(k_cuts) < nb - 1 else nb - 1
    out_s = torch.full((M, K), float("-inf"), dtype=torch.float32, device=dev)
    out_t = torch.full((M, K), -1, dtype=torch.int32, device=dev)
    out_g = torch.zeros((M, K), dtype=torch.float32, device=dev)
    out_h = torch.zeros((M, K), dtype=torch.float32, device=dev)
    out_c = torch.zeros((M, K), dtype=torch.int64, device=dev)
    p = _hip.PbSplitParams(lambda_l2=float(lambda_l2), lambda_dro=float(lambda_dro),
                           direction_weight=float(direction_weight), era_alpha=alpha,
                           min_samples_leaf=int(min_samples_leaf), k_cuts=int(k_cuts),
                           cut_selection=1 if str(cut_selection) == "mass" else 0, reserved=0)
    t0 = time.perf_counter()
    pos_all = torch.arange(int(rows_index.numel()), device=dev)
    for m0 in range(0, M, _NODE_CHUNK):
        m1 = min(M, m0 + _NODE_CHUNK)
        sel = (node_of >= m0) & (node_of < m1)
        pos = pos_all[sel]
        # era-major, then node, then list order: the rows of era e are contiguous
        key = era_of[sel] * (m1 - m0) + (node_of[sel] - m0)
        order = torch.sort(key, stable=True).indices
        pos = pos[order]
        node = (node_of[pos] - m0).to(torch.int32)
        R = int(pos.numel())
        if R == 0:
            continue
        era_sizes = torch.bincount(era_of[pos], minlength=E)
        era_off = np.zeros(E + 1, dtype=np.int32)
        era_off[1:] = np.cumsum(era_sizes.cpu().numpy())
        if int(era_sizes.max()) > 65535:
            raise RuntimeError("HIP backend: an era holds more than 65535 rows of the listed nodes")
        ld = (R + 15) // 16 * 16
        rows = rows_index.to(dev, torch.int64)[pos]
        b = torch.zeros((K, ld), dtype=torch.uint8, device=dev)
        b[:, :R] = bins.index_select(0, feats_all).index_select(1, rows).view(torch.uint8) \
            if bins.dtype in (torch.int8, torch.uint8) else \
            bins.index_select(0, feats_all).index_select(1, rows).to(torch.uint8)
        preds = torch.zeros(ld, dtype=torch.float32, device=dev)
        preds[:R] = grad.to(dev, torch.float32)[pos]
        zeros = torch.zeros(ld, dtype=torch.float32, device=dev)
        g = torch.zeros(ld, dtype=torch.float32, device=dev)
        nid = torch.full((ld,), -1, dtype=torch.int16, device=dev)   # 0xFFFF: pad rows
        tnode = torch.zeros(ld, dtype=torch.int16, device=dev)
        U = m1 - m0
        depth = max(0, math.ceil(math.log2(U)))
        dims = _hip.PbDims(num_rows=R, ld=ld, num_features=K, num_eras=E, max_bins=nb,
                           max_depth=depth + 1, max_feats=K, min_samples_leaf=1)
        ctx = ctypes.c_void_p()
        _hip.check(lib.pb_ctx_create(ctypes.byref(dims), era_off.ctypes.data, ctypes.byref(ctx)),
                   "pb_ctx_create")
        try:
            s = _hip.stream_ptr()
            # grad = preds - 0 (exact), max|grad| for the fixed-point scale
            _hip.check(lib.pb_round_begin(ctx, preds.data_ptr(), zeros.data_ptr(), g.data_ptr(),
                                          nid.data_ptr(), tnode.data_ptr(), s), "pb_round_begin")
            nid[:R] = node.to(torch.int16)
            nid[R:] = -1
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
            cand = torch.zeros(mx * K * T * _hip.CANDIDATE_DTYPE.itemsize, dtype=torch.uint8, device=dev)
            fid = feature_ids.to(dev, torch.int32).contiguous()
            _hip.check(lib.pb_des_score(ctx, cnt.data_ptr(), gp.data_ptr(), fid.data_ptr(), K, depth,
                                        mx, ctypes.byref(p), cand.data_ptr(), s), "pb_des_score")
            rec = cand.view(torch.int32).reshape(mx, K, T, 8)[:U]
        finally:
            torch.cuda.synchronize(dev)
            lib.pb_ctx_destroy(ctx)
        score = rec[..., 0].view(torch.float32)
        lt = rec[..., 1].to(torch.int64)
        lg = rec[..., 2].view(torch.float32)
        thr = rec[..., 4]
        valid = rec[..., 5] != 0
        # per (node, feature): the CUDA path's tie-break over thresholds
        s_ok = torch.where(valid, score, torch.full_like(score, float("-inf")))
        best = s_ok.max(dim=2, keepdim=True).values
        elig = valid & (s_ok >= best - 1e-12)
        lt_e = torch.where(elig, lt, torch.full_like(lt, -1))
        lt_best = lt_e.max(dim=2, keepdim=True).values
        elig = elig & (lt == lt_best)
        thr_e = torch.where(elig, thr, torch.full_like(thr, -1))
        pick = thr_e.argmax(dim=2, keepdim=True)
        has = elig.any(dim=2)
        out_s[m0:m1] = torch.where(has, s_ok.gather(2, pick)[..., 0], out_s[m0:m1])
        out_t[m0:m1] = torch.where(has, thr.gather(2, pick)[..., 0], out_t[m0:m1])
        out_g[m0:m1] = torch.where(has, lg.gather(2, pick)[..., 0], out_g[m0:m1])
        cnt_pick = lt.gather(2, pick)[..., 0]
        out_c[m0:m1] = torch.where(has, cnt_pick, out_c[m0:m1])
        out_h[m0:m1] = torch.where(has, cnt_pick.to(torch.float32), out_h[m0:m1])
    kernel_ms = (time.perf_counter() - t0) * 1e3
    return {"scores": out_s, "thresholds": out_t, "left_grad": out_g, "left_hess": out_h,
            "left_count": out_c, "kernel_ms": kernel_ms}


def partition_frontier_rowlist(bins, rows_index, node_row_splits, node_era_splits, feat_per_node,
                               thr_per_node):
    dev = bins.device
    S = int(node_row_splits.numel()) - 1
    if S <= 0:
        z = torch.empty(0, dtype=torch.int32, device=dev)
        return {"left_index": z, "right_index": z.clone(),
                "left_splits": torch.empty((0, 0), dtype=torch.int32, device=dev),
                "right_splits": torch.empty((0, 0), dtype=torch.int32, device=dev)}
    counts, node, era = _segments(node_row_splits.to(dev), node_era_splits.to(dev))
    E = int(counts.shape[1])
    rows = rows_index.to(dev, torch.int64)
    f = feat_per_node.to(dev, torch.int64)[node]
    t = thr_per_node.to(dev, torch.int32)[node]
    bv = bins.view(torch.uint8) if bins.dtype == torch.int8 else bins
    go_left = bv[f, rows].to(torch.int32) <= t   # left iff bin <= threshold
    left_index = rows_index.to(dev, torch.int32)[go_left]
    right_index = rows_index.to(dev, torch.int32)[~go_left]
    seg = node * E + era
    lc = torch.zeros(S * E, dtype=torch.int64, device=dev).index_add_(0, seg, go_left.to(torch.int64))
    lc = lc.reshape(S, E)
    rc = counts - lc
    zero = torch.zeros((S, 1), dtype=torch.int64, device=dev)

    def absolute(c):
        local = torch.cat([zero, c.cumsum(1)], 1)
        base = torch.cat([zero[:1, 0], c.sum(1).cumsum(0)[:-1]])
        return (local + base[:, None]).to(torch.int32)

    return {"left_index": left_index, "right_index": right_index,
            "left_splits": absolute(lc), "right_splits": absolute(rc)}
