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
    # bins >= max_bins: the reference leaves those rows out of the histogram and sends them
    # right (frontier_cuda.cu:451, frontier_cpu.cpp:278-281, 464-470); here the subset's columns
    # are copied with such bins set to max_bins, one extra plane bin that the scorer skips
    fid_gather, skip = fid, 0
    sel = None
    if K and N:
        # ids out of range are left to the gather kernel's own check (it raises "feature id");
        # index_select would read out of bounds with them
        lo, hi = (int(v) for v in torch.aminmax(fid))
        if 0 <= lo and hi < F:
            sel = b_fm.index_select(0, fid.long())
    if sel is not None and int(sel.max()) >= nb:
        if nb + 1 > 255:
            raise ValueError("bins >= max_bins need max_bins <= 254 on the HIP backend")
        b_fm = torch.clamp(sel, max=nb).contiguous()
        F, ld_in = K, int(b_fm.stride(0))
        fid_gather, skip = torch.arange(K, dtype=torch.int32, device=dev), 1
    del sel
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
                           cut_selection=1 if str(cut_selection) == "mass" else 0, skip_last_bin=skip)
    t0 = time.perf_counter()

    def consume(m0, U, mx, cand, cnt, gp):
        _hip.check(lib.pb_best_thresholds(cand.data_ptr(), U, K, T, out_s[m0].data_ptr(),
                                          out_t[m0].data_ptr(), out_g[m0].data_ptr(),
                                          out_h[m0].data_ptr(), out_c[m0].data_ptr(), _hip.stream_ptr()),
                   "pb_best_thresholds")

    _score_node_chunks(lib, b_fm, F, N, ld_in, fid_gather, fid, K, vals, rows, R, nrs, nes, M, E, nb + skip,
                       T, p, _NODE_CHUNK, consume, "find_best_splits_batched_cuda")
    kernel_ms = (time.perf_counter() - t0) * 1e3
    return {"scores": out_s, "thresholds": out_t, "left_grad": out_g, "left_hess": out_h,
            "left_count": out_c, "kernel_ms": kernel_ms}


def _score_node_chunks(lib, b_fm, F, N, ld_in, fid_gather, fid_score, K, vals, rows, R, nrs, nes, M, E, nb, T,
                       p, chunk, consume, what, times=None):
    """For nodes [m0, m0 + chunk) at a time: pb_rowlist_gather of their listed rows (feature
    columns fid_gather of b_fm), pb_round_begin / pb_hist_build / pb_des_score over them (the
    candidates' feature ids are fid_score), then consume(m0, U, max_nodes, cand, cnt, gp) with
    the candidate records [max_nodes][K][T] and the histogram planes, before the chunk's
    context is released. Chunks whose lists hold no row are skipped. `times` (optional dict)
    accumulates the milliseconds of gather + histogram ("hist_ms") and of the scorer
    ("score_ms"), from HIP events."""
    dev = b_fm.device
    # rows listed per node (the gather places exactly these when the segments are consistent)
    node_rows = (nes[:, E] - nes[:, 0]).to(torch.int64).clamp_min(0).cpu()
    s = _hip.stream_ptr()
    for m0 in range(0, M, chunk):
        m1 = min(M, m0 + chunk)
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
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)] if times is not None else None
        if ev:
            ev[0].record()
        _hip.check(lib.pb_rowlist_gather(b_fm.data_ptr(), N, ld_in, F, fid_gather.data_ptr(), K, vals.data_ptr(),
                                         rows.data_ptr(), R, nrs.data_ptr(), nes.data_ptr(), m0, m1, E,
                                         b.data_ptr(), ld, preds.data_ptr(), nid.data_ptr(),
                                         era_off_dev.data_ptr(), work.data_ptr(), s), "pb_rowlist_gather")
        _check_status(work, what)
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
            if ev:
                ev[1].record()
            _hip.check(lib.pb_des_score(ctx, cnt.data_ptr(), gp.data_ptr(), fid_score.data_ptr(), K, depth,
                                        mx, ctypes.byref(p), cand.data_ptr(), s), "pb_des_score")
            if ev:
                ev[2].record()
            consume(m0, U, mx, cand, cnt, gp)
            if ev:
                torch.cuda.synchronize(dev)
                times["hist_ms"] = times.get("hist_ms", 0.0) + ev[0].elapsed_time(ev[1])
                times["score_ms"] = times.get("score_ms", 0.0) + ev[1].elapsed_time(ev[2])
        finally:
            torch.cuda.synchronize(dev)
            lib.pb_ctx_destroy(ctx)


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


_STATS_ZERO = {"nodes_processed": 0, "nodes_skipped": 0, "rows_total": 0, "feature_blocks": 0,
               "bincount_calls": 0, "hist_ms": 0.0, "scan_ms": 0.0, "score_ms": 0.0, "partition_ms": 0.0,
               "nodes_subtract_ok": 0, "nodes_subtract_fallback": 0, "nodes_rebuild": 0, "block_size": 0}
_HOST_CHUNK = 1 << 15  # nodes per HIP context (frontier depth 15): one chunk for any real frontier


def find_best_splits_batched_host(bins, grad, nodes_era_rows, feature_subset, max_bins, k_cuts, cut_selection,
                                  lambda_l2, lambda_dro, direction_weight, era_alpha, min_samples_leaf):
    """find_best_splits_batched_cpu (frontier_cpu.cpp:111-515) with its host schema, computed on
    the HIP device: bins int8 [N, F] (rows, features), grad float32 [N], nodes_era_rows a list
    (per node) of lists (per era) of row-id arrays, feature_subset int32 [K]. Returns
    (decisions, stats): decisions[i] is None for a node without a valid split (or without rows),
    else a dict of feature, threshold, score, left/right grad and hess, left/right count and
    left_rows / right_rows (per era, int64 row ids in list order); stats the reference's keys
    (booster.py:1094-1110), its timings measured here with HIP events per phase.

    The listed rows of the subset's columns go to the device once per call; gather, histogram,
    scorer, sequential pick and partition are the HIP kernels (pb_rowlist_gather, pb_hist_build,
    pb_des_score, pb_pick_sequential, pb_rowlist_partition). Differences from the reference:
    a node's left/right sums come from exact fixed-point histograms rounded once to float32
    (the reference adds float32 in row order); every node must list the same number of eras;
    bins >= max_bins are skipped in the histogram and sent right, as the reference does, for
    max_bins up to 254; mass K-cuts are taken over the whole call up to 32768 nodes."""
    lib = _hip.load()
    bins_np = np.asarray(bins)
    grad_np = np.asarray(grad, dtype=np.float32)
    if bins_np.ndim != 2:
        raise ValueError("bins must be 2D (rows, features)")
    if grad_np.ndim != 1:
        raise ValueError("grad must be 1D")
    N, F = int(bins_np.shape[0]), int(bins_np.shape[1])
    if grad_np.shape[0] != N:
        raise ValueError("grad length must match bins rows")
    nb = max(1, int(max_bins))
    n_in = len(nodes_era_rows)
    index_map, node_lists, rows_total = [], [], 0
    for idx in range(n_in):
        item = nodes_era_rows[idx]
        if not isinstance(item, list):
            raise ValueError("Each node entry must be a list of era row arrays")
        if len(item) == 0:
            continue
        arrs = []
        for e in item:
            a = np.asarray(e)
            if a.ndim != 1:
                raise ValueError("era row array must be 1D")
            a = a.astype(np.int64, copy=False)
            if a.size and (int(a.min()) < 0 or int(a.max()) >= N):
                raise IndexError("row index out of bounds")
            arrs.append(a)
        cnt = sum(int(a.size) for a in arrs)
        if cnt == 0:
            continue
        rows_total += cnt
        index_map.append(idx)
        node_lists.append(arrs)
    stats = dict(_STATS_ZERO)
    decisions = [None] * n_in
    stats["rows_total"] = rows_total
    stats["nodes_skipped"] = n_in - len(index_map)
    M = len(index_map)
    if M == 0:
        return decisions, stats
    feats = np.asarray(feature_subset)
    if feats.ndim != 1:
        raise ValueError("feature_subset must be 1D")
    feats = feats.astype(np.int32, copy=False)
    K = int(feats.shape[0])
    if K and (int(feats.min()) < 0 or int(feats.max()) >= F):
        raise IndexError("feature index out of range")
    E = len(node_lists[0])
    if any(len(a) != E for a in node_lists):
        raise ValueError("every node must list the same number of eras")
    stats.update(nodes_processed=M, feature_blocks=1 if K else 0, bincount_calls=2 if K else 0,
                 nodes_subtract_ok=M, block_size=K)
    if K == 0:
        return decisions, stats
    if not 2 <= nb <= 255:
        raise ValueError("max_bins must lie in [2, 255]")
    sub = np.ascontiguousarray(bins_np[:, feats]).astype(np.int8, copy=False).view(np.uint8)  # [N, K]
    # bins >= max_bins (int8 bins read unsigned, as the reference's cast does): the reference
    # leaves those rows out of the feature's histogram and sends them right (frontier_cpu.cpp:
    # 278-281, 464-470). They go to one extra plane bin, max_bins, that the scorer skips
    # (pb_split_params.skip_last_bin); the partition's bin <= threshold sends them right.
    skip = 0
    if int(sub.max()) >= nb:
        if nb + 1 > 255:
            raise ValueError("bins >= max_bins need max_bins <= 254 on the HIP backend")
        sub = np.minimum(sub, np.uint8(nb))
        skip = 1
    nbp = nb + skip  # bins of the histogram planes
    dev = torch.device("cuda")
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]  # around the partition
    b_fm = torch.from_numpy(sub).to(dev).t().contiguous()  # [K, N] feature-major
    flat = [a for arrs in node_lists for a in arrs]
    sizes = np.array([a.size for a in flat], dtype=np.int64).reshape(M, E)
    # the CUDA path's list layout: node_row_splits absolute, node_era_splits relative to the node
    nes_np = np.zeros((M, E + 1), dtype=np.int64)
    nes_np[:, 1:] = np.cumsum(sizes, axis=1)
    nrs_np = np.zeros(M + 1, dtype=np.int64)
    nrs_np[1:] = np.cumsum(sizes.sum(axis=1))
    R = int(nrs_np[-1])
    if R >= 2 ** 31:
        raise ValueError("more than 2^31 - 1 listed rows")
    rows = torch.from_numpy(np.concatenate(flat).astype(np.int32)).to(dev)
    nes = torch.from_numpy(nes_np.astype(np.int32)).to(dev)
    nrs = torch.from_numpy(nrs_np.astype(np.int32)).to(dev)
    vals = torch.from_numpy(grad_np).to(dev)[rows.long()]  # per list position, as the gather reads
    fid = torch.from_numpy(feats).to(dev)
    local = torch.arange(K, dtype=torch.int32, device=dev)
    T = k_cuts if 0 < int(k_cuts) < nb - 1 else nb - 1
    p = _hip.PbSplitParams(lambda_l2=float(lambda_l2), lambda_dro=float(lambda_dro),
                           direction_weight=float(direction_weight), era_alpha=max(0.0, float(era_alpha)),
                           min_samples_leaf=int(min_samples_leaf), k_cuts=int(k_cuts),
                           cut_selection=1 if str(cut_selection) == "mass" else 0, skip_last_bin=skip)
    win = torch.zeros(M * _hip.CANDIDATE_DTYPE.itemsize, dtype=torch.uint8, device=dev)  # valid = 0
    tot_g = np.zeros((M, E), dtype=np.float32)
    sc_ms = [0.0]

    def consume(m0, U, mx, cand, cnt, gp):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        band = torch.empty(U * K * T, dtype=torch.int32, device=dev)
        _hip.check(lib.pb_pick_sequential(cand.data_ptr(), U, K, T, band.data_ptr(),
                                          win.data_ptr() + m0 * _hip.CANDIDATE_DTYPE.itemsize,
                                          _hip.stream_ptr()), "pb_pick_sequential")
        e1.record()
        # era totals [E][mx] after the prefix planes (pb_hist_build's layout)
        off = (E * mx * K * (nbp - 1) + 63) // 64 * 64
        tot_g[m0:m0 + U] = gp[off:off + E * mx].view(E, mx)[:, :U].t().cpu().numpy()
        sc_ms[0] += e0.elapsed_time(e1)

    times = {}
    _score_node_chunks(lib, b_fm, K, N, int(b_fm.stride(0)), local, fid, K, vals, rows, R, nrs, nes, M, E, nbp,
                       T, p, _HOST_CHUNK, consume, "find_best_splits_batched", times)
    w = np.frombuffer(win.cpu().numpy().tobytes(), dtype=_hip.CANDIDATE_DTYPE)
    split = w["valid"] != 0
    # partition every node (nodes without a split go all left and are not read)
    f_loc = np.zeros(M, dtype=np.int32)
    t_loc = np.full(M, 255, dtype=np.int32)
    if split.any():
        where = {int(f): i for i, f in enumerate(feats.tolist())}  # first subset slot of a feature id
        f_loc[split] = [where[int(f)] for f in w["feature"][split]]
        t_loc[split] = w["threshold"][split]
    ev[0].record()
    part = partition_frontier_rowlist(b_fm, rows, nrs, nes, torch.from_numpy(f_loc), torch.from_numpy(t_loc))
    ev[1].record()
    torch.cuda.synchronize(dev)
    left = part["left_index"].cpu().numpy().astype(np.int64)
    right = part["right_index"].cpu().numpy().astype(np.int64)
    ls = part["left_splits"].cpu().numpy().astype(np.int64)
    rs = part["right_splits"].cpu().numpy().astype(np.int64)
    for j in range(M):
        if not split[j]:
            continue
        total_count = int(sizes[j].sum())
        total_grad = np.cumsum(tot_g[j], dtype=np.float32)[-1]  # float32 era-order sum, as the reference
        lg = np.float32(w["left_grad"][j])
        lc = int(w["left_total"][j])
        lh = np.float32(lc)
        decisions[index_map[j]] = {
            "feature": int(w["feature"][j]), "threshold": int(w["threshold"][j]), "score": float(w["score"][j]),
            "left_grad": float(lg), "left_hess": float(lh), "right_grad": float(np.float32(total_grad - lg)),
            "right_hess": float(np.float32(np.float32(total_count) - lh)), "left_count": lc,
            "right_count": total_count - lc,
            "left_rows": [left[ls[j, e]:ls[j, e + 1]] for e in range(E)],
            "right_rows": [right[rs[j, e]:rs[j, e + 1]] for e in range(E)],
        }
    stats["hist_ms"] = times.get("hist_ms", 0.0)
    stats["score_ms"] = times.get("score_ms", 0.0) + sc_ms[0]
    stats["partition_ms"] = ev[0].elapsed_time(ev[1])
    return decisions, stats
