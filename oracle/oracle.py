"""ORACLE — test infrastructure only (never imported by packboost_amd).

Python side of the CPU restatement of the reference's native-CPU training path:
  * split_batch(): ctypes wrapper of frontier_ref.c:oracle_split_batch, the restated
    find_best_splits_batched_cpu (frontier_cpu.cpp:111-515);
  * fit(): the PackBoost.fit round/depth loop on device="cpu" with the native split finder
    (booster.py:375-599, 1012-1293): per-era row lists, shard dedup, RNG draws only while a
    depth has active nodes, TreeBuilder numbering, leaf values in Python double, pack_sum via
    float32 adds in tree order, preds += float32(lr) * pack_sum;
  * predict(): booster.py:709-712 with Tree.predict_bins (booster.py:131-169).
Float32 sums the reference takes with torch (root and no-split leaf values,
booster.py:499-513, 531-542) are taken with the same torch CPU routine here.
"""

from __future__ import annotations

import ctypes
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_DIR = HERE / "_ref"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = load_library(LIB_PATH)
    return _lib


def build_mutant(n: int, out_dir: Path) -> Path:
    """Compiles the restatement with planted mistake `n` (frontier_ref.c, ORACLE_MUTANT)."""
    out = Path(out_dir) / f"liboracle_mutant{n}.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-fopenmp", "-std=c11", f"-DORACLE_MUTANT={n}",
                    "-shared", "-o", str(out), str(HERE / "frontier_ref.c"), "-lm"], check=True)
    return out


class use_library:
    """Context manager: route every oracle call through another build of frontier_ref.c."""

    def __init__(self, path: Path) -> None:
        self.path = path

    def __enter__(self):
        global _lib
        self.saved = _lib
        _lib = load_library(self.path)
        return _lib

    def __exit__(self, *exc) -> None:
        global _lib
        _lib = self.saved


def load_library(path: Path) -> ctypes.CDLL:
    L = ctypes.CDLL(str(path))
    P = ctypes.c_void_p
    L.oracle_split_batch.restype = ctypes.c_int
    L.oracle_split_batch.argtypes = (
        [P, ctypes.c_int64, ctypes.c_int64, P, ctypes.c_int32, ctypes.c_int32, P, P, P,
         ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_float,
         ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_int32] + [P] * 17)
    L.oracle_score_planes.restype = ctypes.c_int
    L.oracle_score_planes.argtypes = (
        [P, P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, P, P,
         ctypes.c_int32, ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float,
         ctypes.c_int32] + [P] * 9)
    L.oracle_even_cuts.restype = ctypes.c_int
    L.oracle_even_cuts.argtypes = [ctypes.c_int, ctypes.c_int, P]
    L.oracle_mass_cuts.restype = ctypes.c_int
    L.oracle_mass_cuts.argtypes = [P, ctypes.c_int, ctypes.c_int, P]
    L.oracle_num_threads.restype = ctypes.c_int
    return L


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def f32(x) -> float:
    """float32 rounding of a Python number (pybind's double -> float cast)."""
    return float(np.float32(x))


@dataclass
class SplitResult:
    feature: np.ndarray
    threshold: np.ndarray
    score: np.ndarray
    left_grad: np.ndarray
    left_hess: np.ndarray
    right_grad: np.ndarray
    right_hess: np.ndarray
    left_count: np.ndarray
    right_count: np.ndarray
    go_left: np.ndarray
    planes: tuple[np.ndarray, np.ndarray] | None
    cands: tuple | None
    timings: np.ndarray


def split_batch(bins: np.ndarray, grad: np.ndarray, nodes_era_rows: list[list[np.ndarray]],
                feats: np.ndarray, max_bins: int, k_cuts: int = 0, cut_selection: str = "mass",
                lambda_l2: float = 1e-6, lambda_dro: float = 0.0, direction_weight: float = 0.0,
                era_alpha: float = 0.0, min_samples_leaf: int = 20, want_planes: bool = False,
                want_cands: bool = False) -> SplitResult:
    """Restated find_best_splits_batched_cpu on per-node, per-era row lists."""
    bins = np.ascontiguousarray(bins, dtype=np.uint8)
    grad = np.ascontiguousarray(grad, dtype=np.float32)
    feats = np.ascontiguousarray(feats, dtype=np.int32)
    M = len(nodes_era_rows)
    E = len(nodes_era_rows[0]) if M else 1
    rows_parts, splits = [], np.zeros((M, E + 1), dtype=np.int64)
    pos = 0
    for m, eras in enumerate(nodes_era_rows):
        splits[m, 0] = pos
        for e, r in enumerate(eras):
            r = np.asarray(r, dtype=np.int64).reshape(-1)
            rows_parts.append(r)
            pos += r.shape[0]
            splits[m, e + 1] = pos
    rows = np.concatenate(rows_parts) if rows_parts else np.zeros(0, np.int64)
    n = max(M, 1)
    out = {k: np.zeros(n, dt) for k, dt in [
        ("feature", np.int32), ("threshold", np.int32), ("score", np.float32),
        ("left_grad", np.float32), ("left_hess", np.float32), ("right_grad", np.float32),
        ("right_hess", np.float32), ("left_count", np.int64), ("right_count", np.int64)]}
    go_left = np.zeros(max(rows.shape[0], 1), dtype=np.uint8)
    K = feats.shape[0]
    full = max(1, max_bins - 1)
    T = k_cuts if (0 < k_cuts < full) else full
    planes = None
    if want_planes:
        planes = (np.zeros((E, M, K, max_bins), np.int32), np.zeros((E, M, K, max_bins), np.float32))
    cands = None
    if want_cands:
        cands = (np.zeros((M, K, T), np.float32), np.zeros((M, K, T), np.int64),
                 np.zeros((M, K, T), np.float32), np.zeros((M, K, T), np.uint8))
    tim = np.zeros(4, dtype=np.float64)
    rc = lib().oracle_split_batch(
        _p(bins), bins.shape[0], bins.shape[1], _p(grad), M, E, _p(rows), _p(splits), _p(feats), K,
        int(max_bins), int(k_cuts), 1 if cut_selection == "mass" else 0, f32(lambda_l2),
        f32(lambda_dro), f32(direction_weight), f32(era_alpha), int(min_samples_leaf),
        _p(out["feature"]), _p(out["threshold"]), _p(out["score"]), _p(out["left_grad"]),
        _p(out["left_hess"]), _p(out["right_grad"]), _p(out["right_hess"]), _p(out["left_count"]),
        _p(out["right_count"]), _p(go_left), _p(planes[0]) if planes else None,
        _p(planes[1]) if planes else None, *(_p(c) for c in cands) if cands else (None,) * 4,
        _p(tim))
    if rc == -2:
        raise IndexError("row or feature index out of range")
    if rc != 0:
        raise RuntimeError(f"oracle_split_batch failed: {rc}")
    return SplitResult(**{k: v[:M] for k, v in out.items()}, go_left=go_left[: rows.shape[0]],
                       planes=planes, cands=cands, timings=tim)


def score_planes(plane_cnt: np.ndarray, plane_g: np.ndarray, feats: np.ndarray,
                 thr_tab: np.ndarray | None, *, lambda_l2: float, lambda_dro: float,
                 direction_weight: float, era_alpha: float, min_samples_leaf: int):
    """Restated scorer (frontier_cpu.cpp:342-444) on planes [E][M][K][nb]."""
    plane_cnt = np.ascontiguousarray(plane_cnt, dtype=np.int32)
    plane_g = np.ascontiguousarray(plane_g, dtype=np.float32)
    E, M, K, nb = plane_cnt.shape
    feats = np.ascontiguousarray(feats, dtype=np.int32)
    T = thr_tab.shape[1] if thr_tab is not None else max(1, nb - 1)
    tt = None if thr_tab is None else np.ascontiguousarray(thr_tab, dtype=np.int32)
    cs, cl, cg, cv = (np.zeros((M, K, T), np.float32), np.zeros((M, K, T), np.int64),
                      np.zeros((M, K, T), np.float32), np.zeros((M, K, T), np.uint8))
    bf, bt, bs = np.zeros(M, np.int32), np.zeros(M, np.int32), np.zeros(M, np.float32)
    bl, blg = np.zeros(M, np.int64), np.zeros(M, np.float32)
    rc = lib().oracle_score_planes(
        _p(plane_cnt), _p(plane_g), E, M, K, nb, _p(feats), _p(tt), T, f32(lambda_l2),
        f32(lambda_dro), f32(direction_weight), f32(era_alpha), int(min_samples_leaf), _p(cs),
        _p(cl), _p(cg), _p(cv), _p(bf), _p(bt), _p(bs), _p(bl), _p(blg))
    if rc != 0:
        raise RuntimeError(f"oracle_score_planes failed: {rc}")
    return {"score": cs, "left_total": cl, "left_grad": cg, "valid": cv,
            "best_feature": bf, "best_threshold": bt, "best_score": bs, "best_left": bl,
            "best_left_grad": blg}


def even_cuts(max_bins: int, k: int) -> np.ndarray:
    out = np.zeros(512, np.int32)
    n = lib().oracle_even_cuts(max_bins, k, _p(out))
    return out[:n].copy()


def mass_cuts(counts: np.ndarray, max_bins: int, k: int) -> np.ndarray:
    c = np.ascontiguousarray(counts, dtype=np.int64)
    out = np.zeros(512, np.int32)
    n = lib().oracle_mass_cuts(_p(c), max_bins, k, _p(out))
    return out[:n].copy()


# ------------------------------------------------------------ the compiled reference frontier
_ref_mod = None


def ref_module():
    """The reference's own find_best_splits_batched_cpu (frontier_cpu.cpp + bindings.cpp,
    compiled by `make -C oracle ref` into oracle/_ref), or None when it is not built."""
    global _ref_mod
    if _ref_mod is None:
        import glob
        import importlib.util

        hits = glob.glob(str(REF_DIR / "_backend*.so"))
        if not hits:
            return None
        spec = importlib.util.spec_from_file_location("_backend", hits[0])
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _ref_mod = mod
    return _ref_mod


def ref_split_batch(bins: np.ndarray, grad: np.ndarray, nodes_era_rows: list[list[np.ndarray]],
                    feats: np.ndarray, max_bins: int, k_cuts: int = 0, cut_selection: str = "mass",
                    lambda_l2: float = 1e-6, lambda_dro: float = 0.0, direction_weight: float = 0.0,
                    era_alpha: float = 0.0, min_samples_leaf: int = 20) -> SplitResult:
    """split_batch through the compiled reference frontier (frontier_cpu.cpp:111-515) instead of
    the restatement; its decisions and left/right row lists are mapped onto SplitResult."""
    mod = ref_module()
    if mod is None:
        raise RuntimeError("oracle/_ref is not built (`make -C oracle ref`)")
    M = len(nodes_era_rows)
    decs, stats = mod.find_best_splits_batched_cpu(
        np.ascontiguousarray(bins, dtype=np.uint8).view(np.int8), np.ascontiguousarray(grad, np.float32),
        nodes_era_rows, np.ascontiguousarray(feats, np.int32), int(max_bins), int(k_cuts), cut_selection,
        float(lambda_l2), float(lambda_dro), float(direction_weight), float(era_alpha),
        int(min_samples_leaf))
    n = max(M, 1)
    out = {k: np.zeros(n, dt) for k, dt in [
        ("feature", np.int32), ("threshold", np.int32), ("score", np.float32),
        ("left_grad", np.float32), ("left_hess", np.float32), ("right_grad", np.float32),
        ("right_hess", np.float32), ("left_count", np.int64), ("right_count", np.int64)]}
    # go_left per entry of the node-major, era-major row lists: the rows are distinct, so a
    # mask over all rows marks the reference's left lists
    left = np.zeros(bins.shape[0], dtype=np.uint8)
    for m, eras in enumerate(nodes_era_rows):
        d = decs[m]
        if d is None:
            out["feature"][m] = -1
            continue
        for key in out:
            out[key][m] = d[key]
        lr = [np.asarray(x, dtype=np.int64) for x in d["left_rows"] if len(x)]
        if lr:
            left[np.concatenate(lr)] = 1
    rows = [np.asarray(r, dtype=np.int64) for eras in nodes_era_rows for r in eras]
    go_left = left[np.concatenate(rows)] if rows else np.zeros(0, np.uint8)
    tim = np.array([stats.get("hist_ms", 0.0), stats.get("scan_ms", 0.0), stats.get("score_ms", 0.0),
                    stats.get("partition_ms", 0.0)], dtype=np.float64)
    return SplitResult(**{k: v[:M] for k, v in out.items()}, go_left=go_left, planes=None,
                       cands=None, timings=tim)


# ----------------------------------------------------------------------------- fit loop
@dataclass
class FitResult:
    rounds: list[dict[str, np.ndarray]]   # one tree per round (all B trees are identical)
    preds: np.ndarray                     # float32 training predictions after the last round
    depth_logs: list[dict]
    split_ms: float                       # time inside oracle_split_batch
    round_seconds: list[float]


def _torch_sum_f32(grad_t: torch.Tensor, rows: np.ndarray) -> float:
    if rows.size == 0:
        return 0.0
    return float(grad_t[torch.from_numpy(rows)].sum().item())


def fit(bins: np.ndarray, y: np.ndarray, era_codes: np.ndarray | None, *, num_rounds: int,
        pack_size: int = 8, max_depth: int = 6, learning_rate: float = 0.1,
        lambda_l2: float = 1e-6, lambda_dro: float = 0.0, direction_weight: float = 0.0,
        min_samples_leaf: int = 20, max_bins: int = 63, k_cuts: int = 0,
        cut_selection: str = "mass", layer_feature_fraction: float = 1.0, era_alpha: float = 0.0,
        random_state: int | None = None, rng: torch.Generator | None = None,
        stop_after_depths: int | None = None, trace: list | None = None,
        splitter: str = "restated", init_preds: np.ndarray | None = None) -> FitResult:
    """PackBoost.fit on the native CPU path, restated (booster.py:375-599). splitter
    "reference" runs each depth's split finder on the compiled reference frontier
    (ref_split_batch) instead of the C restatement. init_preds (float32 [N]) continues a fit
    from those training predictions (with `rng` left where the earlier rounds took it, a fit
    split into calls grows the same trees as one call)."""
    split_fn = ref_split_batch if splitter == "reference" else split_batch
    import time

    bins = np.ascontiguousarray(bins, dtype=np.uint8)
    y = np.asarray(y, dtype=np.float32)
    N, F = bins.shape
    if era_codes is None:
        era_codes = np.zeros(N, dtype=np.int64)
    codes = np.asarray(era_codes).astype(np.int64)
    E = int(codes.max()) + 1 if N else 1
    base_era_rows = [np.nonzero(codes == e)[0].astype(np.int64) for e in range(E)]
    if rng is None:
        rng = torch.Generator(device="cpu")
        if random_state is not None:
            rng.manual_seed(int(random_state))
    k = min(F, max(1, int(round(float(layer_feature_fraction) * F))))
    msl = int(min_samples_leaf)
    preds = np.zeros(N, dtype=np.float32) if init_preds is None else \
        np.array(init_preds, dtype=np.float32, copy=True)
    rounds, logs, rsec = [], [], []
    split_ms = 0.0
    lr32 = np.float32(learning_rate)
    for _ in range(num_rounds):
        t0 = time.perf_counter()
        grad = (preds - y).astype(np.float32)
        grad_t = torch.from_numpy(grad)
        # one tree per pack: every tree starts from the same shards and shares each depth's
        # feature subset; the reference's dedup hands all of them the same decisions.
        nodes = [dict(feature=-1, threshold=0, left=-1, right=-1, value=0.0, is_leaf=True)]
        root_rows = np.concatenate([r for r in base_era_rows if r.size] or [np.zeros(0, np.int64)])
        leaf_rows = {0: root_rows}
        if root_rows.size:
            g = _torch_sum_f32(grad_t, root_rows)
            h = float(np.float32(root_rows.size))
            nodes[0]["value"] = -g / (h + lambda_l2)
        frontier = [(0, list(base_era_rows))]
        for depth in range(max_depth):
            if stop_after_depths is not None and depth >= stop_after_depths:
                break
            active = [(nid, er) for nid, er in frontier if sum(r.size for r in er) >= 2 * msl]
            if not active:
                break
            feat_subset = torch.randperm(F, generator=rng)[:k].numpy().astype(np.int32)
            res = split_fn(bins, grad, [er for _, er in active], feat_subset, max_bins, k_cuts,
                           cut_selection, lambda_l2, lambda_dro, direction_weight, era_alpha, msl)
            split_ms += float(res.timings.sum())
            if trace is not None:
                trace.append({"round": len(rounds), "depth": depth, "node_ids": [n for n, _ in active],
                              "feats": feat_subset, "nodes_era_rows": [er for _, er in active],
                              "grad": grad, "result": res})
            nxt = []
            pos = 0
            for m, (nid, er) in enumerate(active):
                lens = [r.size for r in er]
                gl = res.go_left[pos: pos + sum(lens)].astype(bool)
                pos += sum(lens)
                if res.feature[m] < 0:
                    rows_all = np.concatenate([r for r in er if r.size] or [np.zeros(0, np.int64)])
                    val = 0.0
                    if rows_all.size:
                        g = _torch_sum_f32(grad_t, rows_all)
                        h = float(np.float32(rows_all.size))
                        val = -g / (h + lambda_l2)
                    nodes[nid].update(value=val, is_leaf=True, feature=-1, threshold=0, left=-1, right=-1)
                    leaf_rows.setdefault(nid, rows_all)
                    continue
                li, ri = len(nodes), len(nodes) + 1
                nodes[nid].update(feature=int(res.feature[m]), threshold=int(res.threshold[m]),
                                  is_leaf=False, left=li, right=ri)
                lv = -float(res.left_grad[m]) / (float(res.left_hess[m]) + lambda_l2)
                rv = -float(res.right_grad[m]) / (float(res.right_hess[m]) + lambda_l2)
                nodes.append(dict(feature=-1, threshold=0, left=-1, right=-1, value=lv, is_leaf=True))
                nodes.append(dict(feature=-1, threshold=0, left=-1, right=-1, value=rv, is_leaf=True))
                lrows, rrows = [], []
                off = 0
                for r in er:
                    sel = gl[off: off + r.size]
                    off += r.size
                    lrows.append(r[sel])
                    rrows.append(r[~sel])
                leaf_rows.pop(nid, None)
                leaf_rows[li] = np.concatenate(lrows) if lrows else np.zeros(0, np.int64)
                leaf_rows[ri] = np.concatenate(rrows) if rrows else np.zeros(0, np.int64)
                nxt.append((li, lrows))
                nxt.append((ri, rrows))
            logs.append({"depth": depth, "nodes_processed": len(active),
                         "nodes_collapsed": (pack_size - 1) * len(active),
                         "rows_total": int(sum(r.size for _, er in active for r in er))})
            frontier = nxt
        arrs = {key: np.array([n[key] for n in nodes]) for key in
                ("feature", "threshold", "left", "right", "value", "is_leaf")}
        leaf_val = np.zeros(N, dtype=np.float32)
        for nid, rows in leaf_rows.items():
            if rows.size:
                leaf_val[rows] = np.float32(nodes[nid]["value"])
        preds = pack_update(preds, leaf_val, pack_size, lr32)
        rounds.append(arrs)
        rsec.append(time.perf_counter() - t0)
    return FitResult(rounds=rounds, preds=preds, depth_logs=logs, split_ms=split_ms, round_seconds=rsec)


def pack_update(preds: np.ndarray, leaf_val: np.ndarray, pack_size: int, lr32) -> np.ndarray:
    """End of round (booster.py:581-599): pack_sum = B float32 adds of the row's leaf value (the
    pack's identical trees, in tree order), then preds += float32(lr) * pack_sum."""
    pack_sum = np.zeros(leaf_val.shape[0], dtype=np.float32)
    for _t in range(pack_size):
        pack_sum = (pack_sum + leaf_val).astype(np.float32)
    return (preds + (np.float32(lr32) * pack_sum).astype(np.float32)).astype(np.float32)


def replay_preds(rounds: list[dict[str, np.ndarray]], bins: np.ndarray, pack_size: int,
                 learning_rate: float, rows: np.ndarray | None = None) -> np.ndarray:
    """The training predictions fit() leaves after `rounds`, recomputed from the trees alone: each
    row's leaf by the partition rule bin <= threshold -> left (leaf_index), then pack_update. With
    `rows`, only those rows (bins may then hold just them, in that order)."""
    sub = bins if rows is None else bins[rows]
    preds = np.zeros(sub.shape[0], dtype=np.float32)
    lr32 = np.float32(learning_rate)
    for arrs in rounds:
        leaf_val = np.asarray(arrs["value"]).astype(np.float32)[leaf_index(arrs, sub)]
        preds = pack_update(preds, leaf_val, pack_size, lr32)
    return preds


def predict_tree(arrs: dict[str, np.ndarray], bins: np.ndarray) -> np.ndarray:
    """Tree.predict_bins on CPU (booster.py:131-169): float32 leaf value per row."""
    N = bins.shape[0]
    node = np.zeros(N, dtype=np.int64)
    out = np.zeros(N, dtype=np.float32)
    active = np.arange(N)
    feat, thr = arrs["feature"], arrs["threshold"]
    left, right = arrs["left"], arrs["right"]
    val = arrs["value"].astype(np.float32)
    leaf = arrs["is_leaf"].astype(bool)
    while active.size:
        nd = node[active]
        lm = leaf[nd]
        if lm.any():
            out[active[lm]] = val[nd[lm]]
            active, nd = active[~lm], nd[~lm]
            if not active.size:
                break
        go_left = bins[active, feat[nd]] <= thr[nd]
        node[active] = np.where(go_left, left[nd], right[nd])
    return out


def leaf_index(arrs: dict[str, np.ndarray], bins: np.ndarray) -> np.ndarray:
    N = bins.shape[0]
    node = np.zeros(N, dtype=np.int64)
    leaf = arrs["is_leaf"].astype(bool)
    for _ in range(len(leaf)):
        act = ~leaf[node]
        if not act.any():
            break
        idx = np.nonzero(act)[0]
        nd = node[idx]
        go_left = bins[idx, arrs["feature"][nd]] <= arrs["threshold"][nd]
        node[idx] = np.where(go_left, arrs["left"][nd], arrs["right"][nd])
    return node


def predict(rounds: list[dict[str, np.ndarray]], pack_size: int, tree_weight: float,
            bins: np.ndarray) -> np.ndarray:
    """pred += float32(w) * tree.predict_bins(bins), tree by tree (booster.py:709-712)."""
    w = np.float32(tree_weight)
    pred = np.zeros(bins.shape[0], dtype=np.float32)
    for arrs in rounds:
        v = predict_tree(arrs, bins)
        for _ in range(pack_size):
            pred = (pred + (w * v).astype(np.float32)).astype(np.float32)
    return pred
