"""PackBoost: pack-parallel gradient boosting with Directional Era Splitting on MI355X.

Public surface and model format follow the reference's packboost/booster.py:
  * TreeNode / Tree / TreeBuilder (booster.py:25-190) — same fields and child numbering;
  * PackBoost(config).fit(X, y, era, *, num_rounds, feature_names, eval_sets, round_callback),
    .predict(X), .predict_packwise(X, block_size_trees), .trees, .round_metrics,
    ._depth_logs, ._tree_weight, ._binner (booster.py:289-726).
The split finder, partition, pack aggregation and prediction run as HIP kernels on the
device (engine.DeviceFit); there is no CPU compute path.
"""

from __future__ import annotations

import json
import logging
import os
import warnings
from dataclasses import dataclass, field
from time import perf_counter
from typing import Callable, Iterable, List, Sequence, Tuple

import numpy as np
import torch

from . import backends as native_backends
from .backends import _hip
from .config import PackBoostConfig
from .data import (BinningResult, apply_bins, apply_bins_device, detect_prebinned, encode_eras,
                   era_major_order, feature_names_or_default, preprocess_features,
                   quantile_bin_device)
from .engine import (DeviceFit, column_major_bins, depth_log_from_round, padded_rows,
                     subset_size, tree_arrays_from_log)


# ------------------------------------------------------------------ tree structures
@dataclass(slots=True)
class TreeNode:
    feature: int = -1
    threshold: int = 0
    left: int = -1
    right: int = -1
    value: float = 0.0
    is_leaf: bool = True


@dataclass(slots=True)
class Tree:
    nodes: List[TreeNode]
    _compiled: dict = field(init=False, repr=False, default_factory=dict)

    def _ensure_compiled(self, device: torch.device) -> dict[str, torch.Tensor]:
        key = str(device)
        c = self._compiled.get(key)
        if c is None:
            c = {
                "feature": torch.tensor([n.feature for n in self.nodes], dtype=torch.int32, device=device),
                "threshold": torch.tensor([n.threshold for n in self.nodes], dtype=torch.int32, device=device),
                "left": torch.tensor([n.left for n in self.nodes], dtype=torch.int32, device=device),
                "right": torch.tensor([n.right for n in self.nodes], dtype=torch.int32, device=device),
                "value": torch.tensor([n.value for n in self.nodes], dtype=torch.float32, device=device),
                "is_leaf": torch.tensor([n.is_leaf for n in self.nodes], dtype=torch.bool, device=device),
            }
            self._compiled[key] = c
        return c

    def predict_bins(self, bins: torch.Tensor) -> torch.Tensor:
        """Leaf value per row of integer bins [N, F] (left iff bin <= threshold), on the GPU."""
        N = int(bins.shape[0])
        device = _device_of(bins)
        if N == 0:
            return torch.empty(0, dtype=torch.float32, device=bins.device)
        bins_fm = _to_column_major(bins, device)
        c = self._ensure_compiled(device)
        out = torch.empty(N, dtype=torch.float32, device=device)
        lib = _hip.load()
        _hip.check(lib.pb_predict_bins(
            bins_fm.data_ptr(), N, bins_fm.shape[1], bins_fm.shape[0], c["feature"].data_ptr(),
            c["threshold"].data_ptr(), c["left"].data_ptr(), c["right"].data_ptr(),
            c["value"].data_ptr(), c["is_leaf"].to(torch.uint8).data_ptr(), len(self.nodes),
            out.data_ptr(), _hip.stream_ptr()), "pb_predict_bins")
        return out.to(bins.device)


class TreeBuilder:
    """Grows one tree in breadth-first id order (booster.py:172-190): node 0 is the root and a
    split appends the two children at the end of the node list, so the ids a depth creates are
    consecutive and follow the order in which its nodes split."""

    def __init__(self) -> None:
        self.nodes: List[TreeNode] = [TreeNode()]

    def set_leaf(self, node_id: int, value: float) -> None:
        """Turns node_id into a leaf holding `value` (clearing any split it held)."""
        self.nodes[node_id] = TreeNode(value=float(value))

    def split(self, node_id: int, feature: int, threshold: int) -> Tuple[int, int]:
        """Splits node_id on (feature, threshold); returns the ids of its new children."""
        first_child = len(self.nodes)
        node = self.nodes[node_id]
        node.is_leaf = False
        node.feature, node.threshold = int(feature), int(threshold)
        node.left, node.right = first_child, first_child + 1
        self.nodes.extend((TreeNode(), TreeNode()))
        return node.left, node.right

    def build(self) -> Tree:
        return Tree(nodes=self.nodes)


def _tree_from_arrays(a: dict[str, np.ndarray]) -> Tree:
    nodes = [TreeNode(int(f), int(t), int(l), int(r), float(v), bool(lf))
             for f, t, l, r, v, lf in zip(a["feature"], a["threshold"], a["left"], a["right"],
                                          a["value"], a["is_leaf"])]
    return Tree(nodes=nodes)


def _device_of(x) -> torch.device:
    if isinstance(x, torch.Tensor) and x.is_cuda:
        return x.device
    return torch.device("cuda", torch.cuda.current_device())


def _to_column_major(bins, device: torch.device) -> torch.Tensor:
    """Row-major integer bins [N, F] (numpy or torch) -> contiguous uint8 [F, ld] on device."""
    if isinstance(bins, torch.Tensor):
        t = bins
    else:
        t = torch.from_numpy(np.ascontiguousarray(bins))
    if t.dtype not in (torch.uint8, torch.int8):
        t = t.to(torch.uint8)
    N, F = t.shape
    ld = padded_rows(int(N))
    out = torch.zeros((int(F), ld), dtype=torch.uint8, device=device)
    out[:, :N] = t.to(device).view(torch.uint8).t()
    return out


def _is_float_input(X) -> bool:
    if isinstance(X, torch.Tensor):
        return X.dtype.is_floating_point
    arr = X.to_numpy() if hasattr(X, "to_numpy") else X
    return not np.issubdtype(np.asarray(arr).dtype, np.integer)


def _bins_fm_for(X, bin_edges, max_bins: int, device: torch.device,
                 perm: np.ndarray | None = None) -> tuple[torch.Tensor, int]:
    """Column-major uint8 bins [F, ld] on the device for prediction / evaluation: float inputs
    are binned on the device with the model's edges (apply_bins_device); integer inputs are
    taken as bins (apply_bins' prebinned rule)."""
    if bin_edges is not None and _is_float_input(X):
        out = apply_bins_device(X, bin_edges, max_bins, device, perm=perm)
        return out, int(X.shape[0])
    if isinstance(X, torch.Tensor):
        if X.dtype.is_floating_point:
            raise ValueError("float inputs need the model's bin edges (the model was trained on bins)")
        bins = X if perm is None else X[torch.as_tensor(perm, device=X.device)]
    else:
        bins = apply_bins(X, bin_edges, max_bins)
        if perm is not None:
            bins = bins[perm]
    return _to_column_major(bins, device), int(bins.shape[0])


def _require_backend(device: torch.device) -> None:
    if device.type != "cuda":
        raise RuntimeError(
            "packboost_amd runs on the MI355X HIP backend only; use PackBoostConfig(device='cuda')")
    if not torch.cuda.is_available():
        raise RuntimeError("HIP error: no GPU device is visible to torch")
    _hip.load()


# ------------------------------------------------------------------ booster
class PackBoost:
    """Pack-parallel gradient booster with DES scoring (squared loss)."""

    NONFINITE_POLICIES = ("raise", "truncate")

    def __init__(self, config: PackBoostConfig, *, nonfinite: str | None = None) -> None:
        """nonfinite: what fit does at the first round whose gradients (preds - y) are not all
        finite (y holding NaN/inf, or predictions that overflowed). "raise" (the default, or
        PACKBOOST_NONFINITE) raises FloatingPointError; "truncate" warns (RuntimeWarning) and
        ends the fit with the rounds before it, whose trees and training predictions stand.
        The reference has no such check: its float sums carry NaN into the scores
        (frontier_cpu.cpp:363-432), a candidate whose era sums hold a NaN never wins, and the
        failed-split leaf is -NaN/(h + lambda) (booster.py:532-542), so from that round on its
        trees hold NaN values and its predictions turn NaN. The fixed-point histograms here
        have no NaN to carry, so neither policy reproduces that; both stop before it."""
        self.config = config
        policy = (nonfinite or os.getenv("PACKBOOST_NONFINITE") or "raise").lower()
        if policy not in self.NONFINITE_POLICIES:
            raise ValueError(f"nonfinite must be one of {self.NONFINITE_POLICIES}, got {policy!r}")
        self.nonfinite = policy
        self._device = torch.device(config.device)
        self._rng = torch.Generator(device="cpu")
        if config.random_state is not None:
            self._rng.manual_seed(int(config.random_state))
        mode = (os.getenv("PACKBOOST_HIST_MODE") or config.histogram_mode).lower()
        if mode not in {"rebuild", "subtract", "auto"}:
            raise ValueError(f"Unsupported histogram_mode: {mode}")
        if config.cut_selection not in ("even", "mass"):
            raise ValueError(f"Unsupported cut_selection: {config.cut_selection}")
        self._histogram_mode = mode
        self._logger = logging.getLogger(__name__)
        self._depth_logs: list[dict[str, object]] = []
        self._binner: BinningResult | None = None
        self._rounds: list[dict[str, np.ndarray]] = []   # one tree's arrays per round
        self._trees_cache: list[Tree] | None = None
        self._era_unique: np.ndarray | None = None
        self._feature_names: list[str] | None = None
        self._tree_weight: float | None = None
        self._trained_pack_size: int | None = None
        self._round_metrics: list[dict[str, float]] = []
        self._packed_forest: list[dict[str, torch.Tensor]] = []
        self._num_features: int | None = None
        self._use_native_cuda = self._device.type == "cuda" and native_backends.cuda_available()
        # per-depth phase times in the depth logs (hist_ms, score_ms, partition_ms): every
        # PACKBOOST_PHASE_EVERY-th round (default 8, round 1 included) is timed phase by phase
        # with HIP events while the round loop stays pipelined, and the other rounds' logs carry
        # the last timed round's values (phase_ms_round names it). profile_phases (or
        # PACKBOOST_PROFILE_PHASES=1) times every round, one round at a time.
        self.profile_phases = os.getenv("PACKBOOST_PROFILE_PHASES", "0") not in ("", "0")
        try:
            self.phase_every = max(1, int(os.getenv("PACKBOOST_PHASE_EVERY", "8")))
        except ValueError:
            self.phase_every = 8

    def _phase_times(self) -> bool:
        return bool(self.profile_phases)

    # ---------------------------------------------------------------- public
    @property
    def trees(self) -> Sequence[Tree]:
        if self._trees_cache is None:
            B = int(self._trained_pack_size or self.config.pack_size)
            out: list[Tree] = []
            for arrs in self._rounds:
                for _ in range(B):
                    out.append(_tree_from_arrays(arrs))
            self._trees_cache = out
        return self._trees_cache

    @property
    def round_metrics(self) -> Sequence[dict[str, float]]:
        return self._round_metrics

    def fit(self, X, y, era: Iterable[int] | None, *, num_rounds: int,
            feature_names: Sequence[str] | None = None,
            eval_sets: Sequence[tuple] | None = None,
            round_callback: Callable[[int, dict[str, float]], None] | None = None) -> "PackBoost":
        """Squared-loss boosting with pack-synchronous growth and DES (booster.py:375-656)."""
        _require_backend(self._device)
        cfg = self.config
        y_np = np.asarray(y.detach().cpu().numpy() if isinstance(y, torch.Tensor) else y,
                          dtype=np.float32)
        if y_np.ndim != 1:
            raise ValueError("y must be 1-D")
        if isinstance(X, torch.Tensor):
            N, F = int(X.shape[0]), int(X.shape[1])
        else:
            X_arr = np.asarray(X.to_numpy() if hasattr(X, "to_numpy") else X)
            N, F = X_arr.shape
        if N != y_np.shape[0]:
            raise ValueError("X and y row mismatch")
        codes, uniq = encode_eras(era, N)
        self._era_unique = uniq
        E = int(uniq.shape[0])
        self._feature_names = feature_names_or_default(feature_names, F)
        self._num_features = F

        perm, offsets = era_major_order(codes, E)
        device = self._device if self._device.index is not None else torch.device(
            "cuda", torch.cuda.current_device())
        if isinstance(X, torch.Tensor) and not X.dtype.is_floating_point:
            self._binner = BinningResult(bins=np.empty((0, F), np.uint8), bin_edges=None, prebinned=True)
            bins_fm = column_major_bins(X, perm, device)
        elif not isinstance(X, torch.Tensor) and (bool(cfg.prebinned) or detect_prebinned(X_arr, cfg.max_bins)):
            self._binner = preprocess_features(X_arr, cfg.max_bins, assume_prebinned=bool(cfg.prebinned))
            bins_fm = column_major_bins(self._binner.bins, perm, device)
        else:
            # quantile binning on the device, rows gathered era-major (data.py:44-56)
            bins_fm, edges = quantile_bin_device(X if isinstance(X, torch.Tensor) else X_arr,
                                                 cfg.max_bins, device, perm=perm)
            self._binner = BinningResult(bins=np.empty((0, F), np.uint8), bin_edges=edges,
                                         prebinned=False)
        if N and int(bins_fm[:, :N].max().item()) >= cfg.max_bins:
            raise ValueError("bins must lie in [0, max_bins)")
        y_dev = torch.from_numpy(y_np if perm is None else y_np[perm]).to(device)
        self._perm = perm
        self._depth_logs = []
        self._round_metrics = []
        self._rounds = []
        self._trees_cache = None
        self._packed_forest = []
        self._tree_weight = None
        self._trained_pack_size = None

        fitter = DeviceFit(bins_fm, N, y_dev, offsets, cfg)
        self._fitter = fitter
        k = subset_size(cfg, F)
        era_off_dev = torch.from_numpy(np.asarray(offsets, dtype=np.int32)).to(device)
        corr_scratch = torch.empty(E + 1, dtype=torch.float64, device=device)
        eval_states = self._prepare_eval(eval_sets, device)
        eval_every = _eval_every()
        # metrics and eval predictions run on a side stream so that the next round, already
        # enqueued on the fit's stream, keeps the GPU busy while the host builds trees
        side = torch.cuda.Stream(device)
        truncated = False
        try:
            t0 = perf_counter()
            last_phase: dict[int, tuple[np.ndarray, int]] = {}  # depth -> (times, timed round)
            round_iter = enumerate(fitter.rounds(self._rng, num_rounds, phase_times=self._phase_times(),
                                                 phase_every=self.phase_every))
            while True:
                try:
                    round_idx, (log, preds_after, ready) = next(round_iter)
                except StopIteration:
                    break
                except FloatingPointError as exc:
                    if self.nonfinite != "truncate":
                        raise
                    warnings.warn(f"{exc}; nonfinite='truncate' ends the fit after "
                                  f"{len(self._rounds)} rounds", RuntimeWarning, stacklevel=2)
                    truncated = True
                    break
                arrs = tree_arrays_from_log(log, cfg, N)
                self._rounds.append(arrs)
                self._trees_cache = None
                self._tree_weight = float(cfg.learning_rate)
                self._trained_pack_size = int(cfg.pack_size)
                for d in range(int(cfg.max_depth)):
                    if int(log.u_active[d]) <= 0:
                        break
                    if log.phase_ms is not None:
                        last_phase[d] = (log.phase_ms, round_idx + 1)
                    dl = depth_log_from_round(log, d, cfg, k, self._histogram_mode, last_phase.get(d))
                    self._depth_logs.append(dl)
                    if self._logger.isEnabledFor(logging.INFO):
                        self._logger.info(json.dumps(dl))
                with torch.cuda.stream(side):
                    side.wait_event(ready)
                    if eval_states and eval_every > 0 and (
                            (round_idx + 1) % eval_every == 0 or round_idx + 1 == num_rounds):
                        self._update_eval(eval_states)
                    train_corr = _era_corr_device(fitter.y, preds_after, era_off_dev, corr_scratch)
                    eval_corr = {f"{st['name']}_corr": _era_corr_device(
                        st["y"], st["preds"], st["era_off"], st["corr_scratch"]) for st in eval_states}
                t1 = perf_counter()
                round_time = t1 - t0
                t0 = t1
                metrics = {
                    "round": round_idx + 1,
                    "train_corr": train_corr,
                    "trees_per_second": (cfg.pack_size / round_time) if round_time > 0 else float("inf"),
                    "round_seconds": round_time,
                }
                metrics.update(eval_corr)
                self._round_metrics.append(metrics)
                if round_callback is not None:
                    round_callback(round_idx + 1, metrics)
        except BaseException:
            # e.g. FloatingPointError from a round with non-finite gradients: release the
            # fit's device state before the error propagates
            torch.cuda.synchronize(device)
            fitter.close()
            self._fitter = None
            raise
        finally:
            torch.cuda.synchronize(device)
        if truncated:
            # the device has run the non-finite round (and the one enqueued after it) on
            # `fitter.preds`: the kept rounds' training predictions come from their trees
            self._train_preds = (self._predict_device(bins_fm, N, device) if self._rounds
                                 else torch.zeros(N, dtype=torch.float32, device=device))
        else:
            self._train_preds = fitter.preds[:N].clone()
        self._fit_mode = "segments" if fitter.segments else "planes"
        fitter.close()
        self._fitter = None
        return self

    def predict(self, X) -> np.ndarray:
        """Sum over all trees of float32(tree_weight * leaf value) (booster.py:658-712), on the
        compiled forest's tiled walk: the sums are taken in double and rounded once, so they lie
        within float32 rounding of any of the reference's summation orders (its CPU path adds
        tree by tree in float32, its CUDA path pack by pack)."""
        if self._binner is None:
            raise RuntimeError("Model must be fitted before predict()")
        _require_backend(self._device)
        if self._trained_pack_size is not None and int(self.config.pack_size) != self._trained_pack_size:
            raise RuntimeError("pack_size differs from training; keep it constant.")
        N = int(X.shape[0])
        if not self._rounds:
            return np.zeros(N, dtype=np.float32)
        if self._tree_weight is None:
            raise RuntimeError("Missing _tree_weight; call fit() first.")
        device = self._device if self._device.index is not None else torch.device(
            "cuda", torch.cuda.current_device())
        bins_fm, N = _bins_fm_for(X, self._binner.bin_edges, self.config.max_bins, device)
        out = self._predict_device(bins_fm, N, device)
        return out.cpu().numpy()

    def save(self, path) -> "Path":
        """Writes the fitted model as a versioned .npz bundle (see predictor.save_bundle)."""
        from .predictor import save_bundle

        return save_bundle(self, path)

    def predict_packwise(self, X, block_size_trees: int = 8) -> np.ndarray:
        if block_size_trees <= 0:
            raise ValueError("block_size_trees must be positive")
        if self._binner is None:
            raise RuntimeError("Model must be fitted before predict_packwise()")
        return self.predict(X)

    # ---------------------------------------------------------------- internals
    def _forest_device(self, device: torch.device) -> dict[str, torch.Tensor]:
        key = (str(device), len(self._rounds))
        cached = getattr(self, "_forest_cache", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        forest = pack_forest(self._rounds, int(self._trained_pack_size or self.config.pack_size), device)
        self._forest_cache = (key, forest)
        return forest

    def _predict_device(self, bins_fm: torch.Tensor, N: int, device: torch.device) -> torch.Tensor:
        from .predictor import CompiledForest

        key = (str(device), len(self._rounds))
        cached = getattr(self, "_compiled_forest", None)
        if cached is None or cached[0] != key:
            cached = (key, CompiledForest(self._forest_device(device)))
            self._compiled_forest = cached
        return cached[1].predict(bins_fm, N, float(self._tree_weight))

    def _prepare_eval(self, eval_sets, device) -> list[dict]:
        states = []
        for item in eval_sets or ():
            name, X_eval, y_eval, era_eval = item
            if y_eval is None:
                raise ValueError(f"eval set '{name}' requires y values for correlation logging")
            n = int(X_eval.shape[0])
            codes, uniq = encode_eras(era_eval, n)
            E = int(uniq.shape[0])
            # rows era-major (metrics only: eval predictions never leave the fit)
            perm, offs = era_major_order(codes, E)
            yv = np.asarray(y_eval, dtype=np.float32).reshape(-1)
            if perm is not None:
                yv = yv[perm]
            edges = None if self.config.prebinned else self._binner.bin_edges
            bins_fm, _ = _bins_fm_for(X_eval, edges, self.config.max_bins, device, perm=perm)
            states.append({
                "name": name, "bins_fm": bins_fm, "n": n,
                "y": torch.from_numpy(np.ascontiguousarray(yv)).to(device),
                "era_off": torch.from_numpy(np.asarray(offs, dtype=np.int32)).to(device),
                "corr_scratch": torch.empty(E + 1, dtype=torch.float64, device=device),
                "num_eras": E,
                "preds": torch.zeros(n, dtype=torch.float32, device=device),
                "rounds_done": 0,
            })
        return states

    def _update_eval(self, states: list[dict]) -> None:
        # Like the reference (booster.py:236-274) the eval predictions equal predict() on the
        # same rows: the sum over every tree so far, in tree order, of float32(weight * value).
        # That sum is a left fold, so each state extends its own fold by the rounds it has not
        # seen, one float32 add per tree: the B trees of a round are identical, so the round's
        # tree is walked once (pb_predict_bins) and its weighted value added B times. The host
        # work per eval is the new rounds only.
        B = int(self.config.pack_size)
        w = torch.tensor(np.float32(self._tree_weight), dtype=torch.float32)
        lib = _hip.load()
        for st in states:
            dev = st["preds"].device
            wd = w.to(dev)
            while st["rounds_done"] < len(self._rounds):
                a = self._rounds[st["rounds_done"]]
                t = {k: torch.from_numpy(np.ascontiguousarray(np.asarray(a[k]), dtype=dt)).to(dev)
                     for k, dt in (("feature", np.int32), ("threshold", np.int32), ("left", np.int32),
                                   ("right", np.int32), ("value", np.float32), ("is_leaf", np.uint8))}
                v = torch.empty(st["n"], dtype=torch.float32, device=dev)
                _hip.check(lib.pb_predict_bins(
                    st["bins_fm"].data_ptr(), st["n"], st["bins_fm"].shape[1], st["bins_fm"].shape[0],
                    t["feature"].data_ptr(), t["threshold"].data_ptr(), t["left"].data_ptr(),
                    t["right"].data_ptr(), t["value"].data_ptr(), t["is_leaf"].data_ptr(),
                    int(t["value"].numel()), v.data_ptr(), _hip.stream_ptr()), "pb_predict_bins")
                term = wd * v
                for _ in range(B):
                    st["preds"] = st["preds"] + term
                st["rounds_done"] += 1


def pack_forest(rounds: Sequence[dict[str, np.ndarray]], pack_size: int,
                device: torch.device) -> dict[str, torch.Tensor]:
    """Packed SoA of every tree (booster.py:730-783 layout, children as absolute indices)."""
    feats, thrs, lefts, rights, vals, leafs, offs = [], [], [], [], [], [], [0]
    for a in rounds:
        n = a["feature"].shape[0]
        for _ in range(pack_size):
            base = offs[-1]
            feats.append(a["feature"].astype(np.int32))
            thrs.append(a["threshold"].astype(np.int32))
            lf = a["is_leaf"]
            lefts.append(np.where(lf | (a["left"] < 0), -1, a["left"] + base).astype(np.int32))
            rights.append(np.where(lf | (a["right"] < 0), -1, a["right"] + base).astype(np.int32))
            vals.append(a["value"].astype(np.float32))
            leafs.append(lf.astype(np.uint8))
            offs.append(base + n)
    cat = np.concatenate
    return {
        "feature": torch.from_numpy(cat(feats)).to(device),
        "threshold": torch.from_numpy(cat(thrs)).to(device),
        "left_abs": torch.from_numpy(cat(lefts)).to(device),
        "right_abs": torch.from_numpy(cat(rights)).to(device),
        "value": torch.from_numpy(cat(vals)).to(device),
        "is_leaf": torch.from_numpy(cat(leafs)).to(device),
        "offsets": torch.tensor(offs, dtype=torch.int32, device=device),
    }


def _eval_every() -> int:
    try:
        return int(os.getenv("PACKBOOST_EVAL_EVERY", "1"))
    except ValueError:
        return 1


def _era_corr_device(y: torch.Tensor, p: torch.Tensor, era_off: torch.Tensor,
                     scratch: torch.Tensor) -> float:
    """Mean over eras of the Pearson correlation of y and preds (booster.py:909-929) by the
    pb_era_corr kernel on the current stream; rows are era-major, era_off int32 [E+1]."""
    E = int(era_off.numel()) - 1
    lib = _hip.load()
    _hip.check(lib.pb_era_corr(y.data_ptr(), p.data_ptr(), era_off.data_ptr(), E, scratch.data_ptr(),
                               scratch.data_ptr() + 8 * E, _hip.stream_ptr()), "pb_era_corr")
    return float(scratch[E].item())
