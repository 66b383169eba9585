"""Model bundle and standalone predictor.

The reference plans a versioned bundle (trees, feature names, bin edges, config) with a
lightweight loader and a predictor with parity to the trainer (project.md:536-542; README.md:19-20
advertises `PackBoostPredictor`). The bundle here is one `.npz` (no pickles; load with
`allow_pickle=False`) holding:

  format, version              "packboost-bundle", 1
  config                       JSON of the PackBoostConfig fields
  feature_names                JSON list
  bin_edges                    float32 [max_bins - 1, F] (absent when trained on prebinned X)
  tree_weight, pack_size       the trainer's _tree_weight and pack size
  round_offsets                int64 [R + 1]: node range of each round's tree
  feature, threshold, left, right (int32), value (float64), is_leaf (uint8)
                               one tree per round (the B trees of a pack are identical),
                               TreeBuilder numbering, children relative to the tree

`PackBoostPredictor.predict` expands the rounds into the packed forest of booster.py:730-783
(B copies per round, absolute child indices), compiles it once (pb_forest_create) and runs
pb_forest_predict, which sums the trees in PackBoost.predict's order (booster.py:709-712): its
output is bit-identical to the trainer's.
"""

from __future__ import annotations

import json
from dataclasses import asdict, fields
from pathlib import Path

import numpy as np
import torch

from .backends import _hip
from .config import PackBoostConfig

BUNDLE_FORMAT = "packboost-bundle"
BUNDLE_VERSION = 1
_TREE_KEYS = ("feature", "threshold", "left", "right", "value", "is_leaf")


def save_bundle(model, path: str | Path) -> Path:
    """Writes a fitted PackBoost model to `path` (.npz)."""
    if model._binner is None or model._tree_weight is None:
        raise RuntimeError("Model must be fitted before it can be saved")
    rounds = model._rounds
    offs = np.zeros(len(rounds) + 1, dtype=np.int64)
    for r, a in enumerate(rounds):
        offs[r + 1] = offs[r] + len(a["feature"])

    def cat(key, dtype):
        if not rounds:
            return np.zeros(0, dtype=dtype)
        return np.concatenate([np.asarray(a[key]).astype(dtype) for a in rounds])

    cfg = {k: v for k, v in asdict(model.config).items()}
    out = {
        "format": np.array(BUNDLE_FORMAT),
        "version": np.array(BUNDLE_VERSION, dtype=np.int64),
        "config": np.array(json.dumps(cfg)),
        "feature_names": np.array(json.dumps(list(model._feature_names or []))),
        "tree_weight": np.array(float(model._tree_weight), dtype=np.float64),
        "pack_size": np.array(int(model._trained_pack_size or model.config.pack_size), dtype=np.int64),
        "round_offsets": offs,
        "feature": cat("feature", np.int32),
        "threshold": cat("threshold", np.int32),
        "left": cat("left", np.int32),
        "right": cat("right", np.int32),
        "value": cat("value", np.float64),
        "is_leaf": cat("is_leaf", np.uint8),
    }
    edges = model._binner.bin_edges
    if edges is not None:
        out["bin_edges"] = np.asarray(edges, dtype=np.float32)
    path = Path(path)
    if path.suffix != ".npz":
        path = path.with_suffix(path.suffix + ".npz") if path.suffix else path.with_suffix(".npz")
    np.savez(path, **out)
    return path


def load_bundle(path: str | Path) -> dict:
    """Reads a bundle written by save_bundle; refuses other formats and newer versions."""
    with np.load(path, allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    if str(d.get("format", "")) != BUNDLE_FORMAT:
        raise ValueError(f"{path}: not a PackBoost bundle")
    version = int(d["version"])
    if version > BUNDLE_VERSION:
        raise ValueError(f"{path}: bundle version {version} is newer than this reader ({BUNDLE_VERSION})")
    cfg = json.loads(str(d["config"]))
    known = {f.name for f in fields(PackBoostConfig)}
    d["config"] = PackBoostConfig(**{k: v for k, v in cfg.items() if k in known})
    d["feature_names"] = json.loads(str(d["feature_names"]))
    d["tree_weight"] = float(d["tree_weight"])
    d["pack_size"] = int(d["pack_size"])
    offs = d["round_offsets"]
    d["rounds"] = [{k: d[k][offs[r]:offs[r + 1]] for k in _TREE_KEYS} for r in range(len(offs) - 1)]
    for r in d["rounds"]:
        r["is_leaf"] = r["is_leaf"].astype(bool)
    d["bin_edges"] = d.get("bin_edges")
    return d


class CompiledForest:
    """A packed forest (booster.pack_forest arrays) compiled into device node records
    (pb_forest_create); predict() equals pb_predict_forest bit for bit."""

    def __init__(self, forest: dict[str, torch.Tensor]) -> None:
        import ctypes

        self._lib = _hip.load()
        self.T = int(forest["offsets"].numel() - 1)
        h = ctypes.c_void_p()
        _hip.check(self._lib.pb_forest_create(
            forest["feature"].data_ptr(), forest["threshold"].data_ptr(),
            forest["left_abs"].data_ptr(), forest["right_abs"].data_ptr(),
            forest["value"].data_ptr(), forest["is_leaf"].data_ptr(), forest["offsets"].data_ptr(),
            self.T, int(forest["value"].numel()), ctypes.byref(h)), "pb_forest_create")
        self._h = h
        self.offsets = forest["offsets"]

    def predict(self, bins_fm: torch.Tensor, n: int, tree_weight: float,
                leaves: torch.Tensor | None = None) -> torch.Tensor:
        out = torch.empty(n, dtype=torch.float32, device=bins_fm.device)
        _hip.check(self._lib.pb_forest_predict(
            self._h, bins_fm.data_ptr(), n, bins_fm.shape[1], bins_fm.shape[0], float(tree_weight),
            out.data_ptr(), None if leaves is None else leaves.data_ptr(), _hip.stream_ptr()),
            "pb_forest_predict")
        return out

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            torch.cuda.synchronize()
            self._lib.pb_forest_destroy(self._h)
            self._h = None

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


class PackBoostPredictor:
    """Inference-only view of a fitted model: a bundle path, a loaded bundle, or a model."""

    def __init__(self, source, device: str | torch.device | None = None) -> None:
        if isinstance(source, (str, Path)):
            b = load_bundle(source)
        elif isinstance(source, dict):
            b = source
        else:  # a fitted PackBoost
            b = {"config": source.config, "feature_names": list(source._feature_names or []),
                 "tree_weight": float(source._tree_weight), "rounds": list(source._rounds),
                 "pack_size": int(source._trained_pack_size or source.config.pack_size),
                 "bin_edges": None if source._binner is None else source._binner.bin_edges}
            if source._tree_weight is None:
                raise RuntimeError("Model must be fitted before building a predictor")
        self.config: PackBoostConfig = b["config"]
        self.feature_names: list[str] = b["feature_names"]
        self.tree_weight: float = b["tree_weight"]
        self.pack_size: int = b["pack_size"]
        self.bin_edges = b["bin_edges"]
        self.rounds = b["rounds"]
        self.device = torch.device(device if device is not None else self.config.device)
        if self.device.type != "cuda":
            raise RuntimeError("PackBoostPredictor runs on the HIP device (device='cuda')")
        self._forest = None

    @classmethod
    def load(cls, path: str | Path, device: str | torch.device | None = None) -> "PackBoostPredictor":
        return cls(path, device)

    @property
    def num_trees(self) -> int:
        return len(self.rounds) * self.pack_size

    def _packed(self) -> dict[str, torch.Tensor]:
        if self._forest is None:
            from .booster import pack_forest

            self._forest = pack_forest(self.rounds, self.pack_size, self.device)
        return self._forest

    def _compiled(self) -> CompiledForest:
        if getattr(self, "_cforest", None) is None:
            self._cforest = CompiledForest(self._packed())
        return self._cforest

    def _bins_fm(self, X) -> tuple[torch.Tensor, int]:
        from .booster import _bins_fm_for

        nf = int(X.shape[1])
        if self.feature_names and nf != len(self.feature_names):
            raise ValueError(f"X has {nf} features; the model expects {len(self.feature_names)}")
        return _bins_fm_for(X, self.bin_edges, self.config.max_bins, self.device)

    def predict(self, X) -> np.ndarray:
        """float32 predictions, bit-identical to PackBoost.predict on the same model."""
        bins_fm, n = self._bins_fm(X)
        if not self.rounds or n == 0:
            return np.zeros(n, dtype=np.float32)
        return self._compiled().predict(bins_fm, n, self.tree_weight).cpu().numpy()

    def predict_leaves(self, X) -> np.ndarray:
        """int32 [num_trees, N]: each tree's leaf, as a node index within that tree."""
        bins_fm, n = self._bins_fm(X)
        T = self.num_trees
        if T == 0 or n == 0:
            return np.zeros((T, n), dtype=np.int32)
        cf = self._compiled()
        leaf = torch.empty((T, n), dtype=torch.int32, device=self.device)
        cf.predict(bins_fm, n, self.tree_weight, leaves=leaf)
        offs = cf.offsets[:-1].to(torch.int32)[:, None]
        return (leaf - offs).cpu().numpy()
