"""Writes tests/golden/fit_*.npz: input/output vectors of the reference's own PackBoost.fit.

Run in the build container only (it needs /root/reference and oracle/_ref, which never travel
to the GPU box):

    make -C oracle ref && python tests/golden/make_fit_golden.py

The reference package is imported from /root/reference with its native CPU split finder,
i.e. oracle/_ref/_backend*.so, compiled by oracle/Makefile from the reference's own
frontier_cpu.cpp + bindings.cpp and registered as `packboost._backend` (the module name the
reference's loader imports, backends/__init__.py:20-35). Each case records:
  inputs   X (float32 [N, F]), y, era labels, the config;
  binning  the reference's preprocess_features bins (uint8) and bin edges (data.py:31-111);
  trees    every round's first tree (feature, threshold, left, right, value, is_leaf) after
           checking that all B trees of the pack are identical (booster.py:503-563);
  preds    PackBoost.predict on X (booster.py:658-712).
Only these arrays are committed, never reference code.
"""

from __future__ import annotations

import glob
import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REF = Path("/root/reference")

CASES = {
    # name: (data recipe, config, rounds)
    "fit_config1": (dict(seed=42, n=2400, f=10, eras=8, interleave=False),
                    dict(pack_size=4, max_depth=4, learning_rate=0.05, lambda_l2=1.0,
                         lambda_dro=0.5, min_samples_leaf=20, max_bins=32, random_state=42), 5),
    "fit_dir_alpha": (dict(seed=7, n=2000, f=10, eras=6, interleave=True),
                      dict(pack_size=3, max_depth=4, learning_rate=0.1, lambda_l2=1e-3,
                           lambda_dro=0.1, direction_weight=0.05, min_samples_leaf=8, max_bins=63,
                           layer_feature_fraction=0.6, era_alpha=1.5, random_state=7), 5),
    "fit_early_stop": (dict(seed=9, n=2400, f=10, eras=5, interleave=False),
                       dict(pack_size=2, max_depth=6, learning_rate=0.1, lambda_l2=1e-6,
                            lambda_dro=0.2, min_samples_leaf=150, max_bins=31,
                            layer_feature_fraction=0.5, random_state=23), 5),
    "fit_kcuts_mass": (dict(seed=5, n=2000, f=8, eras=4, interleave=False),
                       dict(pack_size=2, max_depth=3, learning_rate=0.1, lambda_l2=1e-3,
                            lambda_dro=0.3, min_samples_leaf=10, max_bins=48, k_cuts=5,
                            cut_selection="mass", random_state=3), 4),
    "fit_kcuts_even": (dict(seed=6, n=2000, f=8, eras=4, interleave=False),
                       dict(pack_size=2, max_depth=3, learning_rate=0.1, lambda_l2=1e-3,
                            lambda_dro=0.3, min_samples_leaf=10, max_bins=48, k_cuts=6,
                            cut_selection="even", random_state=4), 4),
}


def make_data(seed: int, n: int, f: int, eras: int, interleave: bool):
    """y = 5 random-weight features + 0.5 sin(x0) + N(0, 0.1) (the config-1 recipe)."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, f)).astype(np.float32)
    idx = rng.choice(f, 5, replace=False)
    w = rng.standard_normal(5).astype(np.float32)
    y = (X[:, idx] @ w + 0.5 * np.sin(X[:, 0]) + 0.1 * rng.standard_normal(n)).astype(np.float32)
    if interleave:
        era = (rng.integers(0, eras, size=n) * 3 + 100).astype(np.int64)
    else:
        era = np.repeat(np.arange(eras), n // eras).astype(np.int64)
    return X, y, era


def load_reference():
    hits = glob.glob(str(ROOT / "oracle" / "_ref" / "_backend*.so"))
    if not hits:
        raise SystemExit("oracle/_ref is not built: run `make -C oracle ref` first")
    spec = importlib.util.spec_from_file_location("packboost._backend", hits[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules["packboost._backend"] = mod
    sys.path.insert(0, str(REF))
    import packboost
    from packboost import backends

    assert backends.cpu_available(), "reference CPU backend did not load"
    return packboost


def main() -> None:
    pb = load_reference()
    for name, (recipe, cfg, rounds) in CASES.items():
        X, y, era = make_data(**recipe)
        model = pb.PackBoost(pb.PackBoostConfig(device="cpu", **cfg))
        model.fit(X, y, era, num_rounds=rounds)
        B = cfg["pack_size"]
        trees = model.trees
        assert len(trees) == rounds * B
        out = {"X": X, "y": y, "era": era, "config": np.array(json.dumps(cfg)),
               "rounds": np.array(rounds)}
        binner = model._binner
        out["bins"] = np.asarray(binner.bins).astype(np.uint8)
        edges = binner.bin_edges
        out["has_edges"] = np.array(edges is not None)
        if edges is not None:
            out["edge_lens"] = np.array([len(e) for e in edges], dtype=np.int64)
            out["edges"] = (np.concatenate([np.asarray(e, dtype=np.float64) for e in edges])
                            if len(edges) else np.zeros(0))
        for r in range(rounds):
            pack = trees[r * B:(r + 1) * B]
            sig0 = [(n.feature, n.threshold, n.left, n.right, n.value, n.is_leaf) for n in pack[0].nodes]
            for t in pack[1:]:
                assert [(n.feature, n.threshold, n.left, n.right, n.value, n.is_leaf)
                        for n in t.nodes] == sig0, f"{name}: round {r} trees differ within the pack"
            nodes = pack[0].nodes
            out[f"r{r}_feature"] = np.array([n.feature for n in nodes], dtype=np.int64)
            out[f"r{r}_threshold"] = np.array([n.threshold for n in nodes], dtype=np.int64)
            out[f"r{r}_left"] = np.array([n.left for n in nodes], dtype=np.int64)
            out[f"r{r}_right"] = np.array([n.right for n in nodes], dtype=np.int64)
            out[f"r{r}_value"] = np.array([n.value for n in nodes], dtype=np.float64)
            out[f"r{r}_is_leaf"] = np.array([n.is_leaf for n in nodes], dtype=bool)
        out["preds"] = np.asarray(model.predict(X), dtype=np.float32)
        out["tree_weight"] = np.array(float(model._tree_weight))
        np.savez_compressed(HERE / f"{name}.npz", **out)
        print(f"{name}: {rounds} rounds, {sum(len(t.nodes) for t in trees[::B])} nodes", flush=True)


if __name__ == "__main__":
    main()
