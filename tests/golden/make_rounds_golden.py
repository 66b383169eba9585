"""Writes tests/golden/<case>_rounds.npz: the oracle's whole-round decisions on a BASELINE
workload at its full size, for the GPU tests that compare the HIP fit round by round.

  config3  2,400,000 rows x 2,376 features quantised to 5 levels, 574 eras, B 8, D 6,
           238 features per depth, lr 0.01, lambda_dro 0.5 (5 rounds);
  config2  200,000 x 100 float32 features (10 correlated at 0.6), 50 eras, 128 quantile bins,
           B 8, D 5 (its 100 rounds).

Each workload is a pure function of a NumPy seed (`case_data()`), so the GPU tests regenerate
it on the box and only the oracle's outputs are committed (`load_fixture()` reads them back). The oracle is the restated fit loop
(oracle.fit, booster.py:375-599) with each depth's split finder run by the reference's own
compiled frontier (frontier_cpu.cpp:111-515 via oracle/_ref) when it is built here, else by the
C restatement; the two are bit-identical (tests/test_oracle_reference.py). Per round it records:
  trees   the round's tree (feature, threshold, left, right, value, is_leaf);
  depths  per depth the frontier node ids, the feature subset, and per node the chosen
          (feature, threshold), the split score, the left count and the node's row count;
  preds   the float32 training predictions after the round: their float64 sum over all rows,
          and their values at SAMPLE_ROWS seeded rows (rounds 0-4, every 25th and the last).

Run in the build container (config3: about 45 s per round on 8 cores; config2: about 1 s):

    python tests/golden/make_rounds_golden.py config3 [rounds]
    python tests/golden/make_rounds_golden.py config2 [rounds]
"""

from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent

N3, F3, E3, NB3 = 2_400_000, 2376, 574, 5
CONFIG3 = dict(pack_size=8, max_depth=6, learning_rate=0.01, lambda_l2=1e-6, lambda_dro=0.5,
               min_samples_leaf=20, max_bins=5, layer_feature_fraction=0.1, random_state=42)
CONFIG2 = dict(pack_size=8, max_depth=5, learning_rate=0.1, max_bins=128, min_samples_leaf=20,
               random_state=42)
ROUNDS = {"config3": 5, "config2": 100}
SAMPLE_ROWS = {"config3": 20_000, "config2": 4_000}
SEED = 42


def era_sizes(n: int = N3, e: int = E3) -> np.ndarray:
    """Contiguous eras of np.array_split sizes (config 3: 4181 / 4182 rows)."""
    base, extra = divmod(n, e)
    return np.array([base + 1] * extra + [base] * (e - extra), dtype=np.int64)


def panel(seed: int = SEED, n: int = N3, f: int = F3, e: int = E3):
    """The config-3 panel: row-major uint8 bins [n, f] uniform over {0..4}; eras contiguous;
    y in {0, .25, .5, .75, 1} from quantising a 50-feature linear form whose first 10 weights
    flip sign per era at random, plus noise of half the form's standard deviation."""
    rng = np.random.default_rng(seed)
    bins = rng.integers(0, NB3, size=(n, f), dtype=np.uint8)
    sizes = era_sizes(n, e)
    era = np.repeat(np.arange(e, dtype=np.int64), sizes)
    sel = rng.choice(f, 50, replace=False)
    w = rng.standard_normal(50)
    flips = np.where(rng.random((e, 10)) < 0.5, -1.0, 1.0)
    lin = np.zeros(n, dtype=np.float64)
    for j in range(50):
        col = bins[:, sel[j]].astype(np.float64) - 2.0
        lin += w[j] * col * (flips[era, j] if j < 10 else 1.0)
    lin += rng.standard_normal(n) * lin.std() * 0.5
    q = np.quantile(lin, [0.2, 0.4, 0.6, 0.8])
    y = (np.searchsorted(q, lin, side="right") / 4.0).astype(np.float32)
    return bins, y, era


def case_data(name: str):
    """(X the fit's input, bins row-major uint8 [N, F], y float32, era codes int64, config)."""
    if name == "config3":
        bins, y, era = panel()
        return bins, bins, y, era, dict(CONFIG3)
    if name == "config2":
        sys.path.insert(0, str(ROOT))
        from oracle.calibrate import config2_data
        from packboost_amd.data import preprocess_features

        X, y, era = config2_data(SEED)
        return X, preprocess_features(X, CONFIG2["max_bins"]).bins, y, era.astype(np.int64), dict(CONFIG2)
    raise ValueError(name)


def sample_rows(name: str, n: int) -> np.ndarray:
    rng = np.random.default_rng(SEED + 1)
    return np.sort(rng.choice(n, min(n, SAMPLE_ROWS[name]), replace=False))


def load_fixture(name: str) -> dict:
    """tests/golden/<name>_rounds.npz as {"rounds": R, "trees": [per round dict of arrays],
    "depths": [{"round", "depth", "nodes", "feats", "feature", "threshold", "score",
    "left_count", "rows"} per traced depth], "preds_sum": [R], "preds_sample": {round: array}}."""
    with np.load(HERE / f"{name}_rounds.npz", allow_pickle=False) as z:
        f = {k: z[k] for k in z.files}
    R = int(f["rounds"][0])
    trees, t0 = [], 0
    for r in range(R):
        n = int(f["t_len"][r])
        trees.append({k: f[f"t_{k}"][t0:t0 + n] for k in
                      ("feature", "threshold", "left", "right", "value", "is_leaf")})
        t0 += n
    depths, d0 = [], 0
    for i in range(len(f["d_len"])):
        n = int(f["d_len"][i])
        e = {k: f[f"d_{k}"][d0:d0 + n] for k in
             ("nodes", "feature", "threshold", "score", "left_count", "rows")}
        e.update(round=int(f["d_round"][i]), depth=int(f["d_depth"][i]), feats=f["d_feats"][i])
        depths.append(e)
        d0 += n
    samples = {r: f[f"r{r}_preds_sample"] for r in range(R) if f"r{r}_preds_sample" in f}
    return {"rounds": R, "trees": trees, "depths": depths, "preds_sum": f["preds_sum"],
            "preds_sample": samples}


def main() -> int:
    name = sys.argv[1] if len(sys.argv) > 1 else "config3"
    rounds = int(sys.argv[2]) if len(sys.argv) > 2 else ROUNDS[name]
    sys.path.insert(0, str(ROOT))
    import torch

    from oracle import oracle as ref

    t0 = time.perf_counter()
    _, bins, y, era, cfg = case_data(name)
    print(f"{name} data {time.perf_counter() - t0:.1f} s", flush=True)
    splitter = "reference" if ref.ref_module() is not None else "restated"
    rng = torch.Generator().manual_seed(cfg["random_state"])
    kw = {k: v for k, v in cfg.items() if k != "random_state"}
    out: dict[str, np.ndarray] = {}
    cols: dict[str, list] = {k: [] for k in (
        "t_feature", "t_threshold", "t_left", "t_right", "t_value", "t_is_leaf", "t_len",
        "d_round", "d_depth", "d_len", "d_feats", "d_nodes", "d_feature", "d_threshold", "d_score",
        "d_left_count", "d_rows")}
    samp = sample_rows(name, bins.shape[0])
    preds = None
    sums = []
    for r in range(rounds):
        t1 = time.perf_counter()
        trace: list = []
        res = ref.fit(bins, y, era, num_rounds=1, rng=rng, trace=trace, splitter=splitter,
                      init_preds=preds, **kw)
        preds = res.preds
        a = res.rounds[0]
        # ids, features and thresholds fit int16 (trees of at most 2^15 nodes, F < 2^15)
        for key in ("feature", "threshold", "left", "right"):
            cols[f"t_{key}"].append(np.asarray(a[key]).astype(np.int16))
        cols["t_value"].append(np.asarray(a["value"], dtype=np.float64))
        cols["t_is_leaf"].append(np.asarray(a["is_leaf"], dtype=bool))
        cols["t_len"].append(len(a["feature"]))
        for t in trace:
            d, rr = t["depth"], t["result"]
            cols["d_round"].append(r)
            cols["d_depth"].append(d)
            cols["d_len"].append(len(t["node_ids"]))
            cols["d_feats"].append(np.asarray(t["feats"], dtype=np.int16))
            cols["d_nodes"].append(np.asarray(t["node_ids"], dtype=np.int16))
            cols["d_feature"].append(rr.feature.astype(np.int16))
            cols["d_threshold"].append(rr.threshold.astype(np.int16))
            cols["d_score"].append(rr.score.astype(np.float32))
            cols["d_left_count"].append(rr.left_count.astype(np.int64))
            cols["d_rows"].append(np.array([sum(x.size for x in er) for er in t["nodes_era_rows"]],
                                           dtype=np.int64))
        if r < 5 or r % 25 == 24 or r == rounds - 1:
            out[f"r{r}_preds_sample"] = preds[samp].astype(np.float32)
        sums.append(preds.astype(np.float64).sum())
        print(f"round {r}: {len(trace)} depths, tree of {a['feature'].shape[0]} nodes, "
              f"{time.perf_counter() - t1:.1f} s", flush=True)
    for k, v in cols.items():
        if k == "d_feats":
            out[k] = np.stack(v)
        elif k in ("t_len", "d_round", "d_depth", "d_len"):
            out[k] = np.asarray(v, dtype=np.int32)
        else:
            out[k] = np.concatenate(v)
    out["preds_sum"] = np.asarray(sums, dtype=np.float64)
    out["rounds"] = np.array([rounds])
    out["splitter"] = np.array([splitter])
    out["config"] = np.array([repr(cfg)])
    path = HERE / f"{name}_rounds.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes, splitter {splitter})")
    return 0


if __name__ == "__main__":
    sys.exit(main())
