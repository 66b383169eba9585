"""Calibrates the CPU baseline: the oracle's fit loop with its C restatement of the split finder
against the same loop with the reference's own compiled frontier (frontier_cpu.cpp, built by
`make -C oracle ref`), on BASELINE config 2 and a 240,000-row slice of config 3.

Test infrastructure (the oracle's checker side); prints one JSON line per workload with the
steady-state seconds per round (rounds 2.., the reference's round_seconds span,
booster.py:495, 654) of each splitter and their ratio. Both splitters must give the same trees.

    python oracle/calibrate.py [--rounds 3]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from oracle import oracle as om  # noqa: E402


def config2_data(seed: int = 42):
    """200,000 x 100 N(0,1) float32 features, 10 of them pairwise
    correlated at 0.6, y = sparse linear over 20 features + tanh interactions + a per-era shift
    N(0, 0.2) + noise, 50 contiguous eras. Returns X, y, era."""
    rng = np.random.default_rng(seed)
    N, F, E = 200_000, 100, 50
    X = rng.standard_normal((N, F)).astype(np.float32)
    z = rng.standard_normal(N).astype(np.float32)
    X[:, :10] = np.sqrt(0.6) * z[:, None] + np.sqrt(0.4) * X[:, :10]
    sel = rng.choice(F, 20, replace=False)
    w = rng.standard_normal(20).astype(np.float32)
    era = np.repeat(np.arange(E), N // E)
    y = X[:, sel] @ w + np.tanh(X[:, 0] * X[:, 1]) + np.tanh(X[:, 2] - X[:, 3])
    y = (y + (rng.standard_normal(E) * 0.2)[era] + 0.1 * rng.standard_normal(N)).astype(np.float32)
    return X, y, era


def config2(seed: int = 42):
    """Config 2 binned on the host into 128 quantile bins (data.py:44-111), with its fit
    parameters (pack 8, depth 5)."""
    from packboost_amd.data import preprocess_features

    X, y, era = config2_data(seed)
    bins = preprocess_features(X, 128).bins
    kw = dict(pack_size=8, max_depth=5, learning_rate=0.1, max_bins=128, min_samples_leaf=20,
              random_state=42)
    return bins, y, era, kw


def config3_slice(rows: int = 240_000, seed: int = 42):
    """Config 3's panel shape on `rows` rows: 2376 features uniform over 5 levels, 574
    contiguous eras, y quantised to {0, .25, .5, .75, 1} from a sparse linear combination of
    50 features with era-specific sign flips on 10 of them plus noise."""
    rng = np.random.default_rng(seed)
    F, E = 2376, 574
    bins = rng.integers(0, 5, size=(rows, F), dtype=np.uint8)
    sizes = np.array([len(a) for a in np.array_split(np.arange(rows), E)])
    era = np.repeat(np.arange(E), sizes)
    sel = rng.choice(F, 50, replace=False)
    w = rng.standard_normal(50)
    flips = np.where(rng.random((E, 10)) < 0.5, -1.0, 1.0)
    lin = np.zeros(rows)
    for j in range(50):
        col = bins[:, sel[j]].astype(np.float64) - 2.0
        lin += w[j] * col * (flips[era, j] if j < 10 else 1.0)
    lin += rng.standard_normal(rows) * lin.std() * 0.5
    y = (np.digitize(lin, np.quantile(lin, [0.2, 0.4, 0.6, 0.8])) / 4.0).astype(np.float32)
    kw = dict(pack_size=8, max_depth=6, learning_rate=0.01, lambda_dro=0.5, max_bins=5,
              min_samples_leaf=20, layer_feature_fraction=0.1, random_state=42)
    return bins, y, era, kw


def time_fit(bins, y, era, kw, rounds: int, splitter: str):
    t0 = time.perf_counter()
    r = om.fit(bins, y, era, num_rounds=rounds, splitter=splitter, **kw)
    wall = time.perf_counter() - t0
    steady = r.round_seconds[1:] if len(r.round_seconds) > 1 else r.round_seconds
    return r, float(np.mean(steady)), wall


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--rounds", type=int, default=3)
    ap.add_argument("--workloads", default="config2,config3_slice")
    ap.add_argument("--write", action="store_true",
                    help="also write the records to oracle/calibration.json (read by bench.py's "
                         "cpu_baseline leg on the GPU box, where the reference is not run)")
    args = ap.parse_args()
    if om.ref_module() is None:
        print("oracle/_ref is not built: run `make -C oracle ref`", file=sys.stderr)
        return 2
    threads = int(om.lib().oracle_num_threads())
    records = []
    for name in args.workloads.split(","):
        bins, y, era, kw = config2() if name == "config2" else config3_slice()
        res = {}
        for splitter in ("restated", "reference"):
            r, sec, wall = time_fit(bins, y, era, kw, args.rounds, splitter)
            res[splitter] = (r, sec)
            print(f"[calibrate] {name} {splitter}: {sec:.3f} s/round (wall {wall:.1f} s)",
                  file=sys.stderr, flush=True)
        (ra, sa), (rb, sb) = res["restated"], res["reference"]
        same = all(np.array_equal(a[k], b[k]) for a, b in zip(ra.rounds, rb.rounds) for k in a)
        rec = {
            "workload": name, "rows": int(bins.shape[0]), "features": int(bins.shape[1]),
            "rounds": args.rounds, "omp_threads": threads, "torch_threads": torch.get_num_threads(),
            "restated_s_per_round": round(sa, 4), "reference_s_per_round": round(sb, 4),
            "reference_over_restated": round(sb / sa, 3), "identical_trees": bool(same),
            "cpu": os.popen("lscpu | grep 'Model name'").read().split(":", 1)[-1].strip(),
        }
        records.append(rec)
        print(json.dumps(rec), flush=True)
    if args.write:
        path = ROOT / "oracle" / "calibration.json"
        path.write_text(json.dumps(records, indent=1) + "\n")
        print(f"wrote {path}", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
