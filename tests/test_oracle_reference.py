"""Pins the oracle to the reference itself: oracle/_ref holds the reference's own
frontier_cpu.cpp + bindings.cpp compiled from /root/reference by oracle/Makefile (`make ref`).
On seeded random batches the restated split finder must return bit-identical decisions
(feature, threshold, score, grad/hess sums, counts) and partitions.
"""

from __future__ import annotations

import glob
import importlib.util
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def _load_ref():
    hits = glob.glob(str(ROOT / "oracle" / "_ref" / "_backend*.so"))
    if not hits:
        pytest.skip("oracle/_ref is not built (needs /root/reference; `make -C oracle ref`)")
    spec = importlib.util.spec_from_file_location("_backend", hits[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


CASES = [
    # seed, N, F, E, nb, U, K, k_cuts, cut, msl, lam, dro, dir_w, alpha
    (1, 3000, 10, 5, 5, 1, 10, 0, "mass", 20, 1e-6, 0.5, 0.0, 0.0),
    (2, 5000, 16, 9, 64, 4, 7, 0, "mass", 10, 1.0, 0.5, 0.0, 0.0),
    (3, 4000, 12, 7, 128, 6, 12, 0, "mass", 5, 1e-3, 0.1, 0.2, 1.5),
    (4, 4000, 12, 7, 32, 3, 12, 5, "mass", 5, 1e-3, 0.1, 0.0, 0.0),
    (5, 4000, 12, 7, 32, 3, 12, 6, "even", 5, 1e-3, 0.1, 0.0, 0.0),
    (6, 2000, 6, 3, 2, 2, 6, 0, "mass", 1, 0.5, 0.0, 0.0, 0.0),
]


@pytest.mark.parametrize("case", CASES, ids=[f"case{c[0]}" for c in CASES])
def test_oracle_matches_reference_cpu(oracle_mod, case):
    from tests.helpers import make_problem

    seed, N, F, E, nb, U, K, kc, cut, msl, lam, dro, dw, alpha = case
    p = make_problem(seed, N, F, E, nb, U, empty_era=(seed % 2 == 0))
    _compare(oracle_mod, p, case)


SKIP_CASES = [
    # bins >= max_bins: skipped in the histogram, sent right (frontier_cpu.cpp:278-281, 464-470)
    (11, 3000, 8, 5, 5, 2, 8, 0, "mass", 10, 1e-6, 0.5, 0.0, 0.0),
    (12, 4000, 10, 7, 32, 3, 10, 6, "mass", 5, 1e-3, 0.1, 0.0, 0.0),
    (13, 4000, 10, 7, 16, 3, 10, 0, "mass", 5, 1e-3, 0.1, 0.2, 1.5),
]


@pytest.mark.parametrize("case", SKIP_CASES, ids=[f"case{c[0]}" for c in SKIP_CASES])
def test_oracle_matches_reference_with_skipped_bins(oracle_mod, case):
    from tests.helpers import make_problem, with_skipped_bins

    seed, N, F, E, nb, U, K, kc, cut, msl, lam, dro, dw, alpha = case
    p = with_skipped_bins(make_problem(seed, N, F, E, nb, U, empty_era=True), seed)
    assert int(p["bins"].max()) >= nb
    _compare(oracle_mod, p, case)


def _compare(oracle_mod, p, case):
    ref = _load_ref()
    from tests.helpers import node_era_rows

    seed, N, F, E, nb, U, K, kc, cut, msl, lam, dro, dw, alpha = case
    feats = np.random.default_rng(seed).permutation(F)[:K].astype(np.int32)
    ner = node_era_rows(p)
    got = oracle_mod.split_batch(p["bins"], p["grad"], ner, feats, nb, kc, cut, lam, dro, dw, alpha, msl)
    decs, stats = ref.find_best_splits_batched_cpu(
        p["bins"].view(np.int8), p["grad"], [[r for r in eras] for eras in ner], feats, nb, kc, cut,
        lam, dro, dw, alpha, msl)
    assert len(decs) == U
    pos = 0
    for u, d in enumerate(decs):
        n_rows = sum(r.size for r in ner[u])
        gl = got.go_left[pos: pos + n_rows].astype(bool)
        pos += n_rows
        if d is None:
            assert got.feature[u] == -1
            continue
        assert (got.feature[u], got.threshold[u]) == (d["feature"], d["threshold"])
        for key in ("score", "left_grad", "left_hess", "right_grad", "right_hess"):
            assert np.float32(getattr(got, key)[u]).view(np.uint32) == np.float32(d[key]).view(np.uint32), key
        assert got.left_count[u] == d["left_count"] and got.right_count[u] == d["right_count"]
        off = 0
        for e, r in enumerate(ner[u]):
            sel = gl[off: off + r.size]
            off += r.size
            np.testing.assert_array_equal(r[sel], np.asarray(d["left_rows"][e]))
            np.testing.assert_array_equal(r[~sel], np.asarray(d["right_rows"][e]))
