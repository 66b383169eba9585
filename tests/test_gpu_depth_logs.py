"""The per-depth instrumentation contract (booster.py:220-270, 565-579) on the HIP fit.

The reference fills a DepthInstrumentation per depth (nodes processed / skipped / collapsed,
rows, phase milliseconds, histogram-mode counters) and its tests pin the accounting invariant
(tests/test_packboost_parity.py:67-87). Here: the same key set, node and row counts equal to
the oracle's restatement of the reference fit, the invariant in all three histogram modes, and
phase times that are measured in a default fit (every 8th round timed, the others carrying the
last timed round's values and naming it) and in every round with phase timing on, without
changing the fit.
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REFERENCE_KEYS = {
    "nodes_processed", "nodes_skipped", "rows_total", "feature_blocks", "bincount_calls",
    "hist_ms", "scan_ms", "score_ms", "partition_ms", "nodes_subtract_ok", "nodes_rebuild",
    "nodes_subtract_fallback", "nodes_collapsed", "feature_block_size", "depth",
    "feature_subset_size", "pack_size", "layer_feature_fraction", "histogram_mode", "seed",
    "torch_threads",
}
# keys this build adds: the round the *_ms values were measured on, and that the prefix scan is
# timed inside hist_ms
EXTRA_KEYS = {"phase_ms_round", "scan_fused"}


def _dataset(seed=123, n_rows=320, n_features=12, n_eras=8):
    """The shape of the reference parity tests' dataset (tests/test_packboost_parity.py:8-15):
    N(0, 1) features, a linear target plus noise, shuffled era labels."""
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n_rows, n_features)).astype(np.float32)
    coefs = rng.normal(size=n_features).astype(np.float32)
    y = (X @ coefs + 0.1 * rng.standard_normal(n_rows)).astype(np.float32)
    eras = np.arange(n_rows, dtype=np.int16) % n_eras
    rng.shuffle(eras)
    return X, y, eras


@pytest.mark.parametrize("hist_mode", ["auto", "subtract", "rebuild"])
def test_depth_log_accounting(hip, oracle_mod, hist_mode):
    from packboost_amd import PackBoost, PackBoostConfig
    from packboost_amd.data import encode_eras, preprocess_features

    X, y, eras = _dataset()
    kw = dict(pack_size=2, max_depth=3, learning_rate=0.1, min_samples_leaf=6, max_bins=63,
              random_state=5)
    booster = PackBoost(PackBoostConfig(histogram_mode=hist_mode, **kw))
    booster.fit(X, y, eras, num_rounds=2)
    logs = booster._depth_logs
    assert logs
    for dl in logs:
        assert set(dl) == REFERENCE_KEYS | EXTRA_KEYS
        n = dl["nodes_processed"]
        assert dl["nodes_subtract_ok"] + dl["nodes_rebuild"] == n
        if hist_mode == "rebuild":
            assert dl["nodes_subtract_ok"] == 0
        else:
            assert dl["nodes_subtract_ok"] >= 0
            assert dl["nodes_subtract_fallback"] <= dl["nodes_rebuild"]
        assert dl["histogram_mode"] == hist_mode
        # a default fit times round 1 (then every 8th): both rounds report round 1's times
        assert dl["phase_ms_round"] == 1
        assert dl["hist_ms"] > 0.0 and dl["score_ms"] > 0.0 and dl["partition_ms"] > 0.0
        assert dl["scan_ms"] == 0.0 and dl["scan_fused"]
    bins = preprocess_features(X, 63).bins
    codes = encode_eras(eras, X.shape[0])[0].astype(np.int64)
    ref = oracle_mod.fit(bins, y, codes, num_rounds=2, **kw)
    got = [(dl["depth"], dl["nodes_processed"], dl["nodes_collapsed"], dl["rows_total"]) for dl in logs]
    exp = [(r["depth"], r["nodes_processed"], r["nodes_collapsed"], r["rows_total"]) for r in ref.depth_logs]
    assert got == exp


def test_depth_log_phase_times(hip):
    """With phase timing on, every processed depth reports GPU milliseconds for its histogram,
    score and partition launches, and the fit is the same as the pipelined one."""
    from packboost_amd import PackBoost, PackBoostConfig

    X, y, eras = _dataset(seed=7, n_rows=4000, n_features=10)
    cfg = PackBoostConfig(pack_size=2, max_depth=4, learning_rate=0.1, min_samples_leaf=8,
                          max_bins=32, random_state=3)
    plain = PackBoost(cfg).fit(X, y, eras, num_rounds=3)
    timed = PackBoost(cfg)
    timed.profile_phases = True
    timed.fit(X, y, eras, num_rounds=3)
    assert len(timed._depth_logs) == len(plain._depth_logs)
    for a, b in zip(timed._depth_logs, plain._depth_logs):
        for key in ("depth", "nodes_processed", "nodes_collapsed", "rows_total"):
            assert a[key] == b[key]
        assert a["hist_ms"] > 0.0 and a["score_ms"] > 0.0 and a["partition_ms"] > 0.0
        assert a["scan_ms"] == 0.0  # the prefix scan is part of the histogram kernel
    # every round timed: each log names its own round; the default fit times rounds 1 and 9
    # here only round 1 (3 rounds), and the later rounds carry its values
    per_round = {}
    for a in timed._depth_logs:
        per_round.setdefault(a["phase_ms_round"], []).append(a)
    assert sorted(per_round) == [1, 2, 3]
    first = {b["depth"]: b for b in plain._depth_logs[: len(per_round[1])]}
    for b in plain._depth_logs:
        assert b["phase_ms_round"] == 1
        assert b["hist_ms"] == first[b["depth"]]["hist_ms"]
    for ra, rb in zip(timed._rounds, plain._rounds):
        for key in ("feature", "threshold", "left", "right", "is_leaf"):
            np.testing.assert_array_equal(ra[key], rb[key])
        np.testing.assert_array_equal(np.asarray(ra["value"]), np.asarray(rb["value"]))
    np.testing.assert_array_equal(timed.predict(X), plain.predict(X))
