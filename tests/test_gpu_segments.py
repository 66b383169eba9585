"""Segment mode (pb_set_segment_mode): rows sorted by frontier node, one fused histogram +
DES kernel per depth from a first fused depth on (the plane path before it) and a stable row
partition between depths, against the plane path of the same fit. The candidates are the plane
scorer's bit for bit, so the whole fit must agree exactly: every tree (features, thresholds,
children, leaf values), the training predictions after every round and the round metrics.
Covers first fused depths 0, 2, 3 and none (the sorted order tracked from the caller's columns
throughout), 255 and 64 bins, an era without rows, nodes that stop splitting
(min_samples_leaf), the direction term, era weights and DRO, and a root too small to split."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _data(seed, N, F, E, empty_era=False):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((N, F)).astype(np.float32)
    w = rng.standard_normal(F).astype(np.float32)
    y = (X @ w * 0.3 + np.tanh(X[:, 0] * X[:, 1]) + 0.5 * rng.standard_normal(N)).astype(np.float32)
    sizes = rng.integers(1, 10, size=E).astype(np.float64)
    if empty_era:
        sizes[E // 2] = 0
    era = np.repeat(np.arange(E), np.floor(sizes / sizes.sum() * N).astype(np.int64))
    era = np.concatenate([era, np.full(N - era.size, E - 1)])
    return X, y, rng.permutation(era)


def _fit(mode, monkeypatch, X, y, era, rounds, from_depth=0, **kw):
    from packboost_amd import PackBoost, PackBoostConfig

    monkeypatch.setenv("PB_FIT_MODE", mode)
    monkeypatch.setenv("PB_SEG_FROM_DEPTH", str(from_depth))
    model = PackBoost(PackBoostConfig(**kw)).fit(X, y, era, num_rounds=rounds)
    assert model._fit_mode == mode
    return model


@pytest.mark.parametrize("case", [
    # seed, N, F, E, nb, D, B, msl, dro, dir, alpha, empty_era, rounds
    (1, 20000, 24, 12, 255, 6, 4, 20, 0.0, 0.0, 0.0, False, 4),
    (2, 12000, 16, 7, 64, 5, 2, 40, 0.5, 0.2, 1.5, True, 4),
    (3, 6000, 10, 5, 255, 7, 1, 10, 0.3, 0.0, 0.0, False, 3),
], ids=["nb255_d6", "nb64_dir_alpha_dro_empty_era", "nb255_d7_small_nodes"])
def test_segments_match_planes(hip, monkeypatch, case):
    seed, N, F, E, nb, D, B, msl, dro, dirw, alpha, empty, rounds = case
    print(f"[segments] {case}", flush=True)
    X, y, era = _data(seed, N, F, E, empty)
    kw = dict(pack_size=B, max_depth=D, learning_rate=0.2, min_samples_leaf=msl, max_bins=nb,
              lambda_dro=dro, direction_weight=dirw, era_alpha=alpha, random_state=seed)
    planes = _fit("planes", monkeypatch, X, y, era, rounds, **kw)
    for from_depth in (0, 2, 3, D):
        print(f"[segments] first fused depth {from_depth}", flush=True)
        seg = _fit("segments", monkeypatch, X, y, era, rounds, from_depth, **kw)
        assert len(seg._rounds) == len(planes._rounds) == rounds
        for r, (a, b) in enumerate(zip(seg._rounds, planes._rounds)):
            for key in ("feature", "threshold", "left", "right", "is_leaf", "value"):
                np.testing.assert_array_equal(np.asarray(a[key]), np.asarray(b[key]),
                                              err_msg=f"from {from_depth} round {r} {key}")
        np.testing.assert_array_equal(seg._train_preds.cpu().numpy(), planes._train_preds.cpu().numpy())
        for ma, mb in zip(seg.round_metrics, planes.round_metrics):
            assert ma["train_corr"] == mb["train_corr"]
        np.testing.assert_array_equal(seg.predict(X[:500]), planes.predict(X[:500]))


def test_segments_root_too_small(hip, monkeypatch):
    X, y, era = _data(5, 300, 6, 3)
    kw = dict(pack_size=2, max_depth=4, learning_rate=0.1, min_samples_leaf=200, max_bins=255, random_state=1)
    planes = _fit("planes", monkeypatch, X, y, era, 2, **kw)
    for from_depth in (0, 2):
        seg = _fit("segments", monkeypatch, X, y, era, 2, from_depth, **kw)
        for a, b in zip(seg._rounds, planes._rounds):
            np.testing.assert_array_equal(np.asarray(a["value"]), np.asarray(b["value"]))
        np.testing.assert_array_equal(seg._train_preds.cpu().numpy(), planes._train_preds.cpu().numpy())


def test_segments_refuse_k_cuts(hip, monkeypatch):
    X, y, era = _data(6, 2000, 6, 3)
    with pytest.raises(ValueError, match="segments"):
        _fit("segments", monkeypatch, X, y, era, 1, pack_size=1, max_depth=3, max_bins=255, k_cuts=8,
             min_samples_leaf=10, random_state=1)


def test_segments_many_eras(hip, monkeypatch):
    """5000 eras, more than the 4096 entries of the 1/n table: past the table the fused kernel's
    Welford factor falls back to IEEE division, as the wide scorer's does."""
    X, y, era = _data(7, 100_000, 8, 5000)
    assert np.unique(era).size > 4096
    kw = dict(pack_size=2, max_depth=4, learning_rate=0.2, min_samples_leaf=5, max_bins=128, random_state=3)
    planes = _fit("planes", monkeypatch, X, y, era, 2, **kw)
    for from_depth in (0, 2):
        seg = _fit("segments", monkeypatch, X, y, era, 2, from_depth, **kw)
        for r, (a, b) in enumerate(zip(seg._rounds, planes._rounds)):
            for key in ("feature", "threshold", "value"):
                np.testing.assert_array_equal(np.asarray(a[key]), np.asarray(b[key]),
                                              err_msg=f"from {from_depth} round {r} {key}")
        np.testing.assert_array_equal(seg._train_preds.cpu().numpy(), planes._train_preds.cpu().numpy())


@pytest.mark.parametrize("case", [
    # seed, N, F, E, nb, D, B, msl, dro, dir, alpha, empty_era, rounds
    (11, 20000, 16, 10, 255, 6, 4, 20, 0.3, 0.0, 0.0, False, 4),
    (12, 12000, 12, 7, 64, 5, 2, 30, 0.5, 0.2, 1.5, True, 4),
], ids=["nb255_d6_dro", "nb64_dir_alpha_dro_empty_era"])
def test_segments_match_oracle(hip, oracle_mod, monkeypatch, case):
    """Segment mode fused from depth 0 (every depth's histogram and DES scores from
    seg_score_kernel) against the oracle's restated reference fit directly: trees identical
    or parted at an asserted near-tie, values and training predictions within 1e-5
    (tests.helpers.live_fit_parity)."""
    from packboost_amd.data import encode_eras, preprocess_features
    from tests.helpers import live_fit_parity

    seed, N, F, E, nb, D, B, msl, dro, dirw, alpha, empty, rounds = case
    print(f"[segments vs oracle] {case}", flush=True)
    X, y, era = _data(seed, N, F, E, empty)
    kw = dict(pack_size=B, max_depth=D, learning_rate=0.2, min_samples_leaf=msl, max_bins=nb,
              lambda_dro=dro, direction_weight=dirw, era_alpha=alpha, random_state=seed)
    bins = preprocess_features(X, nb).bins
    codes = encode_eras(era, N)[0].astype(np.int64)
    _, _, matched, _ = live_fit_parity(
        oracle_mod, lambda n: _fit("segments", monkeypatch, X, y, era, n, 0, **kw), bins, y, codes, kw,
        rounds)
    assert matched >= 1
