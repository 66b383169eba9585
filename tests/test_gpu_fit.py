"""End-to-end parity of PackBoost.fit / predict on the HIP backend against the oracle's
restatement of the reference's native-CPU fit (booster.py:375-599 + frontier_cpu.cpp).

Bars: tree structure (feature, threshold, is_leaf, child ids) identical; leaf values and
training predictions within 1e-5 (abs, plus 1e-5 relative on values); predict() within 1e-5
of the oracle's per-tree accumulation; leaf indices bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def config1_data(seed=42, n=10_000, f=20, eras=10):
    """y = 5 random-weight features + 0.5 sin(x0) + N(0, 0.1)."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, f)).astype(np.float32)
    idx = rng.choice(f, 5, replace=False)
    w = rng.standard_normal(5).astype(np.float32)
    y = (X[:, idx] @ w + 0.5 * np.sin(X[:, 0]) + 0.1 * rng.standard_normal(n)).astype(np.float32)
    era = np.repeat(np.arange(eras), n // eras).astype(np.int16)
    return X, y, era


def _compare_rounds(gpu_rounds, ref_rounds):
    assert len(gpu_rounds) == len(ref_rounds)
    for r, (a, b) in enumerate(zip(gpu_rounds, ref_rounds)):
        for key in ("feature", "threshold", "left", "right", "is_leaf"):
            np.testing.assert_array_equal(np.asarray(a[key]), np.asarray(b[key]),
                                          err_msg=f"round {r} {key}")
        va, vb = np.asarray(a["value"], np.float64), np.asarray(b["value"], np.float64)
        np.testing.assert_allclose(va, vb, rtol=1e-5, atol=1e-5, err_msg=f"round {r} value")


@pytest.mark.parametrize("cfg_kw", [
    dict(pack_size=8, max_depth=5, learning_rate=0.05, lambda_l2=1.0, lambda_dro=0.5,
         min_samples_leaf=20, max_bins=128, random_state=42),
    dict(pack_size=3, max_depth=4, learning_rate=0.1, lambda_l2=1e-3, lambda_dro=0.1,
         direction_weight=0.05, min_samples_leaf=8, max_bins=63, layer_feature_fraction=0.6,
         era_alpha=1.5, random_state=7),
], ids=["config1", "dir_alpha"])
def test_fit_matches_oracle(hip, oracle_mod, cfg_kw):
    """BASELINE config 1 over its 20 rounds (and a direction + era-weight variant): trees
    identical (or parted at an asserted near-tie), values, training predictions and predict()
    within 1e-5, leaf indices bit-exact (tests.helpers.live_fit_parity)."""
    import torch
    from packboost_amd import PackBoost, PackBoostConfig
    from packboost_amd.data import preprocess_features
    from tests.helpers import live_fit_parity

    X, y, era = config1_data()
    rounds = 20
    print(f"[fit parity] {cfg_kw}", flush=True)
    cfg = PackBoostConfig(**cfg_kw)
    bins = preprocess_features(X, cfg.max_bins).bins
    model, ref, matched, bar = live_fit_parity(
        oracle_mod, lambda n: PackBoost(cfg).fit(X, y, era, num_rounds=n), bins, y, era.astype(np.int64),
        dict(cfg_kw), rounds)
    dev = model if matched == rounds else PackBoost(cfg).fit(X, y, era, num_rounds=matched)
    pred = dev.predict(X)
    ref_pred = oracle_mod.predict(ref.rounds[:matched], cfg.pack_size, cfg.learning_rate, bins)
    assert np.all(np.abs(pred.astype(np.float64) - ref_pred) <= bar)
    for r in range(matched):
        np.testing.assert_array_equal(oracle_mod.leaf_index(model._rounds[r], bins),
                                      oracle_mod.leaf_index(ref.rounds[r], bins))
    # model format: B identical Tree objects per round
    assert len(model.trees) == rounds * cfg.pack_size
    t0 = model.trees[0]
    assert [n.feature for n in t0.nodes] == list(ref.rounds[0]["feature"])
    # per-tree GPU predict_bins: traversal bit-exact against the CPU walk of the same tree,
    # values within tolerance of the oracle's tree (its leaf sums are taken in row order)
    v = t0.predict_bins(torch.from_numpy(bins)).cpu().numpy()
    np.testing.assert_array_equal(v, oracle_mod.predict_tree(model._rounds[0], bins))
    np.testing.assert_allclose(v, oracle_mod.predict_tree(ref.rounds[0], bins), rtol=1e-5, atol=1e-6)


def test_fit_determinism(hip):
    from packboost_amd import PackBoost, PackBoostConfig

    X, y, era = config1_data(seed=3, n=4000, f=12, eras=8)
    cfg = PackBoostConfig(pack_size=2, max_depth=4, learning_rate=0.15, min_samples_leaf=8,
                          max_bins=63, random_state=19)
    a = PackBoost(cfg).fit(X, y, era, num_rounds=3)
    b = PackBoost(cfg).fit(X, y, era, num_rounds=3)
    for ta, tb in zip(a.trees, b.trees):
        assert [(n.feature, n.threshold, n.is_leaf, n.value) for n in ta.nodes] == \
               [(n.feature, n.threshold, n.is_leaf, n.value) for n in tb.nodes]


def test_unsorted_eras_and_no_eras(hip, oracle_mod):
    """Interleaved era labels (rows permuted era-major inside fit) and era=None."""
    from packboost_amd import PackBoost, PackBoostConfig
    from packboost_amd.data import encode_eras, preprocess_features

    rng = np.random.default_rng(5)
    X, y, _ = config1_data(seed=5, n=3000, f=10, eras=6)
    era = rng.integers(0, 6, size=3000).astype(np.int16) * 3 + 100  # non-contiguous labels
    cfg_kw = dict(pack_size=2, max_depth=3, learning_rate=0.1, min_samples_leaf=10, max_bins=32,
                  lambda_dro=0.3, random_state=11)
    cfg = PackBoostConfig(**cfg_kw)
    bins = preprocess_features(X, cfg.max_bins).bins
    for e in (era, None):
        model = PackBoost(cfg).fit(X, y, e, num_rounds=4)
        codes = encode_eras(e, 3000)[0].astype(np.int64)
        ref = oracle_mod.fit(bins, y, codes, num_rounds=4, **cfg_kw)
        _compare_rounds(model._rounds, ref.rounds)
        pred = model.predict(X)
        np.testing.assert_allclose(pred, oracle_mod.predict(ref.rounds, 2, 0.1, bins), atol=1e-5)


@pytest.mark.parametrize("msl", [150, 2000], ids=["early_stop", "root_leaf"])
def test_early_stopping_rounds(hip, oracle_mod, msl):
    """Trees that stop before max_depth make the reference draw fewer feature subsets
    (booster.py:516-519): the pipelined round loop must rewind its generator and redo the
    round it enqueued ahead. msl=2000 > N/2 leaves every tree a single root leaf."""
    from packboost_amd import PackBoost, PackBoostConfig
    from packboost_amd.data import preprocess_features

    X, y, era = config1_data(seed=9, n=3000, f=16, eras=5)
    cfg_kw = dict(pack_size=4, max_depth=6, learning_rate=0.1, min_samples_leaf=msl, max_bins=31,
                  lambda_dro=0.2, layer_feature_fraction=0.5, random_state=23)
    print(f"[early stop] msl={msl}", flush=True)
    cfg = PackBoostConfig(**cfg_kw)
    model = PackBoost(cfg).fit(X, y, era, num_rounds=6)
    bins = preprocess_features(X, cfg.max_bins).bins
    ref = oracle_mod.fit(bins, y, era.astype(np.int64), num_rounds=6, **cfg_kw)
    _compare_rounds(model._rounds, ref.rounds)
    np.testing.assert_allclose(model._train_preds.cpu().numpy(), ref.preds, atol=1e-5, rtol=0)
    if msl == 150:
        assert max(int(np.count_nonzero(~np.asarray(r["is_leaf"]))) for r in ref.rounds) > 0
        assert all(int(np.count_nonzero(~np.asarray(r["is_leaf"]))) < 63 for r in ref.rounds)


def test_profile_modes(hip):
    """pb_profile_enable: mode 2 times the histogram launches only, mode 1 every phase; the
    events change no result (same trees as an unprofiled run)."""
    import ctypes

    import torch
    from packboost_amd import PackBoostConfig
    from packboost_amd.backends import _hip
    from packboost_amd.data import preprocess_features
    from packboost_amd.engine import DeviceFit, tree_arrays_from_log

    X, y, era = config1_data(seed=4, n=4096, f=12, eras=4)
    cfg = PackBoostConfig(pack_size=2, max_depth=4, learning_rate=0.1, min_samples_leaf=8,
                          max_bins=31, random_state=3, prebinned=True)
    bins = preprocess_features(X, cfg.max_bins).bins
    dev = torch.device("cuda")
    bins_fm = torch.from_numpy(np.ascontiguousarray(bins.T)).to(dev)
    off = np.array([0, 1024, 2048, 3072, 4096], np.int32)
    D, P = cfg.max_depth, _hip.PB_MAX_DEPTH

    def run(every, mode):
        fit = DeviceFit(bins_fm, 4096, torch.from_numpy(y).to(dev), off, cfg)
        trees = [tree_arrays_from_log(log, cfg, 4096)
                 for log, _, _ in fit.rounds(torch.Generator().manual_seed(1), 5,
                                             profile_every=every, profile_mode=mode)]
        torch.cuda.synchronize()
        ms = np.zeros(4 * P, np.float64)
        n = np.zeros(4 * P, np.int64)
        _hip.check(fit.lib.pb_profile_read(fit.ctx, ms.ctypes.data, n.ctypes.data), "read")
        assert fit.lib.pb_profile_enable(fit.ctx, 3) < 0  # modes are 0, 1, 2
        fit.close()
        return trees, ms.reshape(4, P)[:, :D], n.reshape(4, P)[:, :D]

    base, _, n0 = run(0, 0)
    assert n0.sum() == 0
    hist_only, ms2, n2 = run(2, 2)
    all_ph, ms1, n1 = run(1, 1)
    assert n2[0, 0] == 3 and n2[1:].sum() == 0  # rounds 0, 2, 4
    assert (ms2[0][n2[0] > 0] > 0).all()
    assert n1[0, 0] == 5 and (n1[:, 0] == 5).all() and (ms1[:, 0] > 0).all()
    for a, b, c in zip(base, hist_only, all_ph):
        for key in ("feature", "threshold", "left", "right", "is_leaf", "value"):
            np.testing.assert_array_equal(np.asarray(a[key]), np.asarray(b[key]))
            np.testing.assert_array_equal(np.asarray(a[key]), np.asarray(c[key]))
