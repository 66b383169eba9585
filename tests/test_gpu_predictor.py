"""PackBoostPredictor and PackBoostRegressor on the HIP device: a saved-and-loaded bundle
predicts bit-identically to the trainer's predict(), per-tree leaves match the CPU walk of
the same trees, and the wrapper reproduces PackBoost.fit/predict."""

from __future__ import annotations

import numpy as np
import pytest

from tests.test_fit_golden import load_case

pytestmark = pytest.mark.gpu


def test_predictor_matches_trainer(hip, oracle_mod, tmp_path):
    from packboost_amd import PackBoost, PackBoostConfig, PackBoostPredictor
    from packboost_amd.data import apply_bins

    d = load_case("fit_config1")
    cfg = PackBoostConfig(**d["config"])
    print("[predictor] fit_config1", flush=True)
    model = PackBoost(cfg).fit(d["X"], d["y"], d["era"], num_rounds=d["rounds"])
    want = model.predict(d["X"])
    path = model.save(tmp_path / "m.npz")
    pred = PackBoostPredictor.load(path)
    np.testing.assert_array_equal(pred.predict(d["X"]), want)
    np.testing.assert_array_equal(PackBoostPredictor(model).predict(d["X"]), want)
    # new rows through the stored bin edges
    X2 = np.random.default_rng(3).standard_normal((777, d["X"].shape[1])).astype(np.float32)
    np.testing.assert_array_equal(pred.predict(X2), model.predict(X2))
    leaves = pred.predict_leaves(d["X"])
    bins = apply_bins(d["X"], model._binner.bin_edges, cfg.max_bins)
    assert leaves.shape == (pred.num_trees, d["X"].shape[0])
    for r, arrs in enumerate(model._rounds):
        want_leaf = oracle_mod.leaf_index(arrs, bins)
        for t in range(cfg.pack_size):
            np.testing.assert_array_equal(leaves[r * cfg.pack_size + t], want_leaf)
    with pytest.raises(ValueError):
        pred.predict(d["X"][:, :5])


def test_regressor_matches_packboost(hip):
    from packboost_amd import PackBoost, PackBoostConfig, PackBoostRegressor

    d = load_case("fit_dir_alpha")
    cfg = d["config"]
    print("[regressor] fit_dir_alpha", flush=True)
    reg = PackBoostRegressor(num_rounds=d["rounds"], **cfg).fit(d["X"], d["y"], era=d["era"])
    model = PackBoost(PackBoostConfig(**cfg)).fit(d["X"], d["y"], d["era"], num_rounds=d["rounds"])
    np.testing.assert_array_equal(reg.predict(d["X"]), model.predict(d["X"]))
    assert reg.score(d["X"], d["y"]) > 0.0
    assert len(reg.round_metrics) == d["rounds"]
    np.testing.assert_array_equal(reg.to_predictor().predict(d["X"]), model.predict(d["X"]))
