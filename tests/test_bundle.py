"""Model bundle round trip and the scikit-learn wrapper's parameter protocol, on the CPU.

The bundle is filled from the reference's own fitted trees (tests/golden/fit_config1.npz):
after save -> load, the oracle's CPU predict of the loaded trees must equal the reference's
predict() bit for bit, which pins the bundle's tree arrays, weight and pack size."""

from __future__ import annotations

import numpy as np
import pytest

from tests.test_fit_golden import load_case


def _model_from_golden(name="fit_config1"):
    from packboost_amd import PackBoost, PackBoostConfig
    from packboost_amd.data import BinningResult

    d = load_case(name)
    cfg = PackBoostConfig(**d["config"])
    m = PackBoost(cfg)
    m._rounds = [{k: np.asarray(v) for k, v in t.items()} for t in d["trees"]]
    edges = None
    if bool(d["has_edges"]):
        lens = d["edge_lens"]
        assert np.all(lens == lens[0])
        edges = d["edges"].reshape(len(lens), -1).astype(np.float32)  # [max_bins - 1, F]
    m._binner = BinningResult(bins=d["bins"], bin_edges=edges, prebinned=edges is None)
    m._tree_weight = float(d["tree_weight"])
    m._trained_pack_size = cfg.pack_size
    m._feature_names = [f"f{i}" for i in range(d["X"].shape[1])]
    return m, d


def test_bundle_round_trip(tmp_path, oracle_mod):
    from packboost_amd import load_bundle, save_bundle

    m, d = _model_from_golden()
    path = save_bundle(m, tmp_path / "model")
    assert path.suffix == ".npz"
    b = load_bundle(path)
    assert b["config"] == m.config
    assert b["feature_names"] == m._feature_names
    assert b["tree_weight"] == m._tree_weight and b["pack_size"] == m.config.pack_size
    assert len(b["rounds"]) == len(m._rounds)
    for got, want in zip(b["rounds"], m._rounds):
        for k in ("feature", "threshold", "left", "right", "is_leaf"):
            np.testing.assert_array_equal(got[k], want[k])
        np.testing.assert_array_equal(got["value"], want["value"])
    np.testing.assert_array_equal(b["bin_edges"], m._binner.bin_edges)
    pred = oracle_mod.predict(b["rounds"], b["pack_size"], b["tree_weight"], d["bins"])
    np.testing.assert_array_equal(pred, d["preds"])


def test_bundle_rejects_foreign_and_newer_files(tmp_path):
    from packboost_amd import load_bundle, save_bundle

    np.savez(tmp_path / "x.npz", a=np.zeros(3))
    with pytest.raises(ValueError):
        load_bundle(tmp_path / "x.npz")
    m, _ = _model_from_golden()
    p = save_bundle(m, tmp_path / "m.npz")
    with np.load(p, allow_pickle=False) as z:
        items = {k: z[k] for k in z.files}
    items["version"] = np.array(99)
    np.savez(tmp_path / "new.npz", **items)
    with pytest.raises(ValueError):
        load_bundle(tmp_path / "new.npz")


def test_unfitted_model_cannot_be_saved(tmp_path):
    from packboost_amd import PackBoost, PackBoostConfig, save_bundle

    with pytest.raises(RuntimeError):
        save_bundle(PackBoost(PackBoostConfig()), tmp_path / "m.npz")


def test_regressor_params_protocol():
    from packboost_amd import PackBoostRegressor

    r = PackBoostRegressor(num_rounds=7, pack_size=4, max_depth=3)
    p = r.get_params()
    assert p["num_rounds"] == 7 and p["pack_size"] == 4 and p["max_depth"] == 3
    assert p["learning_rate"] == 0.1  # PackBoostConfig default
    r.set_params(learning_rate=0.05, num_rounds=3)
    assert r.get_params()["learning_rate"] == 0.05 and r.num_rounds == 3
    with pytest.raises(ValueError):
        r.set_params(bogus=1)
    with pytest.raises(TypeError):
        PackBoostRegressor(bogus=1)
    with pytest.raises(RuntimeError):
        r.predict(np.zeros((2, 3)))
    clone = PackBoostRegressor(**r.get_params())
    assert clone.get_params() == r.get_params()
