"""Round metrics on the device (pb_era_corr) against the reference's era correlation
(PackBoost._era_correlation_np, booster.py:909-929), computed here in float64 NumPy.

Bars: per-era and mean correlations within 1e-9 (both sides in double) on data with empty,
single-row and constant eras; the fit's train metric within 1e-5 of the NumPy metric of
predict() (the fit's running predictions and predict() sum trees in different orders); the
eval metric within 1e-9 of the NumPy metric of the oracle's tree-order float32 sum, the order
in which the eval predictions accumulate."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def era_corr_np(era, y, p):
    """The reference's metric (booster.py:909-929) in float64."""
    cors = []
    for e in np.unique(era):
        m = era == e
        yy, pp = y[m].astype(np.float64), p[m].astype(np.float64)
        if yy.size < 2:
            continue
        sy, sp = yy.std(), pp.std()
        if sy <= 1e-12 or sp <= 1e-12:
            continue
        c = float(((yy - yy.mean()) * (pp - pp.mean())).mean()) / (sy * sp)
        if np.isfinite(c):
            cors.append(c)
    return float(np.mean(cors)) if cors else float("nan")


def test_era_corr_kernel(hip):
    import torch

    rng = np.random.default_rng(0)
    sizes = [500, 0, 1, 300, 40, 1000, 2, 700]
    E = len(sizes)
    era = np.repeat(np.arange(E), sizes)
    N = era.size
    y = rng.standard_normal(N).astype(np.float32)
    p = (0.3 * y + rng.standard_normal(N)).astype(np.float32)
    y[era == 4] = 1.25  # constant target: skipped
    offs = np.zeros(E + 1, np.int32)
    offs[1:] = np.cumsum(sizes)
    dev = torch.device("cuda")
    yd, pd_ = torch.from_numpy(y).to(dev), torch.from_numpy(p).to(dev)
    od = torch.from_numpy(offs).to(dev)
    scratch = torch.empty(E + 1, dtype=torch.float64, device=dev)
    lib = hip.load()
    hip.check(lib.pb_era_corr(yd.data_ptr(), pd_.data_ptr(), od.data_ptr(), E, scratch.data_ptr(),
                              scratch.data_ptr() + 8 * E, hip.stream_ptr()), "pb_era_corr")
    got = scratch.cpu().numpy()
    for e in range(E):
        want = era_corr_np(np.zeros(sizes[e]), y[era == e], p[era == e])
        if np.isnan(want):
            assert np.isnan(got[e]), e
        else:
            assert abs(got[e] - want) <= 1e-9, (e, got[e], want)
    assert abs(got[E] - era_corr_np(era, y, p)) <= 1e-9
    # no era counts -> NaN
    hip.check(lib.pb_era_corr(yd.data_ptr(), yd.data_ptr(), od[2:4].data_ptr(), 1, scratch.data_ptr(),
                              scratch.data_ptr() + 8, hip.stream_ptr()), "pb_era_corr")
    assert np.isnan(scratch[1].item())


def test_fit_round_metrics(hip):
    from packboost_amd import PackBoost, PackBoostConfig
    from tests.test_fit_golden import load_case

    d = load_case("fit_dir_alpha")  # interleaved era labels
    rng = np.random.default_rng(1)
    X2 = rng.standard_normal((900, d["X"].shape[1])).astype(np.float32)
    y2 = (X2[:, 0] + 0.1 * rng.standard_normal(900)).astype(np.float32)
    era2 = rng.integers(0, 7, size=900) * 5
    print("[round metrics]", flush=True)
    model = PackBoost(PackBoostConfig(**d["config"])).fit(
        d["X"], d["y"], d["era"], num_rounds=d["rounds"], eval_sets=[("valid", X2, y2, era2)])
    m = model.round_metrics[-1]
    assert m["round"] == d["rounds"]
    assert abs(m["train_corr"] - era_corr_np(d["era"], d["y"], model.predict(d["X"]))) <= 1e-5
    # the eval predictions accumulate float32(w * leaf) tree by tree, the reference's eval and
    # CPU predict order (booster.py:604-655, 709-712): the metric is exact on that sum
    from oracle import oracle as om
    from packboost_amd.data import apply_bins

    bins2 = apply_bins(X2, model._binner.bin_edges, model.config.max_bins)
    p_eval = om.predict(model._rounds, model.config.pack_size, model._tree_weight, bins2)
    assert abs(m["valid_corr"] - era_corr_np(era2, y2, p_eval)) <= 1e-9
    # PackBoost.predict (the compiled forest's double sums, rounded once) within 1e-5 of it
    np.testing.assert_allclose(model.predict(X2), p_eval, rtol=0, atol=1e-5)
    assert all(np.isfinite(r["train_corr"]) for r in model.round_metrics)
