"""Edge shapes of the HIP path against the oracle: the largest era the 16-bit count field
holds (65535 rows), eras split into segments (up to 100k rows, and a fit without eras), a
thousand eras of 0-5 rows, minimal
shapes (one feature, two bins, depth 1), deep trees whose frontiers need node tiles, and a
255-bin fit.

Bars as in test_gpu_fit / test_gpu_depth: counts bit-exact, grads within 1e-5 of the per-cell
mass; tree structure identical, leaf values and predictions within 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import GpuDepth, make_problem, node_era_rows
from tests.test_gpu_fit import _compare_rounds

pytestmark = pytest.mark.gpu


def _abs_mass(p, U):
    nid = p["nid"].astype(np.int64)
    m = np.zeros((p["E"], U))
    act = nid < U
    np.add.at(m, (p["era"][act], nid[act]), np.abs(p["grad"][act].astype(np.float64)))
    return m


@pytest.mark.parametrize("layout", ["u8", "nibble"])
def test_largest_era(hip, oracle_mod, layout):
    """An era of exactly 65535 rows (all in one node): every count reaches the top of the
    16-bit count field of the LDS addend without carrying into the grad bits."""
    print(f"[largest era] {layout}", flush=True)
    N, F, E, nb, U = 65535 + 1000, 6, 2, 5, 1
    p = make_problem(3, N, F, E, nb, U, ragged=False, inactive_frac=0.0)
    offs = np.array([0, 65535, N], np.int32)
    p["era_off"] = offs
    p["era"] = np.repeat(np.arange(E), np.diff(offs))
    p["bins"][:65535, 0] = 2  # one bin holds the whole era for feature 0
    feats = np.arange(F, dtype=np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb, want_planes=True)
    g = GpuDepth(hip, p, F, msl=1, layout=layout)
    try:
        g.hist(feats)
        cnt, gp = g.planes()
        np.testing.assert_array_equal(cnt, ref.planes[0])
        assert cnt[0, 0, 0, nb - 1] == 65535
        err = np.abs(gp.astype(np.float64) - ref.planes[1].astype(np.float64))
        assert np.all(err <= 1e-5 * np.maximum(_abs_mass(p, U)[:, :, None, None], 1.0))
    finally:
        g.close()


@pytest.mark.parametrize("sizes,nb,U,layout", [
    ((100_000, 7_000), 5, 2, "u8"),           # above the 16-bit count field: 32-bit planes
    ((100_000, 7_000), 5, 2, "nibble"),
    ((20_000, 41_000, 9_000, 16_385), 9, 3, "nibble"),  # split eras, 16-bit planes
    ((70_001,), 200, 2, "u8"),                # one big era, single-feature histograms
], ids=["big-u8", "big-nibble", "split", "one-era-200bins"])
def test_split_eras(hip, oracle_mod, sizes, nb, U, layout):
    """Eras above the segment size are built in parts whose exact sums are added up before the
    planes are written: the planes equal the oracle's whatever the split."""
    print(f"[split eras] {sizes} nb={nb} U={U} {layout}", flush=True)
    N, F, E = int(sum(sizes)), 5, len(sizes)
    p = make_problem(len(sizes) * 7 + nb, N, F, E, nb, U, ragged=False)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    p["era_off"] = offs
    p["era"] = np.repeat(np.arange(E), sizes)
    feats = np.arange(F, dtype=np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb, want_planes=True)
    g = GpuDepth(hip, p, F, msl=1, layout=layout)
    try:
        g.hist(feats)
        cnt, gp = g.planes()
        np.testing.assert_array_equal(cnt, ref.planes[0])
        err = np.abs(gp.astype(np.float64) - ref.planes[1].astype(np.float64))
        assert np.all(err <= 1e-5 * np.maximum(_abs_mass(p, U)[:, :, None, None], 1.0))
        # the split-era sums are cleared for the next build: a second build gives the same planes
        g.hist(feats)
        cnt2, gp2 = g.planes()
        np.testing.assert_array_equal(cnt2, cnt)
        np.testing.assert_array_equal(gp2, gp)
    finally:
        g.close()


def _fit_vs_oracle(oracle_mod, bins, y, era, rounds, **cfg_kw):
    from packboost_amd import PackBoost, PackBoostConfig

    cfg = PackBoostConfig(**cfg_kw, prebinned=True)
    model = PackBoost(cfg).fit(bins, y, era, num_rounds=rounds)
    ref = oracle_mod.fit(bins, y, None if era is None else era.astype(np.int64), num_rounds=rounds,
                         **cfg_kw)
    _compare_rounds(model._rounds, ref.rounds)
    np.testing.assert_allclose(model._train_preds.cpu().numpy(), ref.preds, atol=1e-5, rtol=0)
    return model, ref


def _target(rng, bins, k=3):
    """A linear target in O(1) units (bins scaled to [0, 1]) plus noise."""
    cols = rng.choice(bins.shape[1], size=min(k, bins.shape[1]), replace=False)
    x = bins[:, cols].astype(np.float32) / max(1, int(bins.max()))
    y = x @ rng.standard_normal(len(cols)).astype(np.float32)
    return (y + 0.1 * rng.standard_normal(len(y))).astype(np.float32)


@pytest.mark.parametrize("layout", ["u8", "nibble"])
def test_tiny_eras(hip, oracle_mod, layout):
    """1000 eras of 0-5 rows: era starts fall anywhere inside the 4- and 8-row load groups.
    Planes (counts bit-exact) and partition against the oracle; fits on such data are full of
    exact and near ties, which the parity bar lets flip, so the check stays at one depth."""
    print(f"[tiny eras] {layout}", flush=True)
    p = make_problem(8, 3000, 9, 1000, 7, 3)
    sizes = np.diff(p["era_off"])  # the last era takes the rounding remainder
    assert (sizes[:-1] <= 6).all() and (sizes == 0).any()
    feats = np.arange(9, dtype=np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, 7, want_planes=True,
                                 min_samples_leaf=1)
    g = GpuDepth(hip, p, 9, msl=1, layout=layout)
    try:
        g.hist(feats)
        cnt, gp = g.planes()
        np.testing.assert_array_equal(cnt, ref.planes[0])
        err = np.abs(gp.astype(np.float64) - ref.planes[1].astype(np.float64))
        assert np.all(err <= 1e-5 * np.maximum(_abs_mass(p, 3)[:, :, None, None], 1.0))
    finally:
        g.close()


@pytest.mark.parametrize("F,nb,D", [(1, 2, 1), (1, 2, 3), (2, 3, 2)])
def test_minimal_shapes_fit(hip, oracle_mod, F, nb, D):
    print(f"[minimal] F={F} nb={nb} D={D}", flush=True)
    rng = np.random.default_rng(F * 10 + nb + D)
    N = 800
    bins = rng.integers(0, nb, size=(N, F)).astype(np.int8)
    y = _target(rng, bins, k=F)
    era = np.repeat(np.arange(4), N // 4).astype(np.int16)
    _fit_vs_oracle(oracle_mod, bins, y, era, 3, pack_size=1, max_depth=D, learning_rate=0.3,
                   lambda_l2=1.0, lambda_dro=0.2, min_samples_leaf=5, max_bins=nb, random_state=2)


@pytest.mark.parametrize("nb", [16, 40])
def test_deep_tree_fit(hip, oracle_mod, nb):
    """Depth 9 on 60k rows: frontiers of up to 256 nodes, whose joint-bin (nb 16) or
    single-feature (nb 40) histograms exceed the LDS and run in node tiles. (Leaves of at least
    12 rows and a noisy target keep near-ties, which the parity bar allows to flip, unlikely.)"""
    print(f"[deep] nb={nb}", flush=True)
    rng = np.random.default_rng(nb)
    N, F = 60000, 10
    bins = rng.integers(0, nb, size=(N, F)).astype(np.int8)
    y = (_target(rng, bins, k=6) + 0.3 * rng.standard_normal(N).astype(np.float32)).astype(np.float32)
    era = np.repeat(np.arange(6), N // 6).astype(np.int16)
    model, ref = _fit_vs_oracle(oracle_mod, bins, y, era, 2, pack_size=2, max_depth=9,
                                learning_rate=0.1, lambda_l2=0.1, lambda_dro=0.1,
                                min_samples_leaf=12, max_bins=nb, random_state=6)
    assert max(int(np.count_nonzero(~np.asarray(r["is_leaf"]))) for r in ref.rounds) > 128


def test_deepest_tree_fit(hip, oracle_mod):
    """max_depth 15, the library's limit, on 24k rows with min_samples_leaf 2: frontiers of
    thousands of nodes (node tiles of single features), tree node ids into the tens of
    thousands (uint16 ids), and the last depths' tiny nodes. The tree matches the oracle's
    node for node, or up to its first differing node, which must be a near-tie
    (compare_fit_rounds); depth 16 is refused."""
    from packboost_amd import PackBoost, PackBoostConfig
    from tests.helpers import compare_fit_rounds

    print("[deepest] D=15", flush=True)
    rng = np.random.default_rng(15)
    N, F, nb = 24000, 6, 8
    bins = rng.integers(0, nb, size=(N, F)).astype(np.int8)
    y = (_target(rng, bins, k=4) + 0.5 * rng.standard_normal(N).astype(np.float32)).astype(np.float32)
    era = np.repeat(np.arange(4), N // 4).astype(np.int16)
    kw = dict(pack_size=1, max_depth=15, learning_rate=0.1, lambda_l2=0.5, lambda_dro=0.0,
              min_samples_leaf=2, max_bins=nb, random_state=15)
    model = PackBoost(PackBoostConfig(**kw, prebinned=True)).fit(bins, y, era, num_rounds=1)
    trace: list = []
    ref = oracle_mod.fit(bins, y, era.astype(np.int64), num_rounds=1, trace=trace, **kw)
    sizes = (len(model._rounds[0]["feature"]), len(ref.rounds[0]["feature"]))
    matched, _ = compare_fit_rounds(oracle_mod, model._rounds, ref, trace, bins, kw)
    print(f"[deepest] tree nodes {sizes}, {matched} of 1 rounds identical", flush=True)
    assert min(sizes) > 4000 and max(t["depth"] for t in trace) == 14, sizes
    with pytest.raises(Exception, match="max_depth"):
        PackBoost(PackBoostConfig(max_depth=16, max_bins=nb, prebinned=True)).fit(bins, y, era, num_rounds=1)


def test_fit_without_eras_large(hip, oracle_mod):
    """era=None puts all 150k rows in one era: built in segments, 32-bit counts."""
    print("[no eras, 150k rows]", flush=True)
    rng = np.random.default_rng(15)
    N, F = 150_000, 8
    bins = rng.integers(0, 12, size=(N, F)).astype(np.int8)
    y = (_target(rng, bins, k=4) + 0.3 * rng.standard_normal(N).astype(np.float32)).astype(np.float32)
    _fit_vs_oracle(oracle_mod, bins, y, None, 3, pack_size=2, max_depth=5, learning_rate=0.1,
                   lambda_l2=1.0, lambda_dro=0.0, min_samples_leaf=50, max_bins=12, random_state=3)


def test_255_bins_fit(hip, oracle_mod):
    """Float features quantile-binned into 255 bins on the device (uint8 layout, one feature
    per LDS atomic) against the oracle on NumPy-binned data."""
    from packboost_amd import PackBoost, PackBoostConfig
    from packboost_amd.data import preprocess_features

    print("[255 bins]", flush=True)
    rng = np.random.default_rng(255)
    N, F = 6000, 8
    X = rng.standard_normal((N, F)).astype(np.float32)
    y = (X[:, 0] - 0.5 * X[:, 3] + 0.1 * rng.standard_normal(N)).astype(np.float32)
    era = np.repeat(np.arange(5), N // 5).astype(np.int16)
    kw = dict(pack_size=2, max_depth=4, learning_rate=0.1, lambda_l2=1.0, lambda_dro=0.4,
              min_samples_leaf=10, max_bins=255, random_state=9)
    model = PackBoost(PackBoostConfig(**kw)).fit(X, y, era, num_rounds=3)
    bins = preprocess_features(X, 255).bins
    ref = oracle_mod.fit(bins, y, era.astype(np.int64), num_rounds=3, **kw)
    _compare_rounds(model._rounds, ref.rounds)
    np.testing.assert_allclose(model.predict(X), oracle_mod.predict(ref.rounds, 2, 0.1, bins), atol=1e-5)


@pytest.mark.parametrize("case", ["nan_target", "overflowing_predictions", "root_too_small",
                                  "overflowing_segments"])
def test_nonfinite_gradients_stop_the_fit(hip, monkeypatch, case):
    """Gradients that are not finite have no fixed-point value: the round is flagged on the
    device (pb_round_header.reserved[0]; the per-phase path checks the gradients) and the fit
    raises FloatingPointError instead of growing trees from meaningless histograms (nonfinite
    "raise"), or keeps the finite rounds before it (nonfinite "truncate"). The reference's float
    sums would carry the NaN into its scores instead (tests/test_oracle_nonfinite.py pins what it
    produces). "overflowing_segments" runs the fused segment-mode scorer from depth 0."""
    from packboost_amd import PackBoost, PackBoostConfig

    if case == "overflowing_segments":
        monkeypatch.setenv("PB_FIT_MODE", "segments")
        monkeypatch.setenv("PB_SEG_FROM_DEPTH", "0")

    rng = np.random.default_rng(11)
    N, F = 3000, 6
    X = rng.standard_normal((N, F)).astype(np.float32)
    y = (X[:, 0] + 0.1 * rng.standard_normal(N)).astype(np.float32)
    era = np.repeat(np.arange(6), N // 6)
    kw = dict(max_depth=3, max_bins=16, min_samples_leaf=10, random_state=0)
    if case == "nan_target":
        y[17] = np.nan
        cfg, rounds = PackBoostConfig(pack_size=2, learning_rate=0.1, **kw), 2
    elif case in ("overflowing_predictions", "overflowing_segments"):
        # learning_rate x pack_size = 128: the residuals grow ~127x per round and the
        # predictions pass float32's range within about 20 rounds
        cfg, rounds = PackBoostConfig(pack_size=64, learning_rate=2.0, **kw), 60
    else:  # a root below 2 x min_samples_leaf runs the per-phase path
        y[5] = np.inf
        cfg, rounds = PackBoostConfig(pack_size=2, learning_rate=0.1, **{**kw, "min_samples_leaf": 2000}), 2
    print(f"[nonfinite] {case}", flush=True)
    model = PackBoost(cfg)
    assert model.nonfinite == "raise"
    with pytest.raises(FloatingPointError, match="not finite"):
        model.fit(X, y, era, num_rounds=rounds)
    assert model._fitter is None
    kept = len(model._rounds)  # the rounds before the non-finite one
    assert kept < rounds

    # nonfinite="truncate": a warning, and the fit ends with the same finite rounds
    print(f"[nonfinite] {case} truncate ({kept} finite rounds)", flush=True)
    trunc = PackBoost(cfg, nonfinite="truncate")
    with pytest.warns(RuntimeWarning, match="not finite"):
        trunc.fit(X, y, era, num_rounds=rounds)
    assert trunc._fitter is None and len(trunc._rounds) == kept
    for a, b in zip(model._rounds, trunc._rounds):
        for key in a:
            np.testing.assert_array_equal(a[key], b[key], err_msg=key)
    p = trunc.predict(X)
    assert np.all(np.isfinite(p))
    # the training predictions are the kept trees' (era-major row order)
    order = np.argsort(era, kind="stable")
    np.testing.assert_allclose(trunc._train_preds.cpu().numpy(), p[order], rtol=1e-6,
                               atol=1e-6 * max(1.0, float(np.abs(p).max())))
    if not case.startswith("overflowing"):
        assert kept == 0 and np.all(p == 0.0)
    # the same model object fits again on finite data
    y_ok = np.nan_to_num(y, nan=0.0, posinf=0.0)
    model2 = PackBoost(PackBoostConfig(pack_size=2, learning_rate=0.1, **kw)).fit(X, y_ok, era, num_rounds=2)
    assert np.all(np.isfinite(model2.predict(X[:100])))
