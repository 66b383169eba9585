"""Quantile binning on the device (pb_quantile_edges, pb_apply_bins) against the reference's
NumPy binning (data.py:44-111: np.quantile(method="linear") edges cast to float32,
searchsorted(side="left") clipped): bins bit-identical and edges bit-identical except for
the sign of a zero edge (-0.0 and +0.0 tie in a sort, so which one a quantile picks is the
sorting routine's choice; searchsorted treats them alike), including ties, a constant
column, a column holding NaN, NaN values against finite edges, a single row, and the row
gather the fit uses (era-major order); and against the reference's own bins and edges in the
golden fits."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def assert_edges_equal(got, want, msg=""):
    """Bitwise, except that -0.0 and +0.0 compare equal."""
    g = np.where(got == 0, np.float32(0), got)
    w = np.where(want == 0, np.float32(0), want)
    np.testing.assert_array_equal(g.view(np.uint32), w.view(np.uint32), err_msg=msg)


def _host_bins(X, nb):
    from packboost_amd.data import quantile_bin

    return quantile_bin(X, nb)


def _dev(X, nb, perm=None):
    import torch

    from packboost_amd.data import quantile_bin_device

    bins_fm, edges = quantile_bin_device(X, nb, torch.device("cuda"), perm=perm, chunk_features=3)
    n = X.shape[0]
    return bins_fm[:, :n].cpu().numpy().T, edges


def _data(seed, n, f):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, f)).astype(np.float32)
    X[:, 1] = np.round(X[:, 1] * 2) / 2          # heavy ties
    X[:, 2] = 3.5                                 # constant
    if f > 4:
        X[rng.integers(0, n, 5), 4] = np.nan      # NaN column -> NaN edges
    X[rng.integers(0, n, 7), 0] = np.nan if f <= 4 else X[0, 0]
    return X


@pytest.mark.parametrize("nb", [2, 5, 63, 128, 255])
def test_device_binning_matches_numpy(hip, nb):
    X = _data(nb, 3001, 7)
    print(f"[binning] nb={nb}", flush=True)
    hb, he = _host_bins(X, nb)
    db, de = _dev(X, nb)
    assert_edges_equal(de, he)
    np.testing.assert_array_equal(db, hb)
    perm = np.random.default_rng(1).permutation(X.shape[0])
    pb, _ = _dev(X, nb, perm=perm)
    np.testing.assert_array_equal(pb, hb[perm])


def test_device_binning_small_and_nan_values(hip):
    import torch

    from packboost_amd.data import apply_bins, apply_bins_device

    X1 = np.array([[1.5, -2.0, 0.0]], np.float32)
    hb, he = _host_bins(X1, 8)
    db, de = _dev(X1, 8)
    assert_edges_equal(de, he)
    np.testing.assert_array_equal(db, hb)
    X = _data(9, 2000, 4)  # NaN values in column 0, finite edges elsewhere
    hb, he = _host_bins(X, 16)
    db, de = _dev(X, 16)
    assert_edges_equal(de, he)
    np.testing.assert_array_equal(db, hb)
    Xn = np.random.default_rng(5).standard_normal((999, 4)).astype(np.float32) * 3
    Xn[::37, 1] = np.nan
    got = apply_bins_device(Xn, he, 16, torch.device("cuda"))[:, :999].cpu().numpy().T
    np.testing.assert_array_equal(got, apply_bins(Xn, he, 16))


def test_device_binning_matches_reference_golden(hip):
    from tests.test_fit_golden import CASES, load_case

    for name in CASES:
        d = load_case(name)
        nb = d["config"]["max_bins"]
        db, de = _dev(d["X"], nb)
        np.testing.assert_array_equal(db, d["bins"], err_msg=name)
        want = d["edges"].reshape(len(d["edge_lens"]), -1).astype(np.float32)  # [max_bins - 1, F]
        assert_edges_equal(de, want, name)
