"""HIP PackBoost.fit / predict against the reference's own fit (tests/golden/fit_*.npz).

Same inputs and config as the reference run; the HIP path bins X itself. Bars: tree
structure (feature, threshold, children, is_leaf) identical in every round; leaf values
within 1e-5 (relative, plus 1e-6 absolute: grad sums are exact fixed-point integers here
and float32 row-order sums in the reference); predictions within 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.test_fit_golden import CASES, load_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", CASES)
def test_fit_matches_reference_golden(hip, name):
    from packboost_amd import PackBoost, PackBoostConfig

    d = load_case(name)
    cfg = d["config"]
    print(f"[golden fit] {name} {cfg}", flush=True)
    model = PackBoost(PackBoostConfig(**cfg)).fit(d["X"], d["y"], d["era"], num_rounds=d["rounds"])
    assert len(model._rounds) == d["rounds"]
    for r, (got, want) in enumerate(zip(model._rounds, d["trees"])):
        for key in ("feature", "threshold", "left", "right", "is_leaf"):
            np.testing.assert_array_equal(np.asarray(got[key]), want[key], err_msg=f"round {r} {key}")
        np.testing.assert_allclose(np.asarray(got["value"], np.float64), want["value"],
                                   rtol=1e-5, atol=1e-6, err_msg=f"round {r} value")
    assert len(model.trees) == d["rounds"] * cfg["pack_size"]
    pred = model.predict(d["X"])
    np.testing.assert_allclose(pred, d["preds"], rtol=0, atol=1e-5)
