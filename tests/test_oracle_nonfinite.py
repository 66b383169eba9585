"""What the reference produces from gradients that are not finite, next to what this build does.

The reference has no check: NaN / inf gradients flow through its float sums. A candidate that
sees a NaN in a valid era's sums scores NaN, and `score_f > best` is false for NaN
(frontier_cpu.cpp:363-432). Eras are skipped when one side of the threshold is empty
(`valid_e`, :374-379), so a candidate whose NaN-holding eras all fall on one side still scores
from the other eras and can win. The failed-split leaf is -g/(h + lambda) of the node's float32
gradient sum (booster.py:532-542). A split's right sum is the node total minus the left sum
(frontier_cpu.cpp:476-479), so it is NaN whichever side holds the NaN rows.

Here the oracle's fit loop (oracle.fit, booster.py:375-599) runs those semantics. Its split
finder is checked against the reference's own compiled frontier (oracle/_ref) when that is
built. The HIP fit instead stops at the first such round: `nonfinite="raise"` (the default)
raises FloatingPointError, and `nonfinite="truncate"` keeps the finite rounds before it
(tests/test_gpu_edges.py::test_nonfinite_gradients_stop_the_fit). These tests pin the
reference's outcome that the HIP fit declines to reproduce.
"""

from __future__ import annotations

import numpy as np
import pytest


def _data(seed: int = 3, N: int = 3000, F: int = 4, nb: int = 16):
    rng = np.random.default_rng(seed)
    bins = rng.integers(0, nb, size=(N, F), dtype=np.uint8)
    era = np.repeat(np.arange(6), N // 6).astype(np.int64)
    y = (bins[:, 1].astype(np.float32) / nb + 0.1 * rng.standard_normal(N)).astype(np.float32)
    return bins, y, era


KW = dict(pack_size=2, max_depth=3, max_bins=16, min_samples_leaf=10, learning_rate=0.1,
          random_state=0)


def _fits(oracle_mod, bins, y, era, rounds):
    """The oracle fit with the restated splitter, and with the reference's compiled frontier
    when oracle/_ref is built; the two must agree bit for bit, NaN for NaN."""
    out = oracle_mod.fit(bins, y, era, num_rounds=rounds, splitter="restated", **KW)
    if oracle_mod.ref_module() is not None:
        ref = oracle_mod.fit(bins, y, era, num_rounds=rounds, splitter="reference", **KW)
        for a, b in zip(out.rounds, ref.rounds):
            for key in a:
                np.testing.assert_array_equal(a[key], b[key], err_msg=key)
        np.testing.assert_array_equal(out.preds, ref.preds)
    return out


def _leaf(a) -> bool:
    return a["feature"].shape[0] == 1 and bool(a["is_leaf"][0])


def test_reference_nan_target_gives_nan_leaves(oracle_mod):
    bins, y, era = _data()
    y[17] = np.nan
    res = _fits(oracle_mod, bins, y, era, 3)
    for a in res.rounds:  # every root candidate sees the NaN era valid: no split, NaN leaf
        assert _leaf(a) and np.isnan(a["value"][0])
    assert np.all(np.isnan(res.preds))


def test_reference_inf_target_turns_nan_in_the_next_round(oracle_mod):
    bins, y, era = _data()
    y[5] = np.inf  # grad -inf: the root leaf is +inf, then inf - inf = NaN
    res = _fits(oracle_mod, bins, y, era, 2)
    assert _leaf(res.rounds[0]) and res.rounds[0]["value"][0] == np.inf
    assert _leaf(res.rounds[1]) and np.isnan(res.rounds[1]["value"][0])
    assert np.all(np.isnan(res.preds))
    one = _fits(oracle_mod, bins, y, era, 1)
    assert np.all(one.preds == np.inf)


def test_reference_splits_around_an_era_it_skips(oracle_mod):
    """Era 0 is constant on every feature, so every threshold leaves it on one side and the
    reference skips it; the NaN there does not reach the scores. The root splits on the other
    eras, and the NaN reaches only the values: the nodes that hold era 0's rows, and every
    right child (its sum is the NaN total minus the left sum)."""
    bins, y, era = _data()
    bins[era == 0] = 3
    y[7] = np.nan
    res = _fits(oracle_mod, bins, y, era, 2)
    t0 = res.rounds[0]
    assert int((~t0["is_leaf"]).sum()) > 0
    vals = t0["value"][t0["is_leaf"]]
    assert np.isnan(vals).any() and np.isfinite(vals).any()
    assert np.isnan(t0["value"][0])
    # the rows in finite leaves get finite predictions after round 1; the NaN leaves spread
    # NaN gradients to every era in round 2, whose tree is one NaN leaf
    assert _leaf(res.rounds[1]) and np.isnan(res.rounds[1]["value"][0])
    assert np.all(np.isnan(res.preds))


def test_hip_fit_policy_is_explicit():
    """The policy is a constructor option (or PACKBOOST_NONFINITE); unknown values are refused
    before any device work."""
    from packboost_amd import PackBoost, PackBoostConfig

    assert PackBoost(PackBoostConfig()).nonfinite == "raise"
    assert PackBoost(PackBoostConfig(), nonfinite="truncate").nonfinite == "truncate"
    with pytest.raises(ValueError, match="nonfinite"):
        PackBoost(PackBoostConfig(), nonfinite="propagate")
