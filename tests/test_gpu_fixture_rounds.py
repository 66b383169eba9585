"""Whole rounds of BASELINE configs 3 and 2 at full size against the oracle.

Config 3 (the headline): 2,400,000 rows x 2,376 features quantised to 5 levels, 574 eras,
B 8, D 6, 238 features per depth, lr 0.01, lambda_dro 0.5; the HIP fit takes the path the bench
times (nibble bins, joint-bin histograms, producer/consumer scorer, pipelined rounds).
Config 2: 200,000 x 100 float32 features binned on the device into 128 quantile bins, 50 eras,
B 8, D 5, all 100 of its rounds.

Each is compared round by round with tests/golden/<config>_rounds.npz, the oracle's fit
(booster.py:494-599 restated, each depth's split finder the reference's own compiled
frontier_cpu.cpp:111-515) written in the build container by tests/golden/make_rounds_golden.py
from the same seeded workload: trees identical up to an asserted near-tie (1e-6), node values
and training predictions within 1e-5, frontier sizes and rows per depth exact
(tests.helpers.fixture_fit_parity).
"""

from __future__ import annotations

import pytest

from tests.helpers import fixture_fit_parity

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["config3", "config2"])
def test_rounds_match_oracle_fixture(hip, oracle_mod, name):
    from packboost_amd import PackBoost, PackBoostConfig
    from tests.golden.make_rounds_golden import case_data

    X, _, y, era, cfg = case_data(name)

    def fit_rounds(n):
        model = PackBoost(PackBoostConfig(**cfg)).fit(X, y, era, num_rounds=n)
        assert model._fit_mode == "planes"
        return model

    matched = fixture_fit_parity(oracle_mod, name, fit_rounds)
    assert matched >= 1
