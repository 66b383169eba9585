"""scikit-learn style estimator over PackBoost (the reference's README.md:92-100 usage:
``PackBoostRegressor(pack_size=8, max_depth=5, learning_rate=0.05).fit(X, y, era=...)``).

Constructor keywords are PackBoostConfig fields plus ``num_rounds``; ``get_params`` /
``set_params`` follow scikit-learn's estimator protocol, so the wrapper can be cloned and
grid-searched. Prediction goes through the same HIP kernels as PackBoost.predict.
"""

from __future__ import annotations

from dataclasses import fields
from pathlib import Path

import numpy as np

from .booster import PackBoost
from .config import PackBoostConfig
from .predictor import PackBoostPredictor, save_bundle

_CONFIG_FIELDS = tuple(f.name for f in fields(PackBoostConfig))


class PackBoostRegressor:
    """Squared-loss PackBoost regressor with the scikit-learn fit/predict/score protocol."""

    def __init__(self, num_rounds: int = 100, **config) -> None:
        unknown = set(config) - set(_CONFIG_FIELDS)
        if unknown:
            raise TypeError(f"unknown PackBoostConfig fields: {sorted(unknown)}")
        self.num_rounds = int(num_rounds)
        self._config = dict(config)
        self.model_: PackBoost | None = None

    # scikit-learn estimator protocol -------------------------------------------------
    def get_params(self, deep: bool = True) -> dict:
        defaults = PackBoostConfig()
        out = {name: self._config.get(name, getattr(defaults, name)) for name in _CONFIG_FIELDS}
        out["num_rounds"] = self.num_rounds
        return out

    def set_params(self, **params) -> "PackBoostRegressor":
        for k, v in params.items():
            if k == "num_rounds":
                self.num_rounds = int(v)
            elif k in _CONFIG_FIELDS:
                self._config[k] = v
            else:
                raise ValueError(f"invalid parameter {k!r}")
        return self

    def __repr__(self) -> str:
        args = ", ".join(f"{k}={v!r}" for k, v in sorted(self._config.items()))
        return f"PackBoostRegressor(num_rounds={self.num_rounds}{', ' + args if args else ''})"

    # estimator -------------------------------------------------------------------------
    def fit(self, X, y, era=None, **fit_kwargs) -> "PackBoostRegressor":
        """Fits a fresh model; extra keywords (feature_names, eval_sets, round_callback) are
        passed to PackBoost.fit."""
        cfg = PackBoostConfig(**self._config)
        self.model_ = PackBoost(cfg).fit(X, y, era, num_rounds=self.num_rounds, **fit_kwargs)
        self.n_features_in_ = int(np.asarray(X.shape)[1])
        return self

    def _fitted(self) -> PackBoost:
        if self.model_ is None:
            raise RuntimeError("PackBoostRegressor is not fitted yet; call fit() first")
        return self.model_

    def predict(self, X) -> np.ndarray:
        return self._fitted().predict(X)

    def score(self, X, y, sample_weight=None) -> float:
        """Coefficient of determination R^2 of predict(X) against y."""
        y = np.asarray(y, dtype=np.float64).reshape(-1)
        p = self.predict(X).astype(np.float64)
        w = np.ones_like(y) if sample_weight is None else np.asarray(sample_weight, np.float64)
        ybar = np.average(y, weights=w)
        ss_res = float(np.sum(w * (y - p) ** 2))
        ss_tot = float(np.sum(w * (y - ybar) ** 2))
        return 1.0 - ss_res / ss_tot if ss_tot > 0 else 0.0

    @property
    def round_metrics(self):
        return self._fitted().round_metrics

    def save(self, path: str | Path) -> Path:
        return save_bundle(self._fitted(), path)

    def to_predictor(self) -> PackBoostPredictor:
        return PackBoostPredictor(self._fitted())
