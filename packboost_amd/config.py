"""Configuration of a PackBoost fit.

Same fields, defaults and meaning as the reference's ``PackBoostConfig``
(packboost/config.py:9-90), so existing configs construct unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal


@dataclass(frozen=True, slots=True)
class PackBoostConfig:
    """Hyper-parameters steering PackBoost training.

    pack_size: trees grown per boosting round. max_depth: depth limit (root is depth 0).
    learning_rate: per-tree weight. lambda_l2: L2 term added to hessian sums.
    lambda_dro: weight of the per-era gain standard deviation (DES penalty).
    direction_weight: weight of the directional-agreement term. min_samples_leaf: minimum
    rows per child. max_bins: histogram bins per feature (the reference caps this at 128 for
    int8 storage; this backend stores uint8 and accepts up to 255 for quantile-binned data).
    k_cuts / cut_selection: evaluate k thresholds per feature ("even" or "mass"); 0 = all.
    layer_feature_fraction: fraction of features sampled per depth. era_alpha: pseudo-count
    for count-weighted eras (0 = equal era weights). era_tile_size, feature_block_size,
    enable_node_batching, histogram_mode: execution hints kept for API compatibility.
    random_state: seed of the CPU generator that samples features. device: "cuda" (the
    MI355X device; ROCm exposes HIP devices under torch's "cuda" name). prebinned: treat X as
    integer bins in [0, max_bins).
    """

    pack_size: int = 8
    max_depth: int = 6
    learning_rate: float = 0.1
    lambda_l2: float = 1e-6
    lambda_dro: float = 0.0
    direction_weight: float = 0.0
    min_samples_leaf: int = 20
    max_bins: int = 63
    k_cuts: int = 0
    cut_selection: Literal["even", "mass"] = "mass"
    layer_feature_fraction: float = 1.0
    era_alpha: float = 0.0
    era_tile_size: int = 32
    histogram_mode: Literal["rebuild", "subtract", "auto"] = "rebuild"
    feature_block_size: int = 32
    enable_node_batching: bool = True
    random_state: int | None = None
    device: str = "cuda"
    prebinned: bool = False
