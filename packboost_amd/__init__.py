"""packboost_amd — PackBoost's pack-parallel tree growth and pack prediction on MI355X (gfx950).

Exports the reference's public API (packboost/__init__.py:3-6) plus the wrappers its README
advertises (README.md:19-20, 92-100).
"""

from .booster import PackBoost, Tree, TreeBuilder, TreeNode
from .config import PackBoostConfig
from .predictor import PackBoostPredictor, load_bundle, save_bundle
from .wrapper import PackBoostRegressor

__all__ = ["PackBoost", "PackBoostConfig", "PackBoostPredictor", "PackBoostRegressor", "Tree",
           "TreeNode", "TreeBuilder", "load_bundle", "save_bundle"]
__version__ = "0.1.0"
