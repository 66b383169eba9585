"""packboost_amd — PackBoost's pack-parallel tree growth and pack prediction on MI355X (gfx950).

Exports the reference's public API (packboost/__init__.py:3-6) plus the wrappers its README
advertises (README.md:19-20, 92-100).
"""

from .booster import PackBoost, Tree, TreeBuilder, TreeNode
from .config import PackBoostConfig

__all__ = ["PackBoost", "PackBoostConfig", "Tree", "TreeNode", "TreeBuilder"]
__version__ = "0.1.0"
