"""MI355X-native Quiver query path: NumPy interface (python/quiver/__init__.py)."""

from ._lib import QuiverError
from .index import IndexQuiver, build_index, build_nav, mixture

__all__ = ["IndexQuiver", "QuiverError", "build_index", "build_nav", "mixture"]
__version__ = "0.1.0"
