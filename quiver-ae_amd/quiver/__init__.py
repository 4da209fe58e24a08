"""MI355X-native Quiver query path: NumPy interface (python/quiver/__init__.py)."""

from ._lib import QuiverError
from .index import IndexQuiver, build_index, mixture

__all__ = ["IndexQuiver", "QuiverError", "build_index", "mixture"]
__version__ = "0.1.0"
