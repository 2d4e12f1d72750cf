"""MI355X-native neighbor lists: the tonari ``neighbor_list`` API on gfx950 HIP kernels."""

from .api import neighbor_list

__version__ = "0.1.0"
__all__ = ["neighbor_list"]
