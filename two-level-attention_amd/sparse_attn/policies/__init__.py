"""Region geometry shared by the cache and the selector."""
from .region_geometry import RegionGeometry

__all__ = ['RegionGeometry']
