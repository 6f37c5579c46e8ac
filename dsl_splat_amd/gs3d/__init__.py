"""Original 3D Gaussian Splatting on hand-written HIP kernels for MI355X."""

from .api import RasterizationResult, rasterize
from . import ops

__all__ = ["rasterize", "RasterizationResult", "ops"]
