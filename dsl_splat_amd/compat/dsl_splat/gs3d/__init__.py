"""``dsl_splat.gs3d``: the HIP build's rasterizer (dsl_splat_amd.gs3d)."""

from dsl_splat_amd.gs3d import RasterizationResult, ops, rasterize

__all__ = ["rasterize", "RasterizationResult", "ops"]
