"""Projected footprint storage (splatting/geometry.py:9-19 of the reference).

Only rows with radii > 0 define centres and conics; the HIP projection writes
zeros into culled rows (the reference leaves them unwritten)."""

from dataclasses import dataclass

from torch import Tensor


@dataclass(slots=True)
class ProjectedFootprint:
    centers: Tensor
    conics: Tensor


@dataclass(slots=True)
class ProjectedGaussians(ProjectedFootprint):
    radii: Tensor
    tile_counts: Tensor
    depths: Tensor
