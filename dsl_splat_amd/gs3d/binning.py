"""Original 3DGS square intersections and centre-Z sorting
(gs3d/binning.py:10-28 of the reference)."""

from ..primitives.tiling import TileBins
from ..splatting.binning import bin_and_sort as bin_arrays
from ..splatting.geometry import ProjectedGaussians


def bin_and_sort(state: ProjectedGaussians, width: int, height: int, bindings=None, *,
                 tile_mode: str = "radius") -> TileBins:
    return bin_arrays(state.centers, state.radii, state.tile_counts, state.depths, width, height, bindings,
                      conics=state.conics, tile_mode=tile_mode)
