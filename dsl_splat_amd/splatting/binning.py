"""Square-tile duplication and sorting (splatting/binning.py:16-117 of the
reference) for one or several views at once.

Rows of all views form one flat array (views*N); a pair of view v gets the
global tile id v*tiles + y*gx + x, so one radix sort over
32 + bit_length(views*tiles) key bits orders every view and ``ranges`` has
one row per (view, tile).  With one view this is exactly the reference's
per-view binning.
"""

import ctypes

import torch
from torch import Tensor

from ..primitives.tiling import TileBins, _scratch, identify_ranges, scan_counts, sort_pairs
from ..runtime import abi, native

TILE_MODES = ("radius", "snugbox", "accutile")


def validate_tile_mode(mode) -> None:
    if mode not in TILE_MODES:
        raise ValueError("tile_mode must be 'radius', 'snugbox' or 'accutile'")


def require_radius_mode(mode) -> None:
    validate_tile_mode(mode)
    if mode != "radius":
        raise NotImplementedError(
            f"tile_mode={mode!r} (SnugBox/AccuTile intersections) is not implemented in the HIP "
            "rasterizer yet; use tile_mode='radius'"
        )


def tile_count(width: int, height: int, views: int = 1) -> int:
    return views * ((width + 15) // 16) * ((height + 15) // 16)


@torch.no_grad()
def emit_keys(centers: Tensor, radii: Tensor, depths: Tensor, offsets: Tensor, count: int, width: int,
              height: int) -> tuple[Tensor, Tensor]:
    """Keys/ids (2*count storage each) of the (views, N) rows' tile pairs."""
    device = radii.device
    views, n = (1, radii.numel()) if radii.ndim == 1 else radii.shape
    keys = torch.empty(2 * count, dtype=torch.int64, device=device)
    ids = torch.empty(2 * count, dtype=torch.int32, device=device)
    if count:
        a = abi.EmitArgs()
        a.n, a.views, a.width, a.height = n, views, width, height
        centers, radii, depths = centers.contiguous(), radii.contiguous(), depths.contiguous()
        a.centers, a.radii, a.depths, a.offsets = (
            native.ptr(centers), native.ptr(radii), native.ptr(depths), native.ptr(offsets))
        a.keys, a.values = native.ptr(keys), native.ptr(ids)
        scratch = _scratch(native.query("gs3d_emit_scratch_bytes", views * n), device)
        native.call("gs3d_emit_keys", ctypes.byref(a), native.ptr(scratch), scratch.numel(), native.stream(device))
    return keys, ids


@torch.no_grad()
def emit_and_sort(centers: Tensor, radii: Tensor, depths: Tensor, offsets: Tensor, count: int, width: int,
                  height: int) -> TileBins:
    """Emit keys for (views, N) rows given inclusive offsets and their total,
    then sort them and extract per-(view, tile) ranges."""
    views = 1 if radii.ndim == 1 else radii.shape[0]
    tiles = tile_count(width, height, views)
    keys, ids = emit_keys(centers, radii, depths, offsets, count, width, height)
    ranges = torch.zeros((tiles, 2), dtype=torch.int32, device=radii.device)
    if count:
        sort_pairs(keys, ids, count, 32 + int(tiles).bit_length())
        identify_ranges(keys[:count], ranges)
    return dict(point_list=ids[:count], ranges=ranges, point_list_keys=keys[:count], point_offsets=offsets)


@torch.no_grad()
def bin_and_sort(centers: Tensor, radii: Tensor, tile_counts: Tensor, depths: Tensor, width: int, height: int,
                 bindings=None, *, conics: Tensor | None = None, tile_mode="radius") -> TileBins:
    """Scan, duplicate, sort and range one view's (N,) or several views'
    (C, N) projected Gaussians."""
    if tile_mode != "radius" and conics is None:
        raise ValueError("SnugBox/AccuTile require projected conics")
    require_radius_mode(tile_mode)
    offsets, count = scan_counts(tile_counts)
    return emit_and_sort(centers, radii, depths, offsets, count, width, height)
