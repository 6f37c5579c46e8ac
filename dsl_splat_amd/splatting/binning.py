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
def depth_order(depths: Tensor, tile_counts: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Rows (views*N) stably sorted by depth bits; inclusive offsets of their
    tile counts in that order and the int64 total (all left on the device).
    Returns (order with 2*rows storage, offsets, total)."""
    device = depths.device
    rows = depths.numel()
    order = torch.empty(2 * rows, dtype=torch.int32, device=device)
    offsets = torch.empty(rows, dtype=torch.int32, device=device)
    total = torch.zeros(1, dtype=torch.int64, device=device)
    if rows:
        depths, tile_counts = depths.contiguous(), tile_counts.contiguous()
        scratch = _scratch(native.query("gs3d_depth_order_scratch_bytes", rows), device)
        native.call("gs3d_depth_order", native.ptr(depths), native.ptr(tile_counts), rows, native.ptr(order),
                    native.ptr(offsets), native.ptr(total), native.ptr(scratch), scratch.numel(),
                    native.stream(device))
    return order, offsets, total


@torch.no_grad()
def emit_ordered(centers: Tensor, radii: Tensor, order: Tensor, offsets: Tensor, count: int, width: int,
                 height: int) -> tuple[Tensor, Tensor]:
    """(uint32 global tile ids stored as int32, int32 Gaussian ids), each with
    2*count storage, of the ordered rows' tile pairs."""
    device = radii.device
    views, n = (1, radii.numel()) if radii.ndim == 1 else radii.shape
    tiles = torch.empty(2 * count, dtype=torch.int32, device=device)
    ids = torch.empty(2 * count, dtype=torch.int32, device=device)
    if count:
        a = abi.EmitOrderedArgs()
        a.n, a.views, a.width, a.height = n, views, width, height
        centers, radii = centers.contiguous(), radii.contiguous()
        a.centers, a.radii, a.order, a.offsets = (native.ptr(centers), native.ptr(radii), native.ptr(order),
                                                  native.ptr(offsets))
        a.tile_keys, a.values = native.ptr(tiles), native.ptr(ids)
        native.call("gs3d_emit_ordered", ctypes.byref(a), native.stream(device))
    return tiles, ids


@torch.no_grad()
def sort_by_tile(tiles: Tensor, ids: Tensor, count: int, tile_total: int) -> None:
    """Stable sort of the (tile, id) pairs on the tile id, in place."""
    if count > 1:
        scratch = _scratch(native.query("gs3d_sort_scratch_bytes", count), tiles.device)
        native.call("gs3d_sort_pairs_u32", native.ptr(tiles), native.ptr(ids), count, int(tile_total).bit_length(),
                    native.ptr(scratch), scratch.numel(), native.stream(tiles.device))


@torch.no_grad()
def ranges_of(sorted_tiles: Tensor, count: int, tile_total: int) -> Tensor:
    ranges = torch.zeros((tile_total, 2), dtype=torch.int32, device=sorted_tiles.device)
    if count:
        native.call("gs3d_tile_ranges_u32", native.ptr(sorted_tiles), count, native.ptr(ranges), tile_total,
                    native.stream(sorted_tiles.device))
    return ranges


@torch.no_grad()
def expand_keys(sorted_tiles: Tensor, ids: Tensor, count: int, depths: Tensor, width: int, height: int) -> Tensor:
    """The reference's 64-bit keys (tile << 32 | depth bits) of sorted pairs."""
    n = depths.shape[-1]
    keys = torch.empty(count, dtype=torch.int64, device=depths.device)
    if count:
        native.call("gs3d_expand_keys", native.ptr(sorted_tiles), native.ptr(ids), count,
                    native.ptr(depths.contiguous()), n, tile_count(width, height), native.ptr(keys),
                    native.stream(depths.device))
    return keys


@torch.no_grad()
def finish_binning(centers: Tensor, radii: Tensor, depths: Tensor, order: Tensor, offsets: Tensor, count: int,
                   width: int, height: int, *, with_keys: bool = False) -> TileBins:
    """Emission in depth order, stable tile sort and ranges for a known pair
    count (the host has read the total of ``depth_order``)."""
    views = 1 if radii.ndim == 1 else radii.shape[0]
    tile_total = tile_count(width, height, views)
    tiles, ids = emit_ordered(centers, radii, order, offsets, count, width, height)
    sort_by_tile(tiles, ids, count, tile_total)
    bins: TileBins = dict(point_list=ids[:count], ranges=ranges_of(tiles, count, tile_total))
    if with_keys:
        bins["point_list_keys"] = expand_keys(tiles, ids, count, depths, width, height)
    return bins


@torch.no_grad()
def bin_and_sort(centers: Tensor, radii: Tensor, tile_counts: Tensor, depths: Tensor, width: int, height: int,
                 bindings=None, *, conics: Tensor | None = None, tile_mode="radius",
                 with_keys: bool = False) -> TileBins:
    """Bin one view's (N,) or several views' (C, N) projected Gaussians into
    depth-sorted per-tile lists (same order and ranges as the reference's
    scan + duplicate + 64-bit key sort)."""
    if tile_mode != "radius" and conics is None:
        raise ValueError("SnugBox/AccuTile require projected conics")
    require_radius_mode(tile_mode)
    order, offsets, total = depth_order(depths, tile_counts)
    count = int(total.item()) if depths.numel() else 0
    if count > 2**31 - 1:
        raise OverflowError("tile pair count exceeds int32 offsets")
    return finish_binning(centers, radii, depths, order, offsets, count, width, height, with_keys=with_keys)
