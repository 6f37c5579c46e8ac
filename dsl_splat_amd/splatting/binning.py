"""Tile binning (splatting/binning.py:16-117 of the reference) for one or
several views at once, in the three tile modes of
splatting/intersections.py: "radius" (3-sigma squares), "snugbox"
(opacity-aware rectangles) and "accutile" (per-strip ellipse spans).

Rows of all views form one flat array (views*N); a tile of view v has the
global id v*tiles + y*gx + x and ``ranges`` has one row per (view, tile).
``emit_and_sort`` is the reference's own sequence (inclusive scan, 64-bit
(tile << 32 | depth bits) keys, stable radix sort, ranges); the rasterizer
uses ``order_rows`` + ``bin_rows``, which produce the same lists and ranges
without sorting the pairs (depth-ordered rows, 8x8-tile groups, wavefront
ballot ranking).  With one view either is exactly the reference's per-view
binning.
"""

import ctypes
from dataclasses import dataclass

import torch
from torch import Tensor

from ..primitives.tiling import TileBins, _scratch, identify_ranges, scan_counts, sort_pairs
from ..runtime import abi, native

TILE_MODES = ("radius", "snugbox", "accutile")


def validate_tile_mode(mode) -> None:
    if mode not in TILE_MODES:
        raise ValueError("tile_mode must be 'radius', 'snugbox' or 'accutile'")


def _mode(mode, conics) -> int:
    validate_tile_mode(mode)
    if mode != "radius" and conics is None:
        raise ValueError("SnugBox/AccuTile require projected conics")
    return abi.TILE_MODES[mode]


def tile_count(width: int, height: int, views: int = 1) -> int:
    return views * ((width + 15) // 16) * ((height + 15) // 16)


@native.no_grad
def emit_keys(centers: Tensor, radii: Tensor, depths: Tensor, offsets: Tensor, count: int, width: int,
              height: int, *, conics: Tensor | None = None, tile_mode="radius") -> tuple[Tensor, Tensor]:
    """Keys/ids (2*count storage each) of the (views, N) rows' tile pairs."""
    mode = _mode(tile_mode, conics)
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
        a.tile_mode = mode
        if mode:
            conics = conics.contiguous()
            a.conics = native.ptr(conics)
        scratch = _scratch(native.query("gs3d_emit_scratch_bytes", views * n), device)
        native.call("gs3d_emit_keys", ctypes.byref(a), native.ptr(scratch), scratch.numel(), native.stream(device))
    return keys, ids


@native.no_grad
def emit_and_sort(centers: Tensor, radii: Tensor, depths: Tensor, offsets: Tensor, count: int, width: int,
                  height: int, *, conics: Tensor | None = None, tile_mode="radius") -> TileBins:
    """Emit keys for (views, N) rows given inclusive offsets and their total,
    then sort them and extract per-(view, tile) ranges."""
    views = 1 if radii.ndim == 1 else radii.shape[0]
    tiles = tile_count(width, height, views)
    keys, ids = emit_keys(centers, radii, depths, offsets, count, width, height, conics=conics, tile_mode=tile_mode)
    ranges = torch.zeros((tiles, 2), dtype=torch.int32, device=radii.device)
    if count:
        sort_pairs(keys, ids, count, 32 + int(tiles).bit_length())
        identify_ranges(keys[:count], ranges)
    return dict(point_list=ids[:count], ranges=ranges, point_list_keys=keys[:count], point_offsets=offsets)


@native.no_grad
def order_rows(centers: Tensor, radii: Tensor, depths: Tensor, width: int, height: int, *,
               conics: Tensor | None = None, tile_mode="radius",
               tiles_out: Tensor | None = None, totals: Tensor | None = None,
               sort_bits: int = 0, key_bits_out: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """Depth order of the (views, N) rows.

    Returns (ordered row records with 2*rows storage -- followed, for
    AccuTile, by the rows' compact footprints, 32 bytes each --, inclusive
    group offsets, totals = [group pairs, tile pairs]), all left on the
    device.  ``tiles_out`` (int32, views*N), if given, receives every row's
    tile count in ``tile_mode``; ``totals`` (contiguous int64, 2), if given,
    receives the totals.  ``sort_bits`` (0 = 32) sorts only the low depth-key
    bits, valid when the kept rows' keys agree above them; ``key_bits_out``
    (int32, 1), if given, receives the bits they need (the order must be
    redone with at least that many when it exceeds ``sort_bits``)."""
    mode = _mode(tile_mode, conics)
    device = radii.device
    views, n = (1, radii.numel()) if radii.ndim == 1 else radii.shape
    rows = views * n
    accu = mode == abi.TILE_MODES["accutile"]
    order = torch.empty(2 * rows + (4 * rows if accu else 0), dtype=torch.int64, device=device)
    offsets = torch.empty(rows, dtype=torch.int32, device=device)
    if totals is None:
        totals = torch.empty(2, dtype=torch.int64, device=device)
    elif totals.dtype != torch.int64 or not totals.is_contiguous() or totals.numel() != 2:
        raise ValueError("totals must be a contiguous int64 tensor of two entries")
    a = abi.OrderArgs()
    a.n, a.views, a.width, a.height = n, views, width, height
    depths, centers, radii = depths.contiguous(), centers.contiguous(), radii.contiguous()
    a.depths, a.centers, a.radii = native.ptr(depths), native.ptr(centers), native.ptr(radii)
    a.order, a.group_offsets, a.totals = native.ptr(order), native.ptr(offsets), native.ptr(totals)
    a.tile_mode = mode
    if mode:
        conics = conics.contiguous()
        a.conics = native.ptr(conics)
    if accu:
        a.footprints = native.ptr(order, 2 * rows)
    if tiles_out is not None:
        if tiles_out.dtype != torch.int32 or not tiles_out.is_contiguous() or tiles_out.numel() != rows:
            raise ValueError("tiles_out must be a contiguous int32 tensor with one entry per row")
        a.tiles_out = native.ptr(tiles_out)
    if not 0 <= sort_bits <= 32:
        raise ValueError("sort_bits must be in [0, 32]")
    a.sort_bits = int(sort_bits)
    if key_bits_out is not None:
        if key_bits_out.dtype != torch.int32 or key_bits_out.numel() < 1:
            raise ValueError("key_bits_out must be an int32 tensor of at least one entry")
        a.key_bits_out = native.ptr(key_bits_out)
    scratch = _scratch(native.query("gs3d_order_rows_scratch_bytes", rows), device)
    native.call("gs3d_order_rows", ctypes.byref(a), native.ptr(scratch), scratch.numel(), native.stream(device))
    return order, offsets, totals


def order_pass_count(sort_bits: int) -> int:
    """Radix passes of gs3d_order_rows for ``sort_bits`` (0 = 32): bits 0-7,
    then 8-bit passes, the last one widened to up to 10 bits."""
    end = 32 if sort_bits <= 0 else max(9, min(32, sort_bits))
    passes, rest = 1, end - 8
    while rest > 10:
        passes, rest = passes + 1, rest - 8
    return passes + 1


def _pass_ceiling(bits: int) -> int:
    """Most key bits sorted in as many passes as ``bits`` take (18, 26, 32)."""
    passes = order_pass_count(bits)
    return 32 if passes >= 4 else 8 + 8 * (passes - 2) + 10


# Depth-key bits of earlier frames, per order shape (device, N, views,
# width, height, tile mode): the next frame of the shape sorts only those
# bits (three radix passes instead of four for 25 or 26 bits), and its own
# key range, read with the totals, tells whether that was enough.
_KEY_BITS: dict[tuple, int] = {}


def planned_sort_bits(shape: tuple) -> int:
    """Bits the next depth order of ``shape`` sorts (0 = all 32)."""
    return _KEY_BITS.get(shape, 0)


def remember_key_bits(shape: tuple, needed: int, sorted_bits: int) -> bool:
    """Record the bits a frame's kept depth keys needed; True when the
    frame's order sorted fewer (``sorted_bits``, 0 = 32) and must be redone.
    After such a miss the plan takes the most bits of the needed pass count,
    so a key range that keeps growing by a bit does not miss every frame."""
    sorted_bits = 32 if sorted_bits <= 0 else max(9, sorted_bits)
    needed = max(9, min(32, int(needed)))
    miss = needed > sorted_bits
    if shape not in _KEY_BITS and len(_KEY_BITS) >= _CAPACITY_SHAPES:
        del _KEY_BITS[next(iter(_KEY_BITS))]
    if miss:
        _KEY_BITS[shape] = _pass_ceiling(needed)
    elif order_pass_count(needed) < order_pass_count(sorted_bits) or shape not in _KEY_BITS:
        _KEY_BITS[shape] = needed
    return miss


# Largest pair count one binning launch addresses: tile lists, ranges and
# offsets are int32, as the reference's (primitives/tiling.py:57-64,
# splatting/binning.py:88-89), whose limit applies per view.
PAIR_LIMIT = 2**31 - 1


def check_pair_counts(group_pairs: int, tile_pairs: int) -> None:
    if tile_pairs > PAIR_LIMIT or group_pairs > PAIR_LIMIT:
        raise OverflowError(f"{tile_pairs} tile pairs exceed the int32 offsets of the binning stage")


def view_groups(pairs_per_view: list[int]) -> list[tuple[int, int]]:
    """Consecutive view ranges [v0, v1) whose tile-pair totals each fit one
    binning launch (group pairs never exceed tile pairs); OverflowError when
    a single view does not fit, as in the reference."""
    groups, v0, total = [], 0, 0
    for v, pairs in enumerate(pairs_per_view):
        if pairs > PAIR_LIMIT:
            raise OverflowError(f"view {v} has {pairs} tile pairs, more than the int32 offsets of the binning stage")
        if total + pairs > PAIR_LIMIT:
            groups.append((v0, v))
            v0, total = v, 0
        total += pairs
    groups.append((v0, len(pairs_per_view)))
    return groups


@dataclass(slots=True)
class BinLaunch:
    """Arguments of gs3d_bin_rows that do not depend on the totals, built
    while the device still works on the depth order; ``inputs`` keeps the
    tensors behind the pointers alive.  After a launch with caps, ``caps``
    and ``scratch`` hold what gs3d_bin_redo reads."""
    args: abi.BinArgs
    ranges: Tensor
    inputs: tuple
    caps: Tensor | None = None
    scratch: Tensor | None = None


@native.no_grad
def prepare_bin_rows(centers: Tensor, radii: Tensor, order: Tensor, offsets: Tensor, width: int, height: int, *,
                     conics: Tensor | None = None, tile_mode="radius") -> BinLaunch:
    mode = _mode(tile_mode, conics)
    device = order.device
    views, n = (1, radii.numel()) if radii.ndim == 1 else radii.shape
    ranges = torch.empty((tile_count(width, height, views), 2), dtype=torch.int32, device=device)
    centers, radii = centers.contiguous(), radii.contiguous()
    a = abi.BinArgs()
    a.n, a.views, a.width, a.height = n, views, width, height
    a.centers, a.radii = native.ptr(centers), native.ptr(radii)
    a.order, a.group_offsets = native.ptr(order), native.ptr(offsets)
    a.ranges = native.ptr(ranges)
    a.tile_mode = mode
    if mode:
        conics = conics.contiguous()
        a.conics = native.ptr(conics)
    if mode == abi.TILE_MODES["accutile"]:
        if order.numel() < 6 * views * n:
            raise ValueError("AccuTile binning needs the order returned by order_rows in the same mode")
        a.footprints = native.ptr(order, 2 * views * n)
    return BinLaunch(a, ranges, (centers, radii, order, offsets, conics))


# Group-item capacities of earlier frames, per binning shape.  With a known
# capacity the group items are emitted before the host reads the totals, so
# the device emits while the host synchronises (radius and SnugBox modes).
_CAPACITY: dict[tuple, int] = {}
_CAPACITY_SHAPES = 64
CAPACITY_HEADROOM = 1.125


@dataclass(slots=True)
class EarlyItems:
    """Binning scratch holding the group items emitted with ``capacity``
    (dropped, None, once a frame turns out to need more)."""
    scratch: Tensor | None
    capacity: int


def _shape_key(launch: BinLaunch) -> tuple:
    a = launch.args
    return (launch.ranges.device.index, a.n, a.views, a.width, a.height, a.tile_mode)


@native.no_grad
def emit_early(launch: BinLaunch) -> EarlyItems | None:
    """Enqueue the emission of group items before the totals are known, when
    an earlier frame of the same shape gave a capacity; None otherwise."""
    a = launch.args
    capacity = _CAPACITY.get(_shape_key(launch))
    if not capacity or a.tile_mode == abi.TILE_MODES["accutile"]:
        return None
    device = launch.ranges.device
    scratch = _scratch(native.query("gs3d_bin_rows_scratch_bytes", capacity, a.views, a.width, a.height,
                                    a.tile_mode), device)
    a.group_pairs, a.tile_pairs = capacity, 0
    native.call("gs3d_emit_group_items", ctypes.byref(a), native.ptr(scratch), scratch.numel(),
                native.stream(device))
    return EarlyItems(scratch, capacity)


# A stored capacity shrinks by this factor per frame towards the latest need,
# so one unusually large frame does not oversize the early scratch of every
# later frame of its shape.
CAPACITY_DECAY = 0.9


def _remember_capacity(launch: BinLaunch, group_pairs: int) -> None:
    if launch.args.tile_mode == abi.TILE_MODES["accutile"] or group_pairs <= 0:
        return
    key = _shape_key(launch)
    want = min(PAIR_LIMIT, int(group_pairs * CAPACITY_HEADROOM) + 1)
    stored = _CAPACITY.get(key)
    if stored is None and len(_CAPACITY) >= _CAPACITY_SHAPES:
        del _CAPACITY[next(iter(_CAPACITY))]
    _CAPACITY[key] = max(want, int(stored * CAPACITY_DECAY)) if stored else want


@native.no_grad
def launch_bin_rows(launch: BinLaunch, group_pairs: int, tile_pairs: int,
                    early: EarlyItems | None = None, caps: Tensor | None = None,
                    redo_list: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """Ranges (views*tiles, 2) and the tile-ordered Gaussian ids (tile_pairs);
    ``early`` (from emit_early) is used when its capacity holds every item.
    With ``caps`` (views*tiles int32, see gs3d_bin_args.caps) each tile's
    list is written only up to its cap, the first entry of ``redo_list`` (the
    overflow count of the blend that follows) is zeroed, and the launch keeps
    the binning scratch for redo_bin_rows."""
    check_pair_counts(group_pairs, tile_pairs)
    a, device = launch.args, launch.ranges.device
    ids = torch.empty(tile_pairs, dtype=torch.int32, device=device)
    a.group_pairs, a.tile_pairs = group_pairs, tile_pairs
    a.ids = native.ptr(ids)
    if caps is not None:
        if caps.dtype != torch.int32 or not caps.is_contiguous() or caps.numel() != launch.ranges.shape[0]:
            raise ValueError("caps must be a contiguous int32 tensor with one entry per tile")
        launch.caps = caps
        a.caps = native.ptr(caps)
        a.redo_list = native.ptr(redo_list)
    if early is not None and group_pairs <= early.capacity:
        native.call("gs3d_bin_emitted_rows", ctypes.byref(a), native.ptr(early.scratch), early.scratch.numel(),
                    native.stream(device))
        scratch = early.scratch
    else:
        if early is not None:
            # Too small: release the early scratch before the full one is
            # allocated (the allocator reuses it in stream order, after the
            # early emission), so the two are never held together.
            early.scratch = None
        scratch = _scratch(native.query("gs3d_bin_rows_scratch_bytes", group_pairs, a.views, a.width, a.height,
                                        a.tile_mode), device)
        native.call("gs3d_bin_rows", ctypes.byref(a), native.ptr(scratch), scratch.numel(), native.stream(device))
    if caps is not None:
        launch.scratch = scratch
    _remember_capacity(launch, group_pairs)
    return launch.ranges, ids


@native.no_grad
def capped_items_loaded(launch: BinLaunch) -> int:
    """Group items the capped id-write pass of ``launch`` (a launch_bin_rows
    with caps, before redo_bin_rows) read (gs3d_bin_capped_items);
    synchronises."""
    if launch.scratch is None or launch.caps is None:
        raise RuntimeError("capped_items_loaded needs a launch_bin_rows with caps before it")
    device = launch.ranges.device
    out = torch.empty(1, dtype=torch.int64, device=device)
    native.call("gs3d_bin_capped_items", ctypes.byref(launch.args), native.ptr(launch.scratch),
                launch.scratch.numel(), native.ptr(out), native.stream(device))
    return int(out.item())


@native.no_grad
def redo_bin_rows(launch: BinLaunch, redo: Tensor, redo_list: Tensor) -> None:
    """Write the whole lists of the tiles flagged in ``redo`` (views*tiles
    int32, from a capped blend, whose ``redo_list`` starts with their count)
    after a launch_bin_rows with caps, then release the binning scratch."""
    if launch.scratch is None:
        raise RuntimeError("redo_bin_rows needs a launch_bin_rows with caps before it")
    device = launch.ranges.device
    native.call("gs3d_bin_redo", ctypes.byref(launch.args), native.ptr(redo), native.ptr(redo_list),
                native.ptr(launch.scratch), launch.scratch.numel(), native.stream(device))
    launch.scratch = None


def bin_rows(centers: Tensor, radii: Tensor, order: Tensor, offsets: Tensor, group_pairs: int, tile_pairs: int,
             width: int, height: int, *, conics: Tensor | None = None,
             tile_mode="radius") -> tuple[Tensor, Tensor]:
    """Ranges (views*tiles, 2) and the tile-ordered Gaussian ids (tile_pairs)
    of rows ordered by ``order_rows`` (same conics and tile mode)."""
    check_pair_counts(group_pairs, tile_pairs)
    launch = prepare_bin_rows(centers, radii, order, offsets, width, height, conics=conics, tile_mode=tile_mode)
    return launch_bin_rows(launch, group_pairs, tile_pairs)


@native.no_grad
def pair_tiles(ranges: Tensor, count: int) -> Tensor:
    """Global tile id of every listed pair (uint32 values in int32 storage)."""
    tiles = torch.empty(count, dtype=torch.int32, device=ranges.device)
    if count:
        native.call("gs3d_pair_tiles", native.ptr(ranges), ranges.shape[0], native.ptr(tiles), count,
                    native.stream(ranges.device))
    return tiles


@native.no_grad
def expand_keys(sorted_tiles: Tensor, ids: Tensor, count: int, depths: Tensor, width: int, height: int) -> Tensor:
    """The reference's 64-bit keys (tile << 32 | depth bits) of sorted pairs."""
    n = depths.shape[-1]
    keys = torch.empty(count, dtype=torch.int64, device=depths.device)
    if count:
        native.call("gs3d_expand_keys", native.ptr(sorted_tiles), native.ptr(ids), count,
                    native.ptr(depths.contiguous()), n, tile_count(width, height), native.ptr(keys),
                    native.stream(depths.device))
    return keys


@native.no_grad
def finish_binning(centers: Tensor, radii: Tensor, order: Tensor, offsets: Tensor, group_pairs: int,
                   tile_pairs: int, depths: Tensor, width: int, height: int, *, with_keys: bool = False,
                   conics: Tensor | None = None, tile_mode="radius") -> TileBins:
    """Tile lists and ranges once the host has read the totals of
    ``order_rows``."""
    ranges, ids = bin_rows(centers, radii, order, offsets, group_pairs, tile_pairs, width, height, conics=conics,
                           tile_mode=tile_mode)
    bins: TileBins = dict(point_list=ids, ranges=ranges)
    if with_keys:
        bins["point_list_keys"] = expand_keys(pair_tiles(ranges, tile_pairs), ids, tile_pairs, depths, width, height)
    return bins


@native.no_grad
def bin_and_sort(centers: Tensor, radii: Tensor, tile_counts: Tensor, depths: Tensor, width: int, height: int,
                 bindings=None, *, conics: Tensor | None = None, tile_mode="radius",
                 with_keys: bool = False) -> TileBins:
    """Bin one view's (N,) or several views' (C, N) projected Gaussians into
    depth-sorted per-tile lists (same order and ranges as the reference's
    scan + duplicate + 64-bit key sort).  ``tile_counts`` is accepted for
    the reference's signature; the counts follow from centers, radii and,
    outside the radius mode, conics."""
    _mode(tile_mode, conics)
    order, offsets, totals = order_rows(centers, radii, depths, width, height, conics=conics, tile_mode=tile_mode)
    group_pairs, tile_pairs = totals.cpu().tolist()
    return finish_binning(centers, radii, order, offsets, group_pairs, tile_pairs, depths, width, height,
                          with_keys=with_keys, conics=conics, tile_mode=tile_mode)
