"""Capped tile lists: each camera's tile stops carried from one frame of that
camera to the next.

A tile's blend stops reading its depth-ordered list once every pixel of the
tile has terminated (transmittance below 1e-4, gs3d/render.py:107-169 of the
reference), usually after a small part of the list.  The blend reports that
position per tile (its stop), and the next frame of the same camera (same
64-bit key of view matrix and intrinsics, gs3d_camera_prepare_keyed; same
image size and tile mode) writes each tile's list only up to its cap,
stop + stop/4 + 128 entries.  The blend reads no further; a tile whose pixels
are still live at its cap is flagged, and after the blend gs3d_bin_redo
writes the whole lists of the flagged tiles and a second blend launch
renders only those tiles again, from their first entry.  Images,
transmittance, contributor counts and gradients are therefore those of
whole lists whatever the caps were; a stale cap costs only the redo.

The first frame of a camera writes whole lists (no stops known), and so do
frames with statistics, frames binned per camera group and frames of fewer
than MIN_PAIRS tile pairs: a capped frame launches two more kernels
(gs3d_bin_redo and the redo blend; ~9 us on MI355X when no tile overflows)
and does ~15 us more host work, which only a long id-write pass repays (measured per step: 20.8M-pair frames lose 30-50 us, frames of
93M-171M pairs gain 100-170 us in every tile mode).  GS3D_LIST_CAPS=0 turns
the caps off.
"""

from collections import OrderedDict
from dataclasses import dataclass
import os
import threading

import torch
from torch import Tensor

from ..runtime import native
from ..splatting import binning

ENABLED = os.environ.get("GS3D_LIST_CAPS", "1") != "0"
# Frames with fewer tile pairs write whole lists.
MIN_PAIRS = 48 << 20
# The stop cache keeps at most this many bytes of stop rows (one int32 per
# tile per camera, 32 KB per 1920x1080 camera), dropping the least recently
# rendered cameras first.
CACHE_BYTES = 64 << 20

_LOCK = threading.Lock()
# (device index, width, height, tile mode, batch slot, camera key) -> (stops of the
# frame that rendered the camera last, its row in them, the stream its blend
# ran on).  Stops are used on that stream only: the binning and the blend
# of a frame must read equal caps, which a blend still writing them on
# another stream would not guarantee.
_STOPS: "OrderedDict[tuple, tuple[Tensor, int, int]]" = OrderedDict()
_BYTES = 0


@dataclass(slots=True)
class CappedLists:
    """Caps and outputs of one frame's capped lists.

    caps: (views*tiles) int32 caps of the binning and blend, None when no
    camera of the frame was seen before (whole lists; the stops are still
    measured).  stops: (views, tiles) int32 that the blend fills.  With
    caps, redo: (views*tiles) int32 overflow flags, and redo_list:
    (1 + views*tiles) int32, the count of flagged tiles (zeroed by the
    capped binning it is given to) and the tiles.  launch: the binning launch that gs3d_bin_redo repeats for
    the flagged tiles."""

    keys: list
    shape: tuple
    stream: int
    caps: Tensor | None
    stops: Tensor
    redo: Tensor | None = None
    redo_list: Tensor | None = None
    launch: binning.BinLaunch | None = None

    def rewrite(self) -> None:
        """Whole lists for the tiles the capped blend flagged."""
        binning.redo_bin_rows(self.launch, self.redo, self.redo_list)
        self.launch = None


def applies(tile_pairs: int, tiles: int) -> bool:
    """Whether a frame of ``tile_pairs`` pairs over ``tiles`` tiles (all
    cameras) caps its lists once its cameras have stops."""
    return ENABLED and tiles > 0 and tile_pairs >= MIN_PAIRS


def capped_lengths(stops: Tensor, lengths: Tensor) -> Tensor:
    """Entries of each tile's list that a capped id-write pass keeps: the
    list length, or stop + stop/4 + 128 when that is shorter (int64)."""
    s = stops.reshape(-1).to(torch.int64)
    n = lengths.reshape(-1).to(torch.int64)
    return torch.where(s < 0, n, torch.minimum(n, s + s // 4 + 128))


def clear() -> None:
    """Forget every camera's stops."""
    global _BYTES
    with _LOCK:
        _STOPS.clear()
        _BYTES = 0


def plan(device: torch.device, width: int, height: int, tile_mode: str, keys: list, tile_pairs: int,
         tiles_per_view: int, slot: int = 0) -> CappedLists | None:
    """The frame's caps from the stop cache; None when the frame writes whole
    lists without measuring stops (caps off or a small frame).  ``slot``
    tells apart the frames of one call that render different Gaussians (the
    items of a batched call), so that each finds its own stops even when
    they share a camera."""
    if not keys or not applies(tile_pairs, len(keys) * tiles_per_view):
        return None
    shape = (device.index, width, height, tile_mode, slot)
    stream = native.stream(device).value or 0
    views = len(keys)
    with _LOCK:
        rows = []
        for k in keys:
            row = _STOPS.get(shape + (k,))
            if row is not None:
                _STOPS.move_to_end(shape + (k,))
                if row[2] != stream:
                    row = None
            rows.append(row)
    count = views * tiles_per_view
    caps = None
    first = rows[0]
    if first is not None and first[0].shape[0] == views and all(
            r is not None and r[0] is first[0] and r[1] == i for i, r in enumerate(rows)):
        caps = first[0].view(-1)  # the same cameras in the same order as their last frame
    elif any(r is not None for r in rows):
        # One gather launch; cameras without stops read whole lists (-1).
        whole = torch.full((tiles_per_view,), -1, dtype=torch.int32, device=device) if None in rows else None
        caps = torch.stack([whole if r is None else r[0][r[1]] for r in rows]).view(-1)
    if caps is None:
        return CappedLists(list(keys), shape, stream, None,
                           torch.empty((views, tiles_per_view), dtype=torch.int32, device=device))
    # stops | redo flags | count of flagged tiles (cleared by the capped
    # id-write pass, gs3d_bin_args.redo_list), flagged tiles
    buffer = torch.empty(3 * count + 1, dtype=torch.int32, device=device)
    return CappedLists(list(keys), shape, stream, caps, buffer[:count].view(views, tiles_per_view),
                       buffer[count:2 * count], buffer[2 * count:])


def remember(lists: CappedLists) -> None:
    """Store the stops of a blend that has been enqueued: later frames of
    these cameras read them in stream order."""
    global _BYTES
    row_bytes = lists.stops.shape[1] * 4
    with _LOCK:
        for i, k in enumerate(lists.keys):
            key = lists.shape + (k,)
            if key in _STOPS:
                _BYTES -= row_bytes
                del _STOPS[key]
            _STOPS[key] = (lists.stops, i, lists.stream)
            _BYTES += row_bytes
        while _BYTES > CACHE_BYTES and _STOPS:
            _, (t, _, _) = _STOPS.popitem(last=False)
            _BYTES -= t.shape[1] * 4
