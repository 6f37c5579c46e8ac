"""Prefix scans, radix sorting and tile ranges (primitives/tiling.py:16-100 of
the reference) on the HIP library.

Keys are (tile_id << 32) | float_bits(depth) in int64 storage (read as
uint64 by the kernels); ``scan_counts`` is the inclusive int32 scan with the
host-visible total, ``sort_tile_pairs`` sorts the 2*count scratch arrays in
place on key bits [0, 32 + bit_length(tiles)) and fills zeroed ranges.
"""

from typing import TypedDict

import torch
from torch import Tensor

from ..runtime import native


class _TileRanges(TypedDict):
    point_list: Tensor
    ranges: Tensor


class TileBins(_TileRanges, total=False):
    point_offsets: Tensor
    point_list_keys_unsorted: Tensor
    point_list_unsorted: Tensor
    point_list_keys: Tensor


def _scratch(nbytes: int, device) -> Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


@native.no_grad
def scan_device(counts: Tensor) -> tuple[Tensor, Tensor]:
    """Inclusive int32 offsets and the int64 total, both left on the device."""
    counts = counts.contiguous().view(-1)
    n = counts.numel()
    offsets = torch.empty((n,), dtype=torch.int32, device=counts.device)
    total = torch.zeros((1,), dtype=torch.int64, device=counts.device)
    if n:
        scratch = _scratch(native.query("gs3d_scan_scratch_bytes", n), counts.device)
        native.call("gs3d_scan_i32", native.ptr(counts), n, native.ptr(offsets), native.ptr(total),
                    native.ptr(scratch), scratch.numel(), native.stream(counts.device))
    return offsets, total


def scan_counts(counts: Tensor, stream=None) -> tuple[Tensor, int]:
    """Inclusive int32 offsets and the host-visible allocation size."""
    offsets, total = scan_device(counts)
    count = int(total.item()) if len(offsets) else 0
    if count > 2**31 - 1:
        raise OverflowError("tile pair count exceeds int32 offsets")
    return offsets, count


@native.no_grad
def sort_pairs(keys: Tensor, ids: Tensor, count: int, end_bit: int) -> None:
    """Stable LSD radix sort of keys[:count]/ids[:count] in place (2*count storage)."""
    if count <= 0:
        return
    if keys.numel() < 2 * count or ids.numel() < 2 * count:
        raise ValueError("keys/ids need 2*count elements (the second half is ping-pong storage)")
    scratch = _scratch(native.query("gs3d_sort_scratch_bytes", count), keys.device)
    native.call("gs3d_sort_pairs_u64", native.ptr(keys), native.ptr(ids), count, int(end_bit),
                native.ptr(scratch), scratch.numel(), native.stream(keys.device))


@native.no_grad
def identify_ranges(sorted_keys: Tensor, ranges: Tensor) -> None:
    count = sorted_keys.numel()
    if count:
        native.call("gs3d_tile_ranges", native.ptr(sorted_keys), count, native.ptr(ranges), len(ranges),
                    native.stream(sorted_keys.device))


def sort_tile_pairs(keys: Tensor, ids: Tensor, count: int, ranges: Tensor, stream=None, bindings=None, *,
                    sorted_keys: Tensor | None = None) -> None:
    """Sort 2*count scratch arrays in place and fill zero-initialized ranges."""
    if not count:
        return
    sort_pairs(keys, ids, count, 32 + len(ranges).bit_length())
    identify_ranges(keys[:count] if sorted_keys is None else sorted_keys, ranges)
