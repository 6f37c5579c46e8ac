"""Integer pins for the oracle's scan / key emission / sort / ranges
(primitives/tiling.py:28-100, splatting/binning.py:16-37) against NumPy."""

import numpy as np
from hypothesis import given, settings, strategies as st

import torch_ref


def _emit_python(centers, radii, depths, width, height):
    """Straight Python restatement of the emission order: increasing row,
    then row-major tiles of the rectangle."""
    gx, gy = (width + 15) // 16, (height + 15) // 16
    keys, vals = [], []
    c, n = radii.shape
    for v in range(c):
        for i in range(n):
            if radii[v, i] <= 0:
                continue
            x0, y0, x1, y1 = torch_ref.rect_tiles(centers[v, i], radii[v, i], width, height)
            bits = int(np.float32(depths[v, i]).view(np.uint32))
            for y in range(y0, y1):
                for x in range(x0, x1):
                    tile = v * gx * gy + y * gx + x
                    keys.append((tile << 32) | bits)
                    vals.append(i)
    return np.array(keys, np.uint64), np.array(vals, np.int32)


@settings(max_examples=60, deadline=None)
@given(st.integers(1, 3), st.integers(0, 40), st.integers(1, 70), st.integers(1, 50), st.integers(0, 2**31 - 1))
def test_scan_emit_sort_ranges(views, n, width, height, seed):
    import oracle as oracle_lib

    rng = np.random.default_rng(seed)
    centers = rng.uniform(-30, max(width, height) + 30, size=(views, n, 2)).astype(np.float32)
    radii = rng.integers(-2, 40, size=(views, n)).astype(np.int32)
    radii[radii < 0] = 0
    # Duplicate depths on purpose to exercise stability (ties keep id order).
    depths = rng.choice(np.array([0.5, 1.25, 3.0, 7.5, 100.0], np.float32), size=(views, n))
    tiles = np.zeros((views, n), np.int32)
    for v in range(views):
        for i in range(n):
            if radii[v, i] > 0:
                x0, y0, x1, y1 = torch_ref.rect_tiles(centers[v, i], radii[v, i], width, height)
                tiles[v, i] = (x1 - x0) * (y1 - y0)
    radii[tiles == 0] = 0
    offsets, total = oracle_lib.scan_i32(tiles.ravel())
    np.testing.assert_array_equal(offsets, np.cumsum(tiles.ravel()))
    assert total == int(tiles.sum())
    keys, vals = oracle_lib.emit_keys(centers, radii, depths, offsets, total, width, height)
    ek, ev = _emit_python(centers, radii, depths, width, height)
    np.testing.assert_array_equal(keys, ek)
    np.testing.assert_array_equal(vals, ev)
    T = views * ((width + 15) // 16) * ((height + 15) // 16)
    end_bit = 32 + int(T).bit_length()
    sk, sv = oracle_lib.sort_pairs(keys, vals, end_bit)
    order = np.lexsort((np.arange(len(keys)), keys))  # stable by key
    np.testing.assert_array_equal(sk, keys[order])
    np.testing.assert_array_equal(sv, vals[order])
    # Equivalent characterisation: lexsort by (key, gaussian id).
    order2 = np.lexsort((vals, keys))
    np.testing.assert_array_equal(sv, vals[order2])
    ranges = oracle_lib.tile_ranges(sk, T)
    tile_of = (sk >> np.uint64(32)).astype(np.int64)
    lo = np.searchsorted(tile_of, np.arange(T), side="left")
    hi = np.searchsorted(tile_of, np.arange(T), side="right")
    present = hi > lo
    np.testing.assert_array_equal(ranges[present, 0], lo[present])
    np.testing.assert_array_equal(ranges[present, 1], hi[present])
    assert np.all(ranges[~present] == 0)


def test_sort_respects_end_bit(oracle_lib):
    # Bits at or above end_bit do not take part in the order.
    keys = np.array([(1 << 40) | 5, 3, (2 << 40) | 1, 4], np.uint64)
    vals = np.arange(4, dtype=np.int32)
    sk, sv = oracle_lib.sort_pairs(keys, vals, 40)
    assert list(sv) == [2, 1, 3, 0]


def test_ranges_ignore_invalid_tile(oracle_lib):
    keys = np.array([(3 << 32), (3 << 32) | 1, (0xFFFFFFFF << 32)], np.uint64)
    r = oracle_lib.tile_ranges(keys, 5)
    assert r[3].tolist() == [0, 2] and r[0].tolist() == [0, 0]


def test_parallel_sort_path_matches_stable_order(oracle_lib):
    rng = np.random.default_rng(11)
    keys = (rng.integers(0, 1 << 13, 200_000).astype(np.uint64) << np.uint64(32)) | rng.integers(0, 64, 200_000).astype(np.uint64)
    vals = np.arange(200_000, dtype=np.int32)
    oracle_lib.set_threads(4)
    try:
        sk, sv = oracle_lib.sort_pairs(keys, vals, 45)
    finally:
        oracle_lib.set_threads(1)
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(sk, keys[order])
    np.testing.assert_array_equal(sv, vals[order])
