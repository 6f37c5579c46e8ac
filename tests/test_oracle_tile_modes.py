"""Pins for the oracle's SnugBox / AccuTile footprints
(splatting/intersections.py:46-218) from the geometry they must respect,
not from their formulas:

* the alpha >= 1/255 region of a Gaussian with opacity o is the ellipse
  q(d) = a dx^2 + 2b dx dy + c dy^2 <= 2 ln(255 o) (the blend rejects every
  pixel outside it), so every tile holding a pixel strictly inside it must be
  listed (conservative), in every mode;
* AccuTile lists a subset of SnugBox, SnugBox a subset of the radius square;
* every AccuTile tile touches the ellipse widened by the reference's float32
  rounding allowance:
  inside one strip the ellipse's section is convex, so each tile column
  between its extremes meets it;
* axis-aligned ellipses have closed-form extents sigma * sqrt(2 ln(255 o));
* a rendered image does not depend on the mode (pixels only lose Gaussians
  the blend rejects there), while the pair count drops.
"""

import math

import numpy as np
import pytest

from dsl_splat_amd import synthetic
from test_oracle_render import _pipeline


def _tiles_inside(center, conic, level, gx, gy, shrink=1e-4):
    """Tiles holding an integer pixel with q <= level * (1 - shrink), by brute force in float64."""
    a, b, c = (float(v) for v in conic[:3])
    ys, xs = np.mgrid[0:gy * 16, 0:gx * 16].astype(np.float64)
    dx, dy = float(center[0]) - xs, float(center[1]) - ys
    q = a * dx * dx + 2.0 * b * dx * dy + c * dy * dy
    hit = q <= level * (1.0 - shrink)
    ty, tx = np.nonzero(hit)
    return set((ty // 16 * gx + tx // 16).tolist())


def _min_q_over_tile(center, conic, tile, gx, steps=65):
    ty, tx = divmod(int(tile), gx)
    xs = np.linspace(16 * tx, 16 * tx + 16, steps)
    ys = np.linspace(16 * ty, 16 * ty + 16, steps)
    X, Y = np.meshgrid(xs, ys)
    dx, dy = float(center[0]) - X, float(center[1]) - Y
    a, b, c = (float(v) for v in conic[:3])
    return float((a * dx * dx + 2 * b * dx * dy + c * dy * dy).min())


def _random_gaussian(rng, gx, gy):
    W, H = 16 * gx, 16 * gy
    center = rng.uniform([-20, -20], [W + 20, H + 20]).astype(np.float32)
    sx, sy = np.exp(rng.uniform(np.log(1.0), np.log(30.0), 2))
    th = rng.uniform(0, np.pi)
    if rng.random() < 0.3:  # thin, strongly rotated ellipses
        sx, sy = sx * 4, sy / 4
    R = np.array([[np.cos(th), -np.sin(th)], [np.sin(th), np.cos(th)]])
    cov = R @ np.diag([sx * sx, sy * sy]) @ R.T + 0.3 * np.eye(2)
    inv = np.linalg.inv(cov)
    o = float(rng.choice([0.005, 0.05, 0.3, 0.9, 0.999]))
    conic = np.array([inv[0, 0], inv[0, 1], inv[1, 1], o], np.float32)
    lam = np.linalg.eigvalsh(cov).max()
    radius = int(math.ceil(3.0 * math.sqrt(lam)))
    return center, conic, radius


def test_footprints_are_conservative_nested_and_tight(oracle_lib):
    rng = np.random.default_rng(7)
    gx, gy = 12, 9
    checked = fewer = 0
    for _ in range(300):
        center, conic, radius = _random_gaussian(rng, gx, gy)
        bounds_r, radius_tiles = oracle_lib.tile_footprint("radius", center, conic, radius, gx, gy)
        _, snug = oracle_lib.tile_footprint("snugbox", center, conic, radius, gx, gy)
        _, accu = oracle_lib.tile_footprint("accutile", center, conic, radius, gx, gy)
        R, S, A = set(radius_tiles.tolist()), set(snug.tolist()), set(accu.tolist())
        assert len(S) == len(snug) and len(A) == len(accu), "a tile listed twice"
        assert A <= S <= R
        level = 2.0 * math.log(255.0 * float(conic[3]))
        inside = _tiles_inside(center, conic, level, gx, gy) & R  # the blend only sees the radius square
        assert inside <= A, (center, conic, radius)
        # The footprint widens the level by the float32 rounding bound of q
        # over the reach of the square (intersections.py:72-79).
        a, b, c = (float(v) for v in conic[:3])
        allowance = 2.0 ** -20 * ((a + 2 * abs(b) + c) * (radius + 32) ** 2 + abs(level) + 1.0)
        for t in A:
            assert _min_q_over_tile(center, conic, t, gx) <= (level + allowance) * 1.001 + 0.05
        checked += 1
        fewer += len(A) < len(R)
    assert checked == 300 and fewer > 100


def test_axis_aligned_extents_closed_form(oracle_lib):
    # sigma_x = 6, sigma_y = 3 (conic = diag(1/36, 1/9)), opacity 0.8:
    # extents 6 * sqrt(2 ln 204) = 19.57 px and 9.78 px around (100.3, 60.7).
    gx, gy = 16, 10
    center = np.array([100.3, 60.7], np.float32)
    conic = np.array([1 / 36, 0.0, 1 / 9, 0.8], np.float32)
    ext = math.sqrt(2 * math.log(255 * 0.8))
    x0, x1 = math.floor((100.3 - 6 * ext) / 16), math.floor((100.3 + 6 * ext) / 16) + 1
    y0, y1 = math.floor((60.7 - 3 * ext) / 16), math.floor((60.7 + 3 * ext) / 16) + 1
    bounds, tiles = oracle_lib.tile_footprint("snugbox", center, conic, 20, gx, gy)
    assert tuple(bounds) == (x0, y0, x1, y1) == (5, 3, 8, 5)
    assert sorted(tiles.tolist()) == sorted(y * gx + x for y in range(y0, y1) for x in range(x0, x1))
    # Transposed covariance: the extents swap axes.
    bounds_t, _ = oracle_lib.tile_footprint("snugbox", center[::-1].copy(), np.array([1 / 9, 0.0, 1 / 36, 0.8],
                                            np.float32), 20, gx, gy)
    assert tuple(bounds_t) == (math.floor((60.7 - 3 * ext) / 16), math.floor((100.3 - 6 * ext) / 16),
                               math.floor((60.7 + 3 * ext) / 16) + 1, math.floor((100.3 + 6 * ext) / 16) + 1)


def test_footprint_special_cases(oracle_lib):
    gx, gy = 8, 8
    c = np.array([64.0, 64.0], np.float32)
    # Below the 1/255 opacity threshold nothing is listed (the radius square would be).
    b, t = oracle_lib.tile_footprint("snugbox", c, np.array([0.1, 0.0, 0.1, 1.0 / 300], np.float32), 10, gx, gy)
    assert tuple(b) == (0, 0, 0, 0) and len(t) == 0
    _, t_r = oracle_lib.tile_footprint("radius", c, np.array([0.1, 0.0, 0.1, 1.0 / 300], np.float32), 10, gx, gy)
    assert len(t_r) > 0
    # Not positive definite: the radius square is kept (no precise ellipse).
    bad = np.array([0.1, 0.2, 0.1, 0.5], np.float32)
    for mode in ("snugbox", "accutile"):
        b, t = oracle_lib.tile_footprint(mode, c, bad, 10, gx, gy)
        br, tr = oracle_lib.tile_footprint("radius", c, bad, 10, gx, gy)
        assert tuple(b) == tuple(br) and sorted(t.tolist()) == sorted(tr.tolist())
    # Entirely off screen: nothing.
    b, t = oracle_lib.tile_footprint("accutile", np.array([-200.0, 30.0], np.float32),
                                     np.array([0.5, 0.0, 0.5, 0.9], np.float32), 5, gx, gy)
    assert len(t) == 0
    # A thin diagonal ellipse: AccuTile walks the shorter side and drops the
    # corners SnugBox keeps.
    th = math.pi / 4
    R = np.array([[math.cos(th), -math.sin(th)], [math.sin(th), math.cos(th)]])
    inv = np.linalg.inv(R @ np.diag([40.0 ** 2, 1.0]) @ R.T + 0.3 * np.eye(2))
    conic = np.array([inv[0, 0], inv[0, 1], inv[1, 1], 0.9], np.float32)
    _, snug = oracle_lib.tile_footprint("snugbox", c, conic, 90, gx, gy)
    _, accu = oracle_lib.tile_footprint("accutile", c, conic, 90, gx, gy)
    assert len(accu) < 0.5 * len(snug)


@pytest.mark.parametrize("name,n,W,H,seed", [("small", 300, 96, 80, 5), ("sh3_1080p_4view", 400, 128, 72, 6)])
def test_rendered_image_is_independent_of_tile_mode(oracle_lib, name, n, W, H, seed):
    scene = synthetic.make_scene(name, n=n, width=W, height=H, seed=seed)
    feats = np.random.default_rng(seed).random((n, 3), dtype=np.float32)
    results = {}
    for mode in ("radius", "snugbox", "accutile"):
        results[mode] = _pipeline(oracle_lib, scene, features=feats, tile_mode=mode)
    out_r, _, ids_r, img_r, ft_r, _ = results["radius"]
    counts = {}
    for mode, (out, ranges, ids, image, final_t, contrib) in results.items():
        np.testing.assert_array_equal(out["radii"], out_r["radii"])
        np.testing.assert_array_equal(image, img_r)
        np.testing.assert_array_equal(final_t, ft_r)
        counts[mode] = len(ids)
        assert int(out["tiles"].sum()) == len(ids)
    assert counts["accutile"] <= counts["snugbox"] < counts["radius"]
