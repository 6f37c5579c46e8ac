"""GPU parity of the SnugBox / AccuTile tile modes
(splatting/intersections.py:46-218, gs3d/projection.py:150-161,
splatting/binning.py:40-68) with the oracle, bit-exact:

* projection tile counts (meta ``tiles_per_gauss``);
* the reference's own sequence (duplicate_precise emission + stable 64-bit
  key sort + ranges) through gs3d_emit_keys;
* the grouped binning (gs3d_order_rows + gs3d_bin_rows), whose AccuTile path
  carries a per-(Gaussian, group) tile mask;
* rasterized images identical to the radius mode's (the modes only drop
  Gaussians the blend rejects), with fewer pairs; gradients within
  rtol 1e-4 / atol 1e-5 of their scale.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle_pipeline import compare
from dsl_splat_amd import gs3d, synthetic
from dsl_splat_amd.gs3d import projection as gproj
from dsl_splat_amd.primitives import tiling
from dsl_splat_amd.splatting import binning, cameras
from test_gpu_stages import _np, _say, _scene

pytestmark = pytest.mark.gpu
DEV = "cuda"
MODES = ("snugbox", "accutile")


def _project(scene, degree, mode):
    quats = torch.nn.functional.normalize(scene.quats, dim=-1)
    with_centers = degree is not None and degree > 0
    full, inverse, centers, errors = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height,
                                                            with_centers)
    st = gproj.project_views(scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks,
                             scene.width, scene.height, 0.2, float("inf"), 0.0,
                             sh=scene.sh_coeffs if degree is not None else None, sh_degree=degree or 0,
                             camera_centers=centers if with_centers else None, metadata=True, tile_mode=mode)
    return quats, full, st


def _oracle_lists(centers, conics, radii, depths, tiles, W, H, views, mode):
    ro, rtotal = oracle.scan_i32(tiles.ravel())
    keys, vals = oracle.emit_keys(centers, radii, depths, ro, rtotal, W, H, conics=conics, tile_mode=mode)
    T = views * ((W + 15) // 16) * ((H + 15) // 16)
    sk, sv = oracle.sort_pairs(keys, vals, 32 + int(T).bit_length())
    return sk, sv, oracle.tile_ranges(sk, T)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("key,degree", [("small_rgb", None), ("sh3_4view", 3), ("sh3_720p", 0)])
def test_tile_mode_counts_and_lists_bit_exact(mode, key, degree):
    scene = _scene(key)
    _say(f"tile mode {mode} {key}")
    quats, full, st = _project(scene, degree, mode)
    ref = oracle.project_fwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                             _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height,
                             tile_mode=mode)
    np.testing.assert_array_equal(_np(st.radii), ref["radii"])
    np.testing.assert_array_equal(_np(st.tile_counts), ref["tiles"])
    views, W, H = scene.viewmats.shape[0], scene.width, scene.height
    sk, sv, rr = _oracle_lists(_np(st.centers), _np(st.conics), _np(st.radii), _np(st.depths), ref["tiles"], W, H,
                               views, mode)
    # The reference's sequence.
    offsets, count = tiling.scan_counts(st.tile_counts)
    seq = binning.emit_and_sort(st.centers, st.radii, st.depths, offsets, count, W, H, conics=st.conics,
                                tile_mode=mode)
    np.testing.assert_array_equal(_np(seq["point_list_keys"]).view(np.uint64), sk)
    np.testing.assert_array_equal(_np(seq["point_list"]), sv)
    np.testing.assert_array_equal(_np(seq["ranges"]), rr)
    # The grouped binning.
    bins = binning.bin_and_sort(st.centers, st.radii, st.tile_counts, st.depths, W, H, conics=st.conics,
                                tile_mode=mode, with_keys=True)
    np.testing.assert_array_equal(_np(bins["point_list"]), sv)
    np.testing.assert_array_equal(_np(bins["point_list_keys"]).view(np.uint64), sk)
    np.testing.assert_array_equal(_np(bins["ranges"]), rr)
    radius_pairs = int(oracle.project_fwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                                          _np(scene.viewmats), _np(full), _np(scene.Ks), W, H)["tiles"].sum())
    assert 0 < len(sv) < radius_pairs


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("views,n,W,H,spread,smax", [
    (2, 3000, 200, 120, 1.0, 60.0),      # partial groups at the edges
    (1, 20000, 128, 128, 0.15, 60.0),    # crowded corner: many chunks per group
    (70, 400, 160, 160, 1.0, 60.0),      # 280 groups: two group-sort passes
    (1, 2000, 4200, 64, 1.0, 60.0),      # 263 tiles across: rectangles not packed in the records
    (2, 1500, 640, 480, 1.0, 160.0),     # footprints over 16 tiles both ways: emitted by whole wavefronts
])
def test_tile_mode_grouped_binning_edge_cases(mode, views, n, W, H, spread, smax):
    # Equal depths (ties broken by index), wide and thin rotated ellipses,
    # opacities below the 1/255 threshold, non-positive-definite conics.
    _say(f"tile mode binning {mode} views={views} n={n} {W}x{H}")
    rng = np.random.default_rng(11)
    gx, gy = (W + 15) // 16, (H + 15) // 16
    centers = (rng.random((views, n, 2)) * spread * np.array([W, H])).astype(np.float32)
    s1 = np.exp(rng.uniform(0.0, np.log(smax), (views, n)))
    s2 = s1 * np.exp(rng.uniform(np.log(0.05), 0.0, (views, n)))
    th = rng.uniform(0, np.pi, (views, n))
    ct, sn = np.cos(th), np.sin(th)
    cxx = ct * ct * s1 * s1 + sn * sn * s2 * s2 + 0.3
    cyy = sn * sn * s1 * s1 + ct * ct * s2 * s2 + 0.3
    cxy = ct * sn * (s1 * s1 - s2 * s2)
    det = cxx * cyy - cxy * cxy
    conics = np.stack([cyy / det, -cxy / det, cxx / det, rng.choice([0.003, 0.02, 0.5, 0.99], (views, n))],
                      -1).astype(np.float32)
    conics[:, 3::41, 1] = 10.0  # not positive definite: radius square kept
    radii = np.ceil(3.0 * np.sqrt(np.maximum(cxx, cyy) + np.abs(cxy))).astype(np.int32)
    radii[:, ::97] = 500
    radii[:, 5::13] = 0
    depths = np.full((views, n), 2.5, np.float32)
    depths[:, ::7] = 1.25
    tiles = np.zeros((views, n), np.int32)
    for v in range(views):
        for i in range(n):
            if radii[v, i] > 0:
                tiles[v, i] = len(oracle.tile_footprint(mode, centers[v, i], conics[v, i], radii[v, i], gx, gy)[1])
    if smax > 100.0 and mode == "accutile":
        # some footprints must span more than 16 tiles in both directions
        wide = 0
        for v in range(views):
            for i in range(0, n, 7):
                if radii[v, i] > 0:
                    rect = oracle.tile_footprint("snugbox", centers[v, i], conics[v, i], radii[v, i], gx, gy)[0]
                    wide += min(rect[2] - rect[0], rect[3] - rect[1]) > 16
        assert wide > 0
    sk, sv, rr = _oracle_lists(centers, conics, radii, depths, tiles, W, H, views, mode)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    bins = binning.bin_and_sort(t(centers), t(radii), t(tiles), t(depths), W, H, conics=t(conics), tile_mode=mode,
                                with_keys=True)
    assert len(sv) > 0
    np.testing.assert_array_equal(_np(bins["point_list"]), sv)
    np.testing.assert_array_equal(_np(bins["point_list_keys"]).view(np.uint64), sk)
    np.testing.assert_array_equal(_np(bins["ranges"]), rr)


@pytest.mark.parametrize("mode", MODES)
def test_rasterize_tile_mode_matches_radius_mode(mode):
    scene = synthetic.make_scene("sh3_1080p_4view", n=20000, width=320, height=180, seed=71).to(DEV)
    _say(f"rasterize tile_mode={mode}")
    W, H = scene.width, scene.height
    weights = torch.rand((4, H, W, 3), device=DEV, generator=torch.Generator(DEV).manual_seed(1))

    def run(tile_mode):
        means = scene.means.clone().requires_grad_(True)
        opac = scene.opacities.clone().requires_grad_(True)
        sh = scene.sh_coeffs.clone().requires_grad_(True)
        r = gs3d.rasterize(means, scene.quats, scene.scales, opac, scene.viewmats, scene.Ks, W, H, sh_coeffs=sh,
                           tile_mode=tile_mode)
        ((r.features * weights).sum() + r.alpha.sum()).backward()
        return r, means.grad, opac.grad, sh.grad

    r0, gm0, go0, gs0 = run("radius")
    r1, gm1, go1, gs1 = run(mode)
    np.testing.assert_array_equal(_np(r1.features), _np(r0.features))
    np.testing.assert_array_equal(_np(r1.alpha), _np(r0.alpha))
    assert r1.meta["tile_mode"] == mode
    assert int(r1.meta["tiles_per_gauss"].sum()) < int(r0.meta["tiles_per_gauss"].sum())
    for name, a, b in (("means", gm1, gm0), ("opacities", go1, go0), ("sh", gs1, gs0)):
        compare(f"{mode}_{name}", _np(a), _np(b), rtol=1e-4, atol=1e-5 * float(b.abs().max()))
