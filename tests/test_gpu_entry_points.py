"""Oracle parity of the product entry points besides gs3d.rasterize:

- the gs3d.ops staged API (gs3d/ops.py:27-338): prepare_gaussians ->
  bin_and_sort -> rasterize_to_pixels, forward bit-exact and backward
  through both autograd edges, and the projection edge alone with only the
  centre or only the conic gradient live;
- standalone SH degrees 0-3 with the radii mask (gs3d_sh_fwd/bwd,
  primitives/spherical_harmonics.py:104-159), including the degree-0
  direction detach;
- the standalone metadata pass (gs3d_metadata, splatting/metadata.py:12-31);
- primitives.tiling.sort_tile_pairs in the reference's calling convention
  (2*count key/id scratch sorted in place, zeroed ranges, optional
  sorted_keys; primitives/tiling.py:67-100).

Integer and forward outputs are compared bit-exactly, gradients per entry
within rtol 1e-4 / atol 1e-5 or their float32 error bound.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle
import oracle_pipeline
from oracle_pipeline import check_gradient
from dsl_splat_amd import synthetic
from dsl_splat_amd.cameras import PinholeCamera
from dsl_splat_amd.gs3d import ops
from dsl_splat_amd.gs3d import projection as gproj
from dsl_splat_amd.primitives import tiling
from dsl_splat_amd.primitives.spherical_harmonics import spherical_harmonics
from dsl_splat_amd.runtime import native
from dsl_splat_amd.splatting import binning, cameras

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


def _scene(seed=31, n=4000, width=120, height=88):
    return synthetic.make_scene("small", n=n, width=width, height=height, seed=seed).to(DEV)


def _camera(scene):
    return PinholeCamera(scene.viewmats[0], scene.Ks[0], scene.width, scene.height, near_plane=0.2,
                         far_plane=float("inf"))


@pytest.mark.parametrize("background", [False, True])
def test_ops_pipeline_matches_oracle(background):
    scene = _scene(seed=31 + background)
    print(f"ops pipeline background={background}", flush=True)
    leaves = {k: getattr(scene, k).clone().requires_grad_(True) for k in ("means", "quats", "scales", "opacities")}
    feats = scene.features.clone().requires_grad_(True)
    bg = torch.tensor([0.2, 0.5, 0.7], device=DEV) if background else None
    geometry = ops.prepare_gaussians(leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"],
                                     _camera(scene))
    tiles = ops.bin_and_sort(geometry)
    pix = ops.rasterize_to_pixels(geometry, tiles, feats, bg)
    W = scene.loss_weights[0]
    ((pix.features * W[..., :3]).sum() + (pix.alpha * W[..., 3:]).sum()).backward()
    torch.cuda.synchronize()
    ref = oracle_pipeline.run(_np(scene.means), _np(scene.quats), _np(scene.scales), _np(scene.opacities),
                              _np(scene.viewmats), _np(scene.Ks), scene.width, scene.height, features=_np(scene.features),
                              background=None if bg is None else _np(bg)[None], upstream=_np(scene.loss_weights),
                              normalize_quats=True, bounds=True)
    proj = ref["proj"]
    radii = proj["radii"][0]
    np.testing.assert_array_equal(_np(geometry.radii), radii)
    np.testing.assert_array_equal(_np(geometry.tile_counts), proj["tiles"][0])
    np.testing.assert_array_equal(_np(geometry.depths), proj["depths"][0])
    vis = radii > 0
    np.testing.assert_array_equal(_np(geometry.centers)[vis], proj["centers"][0][vis])
    np.testing.assert_array_equal(_np(geometry.conics)[vis], proj["conics"][0][vis])
    np.testing.assert_array_equal(_np(tiles.ranges), ref["ranges"])
    np.testing.assert_array_equal(_np(tiles.gaussian_ids), ref["sorted_vals"])
    image = torch.cat([pix.features, pix.alpha], -1)
    np.testing.assert_array_equal(_np(image), ref["image"][0])
    pg, bd = ref["proj_grads"], ref["bounds"]
    for name in ("means", "quats", "scales", "opacities"):
        check_gradient(f"ops_{name}", _np(leaves[name].grad), pg[name], bd["proj"][name])
    check_gradient("ops_features", _np(feats.grad), ref["render_grads"]["features"], bd["render"]["features"])


@pytest.mark.parametrize("live", ["centers", "conics"])
def test_ops_projection_edge_with_one_gradient(live):
    # Only one of the projection edge's float outputs reaches the loss: the
    # other arrives as None and counts as zero (gs3d/ops.py:58-86).
    scene = _scene(seed=41)
    print(f"ops projection edge, only {live} live", flush=True)
    leaves = {k: getattr(scene, k).clone().requires_grad_(True) for k in ("means", "quats", "scales", "opacities")}
    geometry = ops.prepare_gaussians(leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"],
                                     _camera(scene))
    n = len(scene.means)
    g = torch.Generator().manual_seed(7)
    gc = torch.randn((n, 2), generator=g).to(DEV) if live == "centers" else torch.zeros((n, 2), device=DEV)
    gk = torch.randn((n, 4), generator=g).to(DEV) * 0.1 if live == "conics" else torch.zeros((n, 4), device=DEV)
    out = geometry.centers if live == "centers" else geometry.conics
    (out * (gc if live == "centers" else gk)).sum().backward()
    torch.cuda.synchronize()
    full, _, _, _ = oracle.camera_prepare(_np(scene.viewmats), _np(scene.Ks), scene.width, scene.height, False)
    args = (_np(scene.means), _np(scene.quats), _np(scene.scales), _np(scene.opacities), _np(scene.viewmats), full,
            _np(scene.Ks), scene.width, scene.height, _np(geometry.radii)[None], _np(gc)[None], _np(gk)[None])
    ref = oracle.project_bwd(*args, normalize_quats=True)
    bound = oracle.project_bwd_bound(*args, np.zeros((1, n, 2)), np.zeros((1, n, 4)), normalize_quats=True)
    for name in ("means", "quats", "scales", "opacities"):
        check_gradient(f"edge_{live}_{name}", _np(leaves[name].grad), ref[name], bound[name])


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_standalone_spherical_harmonics(degree):
    n, rows = 20_000, 16
    g = torch.Generator().manual_seed(degree)
    coef = (torch.randn((n, rows, 3), generator=g) * 0.3).to(DEV).requires_grad_(True)
    dirs = torch.randn((n, 3), generator=g)
    dirs[::501] = 0.0  # zero-length directions
    dirs = dirs.to(DEV).requires_grad_(True)
    radii = torch.randint(-1, 3, (n,), generator=g, dtype=torch.int32).to(DEV)
    print(f"standalone SH degree={degree}", flush=True)
    colors = spherical_harmonics(coef, dirs, degree, radii=radii)
    up = torch.randn((n, 3), generator=g).to(DEV)
    (colors * up).sum().backward()
    torch.cuda.synchronize()
    ref_col, active = oracle.sh_fwd(_np(coef), _np(dirs), degree, radii=_np(radii))
    np.testing.assert_array_equal(_np(colors), ref_col)
    assert np.all(_np(colors)[_np(radii) <= 0] == 0)
    gco, gdir = oracle.sh_bwd(_np(coef), _np(dirs), degree, active, _np(up), radii=_np(radii))
    bco, bdir = oracle.sh_bwd_bound(_np(coef), _np(dirs), degree, active, _np(up), radii=_np(radii))
    got = _np(coef.grad)
    assert np.all(got[:, (degree + 1) ** 2:] == 0)
    check_gradient(f"sh{degree}_coefficients", got, gco, bco)
    if degree == 0:
        # Degree 0 detaches the directions (primitives/spherical_harmonics.py:150-151).
        assert dirs.grad is None
    else:
        check_gradient(f"sh{degree}_directions", _np(dirs.grad), gdir, bdir)


def test_standalone_metadata():
    scene = synthetic.make_scene("sh3_1080p_4view", n=6000, width=160, height=96, seed=17).to(DEV)
    print("standalone metadata", flush=True)
    full, _, _, _ = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height, False)
    st = gproj.project_views(scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, full,
                             scene.Ks, scene.width, scene.height, 0.2, float("inf"), 0.0, normalize_quats=True)
    rows = st.radii.numel()
    means2d = torch.empty((rows, 2), device=DEV)
    opac = torch.empty((rows,), device=DEV)
    conics = torch.empty((rows, 3), device=DEV)
    native.call("gs3d_metadata", native.ptr(st.radii), native.ptr(st.centers), native.ptr(st.conics), rows,
                native.ptr(means2d), native.ptr(opac), native.ptr(conics), native.stream(means2d.device))
    ref = oracle.project_fwd(_np(scene.means), _np(scene.quats), _np(scene.scales), _np(scene.opacities),
                             _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height, metadata=True,
                             normalize_quats=True)
    np.testing.assert_array_equal(_np(means2d).reshape(ref["means2d"].shape), ref["means2d"])
    np.testing.assert_array_equal(_np(opac).reshape(ref["meta_opacities"].shape), ref["meta_opacities"])
    np.testing.assert_array_equal(_np(conics).reshape(ref["meta_conics"].shape), ref["meta_conics"])
    assert (ref["radii"] == 0).any() and (ref["radii"] > 0).any()


@pytest.mark.parametrize("with_sorted_keys", [False, True])
def test_sort_tile_pairs_reference_convention(with_sorted_keys):
    scene = synthetic.make_scene("sh3_1080p_4view", n=8000, width=176, height=112, seed=23).to(DEV)
    print(f"sort_tile_pairs sorted_keys={with_sorted_keys}", flush=True)
    full, _, _, _ = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height, False)
    st = gproj.project_views(scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, full,
                             scene.Ks, scene.width, scene.height, 0.2, float("inf"), 0.0, normalize_quats=True)
    offsets, count = tiling.scan_counts(st.tile_counts)
    keys, ids = binning.emit_keys(st.centers, st.radii, st.depths, offsets, count, scene.width, scene.height)
    tiles = binning.tile_count(scene.width, scene.height, scene.viewmats.shape[0])
    ranges = torch.zeros((tiles, 2), dtype=torch.int32, device=DEV)
    unsorted_keys, unsorted_ids = _np(keys[:count]).view(np.uint64).copy(), _np(ids[:count]).copy()
    tiling.sort_tile_pairs(keys, ids, count, ranges, None, sorted_keys=keys[:count] if with_sorted_keys else None)
    torch.cuda.synchronize()
    sk, sv = oracle.sort_pairs(unsorted_keys, unsorted_ids, 32 + tiles.bit_length())
    np.testing.assert_array_equal(_np(keys[:count]).view(np.uint64), sk)
    np.testing.assert_array_equal(_np(ids[:count]), sv)
    np.testing.assert_array_equal(_np(ranges), oracle.tile_ranges(sk, tiles))
    assert count > 10_000
