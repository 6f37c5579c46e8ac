"""Stage-by-stage parity of the HIP kernels with the CPU oracle.

Integer stages (radii, tile counts, offsets, sorted keys/values, ranges,
contributors) are compared bit-exactly; the forward float stages follow the
same operation sequence as the oracle and are compared bit-exactly too;
every gradient entry (atomically accumulated in another order) is within
rtol 1e-4 / atol 1e-5 of the oracle's or within its stated float32 error
bound (oracle_pipeline.check_gradient).
"""

import numpy as np
import pytest
import torch

import oracle
from oracle_pipeline import check_gradient, compare
from dsl_splat_amd import gs3d, synthetic
from dsl_splat_amd.gs3d import projection as gproj
from dsl_splat_amd.gs3d import render as grender
from dsl_splat_amd.primitives import tiling
from dsl_splat_amd.runtime import native
from dsl_splat_amd.splatting import binning, cameras

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


def _say(*args):
    print(*args, flush=True)


# Frames of fewer than 4096 tiles (all views) blend at one pixel per lane,
# larger ones at two: the "wide" scenes (4320 tiles) cover the two-pixel
# kernels.
SCENES = {
    "small_rgb": dict(name="small", n=4000, width=128, height=96, seed=1),
    "sh3_4view": dict(name="sh3_1080p_4view", n=6000, width=160, height=96, seed=2),
    "sh3_720p": dict(name="sh3_720p", n=5000, width=200, height=120, seed=3),
    "wide_rgb": dict(name="small", n=16000, width=1152, height=960, seed=11),
    "wide_sh3_4view": dict(name="sh3_1080p_4view", n=12000, width=576, height=480, seed=12),
    # 4 tile groups and ~1.5M group items: the group sort's 32 digit rows
    # over more than 512 sort tiles take the two-launch digit scan.
    "dense_small": dict(name="small", n=1_500_000, width=256, height=256, seed=21),
}


def _scene(key):
    cfg = dict(SCENES[key])
    name = cfg.pop("name")
    return synthetic.make_scene(name, **cfg).to(DEV)


def _project(scene, sh_degree=None):
    quats = torch.nn.functional.normalize(scene.quats, dim=-1)
    with_centers = sh_degree is not None and sh_degree > 0
    full, inverse, centers, errors = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height,
                                                            with_centers)
    state = gproj.project_views(
        scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks, scene.width,
        scene.height, 0.2, float("inf"), 0.0, sh=scene.sh_coeffs if sh_degree is not None else None,
        sh_degree=sh_degree or 0, camera_centers=centers if with_centers else None, metadata=True)
    return quats, full, inverse, centers, errors, state


def _oracle_project_bwd(*args, **kw):
    """oracle.project_bwd and the per-entry float32 bounds of its outputs
    (upstream gradients exact: both sides read the same tensors)."""
    ref = oracle.project_bwd(*args, **kw)
    views, n = np.asarray(args[9]).shape
    zeros = dict(e_centers=np.zeros((views, n, 2)), e_conics=np.zeros((views, n, 4)))
    if kw.get("sh") is not None:
        zeros["e_colors"] = np.zeros((views, n, 3))
    bound = oracle.project_bwd_bound(*args, **zeros, **kw)
    return ref, bound


def _oracle_render_bwd(width, height, ranges, ids, centers, conics, feats, final_t, contributors, up, **kw):
    """oracle.render_bwd and the per-entry float32 bounds of its outputs."""
    absgrad = kw.pop("absgrad", False)
    args = (width, height, ranges, ids, centers, conics, feats, final_t, contributors, up)
    return oracle.render_bwd(*args, absgrad=absgrad, **kw), oracle.render_bwd_bound(*args, **kw)


def test_camera_prepare_bit_exact():
    scene = _scene("sh3_4view")
    _say("camera_prepare sh3_4view")
    full, inverse, centers, errors = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height, True)
    torch.cuda.synchronize()
    of, oi, oc, oe = oracle.camera_prepare(_np(scene.viewmats), _np(scene.Ks), scene.width, scene.height, True)
    np.testing.assert_array_equal(_np(errors), oe)
    np.testing.assert_array_equal(_np(full), of)
    np.testing.assert_array_equal(_np(inverse), oi)
    np.testing.assert_array_equal(_np(centers), oc)
    bad = scene.Ks.clone()
    bad[0, 0, 1] = 0.5
    bad[1, 1, 1] = -2.0
    _, _, _, e2 = cameras.launch_prepare(scene.viewmats, bad, scene.width, scene.height, True)
    assert _np(e2).tolist() == [1, 2, 0, 0]


@pytest.mark.parametrize("key,degree", [("small_rgb", None), ("sh3_4view", 3), ("sh3_720p", 0), ("sh3_720p", 1),
                                        ("sh3_720p", 2), ("sh3_720p", 3)])
def test_projection_forward_bit_exact(key, degree):
    scene = _scene(key)
    _say(f"projection fwd {key} degree={degree}")
    quats, full, inverse, centers, errors, st = _project(scene, degree)
    torch.cuda.synchronize()
    ref = oracle.project_fwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                             _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height,
                             sh=_np(scene.sh_coeffs) if degree is not None else None, sh_degree=degree or 0,
                             camera_centers=_np(centers) if degree else None, metadata=True)
    for name, got in (("radii", st.radii), ("tiles", st.tile_counts), ("centers", st.centers),
                      ("conics", st.conics), ("depths", st.depths), ("means2d", st.means2d),
                      ("meta_opacities", st.opacities), ("meta_conics", st.meta_conics)):
        np.testing.assert_array_equal(_np(got), ref[name], err_msg=name)
    if degree is not None:
        np.testing.assert_array_equal(_np(st.colors), ref["colors"], err_msg="colors")
    assert (_np(st.radii) > 0).mean() > 0.3


def test_per_view_sh_projection():
    scene = _scene("sh3_4view")
    per_view = torch.randn((4,) + tuple(scene.sh_coeffs.shape), device=DEV) * 0.3
    scene.sh_coeffs = per_view
    _say("projection fwd per-view SH")
    quats, full, inverse, centers, errors, st = _project(scene, 2)
    ref = oracle.project_fwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                             _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height,
                             sh=_np(per_view), sh_degree=2, camera_centers=_np(centers))
    np.testing.assert_array_equal(_np(st.colors), ref["colors"])


@pytest.mark.parametrize("n", [1, 1000, 4096, 4097, 12_000, 16_384, 16_385, 300_001, 5_000_000])
def test_scan_bit_exact(n):
    _say(f"scan n={n}")
    g = torch.Generator().manual_seed(n)
    counts = torch.randint(0, 50, (n,), generator=g, dtype=torch.int32)
    offsets, total = tiling.scan_device(counts.to(DEV))
    ref = np.cumsum(counts.numpy().astype(np.int64))
    np.testing.assert_array_equal(_np(offsets).astype(np.int64), ref)
    assert int(total.item()) == int(ref[-1])


@pytest.mark.parametrize("count,end_bit", [(1, 45), (5, 41), (4095, 40), (4096, 45), (70_001, 47), (3_000_000, 45)])
def test_radix_sort_stable_bit_exact(count, end_bit):
    _say(f"sort count={count} end_bit={end_bit}")
    rng = np.random.default_rng(count)
    hi = rng.integers(0, 1 << (end_bit - 32), size=count, dtype=np.uint64)
    lo = rng.integers(0, 1 << 10, size=count, dtype=np.uint64) << np.uint64(20)  # many ties
    keys = (hi << np.uint64(32)) | lo
    vals = rng.integers(0, 1 << 30, size=count).astype(np.int32)
    k = torch.empty(2 * count, dtype=torch.int64, device=DEV)
    v = torch.empty(2 * count, dtype=torch.int32, device=DEV)
    k[:count] = torch.from_numpy(keys.view(np.int64)).to(DEV)
    v[:count] = torch.from_numpy(vals).to(DEV)
    tiling.sort_pairs(k, v, count, end_bit)
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(_np(k[:count]).view(np.uint64), keys[order])
    np.testing.assert_array_equal(_np(v[:count]), vals[order])


@pytest.mark.parametrize("key,degree", [("small_rgb", None), ("sh3_4view", 3)])
def test_binning_bit_exact(key, degree):
    scene = _scene(key)
    _say(f"binning {key}")
    quats, full, inverse, centers, errors, st = _project(scene, degree)
    offsets, count = tiling.scan_counts(st.tile_counts)
    bins = binning.emit_and_sort(st.centers, st.radii, st.depths, offsets, count, scene.width, scene.height)
    ro, rtotal = oracle.scan_i32(_np(st.tile_counts).ravel())
    assert rtotal == count
    np.testing.assert_array_equal(_np(offsets), ro)
    keys, vals = oracle.emit_keys(_np(st.centers), _np(st.radii), _np(st.depths), ro, rtotal, scene.width,
                                  scene.height)
    views = scene.viewmats.shape[0]
    T = views * ((scene.width + 15) // 16) * ((scene.height + 15) // 16)
    sk, sv = oracle.sort_pairs(keys, vals, 32 + int(T).bit_length())
    np.testing.assert_array_equal(_np(bins["point_list_keys"]).view(np.uint64), sk)
    np.testing.assert_array_equal(_np(bins["point_list"]), sv)
    np.testing.assert_array_equal(_np(bins["ranges"]), oracle.tile_ranges(sk, T))


def _frame(scene, degree):
    quats, full, inverse, centers, errors, st = _project(scene, degree)
    offsets, count = tiling.scan_counts(st.tile_counts)
    bins = binning.emit_and_sort(st.centers, st.radii, st.depths, offsets, count, scene.width, scene.height)
    return quats, full, inverse, centers, st, bins


@pytest.mark.parametrize("key,degree,extra,bg", [("small_rgb", None, False, True), ("sh3_4view", 3, False, False),
                                                 ("small_rgb", None, True, True), ("wide_rgb", None, True, True),
                                                 ("wide_sh3_4view", 3, False, False)])
def test_render_forward_bit_exact(key, degree, extra, bg):
    scene = _scene(key)
    _say(f"render fwd {key} extra={extra} bg={bg}")
    quats, full, inverse, centers, st, bins = _frame(scene, degree)
    views = scene.viewmats.shape[0]
    feats = st.colors if degree is not None else scene.features
    ex = torch.randn((st.radii.shape[1], 2), device=DEV) if extra else None
    background = torch.rand((views, 3), device=DEV) if bg else None
    out = grender.render_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats, scene.width,
                               scene.height, extra=ex, background=background)
    img, ft, ct = oracle.render_fwd(scene.width, scene.height, _np(bins["ranges"]), _np(bins["point_list"]),
                                    _np(st.centers), _np(st.conics), _np(feats), extra=None if ex is None else _np(ex),
                                    background=None if background is None else _np(background))
    np.testing.assert_array_equal(_np(out.contributors), ct)
    np.testing.assert_array_equal(_np(out.transmittance), ft)
    np.testing.assert_array_equal(_np(out.stacked()), img)
    assert ct.max() > 0


@pytest.mark.parametrize("n,width,height", [(3000, 136, 100), (12000, 1152, 960)])
def test_render_culling_edge_cases(n, width, height):
    # Needle-shaped Gaussians at every orientation and opacities straddling
    # the 1/255 threshold: the per-wavefront strip culling must not change a
    # single forward bit or the gradients (one and two pixels per lane).
    _say(f"render culling edge cases {width}x{height}")
    scene = synthetic.make_scene("small", n=n, width=width, height=height, seed=5)
    g = torch.Generator().manual_seed(7)
    n = scene.means.shape[0]
    long_axis = torch.exp(torch.rand(n, generator=g) * 2.0 - 3.0)
    thin_axis = torch.exp(torch.rand(n, generator=g) * 3.0 - 7.5)
    scene.scales = torch.stack([long_axis, thin_axis, thin_axis], dim=1)
    opac = torch.rand(n, generator=g)
    opac[::3] = 1.0 / 255.0 + (torch.rand(len(opac[::3]), generator=g) - 0.5) * 2e-4
    opac[1::7] = 0.999
    scene.opacities = opac
    scene = scene.to(DEV)
    quats, full, inverse, centers, st, bins = _frame(scene, None)
    feats = scene.features
    out = grender.render_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats, scene.width,
                               scene.height)
    img, ft, ct = oracle.render_fwd(scene.width, scene.height, _np(bins["ranges"]), _np(bins["point_list"]),
                                    _np(st.centers), _np(st.conics), _np(feats))
    np.testing.assert_array_equal(_np(out.contributors), ct)
    np.testing.assert_array_equal(_np(out.transmittance), ft)
    np.testing.assert_array_equal(_np(out.stacked()), img)
    up = torch.randn(out.stacked().shape, device=DEV)
    record, gf, _ = grender.backward_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats,
                                           out.transmittance, out.contributors, up, scene.width, scene.height,
                                           absgrad=True)
    ref, bound = _oracle_render_bwd(scene.width, scene.height, _np(bins["ranges"]), _np(bins["point_list"]),
                                    _np(st.centers), _np(st.conics), _np(feats), _np(out.transmittance),
                                    _np(out.contributors), _np(up), absgrad=True)
    rec = _np(record)
    for name, got in (("centers", rec[..., 0:2]), ("conics", rec[..., 2:6]), ("abs", rec[..., 6:8]),
                      ("features", _np(gf))):
        check_gradient(name, got, ref[name], bound[name])


@pytest.mark.parametrize("key,degree,absgrad", [("small_rgb", None, True), ("sh3_4view", 3, False),
                                                ("wide_rgb", None, True), ("wide_sh3_4view", 3, False)])
def test_render_backward_parity(key, degree, absgrad):
    scene = _scene(key)
    _say(f"render bwd {key}")
    quats, full, inverse, centers, st, bins = _frame(scene, degree)
    views = scene.viewmats.shape[0]
    feats = st.colors if degree is not None else scene.features
    background = torch.rand((views, 3), device=DEV)
    out = grender.render_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats, scene.width,
                               scene.height, background=background)
    up = torch.randn(out.stacked().shape, device=DEV)
    record, gf, _ = grender.backward_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats,
                                           out.transmittance, out.contributors, up, scene.width, scene.height,
                                           background=background, absgrad=absgrad)
    ref, bound = _oracle_render_bwd(scene.width, scene.height, _np(bins["ranges"]), _np(bins["point_list"]),
                                    _np(st.centers), _np(st.conics), _np(feats), _np(out.transmittance),
                                    _np(out.contributors), _np(up), background=_np(background), absgrad=absgrad)
    rec = _np(record)
    for name, got in (("centers", rec[..., 0:2]), ("conics", rec[..., 2:6]), ("features", _np(gf))):
        check_gradient(name, got, ref[name], bound[name])
    if absgrad:
        check_gradient("abs", rec[..., 6:8], ref["abs"], bound["abs"])


@pytest.mark.parametrize("key", ["small_rgb", "wide_rgb"])
def test_render_forward_non_finite_features(key):
    # The forward blend adds a rejected Gaussian's channels with a zero weight
    # only when they are all finite; a Gaussian with a NaN or infinite channel
    # is skipped by a select, as the reference's loop skips it.  The image
    # equals the oracle's bit for bit, NaN and inf included.
    scene = _scene(key)
    _say(f"render fwd non-finite features {key}")
    quats, full, inverse, centers, st, bins = _frame(scene, None)
    visible = torch.nonzero(st.radii[0] > 0).flatten()
    feats = scene.features.clone()
    feats[visible[:3], 0] = float("nan")
    feats[visible[3:5], 2] = float("inf")
    feats[visible[5:7], 1] = -float("inf")
    out = grender.render_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats, scene.width,
                               scene.height)
    img, ft, ct = oracle.render_fwd(scene.width, scene.height, _np(bins["ranges"]), _np(bins["point_list"]),
                                    _np(st.centers), _np(st.conics), _np(feats))
    got = _np(out.stacked())
    assert not np.isfinite(img).all()
    np.testing.assert_array_equal(got, img)
    np.testing.assert_array_equal(_np(out.contributors), ct)
    np.testing.assert_array_equal(_np(out.transmittance), ft)


@pytest.mark.parametrize("key", ["small_rgb", "wide_rgb"])
def test_render_backward_non_finite_inputs(key):
    # The backward's fast traversal adds a rejected pixel's terms with zero
    # weights; whenever an operand may be non-finite it must skip them as the
    # reference's loop does.  NaN features, a NaN upstream gradient and an
    # infinite conic entry (staged after a finite forward, so the lists and
    # transmittances are ordinary) must give the oracle's results: NaN exactly
    # where the oracle has NaN, every other entry within the criterion.
    scene = _scene(key)
    _say(f"render bwd non-finite {key}")
    quats, full, inverse, centers, st, bins = _frame(scene, None)
    feats = scene.features
    out = grender.render_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats, scene.width,
                               scene.height)
    up = torch.randn(out.stacked().shape, device=DEV)
    visible = torch.nonzero(st.radii[0] > 0).flatten()
    feats = feats.clone()
    feats[visible[:3], 1] = float("nan")
    conics = st.conics.clone()
    conics[0, visible[3:5], 0] = float("inf")
    up[0, scene.height // 2, scene.width // 3, 0] = float("nan")
    record, gf, _ = grender.backward_views(bins["ranges"], bins["point_list"], st.centers, conics, feats,
                                           out.transmittance, out.contributors, up, scene.width, scene.height,
                                           absgrad=True)
    ref, bound = _oracle_render_bwd(scene.width, scene.height, _np(bins["ranges"]), _np(bins["point_list"]),
                                    _np(st.centers), _np(conics), _np(feats), _np(out.transmittance),
                                    _np(out.contributors), _np(up), absgrad=True)
    rec = _np(record)
    nans = 0
    for name, got in (("centers", rec[..., 0:2]), ("conics", rec[..., 2:6]), ("abs", rec[..., 6:8]),
                      ("features", _np(gf))):
        nan_got, nan_ref = np.isnan(got), np.isnan(ref[name])
        nans += int(nan_ref.sum())
        np.testing.assert_array_equal(nan_got, nan_ref, err_msg=name)
        keep = ~nan_ref
        check_gradient(name, got[keep], ref[name][keep], np.broadcast_to(bound[name], ref[name].shape)[keep])
    assert nans > 0


# Blended-channel widths D' = features + extra + 1 covering every compiled
# channel window: one window (D' <= 56: kernels of 4, 8, 16, 36 and 56
# channels), the geometry window of 56 followed by feature windows (57-64,
# where all gradient entries no longer fit one 64-lane sum), and forward
# windows of 64 (D' > 64).
@pytest.mark.parametrize("feat,extra,absgrad", [(11, 0, True), (15, 0, False), (37, 2, True), (55, 0, True),
                                                (57, 0, False), (56, 3, True), (60, 3, True), (70, 1, True),
                                                (128, 2, False)])
def test_render_channel_windows(feat, extra, absgrad):
    scene = synthetic.make_scene("small", n=1500, width=72, height=56, seed=feat + extra).to(DEV)
    D = feat + extra + 1
    _say(f"render channel windows D'={D} absgrad={absgrad}")
    quats, full, inverse, centers, st, bins = _frame(scene, None)
    g = torch.Generator().manual_seed(D)
    feats = torch.randn((scene.means.shape[0], feat), generator=g).to(DEV)
    ex = torch.randn((scene.means.shape[0], extra), generator=g).to(DEV) if extra else None
    background = torch.rand((1, feat), generator=g).to(DEV)
    out = grender.render_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats, scene.width,
                               scene.height, extra=ex, background=background)
    img, ft, ct = oracle.render_fwd(scene.width, scene.height, _np(bins["ranges"]), _np(bins["point_list"]),
                                    _np(st.centers), _np(st.conics), _np(feats), extra=None if ex is None else _np(ex),
                                    background=_np(background))
    np.testing.assert_array_equal(_np(out.contributors), ct)
    np.testing.assert_array_equal(_np(out.transmittance), ft)
    np.testing.assert_array_equal(_np(out.stacked()), img)
    up = torch.randn(out.stacked().shape, generator=g).to(DEV)
    record, gf, ge = grender.backward_views(bins["ranges"], bins["point_list"], st.centers, st.conics, feats,
                                            out.transmittance, out.contributors, up, scene.width, scene.height,
                                            extra=ex, background=background, absgrad=absgrad)
    ref, bound = _oracle_render_bwd(scene.width, scene.height, _np(bins["ranges"]), _np(bins["point_list"]),
                                    _np(st.centers), _np(st.conics), _np(feats), _np(out.transmittance),
                                    _np(out.contributors), _np(up), extra=None if ex is None else _np(ex),
                                    background=_np(background), absgrad=absgrad)
    rec = _np(record)
    checks = [("centers", rec[..., 0:2]), ("conics", rec[..., 2:6]), ("features", _np(gf))]
    if absgrad:
        checks.append(("abs", rec[..., 6:8]))
    if extra:
        checks.append(("extra", _np(ge)))
    for name, got in checks:
        check_gradient(name, got, ref[name], bound[name])
    # Every feature channel received gradient (a window that lost its entries
    # would leave zeros).
    assert np.all(np.abs(_np(gf)).max(axis=0) > 0)


@pytest.mark.parametrize("key,degree", [("small_rgb", None), ("sh3_4view", 3), ("sh3_720p", 1)])
def test_projection_backward_parity(key, degree):
    scene = _scene(key)
    _say(f"projection bwd {key} degree={degree}")
    quats, full, inverse, centers, errors, st = _project(scene, degree)
    views, n = st.radii.shape
    g = torch.Generator().manual_seed(5)
    gc = torch.randn((views, n, 2), generator=g).to(DEV)
    gk = torch.randn((views, n, 4), generator=g).to(DEV) * 0.1
    gcol = torch.randn((views, n, 3), generator=g).to(DEV) if degree is not None else None
    res = gproj.backward_views(scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks,
                               scene.width, scene.height, st.radii, gc, gk, (True,) * 6,
                               sh=scene.sh_coeffs if degree is not None else None, sh_degree=degree or 0,
                               camera_centers=centers if degree else None, grad_colors=gcol,
                               need_sh=degree is not None, need_centers=bool(degree), need_screen=True)
    # The contiguous screen gradient is grad_centers where radii > 0 and zero elsewhere, bit for bit.
    visible = (st.radii > 0).unsqueeze(-1)
    assert torch.equal(res["screen"], torch.where(visible, gc, torch.zeros_like(gc)))
    ref, bound = _oracle_project_bwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                             _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height, _np(st.radii),
                             _np(gc), _np(gk), sh=_np(scene.sh_coeffs) if degree is not None else None,
                             sh_degree=degree or 0, camera_centers=_np(centers) if degree else None,
                             grad_colors=None if gcol is None else _np(gcol))
    for name in ("means", "quats", "scales", "opacities"):
        check_gradient(name, _np(res[name]), ref[name], bound[name])
    for name in ("view", "projection"):
        check_gradient(name, _np(res[name]), ref[name], bound[name])
    if degree is not None:
        check_gradient("sh", _np(res["sh"]), ref["sh"], bound["sh"])
    if degree:
        check_gradient("camera_centers", _np(res["camera_centers"]), ref["camera_centers"], bound["camera_centers"])


@pytest.mark.parametrize("degree", [1, 3])
def test_projection_sh_shared_many_views(degree):
    # Shared coefficients seen by 7 cameras: more views than the SH kernels
    # take in one group, so the colour pass loads later radii in the loop
    # and the coefficient gradients of later groups are added to the stored
    # rows; camera-centre gradients on.
    scene = _scene("sh3_4view")
    _say(f"projection shared SH, 7 views, degree={degree}")
    order = [0, 1, 2, 3, 1, 3, 0]
    viewmats = scene.viewmats[order].contiguous()
    viewmats[4:, :3, 3] += torch.tensor([0.3, -0.2, 0.1], device=DEV)
    Ks = scene.Ks[order].contiguous()
    views, n = viewmats.shape[0], scene.means.shape[0]
    quats = torch.nn.functional.normalize(scene.quats, dim=-1)
    full, inverse, centers, errors = cameras.launch_prepare(viewmats, Ks, scene.width, scene.height, True)
    st = gproj.project_views(scene.means, quats, scene.scales, scene.opacities, viewmats, full, Ks,
                             scene.width, scene.height, 0.2, float("inf"), 0.0, sh=scene.sh_coeffs,
                             sh_degree=degree, camera_centers=centers, metadata=True)
    ref_f = oracle.project_fwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                               _np(viewmats), _np(full), _np(Ks), scene.width, scene.height,
                               sh=_np(scene.sh_coeffs), sh_degree=degree, camera_centers=_np(centers), metadata=True)
    assert (st.radii > 0).sum() > 0
    np.testing.assert_array_equal(_np(st.colors), ref_f["colors"])
    g = torch.Generator().manual_seed(13)
    gc = torch.randn((views, n, 2), generator=g).to(DEV)
    gk = torch.randn((views, n, 4), generator=g).to(DEV) * 0.1
    gcol = torch.randn((views, n, 3), generator=g).to(DEV)
    res = gproj.backward_views(scene.means, quats, scene.scales, scene.opacities, viewmats, full, Ks,
                               scene.width, scene.height, st.radii, gc, gk, (True,) * 6, sh=scene.sh_coeffs,
                               sh_degree=degree, camera_centers=centers, grad_colors=gcol, need_sh=True,
                               need_centers=True)
    ref, bound = _oracle_project_bwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                             _np(viewmats), _np(full), _np(Ks), scene.width, scene.height, _np(st.radii),
                             _np(gc), _np(gk), sh=_np(scene.sh_coeffs), sh_degree=degree,
                             camera_centers=_np(centers), grad_colors=_np(gcol))
    got_sh = _np(res["sh"])
    assert np.all(got_sh[..., (degree + 1) ** 2:, :] == 0.0)
    check_gradient("sh", got_sh, ref["sh"], bound["sh"])
    check_gradient("means", _np(res["means"]), ref["means"], bound["means"])
    check_gradient("camera_centers", _np(res["camera_centers"]), ref["camera_centers"], bound["camera_centers"])


@pytest.mark.parametrize("degree", [2, 3])
def test_projection_per_view_sh_parity(degree):
    # Per-view coefficients (C,N,16,3) and, for degree 2, coefficient rows
    # beyond (degree+1)^2 whose gradients must come back as zeros.
    scene = _scene("sh3_4view")
    _say(f"projection per-view SH degree={degree}")
    views, n = scene.viewmats.shape[0], scene.means.shape[0]
    g = torch.Generator().manual_seed(11)
    sh = (scene.sh_coeffs.cpu()[None] + 0.05 * torch.randn((views,) + tuple(scene.sh_coeffs.shape), generator=g))
    sh = sh.contiguous().to(DEV)
    quats = torch.nn.functional.normalize(scene.quats, dim=-1)
    full, inverse, centers, errors = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height, True)
    st = gproj.project_views(scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks,
                             scene.width, scene.height, 0.2, float("inf"), 0.0, sh=sh, sh_degree=degree,
                             camera_centers=centers, metadata=True)
    ref_f = oracle.project_fwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                               _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height, sh=_np(sh),
                               sh_degree=degree, camera_centers=_np(centers), metadata=True)
    np.testing.assert_array_equal(_np(st.colors), ref_f["colors"])
    gc = torch.randn((views, n, 2), generator=g).to(DEV)
    gk = torch.randn((views, n, 4), generator=g).to(DEV) * 0.1
    gcol = torch.randn((views, n, 3), generator=g).to(DEV)
    res = gproj.backward_views(scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks,
                               scene.width, scene.height, st.radii, gc, gk, (True,) * 6, sh=sh, sh_degree=degree,
                               camera_centers=centers, grad_colors=gcol, need_sh=True, need_centers=True)
    ref, bound = _oracle_project_bwd(_np(scene.means), _np(quats), _np(scene.scales), _np(scene.opacities),
                             _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height, _np(st.radii),
                             _np(gc), _np(gk), sh=_np(sh), sh_degree=degree, camera_centers=_np(centers),
                             grad_colors=_np(gcol))
    got_sh = _np(res["sh"])
    assert got_sh.shape == sh.shape
    kc = (degree + 1) ** 2
    assert np.all(got_sh[..., kc:, :] == 0.0)
    check_gradient("sh", got_sh, ref["sh"], bound["sh"])
    check_gradient("means", _np(res["means"]), ref["means"], bound["means"])
    check_gradient("camera_centers", _np(res["camera_centers"]), ref["camera_centers"], bound["camera_centers"])


@pytest.mark.parametrize("key,degree", [("small_rgb", None), ("sh3_4view", 3), ("sh3_720p", 0),
                                        ("dense_small", None)])
def test_grouped_binning_matches_reference_order(key, degree):
    # The production binning (depth-ordered rows, 8x8-tile groups, ballot
    # ranking) must give exactly the reference's ids, ranges and 64-bit keys
    # (scan + duplicate in Gaussian order + stable sort of
    # (tile << 32 | depth bits)).
    scene = _scene(key)
    _say(f"grouped binning {key}")
    quats, full, inverse, centers, errors, st = _project(scene, degree)
    bins = binning.bin_and_sort(st.centers, st.radii, st.tile_counts, st.depths, scene.width, scene.height,
                                with_keys=True)
    ro, rtotal = oracle.scan_i32(_np(st.tile_counts).ravel())
    keys, vals = oracle.emit_keys(_np(st.centers), _np(st.radii), _np(st.depths), ro, rtotal, scene.width,
                                  scene.height)
    views = scene.viewmats.shape[0]
    T = views * ((scene.width + 15) // 16) * ((scene.height + 15) // 16)
    sk, sv = oracle.sort_pairs(keys, vals, 32 + int(T).bit_length())
    assert len(sv) == bins["point_list"].numel() > 0
    np.testing.assert_array_equal(_np(bins["point_list"]), sv)
    np.testing.assert_array_equal(_np(bins["point_list_keys"]).view(np.uint64), sk)
    np.testing.assert_array_equal(_np(bins["ranges"]), oracle.tile_ranges(sk, T))
    if key == "dense_small":
        # Group items = distinct (Gaussian, 8x8-tile group) of the pairs:
        # more than 512 sort tiles of 2048 items.
        gx = (scene.width + 15) // 16
        tile = (sk >> np.uint64(32)).astype(np.int64)
        group = (tile // gx >> 3) * 64 + (tile % gx >> 3)
        assert np.unique(sv.astype(np.int64) * 4096 + group).size > 512 * 2048


@pytest.mark.parametrize("views,n,W,H,spread", [
    (2, 3000, 200, 120, 1.0),      # partial groups at the right/bottom edges, several chunks per group
    (1, 40000, 128, 128, 0.15),    # crowded corner: long group lists, many 512-item chunks
    (70, 400, 160, 160, 1.0),      # 280 groups: one 10-bit pass, ranges from its digit scan
    (12, 200, 1024, 1024, 1.0),    # 768 groups: the most the group sort's 768-counter kernels take
    (13, 200, 1024, 1024, 1.0),    # 832 groups: 1024 counters per digit row
    (16, 200, 1024, 1024, 1.0),    # 1024 groups: the largest one-pass group sort
    (41, 150, 640, 640, 1.0),      # 1025 groups: two 8-bit passes and a range search
    (130, 250, 400, 400, 1.0),     # 2080 groups: 12-bit group keys
    (1, 2000, 4200, 64, 1.0),      # 263 tiles across: rectangles recomputed instead of packed in the records
])
def test_grouped_binning_ties_and_large_rects(views, n, W, H, spread):
    # Equal depths everywhere (ties broken by Gaussian index) and rectangles
    # spanning the whole image (rows touching every group).
    _say(f"grouped binning ties views={views} n={n} {W}x{H}")
    g = torch.Generator().manual_seed(3)
    centers = (torch.rand((views, n, 2), generator=g) * spread * torch.tensor([W, H])).to(DEV)
    radii = torch.randint(1, 40, (views, n), generator=g, dtype=torch.int32)
    radii[:, ::97] = 500
    radii[:, 5::13] = 0
    depths = torch.full((views, n), 2.5)
    depths[:, ::7] = 1.25
    depths[radii == 0] = 0.0
    radii, depths = radii.to(DEV), depths.to(DEV)
    gx, gy = (W + 15) // 16, (H + 15) // 16
    c = _np(centers)
    r = _np(radii)
    tiles = np.zeros((views, n), np.int32)
    import torch_ref
    for v in range(views):
        for i in range(n):
            if r[v, i] > 0:
                x0, y0, x1, y1 = torch_ref.rect_tiles(c[v, i], r[v, i], W, H)
                tiles[v, i] = (x1 - x0) * (y1 - y0)
    r[tiles == 0] = 0
    radii = torch.from_numpy(r).to(DEV)
    tiles_t = torch.from_numpy(tiles).to(DEV)
    bins = binning.bin_and_sort(centers, radii, tiles_t, depths, W, H, with_keys=True)
    ro, rtotal = oracle.scan_i32(tiles.ravel())
    keys, vals = oracle.emit_keys(c, r, _np(depths), ro, rtotal, W, H)
    T = views * gx * gy
    sk, sv = oracle.sort_pairs(keys, vals, 32 + int(T).bit_length())
    np.testing.assert_array_equal(_np(bins["point_list"]), sv)
    np.testing.assert_array_equal(_np(bins["point_list_keys"]).view(np.uint64), sk)
    np.testing.assert_array_equal(_np(bins["ranges"]), oracle.tile_ranges(sk, T))


@pytest.mark.parametrize("key,degree,mode", [("small_rgb", None, "radius"), ("sh3_4view", 3, "radius"),
                                             ("sh3_720p", 0, "snugbox")])
def test_group_items_emitted_before_the_totals(key, degree, mode, monkeypatch):
    # The emission enqueued before the host reads the totals (capacity from an
    # earlier frame) must give exactly gs3d_bin_rows' ids and ranges when the
    # capacity holds every item, and fall back to gs3d_bin_rows when not.
    scene = _scene(key)
    _say(f"early group items {key} {mode}")
    quats, full, inverse, centers, errors, st = _project(scene, degree)
    W, H = scene.width, scene.height
    order, offsets, totals = binning.order_rows(st.centers, st.radii, st.depths, W, H, conics=st.conics,
                                                tile_mode=mode)
    S, M = totals.cpu().tolist()
    assert S > 1
    ref_ranges, ref_ids = binning.bin_rows(st.centers, st.radii, order, offsets, S, M, W, H, conics=st.conics,
                                           tile_mode=mode)
    calls = []
    real_call = binning.native.call
    monkeypatch.setattr(binning.native, "call", lambda name, *a: (calls.append(name), real_call(name, *a))[1])
    for capacity in (S, S + 4097, S - 1, S // 2):
        launch = binning.prepare_bin_rows(st.centers, st.radii, order, offsets, W, H, conics=st.conics,
                                          tile_mode=mode)
        key_ = binning._shape_key(launch)
        binning._CAPACITY[key_] = capacity
        calls.clear()
        try:
            early = binning.emit_early(launch)
            assert early is not None and early.capacity == capacity
            ranges, ids = binning.launch_bin_rows(launch, S, M, early)
        finally:
            binning._CAPACITY.pop(key_, None)
        expect = "gs3d_bin_emitted_rows" if capacity >= S else "gs3d_bin_rows"
        assert calls == ["gs3d_emit_group_items", expect], calls
        np.testing.assert_array_equal(_np(ids), _np(ref_ids))
        np.testing.assert_array_equal(_np(ranges), _np(ref_ranges))


def test_rasterize_reuses_the_group_item_capacity():
    # A second frame of the same shape takes the early emission; its outputs
    # equal the first frame's bit for bit.
    scene = _scene("sh3_4view")
    _say("rasterize twice, early group items")
    binning._CAPACITY.clear()
    args = (scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks, scene.width,
            scene.height)
    first = gs3d.rasterize(*args, sh_coeffs=scene.sh_coeffs, sh_degree=3)
    assert len(binning._CAPACITY) == 1
    second = gs3d.rasterize(*args, sh_coeffs=scene.sh_coeffs, sh_degree=3)
    for a, b in ((first.features, second.features), (first.alpha, second.alpha)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("count,end_bit", [(2, 13), (4097, 15), (1_000_003, 16), (5_000_000, 32), (3, 11),
                                           (4097, 9), (1_000_003, 10), (70_001, 11), (2048, 11),
                                           (14_000_000, 24), (30_000_000, 20)])
def test_u32_radix_sort_stable(count, end_bit):
    # The digit scan's row pass takes 8-48 words a thread by the number of
    # 2048-key tiles per digit row: 1M keys 8, 5M 16, 14M 32, and 30M keys
    # (14,649 tiles) two chunks of 48.
    _say(f"u32 sort count={count} end_bit={end_bit}")
    rng = np.random.default_rng(count + 1)
    keys = rng.integers(0, 1 << end_bit, size=count, dtype=np.uint64).astype(np.uint32)
    vals = np.arange(count, dtype=np.int32)
    k = torch.empty(2 * count, dtype=torch.int32, device=DEV)
    v = torch.empty(2 * count, dtype=torch.int32, device=DEV)
    k[:count] = torch.from_numpy(keys.view(np.int32)).to(DEV)
    v[:count] = torch.from_numpy(vals).to(DEV)
    scratch = torch.empty(native.query("gs3d_sort_scratch_bytes", count), dtype=torch.uint8, device=DEV)
    native.call("gs3d_sort_pairs_u32", native.ptr(k), native.ptr(v), count, end_bit, native.ptr(scratch),
                scratch.numel(), native.stream(k.device))
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(_np(k[:count]).view(np.uint32), keys[order])
    np.testing.assert_array_equal(_np(v[:count]), vals[order])


@pytest.mark.parametrize("key,degree", [("small_rgb", None), ("sh3_4view", 3)])
def test_projection_normalizes_raw_quaternions(key, degree):
    # Raw (unnormalised, some tiny or zero) quaternions: the kernels normalise
    # them as F.normalize does and take the gradient through it; forward
    # bit-exact and gradients within tolerance of the oracle doing the same.
    scene = _scene(key)
    _say(f"projection raw quats {key}")
    g = torch.Generator().manual_seed(9)
    n = scene.means.shape[0]
    raw = scene.quats * (torch.rand((n, 1), generator=g) * 5 + 0.05).to(DEV)
    raw[::97] = 1e-14
    raw[5::211] = 0.0
    with_centers = bool(degree)
    full, inverse, centers, errors = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width, scene.height,
                                                            with_centers)
    st = gproj.project_views(scene.means, raw, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks,
                             scene.width, scene.height, 0.2, float("inf"), 0.0,
                             sh=scene.sh_coeffs if degree is not None else None, sh_degree=degree or 0,
                             camera_centers=centers if with_centers else None, metadata=True, normalize_quats=True)
    ref = oracle.project_fwd(_np(scene.means), _np(raw), _np(scene.scales), _np(scene.opacities),
                             _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height,
                             sh=_np(scene.sh_coeffs) if degree is not None else None, sh_degree=degree or 0,
                             camera_centers=_np(centers) if degree else None, metadata=True, normalize_quats=True)
    for name, got in (("radii", st.radii), ("centers", st.centers), ("conics", st.conics), ("depths", st.depths)):
        np.testing.assert_array_equal(_np(got), ref[name], err_msg=name)
    views = st.radii.shape[0]
    gc = torch.randn((views, n, 2), generator=g).to(DEV)
    gk = torch.randn((views, n, 4), generator=g).to(DEV) * 0.1
    res = gproj.backward_views(scene.means, raw, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks,
                               scene.width, scene.height, st.radii, gc, gk, (True, True, True, True, False, False),
                               normalize_quats=True)
    rb, bound = _oracle_project_bwd(_np(scene.means), _np(raw), _np(scene.scales), _np(scene.opacities),
                                    _np(scene.viewmats), _np(full), _np(scene.Ks), scene.width, scene.height,
                                    _np(st.radii), _np(gc), _np(gk), normalize_quats=True)
    for name in ("means", "quats", "scales", "opacities"):
        check_gradient(f"raw_{name}", _np(res[name]), rb[name], bound[name])


@pytest.mark.parametrize("key,degree", [("small_rgb", None), ("sh3_4view", 3)])
def test_blend_pair_counts_match_the_reference_loop(key, degree):
    # gs3d_render_pair_counts: visited pairs (list entries up to and
    # including the terminating one, gs3d/render.py:82-117) and accepted
    # blends are exact counts of the reference loop; the kernel's evaluated
    # pairs (after strip culling) lie between them.
    scene = _scene(key)
    _say(f"blend pair counts {key}")
    quats, full, inverse, centers, st, bins = _frame(scene, degree)
    feats = st.colors if degree is not None else scene.features
    got = grender.pair_counts(bins["ranges"], bins["point_list"], st.centers, st.conics, feats, scene.width,
                              scene.height)
    visited, accepted = oracle.render_pair_counts(scene.width, scene.height, _np(bins["ranges"]),
                                                  _np(bins["point_list"]), _np(st.centers), _np(st.conics),
                                                  _np(feats))
    assert (got["visited"], got["accepted"]) == (visited, accepted)
    assert accepted <= got["evaluated"] <= visited and accepted > 0


def _kept_key_bits(order, rows, depths):
    """Bit length of (largest key - smallest key with its low byte cleared)
    over the depth keys of the rows that the order kept (records before the
    fillers, packed rectangles)."""
    rec = _np(order[:rows]).view(np.uint64)
    kept = (rec >> np.uint64(32)) != np.uint64(0xFF)
    keys = _np(depths).ravel().view(np.uint32)[(rec[kept] & np.uint64(0xFFFFFFFF)).astype(np.int64)]
    if keys.size == 0:
        return 0
    return (int(keys.max()) - (int(keys.min()) & ~255)).bit_length()


@pytest.mark.parametrize("lo,hi,width", [
    (1.7, 8.3, 640),      # 25 bits of key - base across 2.0: passes of 8, 8 and 9 bits
    (2.1, 40.0, 640),     # 26 bits: 8, 8, 10
    (2.1, 3.9, 640),      # 23 bits: 8, 8, 7
    (2.0, 2.06, 640),     # 18 bits: 8, 10
    (2.0, 2.01, 640),     # 16 bits: 8, 8
    (0.05, 30.0, 640),    # 27 bits: four passes
    (2.5, 2.5, 640),      # one distinct depth: the key's low byte, sorted as 9 bits
    (1.7, 8.3, 4200),     # 263 tiles across: unpacked records
])
def test_depth_order_sorts_only_the_key_bits_in_use(lo, hi, width):
    # gs3d_order_rows with sort_bits = the bits the kept rows' depth keys
    # need (as key_bits_out reports them) gives exactly the 32-bit order:
    # records, group offsets and totals; key_bits_out equals the bit length
    # of the largest kept key minus the smallest with its low byte cleared.
    _say(f"depth order key bits [{lo}, {hi}] width {width}")
    g = torch.Generator().manual_seed(7)
    views, n, height = 3, 30_000, 480
    centers = (torch.rand((views, n, 2), generator=g) * torch.tensor([width * 1.2, height * 1.2])
               - torch.tensor([width * 0.1, height * 0.1]))
    radii = torch.randint(1, 30, (views, n), generator=g, dtype=torch.int32)
    radii[:, 3::11] = 0
    depths = lo + (hi - lo) * torch.rand((views, n), generator=g)
    depths[:, ::5] = depths[:, 1::5][:, : depths[:, ::5].shape[1]]  # ties
    centers, radii, depths = centers.to(DEV), radii.to(DEV), depths.to(DEV)
    rows = views * n
    bits = torch.full((1,), -1, dtype=torch.int32, device=DEV)
    ref_order, ref_offsets, ref_totals = binning.order_rows(centers, radii, depths, width, height, key_bits_out=bits)
    need = int(bits.item())
    packed = (width + 15) // 16 <= 256
    if packed:
        assert need == _kept_key_bits(ref_order, rows, depths)
    plans = {max(need, 9)} | ({26} if need <= 26 else set())
    for sort_bits in sorted(plans):
        bits2 = torch.full((1,), -1, dtype=torch.int32, device=DEV)
        order, offsets, totals = binning.order_rows(centers, radii, depths, width, height, sort_bits=sort_bits,
                                                    key_bits_out=bits2)
        assert int(bits2.item()) == need
        np.testing.assert_array_equal(_np(order[:rows]), _np(ref_order[:rows]))
        np.testing.assert_array_equal(_np(offsets), _np(ref_offsets))
        np.testing.assert_array_equal(_np(totals), _np(ref_totals))


def test_rasterize_redoes_the_depth_order_when_the_key_bits_grow(monkeypatch):
    # Frames of one shape sort the key bits the previous frame needed; a
    # frame whose depths need more is ordered again, and every frame's
    # output equals a frame rendered with no plan (all 32 bits).
    scene = _scene("sh3_720p")
    _say("rasterize, depth-order plan and a miss")
    binning._KEY_BITS.clear()
    calls = []
    real_call = native.call
    monkeypatch.setattr(native, "call", lambda name, *a: (calls.append(name), real_call(name, *a))[1])

    def frame(viewmats):
        calls.clear()
        out = gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, viewmats, scene.Ks,
                             scene.width, scene.height, sh_coeffs=scene.sh_coeffs, sh_degree=3)
        return out, calls.count("gs3d_order_rows")

    near = scene.viewmats.clone()
    near[..., 2, 3] -= 2.0  # camera 2 units closer: depths from ~0.5, more key bits than the 24 of "far"
    outputs = {}
    for name, vm in (("far", scene.viewmats), ("near", near)):
        binning._KEY_BITS.clear()
        outputs[name], orders = frame(vm)
        assert orders == 1
    binning._KEY_BITS.clear()
    first, orders = frame(scene.viewmats)
    plan = binning._KEY_BITS[next(iter(binning._KEY_BITS))]
    assert orders == 1 and plan <= 26, plan
    again, orders = frame(scene.viewmats)
    assert orders == 1
    closer, orders = frame(near)
    assert orders == 2  # the plan missed: ordered again with enough bits
    for got, want in ((first, outputs["far"]), (again, outputs["far"]), (closer, outputs["near"])):
        assert torch.equal(got.features, want.features)
        assert torch.equal(got.alpha, want.alpha)
    binning._KEY_BITS.clear()


@pytest.mark.parametrize("count", [0, 1, 3, 4, 1001, 262_147])
def test_forward_blend_clears_the_given_buffer(count):
    # render_views(zero=...) clears every float of the buffer (float4 body
    # and scalar tail) and blends exactly as without it.
    scene = _scene("wide_sh3_4view")
    _say(f"forward blend clears {count} floats")
    quats, full, inverse, centers, errors, st = _project(scene, 3)
    bins = binning.bin_and_sort(st.centers, st.radii, st.tile_counts, st.depths, scene.width, scene.height)
    args = (bins["ranges"], bins["point_list"], st.centers, st.conics, st.colors, scene.width, scene.height)
    ref = grender.render_views(*args)
    buf = torch.full((count + 8,), float("nan"), device=DEV)
    zero = buf[4:4 + count]  # 16-byte aligned view, NaN guards on both sides
    out = grender.render_views(*args, zero=zero)
    torch.cuda.synchronize()
    assert torch.equal(out.features, ref.features) and torch.equal(out.alpha, ref.alpha)
    assert torch.equal(out.contributors, ref.contributors)
    assert bool((zero == 0).all())
    assert bool(buf[:4].isnan().all()) and bool(buf[4 + count:].isnan().all())


def test_depth_order_plan_over_a_moving_camera():
    # Frames of one shape whose depth ranges shrink and grow (the camera
    # moves along its axis): every frame, planned from the one before, equals
    # the same frame rendered with no plan, gradients included.
    scene = _scene("sh3_720p")
    _say("depth-order plan over a moving camera")
    binning._KEY_BITS.clear()

    def frame(viewmats, plan):
        if not plan:
            saved = dict(binning._KEY_BITS)
            binning._KEY_BITS.clear()
        means = scene.means.clone().requires_grad_(True)
        out = gs3d.rasterize(means, scene.quats, scene.scales, scene.opacities, viewmats, scene.Ks,
                             scene.width, scene.height, sh_coeffs=scene.sh_coeffs, sh_degree=3)
        (out.features.sum() + out.alpha.sum()).backward()
        if not plan:
            binning._KEY_BITS.clear()
            binning._KEY_BITS.update(saved)
        return out.features, out.alpha, means.grad

    for shift in (0.0, -1.5, 0.0, 3.0, 40.0, 0.5, -2.0, -2.0):
        vm = scene.viewmats.clone()
        vm[..., 2, 3] += shift
        got = frame(vm, True)
        want = frame(vm, False)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
        torch.testing.assert_close(got[2], want[2], rtol=1e-4, atol=1e-6 * float(want[2].abs().max().clamp(min=1.0)))
    binning._KEY_BITS.clear()
