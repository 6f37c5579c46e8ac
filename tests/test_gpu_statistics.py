"""GPU parity of the contribution statistics (statistics.py:16-156 of the
reference, observed in the forward blend at gs3d/render.py:109-115).

Kernel level: gs3d_render_fwd_stats against the oracle's observer on the same
GPU-prepared frames -- blend outputs bit-exact and identical to the launch
without statistics, counts bit-exact, sums within rtol 1e-4 / atol 1e-5 of
their scale (the float additions run in another order; the reference's
atomics leave theirs unspecified too).  API level: gs3d.rasterize,
gsplat.rasterization and ops.rasterize_to_pixels return the reference's
names, shapes and dtypes and agree with each other, and at a full 1080p frame
the size-independent identities hold: the all-ones weighted sum over all
Gaussians equals the summed alpha channel, and the all-ones count lies
between the number of covered pixels and the summed last-contributor indices.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle_pipeline import compare
from dsl_splat_amd import gs3d, synthetic
from dsl_splat_amd.cameras import PinholeCamera
from dsl_splat_amd.gs3d import gsplat, ops
from dsl_splat_amd.gs3d import render as grender
from dsl_splat_amd.statistics import MaskedContributionCount, PreparedStatistics, WeightedContributionSum
from test_gpu_stages import _frame, _np, _say, _scene

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _maps(views, H, W, seed):
    g = torch.Generator().manual_seed(seed)
    mask = torch.rand((views, H, W), generator=g) < 0.4
    weights = torch.randn((views, H, W), generator=g)
    weights[torch.rand((views, H, W), generator=g) < 0.2] = 0.0
    shared = torch.rand((H, W), generator=g).expand(views, H, W)
    ones = torch.ones((views, H, W))
    # count(mask), sum(weights), sum(shared map), count(everywhere), sum(ones)
    kinds = (0, 1, 1, 0, 1)
    pv = torch.stack([mask.float(), weights, shared, ones, ones], 1).reshape(views, 5, H * W)
    return kinds, pv.contiguous().to(DEV)


@pytest.mark.parametrize("key,degree", [("small_rgb", None), ("sh3_4view", 3), ("sh3_720p", 1)])
def test_statistics_kernel_matches_oracle(key, degree):
    scene = _scene(key)
    _say(f"statistics kernel {key}")
    quats, full, inverse, centers, st, bins = _frame(scene, degree)
    views, n = st.radii.shape
    H, W = scene.height, scene.width
    feats = st.colors if degree is not None else scene.features
    kinds, pv = _maps(views, H, W, 7)
    counts = torch.zeros((views, 2, n), dtype=torch.int32, device=DEV)
    sums = torch.zeros((views, 3, n), dtype=torch.float32, device=DEV)
    args = (bins["ranges"], bins["point_list"], st.centers, st.conics, feats, W, H)
    out = grender.render_views(*args, statistics=PreparedStatistics(kinds, pv, counts, sums))
    plain = grender.render_views(*args)
    np.testing.assert_array_equal(_np(out.stacked()), _np(plain.stacked()))
    np.testing.assert_array_equal(_np(out.transmittance), _np(plain.transmittance))
    np.testing.assert_array_equal(_np(out.contributors), _np(plain.contributors))
    img, ft, ct, ref_counts, ref_sums = oracle.render_fwd_stats(
        W, H, _np(bins["ranges"]), _np(bins["point_list"]), _np(st.centers), _np(st.conics), _np(feats), kinds,
        _np(pv))
    np.testing.assert_array_equal(_np(out.stacked()), img)
    np.testing.assert_array_equal(_np(counts), ref_counts)
    assert ref_counts[:, 1].sum() > 1000
    compare(f"stat_sums_{key}", _np(sums), ref_sums, rtol=1e-4, atol=1e-5 * float(np.abs(ref_sums).max()))


def _bucket_maps(views, H, W, kinds, seed):
    """Pixel values (views, R, H*W) for the given request kinds: 0/1 masks for
    counts, N(0,1) weights with 20% zeros for sums."""
    g = torch.Generator().manual_seed(seed)
    maps = []
    for kind in kinds:
        if kind == 0:
            maps.append((torch.rand((views, H, W), generator=g) < 0.4).float())
        else:
            w = torch.randn((views, H, W), generator=g)
            w[torch.rand((views, H, W), generator=g) < 0.2] = 0.0
            maps.append(w)
    return torch.stack(maps, 1).reshape(views, len(kinds), H * W).contiguous().to(DEV)


def _stats_against_oracle(scene, feats, st, bins, kinds, pv, nonfinite=False):
    views, n = st.radii.shape
    H, W = scene.height, scene.width
    counts = torch.zeros((views, kinds.count(0), n), dtype=torch.int32, device=DEV)
    sums = torch.zeros((views, kinds.count(1), n), dtype=torch.float32, device=DEV)
    args = (bins["ranges"], bins["point_list"], st.centers, st.conics, feats, W, H)
    out = grender.render_views(*args, statistics=PreparedStatistics(tuple(kinds), pv, counts, sums))
    img, ft, ct, ref_counts, ref_sums = oracle.render_fwd_stats(
        W, H, _np(bins["ranges"]), _np(bins["point_list"]), _np(st.centers), _np(st.conics), _np(feats),
        tuple(kinds), _np(pv))
    np.testing.assert_array_equal(_np(out.stacked()), img)
    np.testing.assert_array_equal(_np(out.contributors), ct)
    np.testing.assert_array_equal(_np(counts), ref_counts)
    got = _np(sums)
    if nonfinite:
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref_sums))
        np.testing.assert_array_equal(np.isinf(got), np.isinf(ref_sums))
        assert not np.isfinite(ref_sums).all()
        keep = np.isfinite(ref_sums)
        got, ref_sums = got[keep], ref_sums[keep]
    if ref_sums.size:
        compare(f"stat_sums_{len(kinds)}", got, ref_sums, rtol=1e-4,
                atol=1e-5 * max(float(np.abs(ref_sums).max()), 1e-30))
    return ref_counts, ref_sums


# Request counts of every compiled bucket (1, 2, 4, 8), every combination of
# kinds of one and two requests (compiled in), at one and two pixels per lane
# and at 4 and 8 blended channels (4-channel launches of up to two requests
# take the pipelined traversal; the others load at use).
@pytest.mark.parametrize("key,channels,kinds", [
    ("small_rgb", 3, (1,)), ("wide_rgb", 3, (1,)), ("wide_rgb", 3, (0,)), ("wide_rgb", 3, (0, 1)),
    ("wide_rgb", 3, (1, 0)), ("wide_rgb", 3, (0, 0)), ("wide_rgb", 3, (1, 1)), ("wide_rgb", 3, (0, 1, 1)),
    ("wide_rgb", 3, (1, 0, 1, 1, 0, 1, 0, 0)), ("wide_rgb", 6, (1,)), ("wide_rgb", 6, (0, 1)),
    ("small_rgb", 6, (0, 1, 0, 1))])
def test_statistics_request_buckets(key, channels, kinds):
    scene = _scene(key)
    _say(f"statistics buckets {key} D={channels} kinds={kinds}")
    quats, full, inverse, centers, st, bins = _frame(scene, None)
    n = st.radii.shape[1]
    g = torch.Generator().manual_seed(5)
    feats = scene.features if channels == 3 else torch.rand((n, channels), generator=g).to(DEV)
    pv = _bucket_maps(st.radii.shape[0], scene.height, scene.width, kinds, 11)
    ref_counts, ref_sums = _stats_against_oracle(scene, feats, st, bins, list(kinds), pv)
    assert (ref_counts.sum() > 0) or (ref_sums != 0).any()


@pytest.mark.parametrize("key", ["small_rgb", "wide_rgb"])
def test_statistics_non_finite_weights(key):
    # A weighted sum whose pixel weights hold NaN and +inf: the product form
    # of the observer (value times a zero weight for rejected pixels) must not
    # be used there; the oracle's sums, NaN and inf included, are reproduced.
    scene = _scene(key)
    _say(f"statistics non-finite weights {key}")
    quats, full, inverse, centers, st, bins = _frame(scene, None)
    views = st.radii.shape[0]
    H, W = scene.height, scene.width
    kinds = [0, 1]
    pv = _bucket_maps(views, H, W, kinds, 13)
    pv[0, 1, (H // 2) * W + W // 2] = float("nan")
    pv[0, 1, (H // 3) * W + W // 4] = float("inf")
    _stats_against_oracle(scene, scene.features, st, bins, kinds, pv, nonfinite=True)


def _requests(views, H, W):
    g = torch.Generator().manual_seed(3)
    mask = (torch.rand((H, W), generator=g) < 0.5).to(DEV)
    weights = torch.randn((views, H, W), generator=g).to(DEV)
    return [MaskedContributionCount("masked", mask), WeightedContributionSum("weighted", weights),
            WeightedContributionSum("ones", torch.ones((H, W), device=DEV)),
            MaskedContributionCount("all", torch.ones((H, W), dtype=torch.bool, device=DEV))]


def test_statistics_through_public_entry_points():
    scene = synthetic.make_scene("sh3_1080p_4view", n=4000, width=128, height=80, seed=51).to(DEV)
    views, n, H, W = scene.viewmats.shape[0], scene.means.shape[0], scene.height, scene.width
    _say("statistics api")
    reqs = _requests(views, H, W)
    feats = torch.rand((n, 3), generator=torch.Generator().manual_seed(52)).to(DEV)
    args = (scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks, W, H)
    r = gs3d.rasterize(*args, features=feats, statistics=reqs)
    plain = gs3d.rasterize(*args, features=feats)
    np.testing.assert_array_equal(_np(r.features), _np(plain.features))
    np.testing.assert_array_equal(_np(r.alpha), _np(plain.alpha))
    assert set(r.statistics) == {"masked", "weighted", "ones", "all"}
    for name, kind in (("masked", torch.int32), ("all", torch.int32), ("weighted", torch.float32),
                       ("ones", torch.float32)):
        assert r.statistics[name].shape == (views, n) and r.statistics[name].dtype == kind
    s = {k: _np(v) for k, v in r.statistics.items()}
    assert np.all(s["masked"] <= s["all"]) and s["all"].sum() > 0
    assert np.all(s["all"][_np(r.radii[..., 0]) == 0] == 0)
    np.testing.assert_allclose(s["ones"].astype(np.float64).sum(-1), _np(r.alpha).astype(np.float64).sum((1, 2, 3)),
                               rtol=1e-5)
    # gsplat adapter: same statistics under meta["statistics"].
    gf, ga, meta = gsplat.rasterization(scene.means, scene.quats, scene.scales, scene.opacities, feats,
                                        scene.viewmats, scene.Ks, W, H, near_plane=0.2, far_plane=float("inf"),
                                        packed=False, statistics=reqs)
    ms = {k: _np(v) for k, v in meta["statistics"].items()}
    np.testing.assert_array_equal(ms["masked"], s["masked"])
    np.testing.assert_array_equal(ms["all"], s["all"])
    compare("gsplat_weighted", ms["weighted"], s["weighted"], rtol=1e-4, atol=1e-5 * float(np.abs(s["weighted"]).max()))
    # Staged ops API on view 0: (N,) results equal to the fused call's view 0.
    cam = PinholeCamera(scene.viewmats[0], scene.Ks[0], W, H, near_plane=0.2, far_plane=float("inf"))
    geometry = ops.prepare_gaussians(scene.means, scene.quats, scene.scales, scene.opacities, cam)
    tiles = ops.bin_and_sort(geometry)
    view0 = [MaskedContributionCount("masked", reqs[0].mask), WeightedContributionSum("weighted", reqs[1].pixel_weights[0])]
    pix = ops.rasterize_to_pixels(geometry, tiles, feats, statistics=view0)
    assert pix.statistics["masked"].shape == (n,) and pix.statistics["weighted"].shape == (n,)
    np.testing.assert_array_equal(_np(pix.statistics["masked"]), s["masked"][0])
    compare("ops_weighted", _np(pix.statistics["weighted"]), s["weighted"][0], rtol=1e-4,
            atol=1e-5 * float(np.abs(s["weighted"][0]).max()))


def test_statistics_full_frame_identities():
    scene = synthetic.make_scene("sh3_1080p_4view", n=400_000, seed=61).to(DEV)
    views, n, H, W = scene.viewmats.shape[0], scene.means.shape[0], scene.height, scene.width
    _say(f"statistics full frame {views}x{W}x{H} n={n}")
    reqs = _requests(views, H, W)
    r = gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks, W, H,
                       sh_coeffs=scene.sh_coeffs, statistics=reqs)
    s = {k: _np(v) for k, v in r.statistics.items()}
    alpha = _np(r.alpha).astype(np.float64).sum((1, 2, 3))
    np.testing.assert_allclose(s["ones"].astype(np.float64).sum(-1), alpha, rtol=1e-5)
    covered = (_np(r.alpha)[..., 0] > 0).sum((1, 2))
    total = s["all"].astype(np.int64).sum(-1)
    assert np.all(total >= covered) and np.all(covered > 0)
    assert np.all(s["masked"] <= s["all"])
    # Masked counts of a complementary pair of masks add up to the count everywhere.
    inv = [MaskedContributionCount("a", reqs[0].mask), MaskedContributionCount("b", ~reqs[0].mask)]
    r2 = gs3d.rasterize(scene.means, scene.quats, scene.scales, scene.opacities, scene.viewmats, scene.Ks, W, H,
                        sh_coeffs=scene.sh_coeffs, statistics=inv)
    np.testing.assert_array_equal(_np(r2.statistics["a"]) + _np(r2.statistics["b"]), s["all"])
    np.testing.assert_array_equal(_np(r2.statistics["a"]), s["masked"])
