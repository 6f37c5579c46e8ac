"""Pins for the float32 error bounds the gradient tests use
(oracle.sum_bound / pair_bound, the running error analysis Err in
gs3d_oracle.cpp).

A bound is only useful if it holds and is not vacuous.  It must hold for the
oracle's own float32 evaluation against the same computation carried out in
double (the blend backward instantiated with double, the projection VJP's
float64 instantiation): the float32 error of one evaluation is part of what
the bound covers.  And it must stay small against the gradients it bounds,
so that a systematic mistake (a dropped or mis-scaled term) exceeds it.
"""

import numpy as np

from dsl_splat_amd import synthetic
from test_oracle_render import _pipeline


def _relative(bound, value):
    return bound / np.maximum(np.abs(value), 1e-30)


def test_render_bound_covers_float32_error(oracle_lib):
    scene = synthetic.make_scene("small", n=400, width=64, height=48, seed=8)
    bg = np.array([[0.3, 0.1, 0.2]], np.float32)
    rng = np.random.default_rng(3)
    extra = rng.normal(size=(400, 2)).astype(np.float32)
    out, ranges, ids, image, final_t, contrib = _pipeline(oracle_lib, scene, background=bg, extra=extra)
    up = rng.normal(size=image.shape).astype(np.float32)
    args = (64, 48, ranges, ids, out["centers"], out["conics"], scene.features.numpy(), final_t, contrib, up)
    g32 = oracle_lib.render_bwd(*args, extra=extra, background=bg, absgrad=True)
    g64 = oracle_lib.render_bwd_bound(*args, extra=extra, background=bg, float64=True)
    bound = oracle_lib.render_bwd_bound(*args, extra=extra, background=bg)
    checked = 0
    for key in ("centers", "conics", "abs", "features", "extra"):
        err = np.abs(g32[key].astype(np.float64) - g64[key])
        assert np.all(err <= bound[key]), (key, float((err / np.maximum(bound[key], 1e-300)).max()))
        live = np.abs(g64[key]) > 0
        checked += int(live.sum())
        # Not vacuous: the median entry's bound is below 3e-5 of its value
        # and most lie below 1e-4 (the plain tolerance), so a systematic
        # relative error of 1e-4 exceeds it; only sums with heavy
        # cancellation get wider bounds.  (Measured here: the float32 error
        # is 1-9% of the bound.)
        rel = _relative(bound[key][live], g64[key][live])
        assert np.median(rel) < 3e-5, key
        assert np.mean(rel < 1e-4) > 0.85, key
    assert checked > 1000


def test_projection_bound_covers_float32_error(oracle_lib):
    scene = synthetic.make_scene("small", n=300, seed=6)
    full, _, _, _ = oracle_lib.camera_prepare(scene.viewmats.numpy(), scene.Ks.numpy(), scene.width, scene.height,
                                              False)
    out = oracle_lib.project_fwd(scene.means.numpy(), scene.quats.numpy(), scene.scales.numpy(),
                                 scene.opacities.numpy(), scene.viewmats.numpy(), full, scene.Ks.numpy(),
                                 scene.width, scene.height)
    rng = np.random.default_rng(11)
    gc = rng.normal(size=(1, 300, 2)).astype(np.float32)
    gk = rng.normal(size=(1, 300, 4)).astype(np.float32)
    common = (scene.means.numpy(), scene.quats.numpy(), scene.scales.numpy(), scene.opacities.numpy(),
              scene.viewmats.numpy(), full, scene.Ks.numpy(), scene.width, scene.height, out["radii"], gc, gk)
    g32 = oracle_lib.project_bwd(*common)
    zero = np.zeros((1, 300, 2)), np.zeros((1, 300, 4))
    bound = oracle_lib.project_bwd_bound(*common, *zero)
    K = scene.Ks[0].numpy()
    view64 = np.zeros((4, 4))
    proj64 = np.zeros((4, 4))
    visible = 0
    rel = {"means": [], "quats": [], "scales": []}
    for i in range(300):
        if out["radii"][0, i] <= 0:
            continue
        visible += 1
        v = oracle_lib.projection_vjp_f64(scene.means[i].numpy(), scene.quats[i].numpy(), scene.scales[i].numpy(),
                                          float(scene.opacities[i]), scene.viewmats[0].numpy(), full[0],
                                          scene.width, scene.height, K[0, 0], K[1, 1], gc[0, i], gk[0, i])
        view64 += v["view"]
        proj64 += v["proj"]
        for name, key in (("means", "mean"), ("quats", "quat"), ("scales", "scale")):
            err = np.abs(g32[name][i].astype(np.float64) - v[key])
            assert np.all(err <= bound[name][i]), (name, i, err, bound[name][i])
            live = np.abs(v[key]) > 0
            rel[name] += list(_relative(bound[name][i][live], v[key][live]))
    assert visible > 100
    # Not vacuous, per parameter (as for the blend): the mean gradients'
    # bound has a median of ~2e-6 of the value and lies below 1e-4 for ~98%
    # of the entries.  The quaternion and scale gradients come out of the
    # covariance chain (Sigma -> M -> R -> q), whose differences of nearly
    # equal products make the worst-case bound ~1000x the typical float32
    # error (median ~2e-7 against bounds of ~1e-4 -- 3e-4); there a
    # systematic relative error of 1e-3 still exceeds the bound for ~80% of
    # the entries.  (Measured over seeds 1, 2, 3, 6: medians 1.8-1.9e-6,
    # 2.5-2.8e-4 and 1.0-1.1e-4; shares below 1e-4 0.98, below 1e-3 0.81-0.84
    # and 0.86-0.87.)
    r = {k: np.array(v) for k, v in rel.items()}
    assert np.median(r["means"]) < 1e-5 and np.mean(r["means"] < 1e-4) > 0.95
    for name in ("quats", "scales"):
        assert np.median(r[name]) < 5e-4, name
        assert np.mean(r[name] < 1e-3) > 0.75, name
    # Camera gradients sum a few hundred per-Gaussian contributions that
    # largely cancel (each Gaussian's pull on the pose), so float32 moves
    # them by ~1e-3 of their largest entry and their bound is of that order.
    for name, ref in (("view", view64), ("projection", proj64)):
        err = np.abs(g32[name][0].astype(np.float64) - ref)
        assert np.all(err <= bound[name][0]), name
        assert np.all(bound[name][0] <= 1e-2 * np.abs(ref).max()), name
