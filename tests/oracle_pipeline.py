"""End-to-end gs3d forward + backward through the CPU oracle (test helper).

Composes the oracle stages in the order the reference composes its kernels
(gs3d/api.py:116-255 and gs3d/autograd.py:91-171): camera rows, projection
(+SH), scan, emission, sort, ranges, blending; then the blend VJP, the
projection (+SH) VJP and the camera VJP.  Inputs are NumPy copies of the
tensors the GPU path consumed; with normalize_quats the quaternions are raw
and the oracle normalises them (and takes their gradient through the
normalisation) exactly as the projection kernels do.
"""

import numpy as np

import oracle


def run(means, quats, scales, opacities, viewmats, Ks, width, height, *, features=None, sh=None, sh_degree=None,
        extra=None, background=None, near=0.2, far=float("inf"), radius_clip=0.0, upstream=None, absgrad=False,
        normalize_quats=False, bounds=False):
    views = viewmats.shape[0]
    with_centers = sh is not None and sh_degree > 0
    full, inverse, centers, errors = oracle.camera_prepare(viewmats, Ks, width, height, with_centers)
    assert np.all(errors == 0), errors
    proj = oracle.project_fwd(means, quats, scales, opacities, viewmats, full, Ks, width, height, near, far,
                              radius_clip, sh=sh, sh_degree=sh_degree or 0,
                              camera_centers=centers if with_centers else None, metadata=True,
                              normalize_quats=normalize_quats)
    offsets, total = oracle.scan_i32(proj["tiles"].ravel())
    keys, vals = oracle.emit_keys(proj["centers"], proj["radii"], proj["depths"], offsets, total, width, height)
    T = views * ((width + 15) // 16) * ((height + 15) // 16)
    sk, sv = oracle.sort_pairs(keys, vals, 32 + int(T).bit_length())
    ranges = oracle.tile_ranges(sk, T)
    blended = proj["colors"] if sh is not None else features
    image, final_t, contrib = oracle.render_fwd(width, height, ranges, sv, proj["centers"], proj["conics"], blended,
                                                extra=extra, background=background)
    out = dict(full=full, inverse=inverse, camera_centers=centers, proj=proj, offsets=offsets, total=total,
               keys=keys, vals=vals, sorted_keys=sk, sorted_vals=sv, ranges=ranges, image=image, final_t=final_t,
               contributors=contrib)
    if upstream is None:
        return out
    g = oracle.render_bwd(width, height, ranges, sv, proj["centers"], proj["conics"], blended, final_t, contrib,
                          upstream, extra=extra, background=background, absgrad=absgrad)
    out["render_grads"] = g
    pg = oracle.project_bwd(means, quats, scales, opacities, viewmats, full, Ks, width, height, proj["radii"],
                            g["centers"], g["conics"], sh=sh, sh_degree=sh_degree or 0,
                            camera_centers=centers if with_centers else None,
                            grad_colors=g["features"] if sh is not None else None, normalize_quats=normalize_quats)
    out["proj_grads"] = pg
    cam_inverse = inverse if with_centers else full
    gview = oracle.camera_backward(Ks, pg["projection"], width, height, cam_inverse,
                                   pg.get("camera_centers") if with_centers else None)
    out["grad_viewmats"] = gview + pg["view"]
    if bounds:
        rb = oracle.render_bwd_bound(width, height, ranges, sv, proj["centers"], proj["conics"], blended, final_t,
                                     contrib, upstream, extra=extra, background=background)
        pb = oracle.project_bwd_bound(means, quats, scales, opacities, viewmats, full, Ks, width, height,
                                      proj["radii"], g["centers"], g["conics"], rb["centers"], rb["conics"], sh=sh,
                                      sh_degree=sh_degree or 0, camera_centers=centers if with_centers else None,
                                      grad_colors=g["features"] if sh is not None else None,
                                      e_colors=rb["features"] if sh is not None else None,
                                      normalize_quats=normalize_quats)
        cb = oracle.camera_backward_bound(Ks, pg["projection"], pb["projection"], width, height, cam_inverse,
                                          pg.get("camera_centers") if with_centers else None,
                                          pb.get("camera_centers") if with_centers else None)
        total = np.abs(out["grad_viewmats"]).astype(np.float64)
        out["bounds"] = dict(render=rb, proj=pb,
                             viewmats=cb + pb["view"] + 2.0 * oracle.UNIT_ROUNDOFF * total)
    return out


# Every check_gradient call of the session (summarised by conftest.py).
GRADIENT_CHECKS = []


def check_gradient(name, got, ref, bound, rtol=1e-4, atol=1e-5, report=None):
    """The gradient criterion: every entry within atol + rtol*|ref| of the
    oracle, or, where float32 evaluation order alone can move it further
    (cancellation across many terms), within its stated error bound (the
    running error analysis of the oracle, oracle.sum_bound/pair_bound).
    Prints the entries outside the plain tolerance and how many of those the
    bound accepts; fails on any entry outside both."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = np.broadcast_to(np.asarray(bound, dtype=np.float64), ref.shape)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    plain = err > atol + rtol * np.abs(ref)
    bad = plain & (err > bound)
    ratio = float((err[plain] / np.maximum(bound[plain], 1e-300)).max()) if plain.any() else 0.0
    stats = dict(name=name, n=int(err.size), max_abs=float(err.max()) if err.size else 0.0,
                 outside_tolerance=int(plain.sum()), outside_bound=int(bad.sum()), max_err_over_bound=ratio)
    if report is not None:
        report.append(stats)
    GRADIENT_CHECKS.append(stats)
    print(f"  {name}: n={stats['n']} max_abs={stats['max_abs']:.3e} outside rtol/atol={stats['outside_tolerance']} "
          f"(max err/bound {ratio:.3f}) outside bound={stats['outside_bound']}", flush=True)
    if bad.any():
        i = np.flatnonzero(bad.ravel())[:5]
        detail = [(int(k), ref.ravel()[k], got.ravel()[k], bound.ravel()[k]) for k in i]
        raise AssertionError(f"{name}: {int(bad.sum())} entries outside tolerance and bound: {detail}")
    return stats


def compare(name, got, ref, rtol=1e-4, atol=1e-5, max_bad_fraction=0.0, report=None):
    """Elementwise |got-ref| <= atol + rtol*|ref|; returns stats, asserts the
    fraction of violating elements is at most max_bad_fraction."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    stats = dict(name=name, n=int(err.size), max_abs=float(err.max()) if err.size else 0.0,
                 mean_abs=float(err.mean()) if err.size else 0.0, bad=int(bad.sum()),
                 scale=float(np.abs(ref).max()) if ref.size else 0.0)
    if report is not None:
        report.append(stats)
    print(f"  {name}: max_abs={stats['max_abs']:.3e} mean_abs={stats['mean_abs']:.3e} "
          f"bad={stats['bad']}/{stats['n']} scale={stats['scale']:.3e}", flush=True)
    assert stats["bad"] <= max_bad_fraction * max(1, stats["n"]), stats
    return stats
