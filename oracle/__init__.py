"""NumPy front end of the CPU oracle (liboracle_gs3d.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always to test results.  The product package
dsl_splat_amd never imports this module.

Each function takes NumPy arrays (converted to contiguous float32/int32),
calls the C restatement in gs3d_oracle.cpp and returns NumPy outputs whose
shapes follow the reference kernels they restate.
"""

import ctypes
import os
import subprocess

import numpy as np

from dsl_splat_amd.runtime import abi

_HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIBRARY selects another build of the same source (the sanitized
# build of the Makefile's "sanitized" target).
_LIB_PATH = os.environ.get("ORACLE_LIBRARY") or os.path.join(_HERE, "liboracle_gs3d.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (g++ only; no GPU needed)."""
    cmd = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        # The default build is brought up to date first: a library built
        # against an older include/gs3d_hip.h would read the argument structs
        # with their old layout.
        if not os.environ.get("ORACLE_LIBRARY") or not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I32, I64 = ctypes.c_int32, ctypes.c_int64
        D = ctypes.c_double
        sig = {
            "oracle_camera_prepare": [P, P, I32, I32, I32, I32, P, P, P, P],
            "oracle_camera_backward": [P, P, I32, I32, P, P, I32, P],
            "oracle_project_fwd": [ctypes.POINTER(abi.ProjectArgs)],
            "oracle_project_bwd": [ctypes.POINTER(abi.ProjectBwdArgs)],
            "oracle_sh_fwd": [P, I32, P, P, I32, I32, P, P],
            "oracle_sh_bwd": [P, I32, P, P, P, P, I32, I32, P, P],
            "oracle_sh_bwd_bound": [P, I32, P, P, P, P, I32, I32, P, P],
            "oracle_scan_i32": [P, I64, P, P],
            "oracle_emit_keys": [ctypes.POINTER(abi.EmitArgs)],
            "oracle_sort_pairs_u64": [P, P, I64, I32],
            "oracle_tile_ranges": [P, I64, P, I64],
            "oracle_render_fwd": [ctypes.POINTER(abi.RenderArgs)],
            "oracle_render_pair_counts": [ctypes.POINTER(abi.RenderArgs), P],
            "oracle_tile_footprint": [I32, P, P, I32, I32, I32, P, P],
            "oracle_logf": [ctypes.c_float],
            "oracle_normalize_quats": [P, I64, P, P, P],
            "oracle_render_fwd_stats": [ctypes.POINTER(abi.RenderArgs), ctypes.POINTER(abi.RenderStatsArgs)],
            "oracle_render_bwd": [ctypes.POINTER(abi.RenderBwdArgs)],
            "oracle_render_bwd_bound": [ctypes.POINTER(abi.RenderBwdArgs), P, P, P, P, P],
            "oracle_render_bwd_f64": [ctypes.POINTER(abi.RenderBwdArgs), P, P, P, P, P],
            "oracle_project_bwd_bound": [ctypes.POINTER(abi.ProjectBwdArgs), P, P, P, P, P, P, P, P, P, P, P],
            "oracle_camera_backward_bound": [P, P, P, I32, I32, P, P, P, I32, P],
            "oracle_projection_loss_f64": [P, P, P, D, P, P, I32, I32, D, D, P, P],
            "oracle_projection_vjp_f64": [P, P, P, D, P, P, I32, I32, D, D, P, P, P],
            "oracle_glm_rotation": [P, P],
            "oracle_sh_basis_grad": [P, I32, P],
        }
        for name, argtypes in sig.items():
            fn = getattr(_lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        _lib.oracle_projection_loss_f64.restype = ctypes.c_double
        _lib.oracle_expf.argtypes = [ctypes.c_float]
        _lib.oracle_expf.restype = ctypes.c_float
        _lib.oracle_logf.restype = ctypes.c_float
        _lib.oracle_sh_basis.argtypes = [P, I32]
        _lib.oracle_sh_basis.restype = ctypes.c_float
        _lib.oracle_set_threads.argtypes = [ctypes.c_int]
        _lib.oracle_set_threads.restype = ctypes.c_int
    return _lib


def set_threads(n: int) -> int:
    """OpenMP threads for the render/projection loops (1 = fully serial)."""
    return lib().oracle_set_threads(int(n))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _ptr(a):
    return None if a is None else a.ctypes.data


def expf(x: float) -> float:
    return float(lib().oracle_expf(ctypes.c_float(x)))


def expf_array(x) -> np.ndarray:
    x = _f32(x).ravel()
    return np.array([lib().oracle_expf(ctypes.c_float(v)) for v in x], dtype=np.float32)


def glm_rotation(q) -> np.ndarray:
    q = _f32(q)
    out = np.empty(9, np.float32)
    lib().oracle_glm_rotation(_ptr(q), _ptr(out))
    return out.reshape(3, 3)


def sh_basis(u, k: int) -> float:
    u = _f32(u)
    return float(lib().oracle_sh_basis(_ptr(u), int(k)))


def sh_basis_grad(u, k: int) -> np.ndarray:
    u = _f32(u)
    g = np.empty(3, np.float32)
    lib().oracle_sh_basis_grad(_ptr(u), int(k), _ptr(g))
    return g


def camera_prepare(views, Ks, width, height, with_centers):
    views, Ks = _f32(views).reshape(-1, 4, 4), _f32(Ks).reshape(-1, 3, 3)
    c = len(views)
    full = np.zeros((c, 4, 4), np.float32)
    inverse = np.zeros((c, 4, 4), np.float32)
    centers = np.zeros((c, 3), np.float32)
    errors = np.zeros(c, np.int32)
    lib().oracle_camera_prepare(
        _ptr(views), _ptr(Ks), c, width, height, int(with_centers),
        _ptr(full), _ptr(inverse), _ptr(centers), _ptr(errors),
    )
    return full, inverse, centers, errors


def camera_backward(Ks, grad_full, width, height, inverse, grad_centers):
    Ks = _f32(Ks).reshape(-1, 3, 3)
    c = len(Ks)
    gf = None if grad_full is None else _f32(grad_full).reshape(c, 4, 4)
    gc = None if grad_centers is None else _f32(grad_centers).reshape(c, 3)
    inv = _f32(inverse).reshape(c, 4, 4)
    out = np.zeros((c, 4, 4), np.float32)
    lib().oracle_camera_backward(_ptr(Ks), _ptr(gf), width, height, _ptr(inv), _ptr(gc), c, _ptr(out))
    return out


def project_fwd(means, quats, scales, opacities, view, projection, intrinsics, width, height,
                near_plane=0.2, far_plane=float("inf"), radius_clip=0.0,
                sh=None, sh_degree=0, camera_centers=None, metadata=False, tile_mode="radius",
                normalize_quats=False):
    """gs3d/projection.py:89-164 for every view; returns a dict of arrays.
    normalize_quats: the quaternions are raw and normalised first, as
    F.normalize does in the reference (inputs.py:252)."""
    means, quats, scales, opacities = _f32(means), _f32(quats), _f32(scales), _f32(opacities)
    view, projection, intrinsics = (
        _f32(view).reshape(-1, 4, 4), _f32(projection).reshape(-1, 4, 4), _f32(intrinsics).reshape(-1, 3, 3))
    n, c = len(means), len(view)
    out = dict(
        centers=np.zeros((c, n, 2), np.float32),
        conics=np.zeros((c, n, 4), np.float32),
        radii=np.zeros((c, n), np.int32),
        tiles=np.zeros((c, n), np.int32),
        depths=np.zeros((c, n), np.float32),
    )
    a = abi.ProjectArgs()
    a.n, a.views, a.width, a.height = n, c, width, height
    a.near_plane, a.far_plane, a.radius_clip = near_plane, far_plane, radius_clip
    a.tile_mode = abi.TILE_MODES[tile_mode]
    a.normalize_quats = int(normalize_quats)
    for name, arr in (("means", means), ("quats", quats), ("scales", scales), ("opacities", opacities),
                      ("view", view), ("projection", projection), ("intrinsics", intrinsics)):
        setattr(a, name, _ptr(arr))
    for name in ("centers", "conics", "radii", "tiles", "depths"):
        setattr(a, name, _ptr(out[name]))
    keep = []
    if sh is not None:
        sh = _f32(sh)
        per_view = sh.ndim == 4
        a.sh = _ptr(sh)
        a.sh_rows = sh.shape[-2]
        a.sh_view_stride = sh.shape[-3] * sh.shape[-2] * 3 if per_view else 0
        a.sh_degree = sh_degree
        cc = _f32(np.zeros((c, 3)) if camera_centers is None else camera_centers).reshape(c, 3)
        keep += [sh, cc]
        a.camera_centers = _ptr(cc)
        out["colors"] = np.zeros((c, n, 3), np.float32)
        a.colors = _ptr(out["colors"])
    if metadata:
        out["means2d"] = np.zeros((c, n, 2), np.float32)
        out["meta_opacities"] = np.zeros((c, n), np.float32)
        out["meta_conics"] = np.zeros((c, n, 3), np.float32)
        a.means2d, a.meta_opacities, a.meta_conics = (
            _ptr(out["means2d"]), _ptr(out["meta_opacities"]), _ptr(out["meta_conics"]))
    lib().oracle_project_fwd(ctypes.byref(a))
    return out


def project_bwd(means, quats, scales, opacities, view, projection, intrinsics, width, height, radii,
                grad_centers, grad_conics, sh=None, sh_degree=0, camera_centers=None, grad_colors=None,
                normalize_quats=False):
    means, quats, scales, opacities = _f32(means), _f32(quats), _f32(scales), _f32(opacities)
    view, projection, intrinsics = (
        _f32(view).reshape(-1, 4, 4), _f32(projection).reshape(-1, 4, 4), _f32(intrinsics).reshape(-1, 3, 3))
    n, c = len(means), len(view)
    radii = _i32(radii).reshape(c, n)
    gc = _f32(grad_centers).reshape(c, n, 2)
    gk = _f32(grad_conics).reshape(c, n, 4)
    out = dict(
        means=np.zeros((n, 3), np.float32), quats=np.zeros((n, 4), np.float32),
        scales=np.zeros((n, 3), np.float32), opacities=np.zeros(n, np.float32),
        view=np.zeros((c, 4, 4), np.float32), projection=np.zeros((c, 4, 4), np.float32),
    )
    a = abi.ProjectBwdArgs()
    a.n, a.views, a.width, a.height = n, c, width, height
    a.normalize_quats = int(normalize_quats)
    for name, arr in (("means", means), ("quats", quats), ("scales", scales), ("opacities", opacities),
                      ("view", view), ("projection", projection), ("intrinsics", intrinsics), ("radii", radii)):
        setattr(a, name, _ptr(arr))
    a.grad_centers, a.grad_centers_stride = _ptr(gc), 2
    a.grad_conics, a.grad_conics_stride = _ptr(gk), 4
    a.grad_means, a.grad_quats, a.grad_scales, a.grad_opacities = (
        _ptr(out["means"]), _ptr(out["quats"]), _ptr(out["scales"]), _ptr(out["opacities"]))
    a.grad_view, a.grad_projection = _ptr(out["view"]), _ptr(out["projection"])
    keep = []
    if sh is not None:
        sh = _f32(sh)
        per_view = sh.ndim == 4
        a.sh = _ptr(sh)
        a.sh_rows = sh.shape[-2]
        a.sh_view_stride = sh.shape[-3] * sh.shape[-2] * 3 if per_view else 0
        a.sh_degree = sh_degree
        cc = _f32(np.zeros((c, 3)) if camera_centers is None else camera_centers).reshape(c, 3)
        gcol = _f32(grad_colors).reshape(c, n, 3)
        keep += [sh, cc, gcol]
        a.camera_centers = _ptr(cc)
        a.grad_colors, a.grad_colors_stride = _ptr(gcol), 3
        out["sh"] = np.zeros(sh.shape, np.float32)
        out["camera_centers"] = np.zeros((c, 3), np.float32)
        a.grad_sh, a.grad_camera_centers = _ptr(out["sh"]), _ptr(out["camera_centers"])
    lib().oracle_project_bwd(ctypes.byref(a))
    return out


def sh_fwd(coefficients, directions, degree, radii=None):
    coefficients, directions = _f32(coefficients), _f32(directions)
    n, rows = coefficients.shape[0], coefficients.shape[1]
    radii = None if radii is None else _i32(radii)
    colors = np.zeros((n, 3), np.float32)
    active = np.zeros((n, 3), np.uint8)
    lib().oracle_sh_fwd(_ptr(coefficients), rows, _ptr(directions), _ptr(radii), n, degree,
                        _ptr(colors), _ptr(active))
    return colors, active


def sh_bwd(coefficients, directions, degree, active, upstream, radii=None):
    coefficients, directions, upstream = _f32(coefficients), _f32(directions), _f32(upstream)
    active = np.ascontiguousarray(active, dtype=np.uint8)
    n, rows = coefficients.shape[0], coefficients.shape[1]
    radii = None if radii is None else _i32(radii)
    gco = np.zeros_like(coefficients)
    gdir = np.zeros((n, 3), np.float32)
    lib().oracle_sh_bwd(_ptr(coefficients), rows, _ptr(directions), _ptr(radii), _ptr(active), _ptr(upstream),
                        n, degree, _ptr(gco), _ptr(gdir))
    return gco, gdir


def sh_bwd_bound(coefficients, directions, degree, active, upstream, radii=None):
    """Per-entry bounds B of sh_bwd's (coefficient, direction) gradients."""
    coefficients, directions, upstream = _f32(coefficients), _f32(directions), _f32(upstream)
    active = np.ascontiguousarray(active, dtype=np.uint8)
    n, rows = coefficients.shape[0], coefficients.shape[1]
    radii = None if radii is None else _i32(radii)
    bco = np.zeros(coefficients.shape + (2,))
    bdir = np.zeros((n, 3, 2))
    lib().oracle_sh_bwd_bound(_ptr(coefficients), rows, _ptr(directions), _ptr(radii), _ptr(active), _ptr(upstream),
                              n, degree, _ptr(bco), _ptr(bdir))
    return pair_bound(bco), pair_bound(bdir)


def scan_i32(counts):
    counts = _i32(counts)
    offsets = np.zeros_like(counts)
    total = ctypes.c_int64(0)
    lib().oracle_scan_i32(_ptr(counts), len(counts), _ptr(offsets), ctypes.addressof(total))
    return offsets, int(total.value)


def emit_keys(centers, radii, depths, offsets, total, width, height, conics=None, tile_mode="radius"):
    """splatting/binning.py:16-37 (:40-68 outside the radius mode) over (views, N) rows."""
    centers = _f32(centers)
    c, n = centers.shape[0], centers.shape[1]
    radii, depths, offsets = _i32(radii).reshape(c, n), _f32(depths).reshape(c, n), _i32(offsets).reshape(-1)
    keys = np.zeros(total, np.uint64)
    values = np.zeros(total, np.int32)
    a = abi.EmitArgs()
    a.n, a.views, a.width, a.height = n, c, width, height
    a.centers, a.radii, a.depths, a.offsets = _ptr(centers), _ptr(radii), _ptr(depths), _ptr(offsets)
    a.keys, a.values = _ptr(keys), _ptr(values)
    a.tile_mode = abi.TILE_MODES[tile_mode]
    if tile_mode != "radius":
        conics = _f32(conics).reshape(c, n, 4)
        a.conics = _ptr(conics)
    lib().oracle_emit_keys(ctypes.byref(a))
    return keys, values


def tile_footprint(mode, center, conic, radius, gx, gy):
    """splatting/intersections.py:46-218 for one projected Gaussian: (bounds
    x0, y0, x1, y1 of the mode's rectangle, listed tile indices in traversal
    order)."""
    center, conic = _f32(center).reshape(2), _f32(conic).reshape(4)
    tiles = np.zeros(max(1, gx * gy), np.int64)
    bounds = np.zeros(4, np.int32)
    count = lib().oracle_tile_footprint(abi.TILE_MODES[mode], _ptr(center), _ptr(conic), int(radius), gx, gy,
                                        _ptr(tiles), _ptr(bounds))
    return bounds, tiles[:count].copy()


def normalize_quats(q, g=None):
    """(unit quaternions, gradient through the normalisation of g or None)."""
    q = _f32(q).reshape(-1, 4)
    u = np.zeros_like(q)
    grad = None if g is None else np.zeros_like(q)
    lib().oracle_normalize_quats(_ptr(q), len(q), _ptr(u), None if g is None else _ptr(_f32(g).reshape(-1, 4)),
                                 _ptr(grad))
    return u, grad


def logf(x: float) -> float:
    """The float32 natural log of the SnugBox/AccuTile alpha level."""
    return float(lib().oracle_logf(float(x)))


def sort_pairs(keys, values, end_bit):
    keys = np.ascontiguousarray(keys, dtype=np.uint64).copy()
    values = _i32(values).copy()
    lib().oracle_sort_pairs_u64(_ptr(keys), _ptr(values), len(keys), end_bit)
    return keys, values


def tile_ranges(sorted_keys, tile_count):
    sorted_keys = np.ascontiguousarray(sorted_keys, dtype=np.uint64)
    ranges = np.zeros((tile_count, 2), np.int32)
    lib().oracle_tile_ranges(_ptr(sorted_keys), len(sorted_keys), _ptr(ranges), tile_count)
    return ranges


def _render_args(width, height, ranges, ids, centers, conics, features, extra, background, keep):
    centers, conics = _f32(centers), _f32(conics)
    c, n = centers.shape[0], centers.shape[1]
    a = abi.RenderArgs()
    a.width, a.height, a.views, a.n = width, height, c, n
    ranges, ids = _i32(ranges), _i32(ids)
    features = _f32(features)
    per_view = features.ndim == 3
    keep += [ranges, ids, centers, conics, features]
    a.ranges, a.ids, a.centers, a.conics = _ptr(ranges), _ptr(ids), _ptr(centers), _ptr(conics)
    a.features = _ptr(features)
    a.feat_channels = features.shape[-1]
    a.feat_stride = features.shape[-1]
    a.feat_view_stride = n * features.shape[-1] if per_view else 0
    if extra is not None:
        extra = _f32(extra)
        keep.append(extra)
        a.extra = _ptr(extra)
        a.extra_channels = extra.shape[-1]
        a.extra_stride = extra.shape[-1]
        a.extra_view_stride = n * extra.shape[-1] if extra.ndim == 3 else 0
    a.one_tail = 1
    if background is not None:
        background = _f32(background).reshape(c, -1)
        keep.append(background)
        a.background = _ptr(background)
        a.background_view_stride = background.shape[-1]
    channels = a.feat_channels + a.extra_channels + 1
    return a, c, n, channels


def render_fwd(width, height, ranges, ids, centers, conics, features, extra=None, background=None):
    """gs3d/render.py:36-126; image is (views,H,W,D') with the alpha channel last."""
    keep = []
    a, c, n, channels = _render_args(width, height, ranges, ids, centers, conics, features, extra, background, keep)
    image = np.zeros((c, height, width, channels), np.float32)
    final_t = np.zeros((c, height, width), np.float32)
    contributors = np.zeros((c, height, width), np.int32)
    a.image, a.final_t, a.contributors = _ptr(image), _ptr(final_t), _ptr(contributors)
    lib().oracle_render_fwd(ctypes.byref(a))
    return image, final_t, contributors


def render_pair_counts(width, height, ranges, ids, centers, conics, features, extra=None, background=None):
    """(visited, accepted) (pixel, Gaussian) pairs of the blend loop
    (gs3d/render.py:82-117): entries visited up to and including the one
    that terminates a pixel, and blends."""
    keep = []
    a, c, n, channels = _render_args(width, height, ranges, ids, centers, conics, features, extra, background, keep)
    image = np.zeros((c, height, width, channels), np.float32)
    final_t = np.zeros((c, height, width), np.float32)
    contributors = np.zeros((c, height, width), np.int32)
    a.image, a.final_t, a.contributors = _ptr(image), _ptr(final_t), _ptr(contributors)
    counts = np.zeros(2, np.int64)
    lib().oracle_render_pair_counts(ctypes.byref(a), _ptr(counts))
    return int(counts[0]), int(counts[1])


def render_fwd_stats(width, height, ranges, ids, centers, conics, features, kinds, pixel_values, extra=None,
                     background=None):
    """render_fwd plus contribution statistics (statistics.py:46-70): kinds[r]
    is 0 (masked count) or 1 (weighted sum), pixel_values (views, R, H, W).
    Returns image, final_t, contributors, counts (views, #counts, N) int32 and
    sums (views, #sums, N) float32."""
    keep = []
    a, c, n, channels = _render_args(width, height, ranges, ids, centers, conics, features, extra, background, keep)
    image = np.zeros((c, height, width, channels), np.float32)
    final_t = np.zeros((c, height, width), np.float32)
    contributors = np.zeros((c, height, width), np.int32)
    a.image, a.final_t, a.contributors = _ptr(image), _ptr(final_t), _ptr(contributors)
    kinds = list(kinds)
    pv = _f32(pixel_values).reshape(c, len(kinds), height * width)
    counts = np.zeros((c, kinds.count(0), n), np.int32)
    sums = np.zeros((c, kinds.count(1), n), np.float32)
    st = abi.RenderStatsArgs()
    st.requests = len(kinds)
    st.sum_mask = sum(1 << r for r, k in enumerate(kinds) if k == 1)
    st.pixel_values, st.pixel_view_stride = _ptr(pv), pv.shape[1] * pv.shape[2]
    st.counts, st.counts_view_stride = _ptr(counts), counts.shape[1] * n
    st.sums, st.sums_view_stride = _ptr(sums), sums.shape[1] * n
    lib().oracle_render_fwd_stats(ctypes.byref(a), ctypes.byref(st))
    return image, final_t, contributors, counts, sums


def render_bwd(width, height, ranges, ids, centers, conics, features, final_t, contributors, upstream,
               extra=None, background=None, absgrad=False):
    """gs3d/render.py:211-356; returns grads for centers, conics, features, extra, abs."""
    keep = []
    a, c, n, channels = _render_args(width, height, ranges, ids, centers, conics, features, extra, background, keep)
    final_t, contributors = _f32(final_t), _i32(contributors)
    upstream = _f32(upstream).reshape(c, height, width, channels)
    a.final_t, a.contributors = _ptr(final_t), _ptr(contributors)
    b = abi.RenderBwdArgs()
    b.fwd = a
    b.upstream = _ptr(upstream)
    features = _f32(features)
    gc = np.zeros((c, n, 2), np.float32)
    gk = np.zeros((c, n, 4), np.float32)
    gf = np.zeros(features.shape, np.float32)
    b.grad_centers, b.grad_centers_stride = _ptr(gc), 2
    b.grad_conics, b.grad_conics_stride = _ptr(gk), 4
    b.grad_features, b.grad_feat_stride = _ptr(gf), features.shape[-1]
    b.grad_feat_view_stride = a.feat_view_stride
    ga = None
    if absgrad:
        ga = np.zeros((c, n, 2), np.float32)
        b.abs_centers, b.abs_stride = _ptr(ga), 2
    ge = None
    if extra is not None:
        extra = _f32(extra)
        ge = np.zeros(extra.shape, np.float32)
        b.grad_extra, b.grad_extra_stride = _ptr(ge), extra.shape[-1]
        b.grad_extra_view_stride = a.extra_view_stride
    lib().oracle_render_bwd(ctypes.byref(b))
    return dict(centers=gc, conics=gk, features=gf, extra=ge, abs=ga)


def projection_loss_f64(mean, quat, scale, opacity, view, proj, width, height, fx, fy, gc, gk):
    f = lambda x: np.ascontiguousarray(x, dtype=np.float64)
    mean, quat, scale, view, proj, gc, gk = map(f, (mean, quat, scale, view, proj, gc, gk))
    return lib().oracle_projection_loss_f64(
        _ptr(mean), _ptr(quat), _ptr(scale), float(opacity), _ptr(view), _ptr(proj),
        width, height, float(fx), float(fy), _ptr(gc), _ptr(gk))


def projection_vjp_f64(mean, quat, scale, opacity, view, proj, width, height, fx, fy, gc, gk):
    f = lambda x: np.ascontiguousarray(x, dtype=np.float64)
    mean, quat, scale, view, proj, gc, gk = map(f, (mean, quat, scale, view, proj, gc, gk))
    out = np.zeros(43, np.float64)
    lib().oracle_projection_vjp_f64(
        _ptr(mean), _ptr(quat), _ptr(scale), float(opacity), _ptr(view), _ptr(proj),
        width, height, float(fx), float(fy), _ptr(gc), _ptr(gk), _ptr(out))
    return dict(mean=out[0:3], quat=out[3:7], scale=out[7:10], opacity=out[10],
                view=out[11:27].reshape(4, 4), proj=out[27:43].reshape(4, 4))


# ---------------------------------------------------------------------------
# Float32 error bounds of the gradient path (running error analysis in the
# C restatement, see Err in gs3d_oracle.cpp).  A gradient entry computed in
# float32 by two implementations that sum the same terms in different orders
# and with different fused operations may differ by at most
#     B = P + 2 R + LAMBDA * sqrt(n) * u * A
# where, over the entry's n terms t, A = sum |t|, P = sum of the bounds the
# terms inherit from their inputs' differences, R = sum of the first-order
# rounding-error bounds of each term's own evaluation (counted once for each
# implementation), and LAMBDA sqrt(n) u A bounds the difference between two
# summation orders (the probabilistic rounding-error bound of Higham and
# Mary, SIAM J. Sci. Comput. 41(5), 2019: it holds with probability at least
# 1 - 2 exp(-LAMBDA^2 / 2) for independent rounding errors; LAMBDA = 6 gives
# 3e-8).  u = 2^-24.
# ---------------------------------------------------------------------------
UNIT_ROUNDOFF = 2.0 ** -24
REORDER_LAMBDA = 6.0


def sum_bound(stats):
    """B of entries given their [sum |t|, sum p, sum r, count] statistics."""
    stats = np.asarray(stats, np.float64)
    A, P, R, n = stats[..., 0], stats[..., 1], stats[..., 2], stats[..., 3]
    return P + 2.0 * R + REORDER_LAMBDA * np.sqrt(n) * UNIT_ROUNDOFF * A


def pair_bound(pr):
    """B of entries computed once per implementation from [p, r] pairs."""
    pr = np.asarray(pr, np.float64)
    return pr[..., 0] + 2.0 * pr[..., 1]


def render_bwd_bound(width, height, ranges, ids, centers, conics, features, final_t, contributors, upstream,
                     extra=None, background=None, float64=False):
    """Per-entry bounds B of render_bwd's gradients (same keys); with
    float64, instead the gradients evaluated in double arithmetic."""
    keep = []
    a, c, n, channels = _render_args(width, height, ranges, ids, centers, conics, features, extra, background, keep)
    final_t, contributors = _f32(final_t), _i32(contributors)
    upstream = _f32(upstream).reshape(c, height, width, channels)
    a.final_t, a.contributors = _ptr(final_t), _ptr(contributors)
    b = abi.RenderBwdArgs()
    b.fwd = a
    b.upstream = _ptr(upstream)
    features = _f32(features)
    b.grad_feat_stride, b.grad_feat_view_stride = features.shape[-1], a.feat_view_stride
    stats = dict(centers=np.zeros((c, n, 2, 4)), conics=np.zeros((c, n, 4, 4)), abs=np.zeros((c, n, 2, 4)),
                 features=np.zeros(features.shape + (4,)))
    if extra is not None:
        extra = _f32(extra)
        b.grad_extra_stride, b.grad_extra_view_stride = extra.shape[-1], a.extra_view_stride
        stats["extra"] = np.zeros(extra.shape + (4,))
    if float64:
        vals = {k: np.zeros(v.shape[:-1]) for k, v in stats.items()}
        lib().oracle_render_bwd_f64(ctypes.byref(b), _ptr(vals["centers"]), _ptr(vals["conics"]),
                                    _ptr(vals["abs"]), _ptr(vals["features"]), _ptr(vals.get("extra")))
        vals.setdefault("extra", None)
        return vals
    lib().oracle_render_bwd_bound(ctypes.byref(b), _ptr(stats["centers"]), _ptr(stats["conics"]),
                                  _ptr(stats["abs"]), _ptr(stats["features"]), _ptr(stats.get("extra")))
    out = {k: sum_bound(v) for k, v in stats.items()}
    out.setdefault("extra", None)
    return out


def project_bwd_bound(means, quats, scales, opacities, view, projection, intrinsics, width, height, radii,
                      grad_centers, grad_conics, e_centers, e_conics, sh=None, sh_degree=0, camera_centers=None,
                      grad_colors=None, e_colors=None, normalize_quats=False):
    """Per-entry bounds B of project_bwd's outputs given bounds e_* of the
    upstream gradients (same keys as project_bwd)."""
    means, quats, scales, opacities = _f32(means), _f32(quats), _f32(scales), _f32(opacities)
    view, projection, intrinsics = (
        _f32(view).reshape(-1, 4, 4), _f32(projection).reshape(-1, 4, 4), _f32(intrinsics).reshape(-1, 3, 3))
    n, c = len(means), len(view)
    radii = _i32(radii).reshape(c, n)
    gc = _f32(grad_centers).reshape(c, n, 2)
    gk = _f32(grad_conics).reshape(c, n, 4)
    ec = np.ascontiguousarray(e_centers, np.float64).reshape(c, n, 2)
    ek = np.ascontiguousarray(e_conics, np.float64).reshape(c, n, 4)
    a = abi.ProjectBwdArgs()
    a.n, a.views, a.width, a.height = n, c, width, height
    a.normalize_quats = int(normalize_quats)
    for name, arr in (("means", means), ("quats", quats), ("scales", scales), ("opacities", opacities),
                      ("view", view), ("projection", projection), ("intrinsics", intrinsics), ("radii", radii)):
        setattr(a, name, _ptr(arr))
    a.grad_centers, a.grad_centers_stride = _ptr(gc), 2
    a.grad_conics, a.grad_conics_stride = _ptr(gk), 4
    pr = dict(means=np.zeros((n, 3, 2)), quats=np.zeros((n, 4, 2)), scales=np.zeros((n, 3, 2)),
              opacities=np.zeros((n, 2)))
    st = dict(view=np.zeros((c, 4, 4, 4)), projection=np.zeros((c, 4, 4, 4)))
    keep, ecol = [], None
    if sh is not None:
        sh = _f32(sh)
        a.sh = _ptr(sh)
        a.sh_rows = sh.shape[-2]
        a.sh_view_stride = sh.shape[-3] * sh.shape[-2] * 3 if sh.ndim == 4 else 0
        a.sh_degree = sh_degree
        cc = _f32(np.zeros((c, 3)) if camera_centers is None else camera_centers).reshape(c, 3)
        gcol = _f32(grad_colors).reshape(c, n, 3)
        ecol = np.ascontiguousarray(e_colors, np.float64).reshape(c, n, 3)
        keep += [sh, cc, gcol]
        a.camera_centers = _ptr(cc)
        a.grad_colors, a.grad_colors_stride = _ptr(gcol), 3
        pr["sh"] = np.zeros(sh.shape + (2,))
        st["camera_centers"] = np.zeros((c, 3, 4))
    lib().oracle_project_bwd_bound(ctypes.byref(a), _ptr(ec), _ptr(ek), _ptr(ecol), _ptr(pr["means"]),
                                   _ptr(pr["quats"]), _ptr(pr["scales"]), _ptr(pr["opacities"]), _ptr(pr.get("sh")),
                                   _ptr(st["view"]), _ptr(st["projection"]), _ptr(st.get("camera_centers")))
    out = {k: pair_bound(v) for k, v in pr.items()}
    out.update({k: sum_bound(v) for k, v in st.items()})
    return out


def camera_backward_bound(Ks, grad_full, e_full, width, height, inverse, grad_centers, e_centers):
    """Per-entry bound B of camera_backward's (C,4,4) result."""
    Ks = _f32(Ks).reshape(-1, 3, 3)
    c = len(Ks)
    gf = None if grad_full is None else _f32(grad_full).reshape(c, 4, 4)
    ef = None if e_full is None else np.ascontiguousarray(e_full, np.float64).reshape(c, 4, 4)
    gc = None if grad_centers is None else _f32(grad_centers).reshape(c, 3)
    ec = None if e_centers is None else np.ascontiguousarray(e_centers, np.float64).reshape(c, 3)
    inv = _f32(inverse).reshape(c, 4, 4)
    out = np.zeros((c, 4, 4, 2))
    lib().oracle_camera_backward_bound(_ptr(Ks), _ptr(gf), _ptr(ef), width, height, _ptr(inv), _ptr(gc), _ptr(ec), c,
                                       _ptr(out))
    return pair_bound(out)
