"""Projection forward/backward launches (gs3d/projection.py:89-428 of the
reference) over gs3d_project_fwd / gs3d_project_bwd.

All cameras of one Gaussian batch go through one launch: each thread reads
its Gaussian (and SH block) once and writes every view's rows, so the
per-view state tensors below have a leading view axis (C, N, ...).  With one
camera and no SH this is exactly the reference's ``project`` kernel; with SH
it also evaluates primitives/sh.py:44-79 on the culled geometry, and with
metadata it also writes splatting/metadata.py:12-31 rows.
"""

from dataclasses import dataclass
import ctypes

import torch
from torch import Tensor

from ..runtime import abi, native
from ..splatting.geometry import ProjectedFootprint, ProjectedGaussians  # noqa: F401  (re-export)


@dataclass(slots=True)
class ProjectedViews:
    """Per-view projected state, all (C, N, ...) contiguous."""

    centers: Tensor
    conics: Tensor
    radii: Tensor
    tile_counts: Tensor
    depths: Tensor
    colors: Tensor | None = None
    means2d: Tensor | None = None
    opacities: Tensor | None = None
    meta_conics: Tensor | None = None

    def view(self, c: int) -> ProjectedGaussians:
        return ProjectedGaussians(self.centers[c], self.conics[c], self.radii[c], self.tile_counts[c], self.depths[c])


def _sh_layout(sh: Tensor, views: int) -> tuple[Tensor, int, int]:
    """(contiguous coefficients, view stride in floats, rows K)."""
    sh = sh.contiguous()
    if sh.ndim == 4:
        if sh.shape[0] != views:
            raise ValueError("per-view SH coefficients need one block per camera")
        return sh, sh.shape[1] * sh.shape[2] * 3, sh.shape[2]
    return sh, 0, sh.shape[1]


@native.no_grad
def project_views(means: Tensor, quats: Tensor, scales: Tensor, opacities: Tensor, view: Tensor,
                  projection: Tensor, intrinsics: Tensor, width: int, height: int, near: float, far: float,
                  radius_clip: float, *, sh: Tensor | None = None, sh_degree: int = 0,
                  camera_centers: Tensor | None = None, metadata: bool = False,
                  tile_mode: str = "radius", normalize_quats: bool = False) -> ProjectedViews:
    """Launch the fused projection for every camera in ``view`` (C,4,4);
    ``tile_counts`` follow ``tile_mode`` (gs3d/projection.py:150-161).  With
    ``normalize_quats`` the quaternions are raw and the kernel normalises
    them as torch.nn.functional.normalize does."""
    device = means.device
    n = len(means)
    views = view.reshape(-1, 4, 4).shape[0]
    f32 = dict(dtype=torch.float32, device=device)
    i32 = dict(dtype=torch.int32, device=device)
    out = ProjectedViews(
        torch.empty((views, n, 2), **f32), torch.empty((views, n, 4), **f32), torch.empty((views, n), **i32),
        torch.empty((views, n), **i32), torch.empty((views, n), **f32),
    )
    keep = [means, quats, scales, opacities]
    a = abi.ProjectArgs()
    a.n, a.views, a.width, a.height = n, views, width, height
    a.near_plane, a.far_plane, a.radius_clip = float(near), float(far), float(radius_clip)
    a.tile_mode = abi.TILE_MODES[tile_mode]
    a.normalize_quats = int(normalize_quats)
    means, quats, scales, opacities = (t.contiguous() for t in (means, quats, scales, opacities))
    view, projection, intrinsics = (t.reshape(views, *t.shape[-2:]).contiguous() for t in (view, projection, intrinsics))
    keep += [means, quats, scales, opacities, view, projection, intrinsics]
    for name, t in (("means", means), ("quats", quats), ("scales", scales), ("opacities", opacities),
                    ("view", view), ("projection", projection), ("intrinsics", intrinsics),
                    ("centers", out.centers), ("conics", out.conics), ("radii", out.radii),
                    ("tiles", out.tile_counts), ("depths", out.depths)):
        setattr(a, name, native.ptr(t))
    if sh is not None:
        sh, stride, rows = _sh_layout(sh, views)
        keep.append(sh)
        out.colors = torch.empty((views, n, 3), **f32)
        a.sh, a.sh_view_stride, a.sh_rows, a.sh_degree = native.ptr(sh), stride, rows, int(sh_degree)
        if sh_degree > 0:
            camera_centers = camera_centers.reshape(views, 3).contiguous()
            keep.append(camera_centers)
            a.camera_centers = native.ptr(camera_centers)
        a.colors = native.ptr(out.colors)
    if metadata:
        out.means2d = torch.empty((views, n, 2), **f32)
        out.opacities = torch.empty((views, n), **f32)
        out.meta_conics = torch.empty((views, n, 3), **f32)
        a.means2d, a.meta_opacities, a.meta_conics = (
            native.ptr(out.means2d), native.ptr(out.opacities), native.ptr(out.meta_conics))
    native.call("gs3d_project_fwd", ctypes.byref(a), native.stream(device))
    return out


# Cameras whose camera gradients one gs3d_project_bwd launch accumulates
# (per-wavefront LDS accumulators); more cameras run in groups of this size.
CAMERA_GRADIENT_GROUP = 16


@native.no_grad
def backward_views(means: Tensor, quats: Tensor, scales: Tensor, opacities: Tensor, view: Tensor,
                   projection: Tensor, intrinsics: Tensor, width: int, height: int, radii: Tensor,
                   grad_centers: Tensor, grad_conics: Tensor, needs: tuple[bool, ...], *,
                   sh: Tensor | None = None, sh_degree: int = 0, camera_centers: Tensor | None = None,
                   grad_colors: Tensor | None = None, need_sh: bool = False, need_centers: bool = False,
                   normalize_quats: bool = False, need_screen: bool = False):
    """Projection (+SH) VJP summed over views; with ``normalize_quats`` the
    quaternions are raw and their gradient includes the normalisation.

    ``needs`` = (means, quats, scales, opacities, view, projection).
    grad_centers / grad_conics may be strided views with unit inner stride;
    ``need_screen`` also returns grad_centers as a contiguous (views, N, 2)
    tensor under "screen" (zero where radii are not positive).
    Returns dict with the requested gradients (None otherwise).

    Any number of cameras: when camera gradients are requested for more than
    CAMERA_GRADIENT_GROUP cameras, the launch runs per group of cameras and
    the per-Gaussian gradients of the groups are summed (the reference
    launches its projection VJP once per view, gs3d/api.py:132-189).
    """
    device = means.device
    n = len(means)
    views = radii.shape[0]
    f32 = dict(dtype=torch.float32, device=device)
    res = dict(means=None, quats=None, scales=None, opacities=None, view=None, projection=None,
               sh=None, camera_centers=None, screen=None)
    if n == 0:
        for key, shape in (("view", (views, 4, 4)), ("projection", (views, 4, 4))):
            res[key] = torch.zeros(shape, **f32)
        return res
    if needs[0] or (sh is not None and sh_degree > 0):
        res["means"] = torch.empty((n, 3), **f32)
    if needs[1]:
        res["quats"] = torch.empty((n, 4), **f32)
    if needs[2]:
        res["scales"] = torch.empty((n, 3), **f32)
    if needs[3]:
        res["opacities"] = torch.empty((n,), **f32)
    if needs[4]:
        res["view"] = torch.zeros((views, 4, 4), **f32)
    if needs[5]:
        res["projection"] = torch.zeros((views, 4, 4), **f32)
    if need_screen:
        res["screen"] = torch.empty((views, n, 2), **f32)
    means, quats, scales, opacities = (t.contiguous() for t in (means, quats, scales, opacities))
    view, projection, intrinsics = (t.reshape(views, *t.shape[-2:]).contiguous() for t in (view, projection, intrinsics))
    radii = radii.contiguous()
    for t in (grad_centers, grad_conics):
        if t.stride(-1) != 1 or t.stride(0) != t.stride(1) * n:
            raise ValueError("gradient rows must be evenly strided (views, N, k)")
    cc = None
    if sh is not None:
        sh, stride, rows = _sh_layout(sh, views)
        if sh_degree > 0:
            cc = camera_centers.reshape(views, 3).contiguous()
            if need_centers:
                res["camera_centers"] = torch.zeros((views, 3), **f32)
        if grad_colors.stride(-1) != 1:
            grad_colors = grad_colors.contiguous()
        if need_sh:
            res["sh"] = torch.empty(sh.shape, **f32)
    camera_grads = needs[4] or needs[5] or res["camera_centers"] is not None
    group = CAMERA_GRADIENT_GROUP if camera_grads else views
    per_gaussian = ("means", "quats", "scales", "opacities") + (("sh",) if sh is not None and stride == 0 else ())
    for v0 in range(0, views, group):
        v1 = min(views, v0 + group)
        out = dict(res)
        if v0 > 0:
            # Later groups write per-Gaussian sums into fresh buffers, added below.
            for key in per_gaussian:
                if res[key] is not None:
                    out[key] = torch.empty_like(res[key])
        a = abi.ProjectBwdArgs()
        a.n, a.views, a.width, a.height = n, v1 - v0, width, height
        a.normalize_quats = int(normalize_quats)
        for name, t in (("means", means), ("quats", quats), ("scales", scales), ("opacities", opacities),
                        ("view", view[v0:v1]), ("projection", projection[v0:v1]),
                        ("intrinsics", intrinsics[v0:v1]), ("radii", radii[v0:v1])):
            setattr(a, name, native.ptr(t))
        a.grad_centers, a.grad_centers_stride = native.ptr(grad_centers[v0:v1]), grad_centers.stride(1)
        a.grad_conics, a.grad_conics_stride = native.ptr(grad_conics[v0:v1]), grad_conics.stride(1)
        a.grad_means = native.ptr(out["means"])
        a.grad_quats = native.ptr(out["quats"])
        a.grad_scales = native.ptr(out["scales"])
        a.grad_opacities = native.ptr(out["opacities"])
        a.grad_view = native.ptr(None if out["view"] is None else out["view"][v0:v1])
        a.grad_projection = native.ptr(None if out["projection"] is None else out["projection"][v0:v1])
        a.screen_grad = native.ptr(None if out["screen"] is None else out["screen"][v0:v1])
        if sh is not None:
            a.sh = native.ptr(sh if stride == 0 else sh[v0:v1])
            a.sh_view_stride, a.sh_rows, a.sh_degree = stride, rows, int(sh_degree)
            if cc is not None:
                a.camera_centers = native.ptr(cc[v0:v1])
                if out["camera_centers"] is not None:
                    a.grad_camera_centers = native.ptr(out["camera_centers"][v0:v1])
            a.grad_colors, a.grad_colors_stride = native.ptr(grad_colors[v0:v1]), grad_colors.stride(1)
            if out["sh"] is not None:
                a.grad_sh = native.ptr(out["sh"] if stride == 0 else out["sh"][v0:v1])
        native.call("gs3d_project_bwd", ctypes.byref(a), native.stream(device))
        if v0 > 0:
            for key in per_gaussian:
                if res[key] is not None:
                    res[key] += out[key]
    return res
