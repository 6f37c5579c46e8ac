"""Differentiable single-view projection and rendering (gs3d/ops.py:27-338 of
the reference): ``prepare_gaussians`` -> ``bin_and_sort`` ->
``rasterize_to_pixels``, each behind its own autograd edge, on the same HIP
kernels as the fused ``rasterize``."""

from dataclasses import dataclass, field, replace
from typing import Any, Sequence

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from . import projection, render
from .cameras import ViewConfig, prepare_camera
from ..cameras import PinholeCamera
from ..inputs import check_tensor, spherical_harmonics
from ..primitives.tiling import TileBins
from ..splatting.binning import bin_and_sort as _bin_arrays, validate_tile_mode
from ..statistics import PreparedStatistics, StatisticsRequest, prepare_statistics


@dataclass(slots=True)
class GaussianGeometry:
    """One camera's projected Gaussians: (N,2) centres, (N,4) conic + opacity,
    (N,) radii, tile counts and depths.  Centres and conics are meaningful only
    where radii > 0."""

    centers: Tensor
    conics: Tensor
    radii: Tensor
    tile_counts: Tensor
    depths: Tensor
    _config: ViewConfig = field(repr=False)


@dataclass(slots=True)
class GaussianTiles:
    ranges: Tensor
    gaussian_ids: Tensor
    _geometry: GaussianGeometry = field(repr=False)


@dataclass(slots=True)
class PixelResult:
    features: Tensor
    alpha: Tensor
    statistics: dict[str, Tensor] = field(default_factory=dict)


class _Project(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, means, quats, scales, opacities, view, full, intrinsics, config: ViewConfig,
                grad_enabled: bool):
        state = projection.project_views(means, quats, scales, opacities, view[None], full[None], intrinsics[None],
                                         config.width, config.height, config.near, config.far, config.radius_clip,
                                         tile_mode=config.tile_mode, normalize_quats=True)
        centers, conics, radii, tiles, depths = (state.centers[0], state.conics[0], state.radii[0],
                                                 state.tile_counts[0], state.depths[0])
        if grad_enabled and any(ctx.needs_input_grad[:6]):
            ctx.save_for_backward(means, quats, scales, opacities, view, full, intrinsics, radii)
            ctx.config = config
        ctx.mark_non_differentiable(radii, tiles, depths)
        ctx.set_materialize_grads(False)
        return centers, conics, radii, tiles, depths

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, centers: Tensor | None, conics: Tensor | None, *unused):
        if centers is None and conics is None:
            return (None,) * 9
        means, quats, scales, opacities, view, full, intrinsics, radii = ctx.saved_tensors
        n = len(means)
        gc = torch.zeros((n, 2), dtype=torch.float32, device=means.device) if centers is None else centers.contiguous()
        gk = torch.zeros((n, 4), dtype=torch.float32, device=means.device) if conics is None else conics.contiguous()
        needs = tuple(ctx.needs_input_grad[:6])
        g = projection.backward_views(means, quats, scales, opacities, view[None], full[None], intrinsics[None],
                                      ctx.config.width, ctx.config.height, radii[None], gc[None], gk[None], needs,
                                      normalize_quats=True)
        out = [g["means"], g["quats"], g["scales"], g["opacities"],
               None if g["view"] is None else g["view"][0],
               None if g["projection"] is None else g["projection"][0]]
        return (*(v if needs[i] else None for i, v in enumerate(out)), None, None, None)


class _Pixels(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, centers, conics, features, radii, ranges, ids, background, config: ViewConfig,
                statistics: PreparedStatistics | None, grad_enabled: bool):
        out = render.render_views(ranges, ids, centers[None], conics[None], features, config.width, config.height,
                                  background=None if background is None else background[None], one_tail=True,
                                  statistics=statistics)
        if grad_enabled and any(ctx.needs_input_grad[:3]):
            ctx.save_for_backward(centers, conics, features, ranges, ids, background, out.transmittance,
                                  out.contributors)
            ctx.config = config
        ctx.set_materialize_grads(False)
        return out.features[0], out.alpha[0]

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, grad_features: Tensor | None, grad_alpha: Tensor | None):
        if grad_features is None and grad_alpha is None:
            return (None,) * 10
        centers, conics, features, ranges, ids, background, final_t, contributors = ctx.saved_tensors
        upstream = (None if grad_features is None else grad_features[None], None,
                    None if grad_alpha is None else grad_alpha[None])
        record, gf, _ = render.backward_views(
            ranges, ids, centers[None], conics[None], features, final_t, contributors, upstream,
            ctx.config.width, ctx.config.height, background=None if background is None else background[None],
            one_tail=True, need_features=ctx.needs_input_grad[2])
        grads = (record[0, :, 0:2], record[0, :, 2:6], gf)
        return (*(g if ctx.needs_input_grad[i] else None for i, g in enumerate(grads)), None, None, None, None, None,
                None, None)


# Per-Gaussian parameters of prepare_gaussians: (name, shape after N).  Their
# validation order, exception types and messages are the reference's
# (gs3d/ops.py:215-249), so a caller sees the same error first.
_GAUSSIAN_PARAMETERS = (("means", (3,)), ("quats", (4,)), ("scales", (3,)), ("opacities", ()))


def _leading_means(means) -> tuple[int, torch.device]:
    """N and the device, fixed by the means."""
    if isinstance(means, Tensor) and means.is_cuda and means.ndim == 2 and means.shape[1] == 3:
        return len(means), means.device
    raise ValueError("means must be CUDA float32 (N,3)")


def prepare_gaussians(means: Tensor, quats: Tensor, scales: Tensor, opacities: Tensor, camera: PinholeCamera, *,
                      radius_clip: float = 0.0, tile_mode: str = "radius") -> GaussianGeometry:
    params = (means, quats, scales, opacities)
    n, device = _leading_means(means)
    validate_tile_mode(tile_mode)
    for (name, tail), value in zip(_GAUSSIAN_PARAMETERS, params):
        check_tensor(name, value, device, (n, *tail))
    view, full, intrinsics, camera_config = prepare_camera(camera, radius_clip)
    if view.device != device:
        raise ValueError("camera and Gaussians must use the same CUDA device")
    config = replace(camera_config, tile_mode=tile_mode)
    centers, conics, radii, tiles, depths = _Project.apply(*(t.contiguous() for t in params), view, full, intrinsics,
                                                           config, torch.is_grad_enabled())
    return GaussianGeometry(centers, conics, radii, tiles, depths, config)


def bin_and_sort(geometry: GaussianGeometry) -> GaussianTiles:
    config = geometry._config
    bins: TileBins = _bin_arrays(geometry.centers.detach(), geometry.radii, geometry.tile_counts,
                                 geometry.depths, config.width, config.height, conics=geometry.conics,
                                 tile_mode=config.tile_mode)
    return GaussianTiles(bins["ranges"], bins["point_list"], geometry)


def _pixel_rules(geometry: GaussianGeometry, tiles: GaussianTiles, features: Tensor, background: Tensor | None):
    """rasterize_to_pixels' input checks as (violated?, exception) pairs, in
    the reference's order (gs3d/ops.py:273-300): each is evaluated only once
    the ones before it hold."""
    n, device = len(geometry.radii), geometry.radii.device
    yield (lambda: tiles._geometry is not geometry), ValueError("tiles must have been built from this geometry")
    yield (lambda: check_tensor("features", features, device)), None
    yield ((lambda: features.ndim != 2 or features.shape[0] != n or features.shape[1] <= 0),
           ValueError("features must have shape (N,D), D>0"))
    if background is not None:
        yield (lambda: check_tensor("background", background, device, (features.shape[1],))), None
        yield ((lambda: torch.is_grad_enabled() and background.requires_grad),
               NotImplementedError("background gradients are not supported"))


def rasterize_to_pixels(geometry: GaussianGeometry, tiles: GaussianTiles, features: Tensor,
                        background: Tensor | None = None, *,
                        statistics: Sequence[StatisticsRequest] = ()) -> PixelResult:
    for violated, error in _pixel_rules(geometry, tiles, features, background):
        # A rule without an exception raises its own (check_tensor).
        if violated() and error is not None:
            raise error
    config = geometry._config
    n = len(geometry.radii)
    prepared, outputs = ([], {})
    if statistics:
        prepared, outputs = prepare_statistics(statistics, batch_dims=(), batch_count=1, cameras=1, n=n,
                                               width=config.width, height=config.height,
                                               device=geometry.radii.device)
    image, alpha = _Pixels.apply(geometry.centers, geometry.conics, features.contiguous(), geometry.radii,
                                 tiles.ranges, tiles.gaussian_ids, background, config,
                                 prepared[0] if statistics else None, torch.is_grad_enabled())
    return PixelResult(image, alpha, {name: value[0] for name, value in outputs.items()})


__all__ = [
    "prepare_gaussians",
    "bin_and_sort",
    "rasterize_to_pixels",
    "spherical_harmonics",
    "GaussianGeometry",
    "GaussianTiles",
    "PixelResult",
]
