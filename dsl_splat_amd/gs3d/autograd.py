"""Original-3DGS blending boundary and its projection/SH/camera VJPs.

Mirrors gs3d/autograd.py:17-171 of the reference, with one Function per
Gaussian batch covering all of its cameras (the reference applies one per
view).  Forward blends the already projected and sorted frame; backward runs
the blend VJP, writes the absolute screen gradients, then one fused
projection + SH VJP over all views and the camera VJP:

    viewmats.grad = d(view) + camera_backward(d(full projection), d(centres))

which is what the reference's separate camera/projection/SH autograd nodes
sum to.  Gradients of means2d are the blend's centre gradients
(screen_gradient_mode "projected_mean").
"""

import math
import os
from dataclasses import dataclass
from typing import Any

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from . import lists as tile_lists, projection, render
from .. import profiling
from ..runtime.gradients import AbsGradientTarget
from ..splatting.cameras import camera_backward
from ..statistics import PreparedStatistics


@dataclass(slots=True)
class ViewBins:
    """Tile lists of cameras [v0, v1): ranges ((v1-v0)*T, 2) into ids."""

    v0: int
    v1: int
    ranges: Tensor
    ids: Tensor


@dataclass(slots=True)
class Frame:
    """Forward state of one Gaussian batch (all C cameras).  ``bins`` is one
    entry for all cameras unless their pairs together exceed the int32
    offsets of one binning launch; then each group of cameras has its own
    lists and is blended by its own launch."""

    width: int
    height: int
    Ks: Tensor                 # (C,3,3) detached
    full: Tensor               # (C,4,4) projection rows
    inverse: Tensor | None     # (C,4,4) view inverse (SH only)
    camera_centers: Tensor | None
    state: projection.ProjectedViews
    bins: list[ViewBins]
    pair_count: int
    sh_degree: int | None
    background: Tensor | None  # (C, D) or None
    lists: "tile_lists.CappedLists | None" = None  # capped lists (one bins entry only), until blended


def _views(t, v0: int, v1: int, views: int, per_view_ndim: int):
    """Cameras [v0, v1) of a per-camera tensor (leading camera axis at
    ``per_view_ndim`` dimensions); shared tensors pass through."""
    if t is None or t.ndim < per_view_ndim or t.shape[0] != views:
        return t
    return t[v0:v1]


# The backward's accumulation buffers (blend gradient record, colour and
# extra-channel gradients) are views of one allocation that the forward blend
# launch clears while it blends (its arithmetic leaves HBM idle; a separate
# fill kernel per buffer cost ~55 us per step at 3M Gaussians, 4 cameras).
# The buffers then live from the forward to the backward: C*N*(6 or 8) + the
# blended channels' C*N*D floats (0.43 GB at 3M Gaussians, 4 cameras, SH
# colours).  GS3D_CLEAR_IN_BACKWARD=1 makes the backward allocate and clear
# them instead, for callers bound by memory rather than time.
CLEAR_DURING_FORWARD = os.environ.get("GS3D_CLEAR_IN_BACKWARD", "0") != "1"


@dataclass(slots=True)
class ClearedBuffers:
    """Accumulation targets of the blend VJP, zeroed by the forward blend."""

    record: Tensor
    features: Tensor | None
    extra: Tensor | None


def _buffers_for_backward(device: torch.device, shapes) -> tuple[ClearedBuffers, Tensor]:
    """(record, features, extra) as views of one float32 allocation, each
    starting on a 16-byte boundary, and that allocation (which the forward
    blend clears)."""
    offsets, total = [], 0
    for shape in shapes:
        offsets.append(total)
        total += 0 if shape is None else (math.prod(shape) + 3) // 4 * 4
    flat = torch.empty(max(total, 4), dtype=torch.float32, device=device)
    views = [None if shape is None else flat[o:o + math.prod(shape)].view(shape) for shape, o in zip(shapes, offsets)]
    return ClearedBuffers(*views), flat


def _statistics_views(statistics, v0: int, v1: int):
    if statistics is None:
        return None
    return PreparedStatistics(statistics.key, statistics.pixel_values[v0:v1], statistics.counts[v0:v1],
                              statistics.sums[v0:v1])


class Rasterize(torch.autograd.Function):
    @staticmethod
    def forward(
        ctx: Any,
        means: Tensor,
        quats: Tensor,
        scales: Tensor,
        opacities: Tensor,
        colors: Tensor,
        extra_features: Tensor | None,
        viewmats: Tensor,
        screen: Tensor | None,
        frame: Frame,
        absolute: list[AbsGradientTarget | None] | None,
        statistics: PreparedStatistics | None,
        grad_enabled: bool,
    ) -> tuple[Tensor, Tensor, Tensor]:
        """Returns the (C,H,W,D) features, (C,H,W,E) extra (E may be 0) and
        (C,H,W,1) alpha planes; statistics, when given, accumulate in the same
        blend launch."""
        st = frame.state
        blended = st.colors if frame.sh_degree is not None else colors
        train = grad_enabled and any(ctx.needs_input_grad[:8])
        ctx.cleared = None
        zero = None
        if train and len(frame.bins) == 1 and CLEAR_DURING_FORWARD:
            needs = ctx.needs_input_grad
            absgrad = absolute is not None and any(t is not None for t in absolute)
            views, n = st.centers.shape[0], st.centers.shape[1]
            need_features = frame.sh_degree is not None or needs[4]
            shapes = ((views, n, render.RECORD_ABS if absgrad else render.RECORD),
                      blended.shape if need_features and blended is not None else None,
                      extra_features.shape if needs[5] and extra_features is not None else None)
            ctx.cleared, zero = _buffers_for_backward(st.centers.device, shapes)
        if len(frame.bins) == 1:
            bins = frame.bins[0]
            lists, frame.lists = frame.lists, None
            output = render.render_views(
                bins.ranges, bins.ids, st.centers, st.conics, blended, frame.width, frame.height,
                extra=extra_features, background=frame.background, one_tail=True, statistics=statistics,
                zero=zero, lists=lists,
            )
            if lists is not None:
                tile_lists.remember(lists)
        else:
            views = st.centers.shape[0]
            parts = []
            for bins in frame.bins:
                v0, v1 = bins.v0, bins.v1
                parts.append(render.render_views(
                    bins.ranges, bins.ids, st.centers[v0:v1], st.conics[v0:v1], _views(blended, v0, v1, views, 3),
                    frame.width, frame.height, extra=_views(extra_features, v0, v1, views, 3),
                    background=_views(frame.background, v0, v1, views, 2), one_tail=True,
                    statistics=_statistics_views(statistics, v0, v1),
                ))
            output = render.RenderedPixels(*(
                None if getattr(parts[0], f) is None else torch.cat([getattr(p, f) for p in parts])
                for f in ("features", "extra", "alpha", "transmittance", "contributors")))
        profiling.mark("blended")
        if train:
            ctx.save_for_backward(means, quats, scales, opacities, colors, extra_features, viewmats,
                                  output.transmittance, output.contributors)
            ctx.frame = frame
            ctx.absolute = absolute
        ctx.set_materialize_grads(False)
        extra = output.extra
        if extra is None:
            extra = output.features.new_empty(output.features.shape[:-1] + (0,))
            ctx.mark_non_differentiable(extra)
        return output.features, extra, output.alpha

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, grad_features: Tensor | None, grad_extra_image: Tensor | None,
                 grad_alpha: Tensor | None) -> tuple[Tensor | None, ...]:
        none = (None,) * 12
        if grad_features is None and grad_extra_image is None and grad_alpha is None:
            return none
        if grad_extra_image is not None and grad_extra_image.numel() == 0:
            grad_extra_image = None
        means, quats, scales, opacities, colors, extra, viewmats, final_t, contributors = ctx.saved_tensors
        frame: Frame = ctx.frame
        st = frame.state
        needs = ctx.needs_input_grad
        sh = frame.sh_degree is not None
        blended = st.colors if sh else colors
        absgrad = ctx.absolute is not None and any(t is not None for t in ctx.absolute)
        profiling.mark("backward")
        upstream = (grad_features, grad_extra_image, grad_alpha)
        blend_args = dict(one_tail=True, absgrad=absgrad, need_features=sh or needs[4], need_extra=needs[5])
        if len(frame.bins) == 1:
            bins = frame.bins[0]
            cleared, ctx.cleared = ctx.cleared, None
            record, grad_blended, grad_extra = render.backward_views(
                bins.ranges, bins.ids, st.centers, st.conics, blended, final_t, contributors, upstream,
                frame.width, frame.height, extra=extra, background=frame.background, cleared=cleared, **blend_args,
            )
        else:
            views = st.centers.shape[0]
            parts = []
            for bins in frame.bins:
                v0, v1 = bins.v0, bins.v1
                parts.append(render.backward_views(
                    bins.ranges, bins.ids, st.centers[v0:v1], st.conics[v0:v1], _views(blended, v0, v1, views, 3),
                    final_t[v0:v1], contributors[v0:v1], tuple(_views(u, v0, v1, views, 1) for u in upstream),
                    frame.width, frame.height, extra=_views(extra, v0, v1, views, 3),
                    background=_views(frame.background, v0, v1, views, 2), **blend_args,
                ))

            def join(k, source):
                items = [p[k] for p in parts]
                if items[0] is None:
                    return None
                # Per-camera sources get per-camera gradients; shared ones sum.
                return torch.cat(items) if source is None or source.ndim == 3 else torch.stack(items).sum(0)

            record, grad_blended, grad_extra = join(0, None), join(1, blended), join(2, extra)
        if absgrad:
            for c, target in enumerate(ctx.absolute):
                if target is not None:
                    target.write(record[c, :, 6:8])
        profiling.mark("blend_vjp")
        grad_centers = record[..., 0:2]
        grad_conics = record[..., 2:6]
        proj_needs = (needs[0], needs[1], needs[2], needs[3], needs[6], needs[6])
        want_sh = sh and (needs[4] or (frame.sh_degree > 0 and (needs[0] or needs[6])))
        grads = dict(means=None, quats=None, scales=None, opacities=None, view=None, projection=None, sh=None,
                     camera_centers=None, screen=None)
        if any(proj_needs) or want_sh:
            grads = projection.backward_views(
                means, quats, scales, opacities, viewmats.detach(), frame.full, frame.Ks, frame.width,
                frame.height, st.radii, grad_centers, grad_conics, proj_needs,
                sh=colors if sh else None, sh_degree=frame.sh_degree or 0, camera_centers=frame.camera_centers,
                grad_colors=grad_blended if sh else None, need_sh=sh and needs[4], normalize_quats=True,
                need_centers=sh and (frame.sh_degree or 0) > 0 and needs[6], need_screen=needs[7],
            )
        profiling.mark("projection_vjp")
        if grads["screen"] is not None:
            # Contiguous rows: the means2d leaf accumulates them without a strided copy.
            grad_centers = grads["screen"]
        grad_view = None
        if needs[6]:
            grad_view = camera_backward(frame.Ks, grads["projection"], frame.width, frame.height,
                                        frame.inverse if frame.inverse is not None else frame.full,
                                        grads["camera_centers"])
            if grads["view"] is not None:
                grad_view = grad_view + grads["view"]
            grad_view = grad_view.reshape(viewmats.shape)
        profiling.mark("camera_vjp")
        return (
            grads["means"] if needs[0] else None,
            grads["quats"] if needs[1] else None,
            grads["scales"] if needs[2] else None,
            grads["opacities"] if needs[3] else None,
            (grads["sh"] if sh else grad_blended) if needs[4] else None,
            grad_extra if needs[5] else None,
            grad_view,
            grad_centers if needs[7] else None,
            None,
            None,
            None,
            None,
        )
