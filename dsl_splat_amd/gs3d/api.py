"""Original 3DGS API with OpenCV cameras (gs3d/api.py:25-265 of the reference).

Same signature, defaults, validation errors, outputs and ``meta`` keys.  Per
Gaussian batch the host issues: one camera launch, one fused projection
(+SH +metadata) launch for all cameras, the depth ordering of all
(camera, Gaussian) rows with their 8x8-tile group counts, ONE host
synchronisation (camera status codes and the group/pair totals together),
the grouped binning that writes every tile's depth-ordered list without
sorting the pairs (its first kernel enqueued before the synchronisation
once an earlier frame of the same shape has given the item capacity), and
one blend launch for all cameras.  ``tile_mode``
selects the reference's radius squares, SnugBox rectangles or AccuTile
strips (splatting/intersections.py).
"""

from dataclasses import dataclass, field
import math
import threading
from numbers import Integral
from typing import Any, Sequence

import torch
from torch import Tensor

from . import lists as tile_lists
from .autograd import Frame, Rasterize, ViewBins
from .. import profiling
from .projection import project_views
from ..cameras import validate_camera_options
from ..inputs import batch_item, normalize_inputs
from ..runtime import native
from ..splatting import binning
from ..splatting.binning import launch_bin_rows, order_rows, prepare_bin_rows, validate_tile_mode
from ..splatting.cameras import launch_prepare, raise_camera_errors
from ..statistics import StatisticsRequest, prepare_statistics
from ..training import prepare_training_metadata

BACKEND = "gs3d-hip"


@dataclass(slots=True)
class RasterizationResult:
    """What ``rasterize`` returns: (..., C, H, W, D) features and (..., C, H, W, 1)
    alpha (channel-last, owned by the call), the meta dictionary and the
    requested contribution statistics."""

    features: Tensor
    alpha: Tensor
    meta: dict[str, Any]
    statistics: dict[str, Tensor] = field(default_factory=dict)

    @property
    def radii(self) -> Tensor:
        return self.meta["radii"]

    @property
    def means2d(self) -> Tensor:
        return self.meta["means2d"]

    @property
    def extra_features(self) -> Tensor | None:
        return self.meta.get("render_extra_signals")


def _sh_degree(features, sh_coeffs, sh_degree) -> int | None:
    """The SH degree in use (None for plain features); ValueError for
    contradictory or malformed colour arguments (gs3d/api.py:86-102)."""
    if (features is None) == (sh_coeffs is None):
        raise ValueError("provide exactly one of features or sh_coeffs")
    if sh_coeffs is None:
        if sh_degree is not None:
            raise ValueError("sh_degree requires sh_coeffs")
        return None
    if not isinstance(sh_coeffs, Tensor) or sh_coeffs.ndim < 3:
        raise ValueError("sh_coeffs must have shape (...,N,K,3) or (...,C,N,K,3)")
    if sh_degree is None:
        rows = sh_coeffs.shape[-2]
        sh_degree = min(3, math.isqrt(rows) - 1)
    if isinstance(sh_degree, bool) or not isinstance(sh_degree, Integral) or not 0 <= sh_degree <= 3:
        raise ValueError("sh_degree must be an integer in [0,3]")
    return sh_degree


# Pinned host buffers the per-frame status word is copied into, one per
# thread and size: a frame waits for its copy before it returns, so the next
# frame of the thread may reuse the buffer.
_PINNED = threading.local()


def _pinned_status(numel: int) -> Tensor:
    cache = getattr(_PINNED, "buffers", None)
    if cache is None:
        cache = _PINNED.buffers = {}
    buf = cache.get(numel)
    if buf is None:
        buf = cache[numel] = torch.empty(numel, dtype=torch.int64, pin_memory=True)
    return buf


@native.no_grad
def _prepare_frame(means, quats, scales, opacities, viewmats, Ks, width, height, near, far, radius_clip,
                   sh, sh_degree, background, tile_mode="radius", capped=True, slot=0) -> Frame:
    """Camera rows, fused projection, depth order, one synchronisation, binning
    (with ``capped``, of lists capped by the cameras' earlier stops; ``slot``:
    the batch item, whose stops are kept apart from the other items')."""
    profiling.mark("start")
    with_centers = sh_degree is not None and sh_degree > 0
    # One int64 status buffer read back once: [group pairs, tile pairs], the
    # depth keys' bit count (int32 in the low half of the third word), the
    # cameras' 64-bit keys and then their int32 status codes.
    cameras = viewmats.numel() // 16
    status = torch.empty(3 + cameras + (cameras + 1) // 2, dtype=torch.int64, device=viewmats.device)
    key_bits = status[2:3].view(torch.int32)[:1]
    camera_keys = status[3:3 + cameras]
    camera_status = status[3 + cameras:].view(torch.int32)[:cameras]
    full, inverse, centers, _ = launch_prepare(viewmats, Ks, width, height, with_centers, errors=camera_status,
                                               keys=camera_keys)
    state = project_views(
        means, quats, scales, opacities, viewmats, full, Ks, width, height, near, far, radius_clip,
        sh=sh if sh_degree is not None else None, sh_degree=sh_degree or 0,
        camera_centers=centers if with_centers else None, metadata=True, normalize_quats=True,
    )
    profiling.mark("projected")
    # The depth ordering computes every row's footprint in the chosen mode
    # once; it also leaves the mode's tile counts in state.tile_counts (the
    # projection counted radius squares).  It sorts the depth-key bits that
    # the last frame of this shape needed; the frame's own need comes back
    # with the totals.
    shape = (status.device.index, state.radii.shape[-1], cameras, width, height, tile_mode)
    sort_bits = binning.planned_sort_bits(shape)
    order, offsets, _ = order_rows(state.centers, state.radii, state.depths, width, height,
                                   conics=state.conics, tile_mode=tile_mode,
                                   tiles_out=None if tile_mode == "radius" else state.tile_counts,
                                   totals=status[:2], sort_bits=sort_bits, key_bits_out=key_bits)
    # Everything the binning launch needs besides the totals is prepared
    # while the device works on the depth order.
    launch = prepare_bin_rows(state.centers, state.radii, order, offsets, width, height, conics=state.conics,
                              tile_mode=tile_mode)
    # The totals are copied to pinned host memory right after the depth
    # order; with a group-item capacity from an earlier frame of this shape,
    # the device then emits the group items while the host waits for them.
    host = _pinned_status(status.numel())
    host.copy_(status, non_blocking=True)
    copied = torch.cuda.Event()
    if status.device.index == torch.cuda.current_device():
        copied.record()  # the current stream, as torch.cuda.current_stream() would give it
    else:
        copied.record(torch.cuda.current_stream(status.device))
    profiling.mark("ordered")
    early = binning.emit_early(launch)
    copied.synchronize()
    profiling.mark("totals_read")
    raise_camera_errors(host[3 + cameras:].view(torch.int32)[:cameras].tolist())
    group_pairs, count = host[:2].tolist()
    if binning.remember_key_bits(shape, int(host[2:3].view(torch.int32)[0]), sort_bits):
        # The depth keys now differ in more bits than were sorted: order
        # again with enough (the totals do not depend on the order).
        early = None
        order, offsets, _ = order_rows(state.centers, state.radii, state.depths, width, height,
                                       conics=state.conics, tile_mode=tile_mode,
                                       sort_bits=binning.planned_sort_bits(shape))
        launch = prepare_bin_rows(state.centers, state.radii, order, offsets, width, height,
                                  conics=state.conics, tile_mode=tile_mode)
    lists = None
    if count <= binning.PAIR_LIMIT and group_pairs <= binning.PAIR_LIMIT:
        if capped:
            lists = tile_lists.plan(status.device, width, height, tile_mode, host[3:3 + cameras].tolist(), count,
                                    launch.ranges.shape[0] // max(cameras, 1), slot=slot)
        caps = lists.caps if lists is not None else None
        ranges, ids = launch_bin_rows(launch, group_pairs, count, early, caps=caps,
                                      redo_list=lists.redo_list if caps is not None else None)
        if caps is not None:
            lists.launch = launch
        bins = [ViewBins(0, cameras, ranges, ids)]
    else:
        del early  # the per-group binning below allocates its own scratch
        bins = _bin_view_groups(state, width, height, tile_mode)
    profiling.mark("binned")
    return Frame(
        width, height, Ks.detach(), full, inverse if with_centers else None, centers if with_centers else None,
        state, bins, count, sh_degree, background, lists,
    )


def _bin_view_groups(state, width: int, height: int, tile_mode: str) -> list[ViewBins]:
    """Binning per group of cameras when all cameras together exceed the
    int32 pair offsets of one binning launch (the reference bins each view
    alone, so its limit is per view)."""
    per_view = state.tile_counts.sum(dim=1, dtype=torch.int64).tolist()
    bins = []
    for v0, v1 in binning.view_groups(per_view):
        sl = slice(v0, v1)
        order, offsets, totals = order_rows(state.centers[sl], state.radii[sl], state.depths[sl], width, height,
                                            conics=state.conics[sl], tile_mode=tile_mode)
        launch = prepare_bin_rows(state.centers[sl], state.radii[sl], order, offsets, width, height,
                                  conics=state.conics[sl], tile_mode=tile_mode)
        group_pairs, count = totals.cpu().tolist()
        ranges, ids = launch_bin_rows(launch, group_pairs, count)
        bins.append(ViewBins(v0, v1, ranges, ids))
    return bins


def rasterize(
    means: Tensor,
    quats: Tensor,
    scales: Tensor,
    opacities: Tensor,
    viewmats: Tensor,
    Ks: Tensor,
    width: int,
    height: int,
    *,
    features: Tensor | None = None,
    sh_coeffs: Tensor | None = None,
    sh_degree: int | None = None,
    backgrounds: Tensor | None = None,
    extra_features: Tensor | None = None,
    near_plane: float = 0.2,
    far_plane: float = math.inf,
    radius_clip: float = 0.0,
    packed: bool = False,
    absgrad: bool = False,
    statistics: Sequence[StatisticsRequest] = (),
    tile_mode: str = "radius",
) -> RasterizationResult:
    """Original 3DGS, forward (and backward through autograd), every camera of
    every batch item.

    Inputs: activated scales and opacities, wxyz quaternions (normalised
    here), either ``features`` (blended as given) or ``sh_coeffs`` (SH colour,
    degree defaulting to min(3, isqrt(K) - 1)); features and SH may be shared
    by the cameras or given per camera.  Pixel (x, y) has its centre at
    (x + 0.5, y + 0.5) in K's coordinates; meta["means2d"] is the projected
    centre in integer-pixel coordinates (K projection - 0.5), zero for culled
    rows.  Gaussians need a centre depth inside (near_plane, far_plane);
    covariances are dilated by 0.3 px.  Gradients reach means, quats, scales,
    opacities, features/SH, extra features, viewmats and means2d; K and
    background gradients are not supported.
    """
    validate_tile_mode(tile_mode)
    validate_camera_options(width, height, near_plane, far_plane, radius_clip)
    sh_degree = _sh_degree(features, sh_coeffs, sh_degree)
    # Quaternions stay raw: the projection kernels normalise them (and take
    # their gradient through the normalisation) as F.normalize does.
    layout = normalize_inputs(
        means, quats, scales, opacities, features if sh_coeffs is None else sh_coeffs, viewmats, Ks,
        backgrounds, extra_features, None, sh_degree, normalize_quats=False,
    )
    frames: list[Frame] = []
    dense: dict[str, list[Tensor]] = {n: [] for n in ("radii", "means2d", "opacities", "tiles_per_gauss", "conics")}
    for b in range(layout.batch_count):
        colors = layout.colors.values[b]
        frame = _prepare_frame(
            layout.means[b], layout.quats[b], layout.scales[b], layout.opacities[b],
            batch_item(layout.viewmats, b), batch_item(layout.Ks, b), width, height, near_plane, far_plane,
            radius_clip, colors if sh_degree is not None else None, sh_degree,
            None if layout.backgrounds is None else batch_item(layout.backgrounds, b), tile_mode,
            capped=not statistics,  # a redone tile would total its statistics twice
            slot=b,
        )
        frames.append(frame)
        st = frame.state
        dense["radii"].append(st.radii[..., None].expand(-1, -1, 2))
        dense["means2d"].append(st.means2d)
        dense["opacities"].append(st.opacities)
        dense["tiles_per_gauss"].append(st.tile_counts)
        dense["conics"].append(st.meta_conics)
    geometry = {
        name: (rows[0] if len(rows) == 1 else torch.stack(rows)).reshape(
            (layout.batch_count, layout.cameras, layout.n) + tuple(rows[0].shape[2:])
        )
        for name, rows in dense.items()
    }
    training = prepare_training_metadata(geometry, layout, packed=packed, absgrad=absgrad)
    meta = training.values
    meta.update(
        width=width,
        height=height,
        tile_size=16,
        tile_width=(width + 15) // 16,
        tile_height=(height + 15) // 16,
        n_cameras=layout.cameras,
        packed=packed,
        backend=BACKEND,
        with_eval3d=False,
        supports_means2d_grad=True,
        screen_gradient_mode="projected_mean",
        tile_mode=tile_mode,
    )
    prepared_stats, statistics_outputs = (
        prepare_statistics(
            statistics, batch_dims=layout.batch_dims, batch_count=layout.batch_count, cameras=layout.cameras,
            n=layout.n, width=width, height=height, device=layout.device,
        )
        if statistics else ([], {})
    )
    planes = []
    grad_enabled = torch.is_grad_enabled()
    for b, frame in enumerate(frames):
        screen = None if training.screen is None else batch_item(training.screen, b)
        targets = training.absolute_targets[b * layout.cameras:(b + 1) * layout.cameras]
        extras = None if layout.extras is None else layout.extras.values[b]
        planes.append(Rasterize.apply(
            layout.means[b], layout.quats[b], layout.scales[b], layout.opacities[b], layout.colors.values[b],
            extras, batch_item(layout.viewmats, b), screen, frame, targets,
            prepared_stats[b] if statistics else None, grad_enabled,
        ))
    shape = layout.batch_dims + (layout.cameras, height, width)

    def gather(k):
        items = [p[k] for p in planes]
        out = items[0] if len(items) == 1 else torch.stack(items)
        return out.reshape(shape + (items[0].shape[-1],))

    features, alpha = gather(0), gather(2)
    if layout.extras is not None:
        meta["render_extra_signals"] = gather(1)
    return RasterizationResult(features, alpha, meta, statistics_outputs)
