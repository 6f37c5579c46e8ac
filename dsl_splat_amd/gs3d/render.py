"""Tile blending forward/backward launches (gs3d/render.py:36-463 of the
reference) over gs3d_render_fwd / gs3d_render_bwd, for all views at once.

The blended vector of a Gaussian is [features | extra | 1] (the constant
alpha channel of gs3d/autograd.py:41-46) assembled inside the kernel from
its sources, so no concatenated copy is made.  The image comes out as the
planes the reference returns after its split (gs3d/api.py:256-265):
features (C,H,W,D), extra (C,H,W,E) and alpha (C,H,W,1), each contiguous, and
the backward reads the upstream gradient of each plane where it lies (any
pixel stride), so autograd never reassembles a full-image gradient.
Backward gradients of centres/conics/abs-centres share one
(C, N, 6) record per Gaussian (centre xy, conic a b c, opacity; |centre| xy
in two more columns with absgrad), so a wavefront's atomics for one Gaussian
land in one 24-byte (32-byte) row.
"""

from dataclasses import dataclass
import ctypes

import torch
from torch import Tensor

from ..runtime import abi, native

# Floats per Gaussian in the gradient record: [dcx, dcy, da, db, dc, dopacity]
# and, with absgrad, [|dcx|, |dcy|].
RECORD = 6
RECORD_ABS = 8


@dataclass(slots=True)
class RenderedPixels:
    features: Tensor       # (C, H, W, D) channel-last
    extra: Tensor | None   # (C, H, W, E) or None
    alpha: Tensor | None   # (C, H, W, 1) when the constant alpha channel is blended
    transmittance: Tensor  # (C, H, W)
    contributors: Tensor   # (C, H, W) int32

    def stacked(self) -> Tensor:
        """All blended channels as one (C, H, W, D') tensor, [features | extra | alpha]."""
        return torch.cat([p for p in (self.features, self.extra, self.alpha) if p is not None], dim=-1)


def _plane(grad: Tensor | None, views: int, height: int, width: int, channels: int):
    """(tensor, pixel stride) of an upstream gradient plane with contiguous
    channels and a uniform pixel stride (copied only when it has neither)."""
    if grad is None or channels == 0:
        return None, 0
    t = grad.reshape(views, height, width, channels)
    s = t.stride(2)
    if (channels > 1 and t.stride(3) != 1) or s < channels or t.stride(1) != width * s or \
            t.stride(0) != height * width * s:
        t = t.contiguous()
        s = channels
    return t, s


def _source(values: Tensor | None, views: int, n: int):
    """(tensor, row stride, view stride) of a (N,k) shared or (C,N,k) per-view source."""
    if values is None:
        return None, 0, 0, 0
    if values.stride(-1) != 1:
        values = values.contiguous()
    if values.ndim == 2:
        if values.stride(0) < values.shape[1] and values.shape[0] > 1:
            values = values.contiguous()
        return values, values.shape[-1], values.stride(0), 0
    if values.ndim == 3 and values.shape[0] == views:
        if values.stride(0) != values.stride(1) * n:
            values = values.contiguous()
        return values, values.shape[-1], values.stride(1), values.stride(0)
    raise ValueError("features must be (N,D) or (C,N,D)")


def _args(width, height, views, n, ranges, ids, centers, conics, features, extra, background, one_tail, keep):
    a = abi.RenderArgs()
    a.width, a.height, a.views, a.n = width, height, views, n
    ranges, ids, centers, conics = ranges.contiguous(), ids.contiguous(), centers.contiguous(), conics.contiguous()
    keep += [ranges, ids, centers, conics]
    a.ranges, a.ids, a.centers, a.conics = (native.ptr(ranges), native.ptr(ids), native.ptr(centers),
                                            native.ptr(conics))
    f, fc, fs, fv = _source(features, views, n)
    keep.append(f)
    a.features, a.feat_channels, a.feat_stride, a.feat_view_stride = native.ptr(f), fc, fs, fv
    e, ec, es, ev = _source(extra, views, n)
    keep.append(e)
    a.extra, a.extra_channels, a.extra_stride, a.extra_view_stride = native.ptr(e), ec, es, ev
    a.one_tail = int(one_tail)
    if background is not None:
        background = background.reshape(views, -1).contiguous()
        keep.append(background)
        a.background, a.background_view_stride = native.ptr(background), background.shape[-1]
    return a, fc + ec + int(one_tail)


def _stats_args(statistics, views: int, n: int, width: int, height: int, keep: list) -> abi.RenderStatsArgs:
    """gs3d_render_stats_args over one frame's PreparedStatistics."""
    key = tuple(statistics.key)
    pv, counts, sums = statistics.pixel_values, statistics.counts, statistics.sums
    if pv.shape != (views, len(key), height * width) or counts.shape[::2] != (views, n) or \
            sums.shape[::2] != (views, n):
        raise ValueError("prepared statistics do not match the rendered views")
    for t in (pv, counts, sums):
        if not t.is_contiguous():
            raise ValueError("prepared statistics must be contiguous")
    keep += [pv, counts, sums]
    st = abi.RenderStatsArgs()
    st.requests = len(key)
    st.sum_mask = sum(1 << r for r, kind in enumerate(key) if kind == 1)
    st.pixel_values, st.pixel_view_stride = native.ptr(pv), pv.stride(0)
    st.counts = native.ptr(counts) if counts.shape[1] else None
    st.counts_view_stride = counts.stride(0)
    st.sums = native.ptr(sums) if sums.shape[1] else None
    st.sums_view_stride = sums.stride(0)
    return st


@native.no_grad
def render_views(ranges: Tensor, ids: Tensor, centers: Tensor, conics: Tensor, features: Tensor,
                 width: int, height: int, *, extra: Tensor | None = None, background: Tensor | None = None,
                 one_tail: bool = True, statistics=None, zero: Tensor | None = None, lists=None) -> RenderedPixels:
    """Blend all views; with a PreparedStatistics, its counts and sums
    accumulate the contribution statistics of the same launch.  ``zero`` (a
    contiguous float32 tensor, 16-byte aligned), if given, is cleared by the
    launch while it blends.  ``lists`` (a CappedLists of the frame whose
    ``ids`` were written up to ``lists.caps``) receives each tile's stop; with
    caps, the tiles the blend flags get their whole lists (lists.rewrite())
    and a second launch blends them again into the same outputs."""
    views, n = centers.shape[0], centers.shape[1]
    device = centers.device
    keep = []
    a, channels = _args(width, height, views, n, ranges, ids, centers, conics, features, extra, background,
                        one_tail, keep)
    f32 = dict(dtype=torch.float32, device=device)
    out = RenderedPixels(
        torch.empty((views, height, width, a.feat_channels), **f32),
        torch.empty((views, height, width, a.extra_channels), **f32) if a.extra_channels else None,
        torch.empty((views, height, width, 1), **f32) if one_tail else None,
        torch.empty((views, height, width), **f32),
        torch.empty((views, height, width), dtype=torch.int32, device=device),
    )
    a.image, a.final_t, a.contributors = (native.ptr(out.features), native.ptr(out.transmittance),
                                          native.ptr(out.contributors))
    a.image_extra, a.image_alpha = native.ptr(out.extra), native.ptr(out.alpha)
    if zero is not None:
        if zero.dtype != torch.float32 or not zero.is_contiguous() or zero.device != device:
            raise ValueError("zero must be a contiguous float32 tensor on the rendering device")
        a.zero_out, a.zero_count = native.ptr(zero), zero.numel()
    capped = lists is not None and lists.caps is not None
    if lists is not None:
        tiles = ranges.shape[0]
        if lists.stops.numel() != tiles or (capped and (lists.caps.numel() != tiles or lists.redo.numel() != tiles
                                                        or lists.redo_list.numel() != tiles + 1)):
            raise ValueError("the capped lists do not match the frame's tiles")
        a.stop_out = native.ptr(lists.stops)
        if capped:
            a.caps, a.redo, a.redo_list = native.ptr(lists.caps), native.ptr(lists.redo), native.ptr(lists.redo_list)
    if statistics is not None and len(statistics.key):
        if capped:
            raise ValueError("statistics need whole tile lists")
        st = _stats_args(statistics, views, n, width, height, keep)
        native.call("gs3d_render_fwd_stats", ctypes.byref(a), ctypes.byref(st), native.stream(device))
    else:
        native.call("gs3d_render_fwd", ctypes.byref(a), native.stream(device))
    if capped:
        lists.rewrite()
        a.caps, a.redo, a.redo_pass = None, None, 1
        a.zero_out, a.zero_count = None, 0
        native.call("gs3d_render_fwd", ctypes.byref(a), native.stream(device))
    return out


@native.no_grad
def backward_views(ranges: Tensor, ids: Tensor, centers: Tensor, conics: Tensor, features: Tensor,
                   final_t: Tensor, contributors: Tensor, upstream, width: int, height: int, *,
                   extra: Tensor | None = None, background: Tensor | None = None, one_tail: bool = True,
                   absgrad: bool = False, need_features: bool = True, need_extra: bool = True, cleared=None):
    """``upstream`` is either the (grad features, grad extra, grad alpha)
    planes (each may be None) or one (C,H,W,D') tensor of all channels.
    Returns (record (C,N,6), or (C,N,8) with absgrad, grad_features like
    features or None, grad_extra like extra or None).  ``cleared``, if
    given, holds zeroed buffers of those shapes (record, features, extra)
    that the launch accumulates into instead of fresh ones."""
    views, n = centers.shape[0], centers.shape[1]
    device = centers.device
    keep = []
    a, channels = _args(width, height, views, n, ranges, ids, centers, conics, features, extra, background,
                        one_tail, keep)
    final_t, contributors = final_t.contiguous(), contributors.contiguous()
    fc, ec = a.feat_channels, a.extra_channels
    if isinstance(upstream, Tensor):
        full = upstream.reshape(views, height, width, channels)
        upstream = (full[..., :fc], full[..., fc:fc + ec] if ec else None, full[..., -1:] if one_tail else None)
    gf_plane, gf_stride = _plane(upstream[0], views, height, width, fc)
    ge_plane, ge_stride = _plane(upstream[1], views, height, width, ec)
    ga_plane, ga_stride = _plane(upstream[2] if one_tail else None, views, height, width, 1)
    keep += [final_t, contributors, gf_plane, ge_plane, ga_plane]
    a.final_t, a.contributors = native.ptr(final_t), native.ptr(contributors)
    b = abi.RenderBwdArgs()
    b.fwd = a
    b.upstream, b.upstream_stride = native.ptr(gf_plane), gf_stride
    b.upstream_extra, b.upstream_extra_stride = native.ptr(ge_plane), ge_stride
    b.upstream_alpha, b.upstream_alpha_stride = native.ptr(ga_plane), ga_stride
    width = RECORD_ABS if absgrad else RECORD

    def zeros(shape, given):
        if given is not None:
            if tuple(given.shape) != tuple(shape) or given.dtype != torch.float32 or not given.is_contiguous():
                raise ValueError(f"cleared buffer of shape {tuple(given.shape)} does not match {tuple(shape)}")
            return given
        return torch.zeros(shape, dtype=torch.float32, device=device)

    record = zeros((views, n, width), cleared and cleared.record)
    b.grad_centers, b.grad_centers_stride = native.ptr(record), width
    b.grad_conics, b.grad_conics_stride = native.ptr(record, 2), width
    if absgrad:
        b.abs_centers, b.abs_stride = native.ptr(record, 6), width
    grad_features = grad_extra = None
    if need_features and features is not None:
        grad_features = zeros(features.shape, cleared and cleared.features)
        b.grad_features = native.ptr(grad_features)
        b.grad_feat_stride = features.shape[-1]
        b.grad_feat_view_stride = n * features.shape[-1] if features.ndim == 3 else 0
    if need_extra and extra is not None:
        grad_extra = zeros(extra.shape, cleared and cleared.extra)
        b.grad_extra = native.ptr(grad_extra)
        b.grad_extra_stride = extra.shape[-1]
        b.grad_extra_view_stride = n * extra.shape[-1] if extra.ndim == 3 else 0
    native.call("gs3d_render_bwd", ctypes.byref(b), native.stream(device))
    return record, grad_features, grad_extra


@native.no_grad
def pair_counts(ranges: Tensor, ids: Tensor, centers: Tensor, conics: Tensor, features: Tensor, width: int,
                height: int, *, extra: Tensor | None = None, background: Tensor | None = None,
                one_tail: bool = True) -> dict[str, int]:
    """(pixel, Gaussian) pairs of one blend of all views: visited as the
    reference's loop visits them, evaluated by the forward kernel after its
    strip culling, and accepted (blended).  A measurement aid: runs the
    forward blend once more (its image is discarded)."""
    views, n = centers.shape[0], centers.shape[1]
    keep = []
    a, _ = _args(width, height, views, n, ranges, ids, centers, conics, features, extra, background, one_tail, keep)
    f32 = dict(dtype=torch.float32, device=centers.device)
    planes = [torch.empty((views, height, width, a.feat_channels), **f32),
              torch.empty((views, height, width, max(a.extra_channels, 1)), **f32),
              torch.empty((views, height, width), **f32), torch.empty((views, height, width), **f32),
              torch.empty((views, height, width), dtype=torch.int32, device=centers.device)]
    a.image = native.ptr(planes[0])
    a.image_extra = native.ptr(planes[1]) if a.extra_channels else None
    a.image_alpha = native.ptr(planes[2]) if one_tail else None
    a.final_t, a.contributors = native.ptr(planes[3]), native.ptr(planes[4])
    counts = torch.zeros(3, dtype=torch.int64, device=centers.device)
    native.call("gs3d_render_pair_counts", ctypes.byref(a), native.ptr(counts), native.stream(centers.device))
    visited, evaluated, accepted = counts.tolist()
    return dict(visited=visited, evaluated=evaluated, accepted=accepted)
