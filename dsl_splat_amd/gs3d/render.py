"""Tile blending forward/backward launches (gs3d/render.py:36-463 of the
reference) over gs3d_render_fwd / gs3d_render_bwd, for all views at once.

The blended vector of a Gaussian is [features | extra | 1] (the constant
alpha channel of gs3d/autograd.py:41-46) assembled inside the kernel from
its sources, so no concatenated copy is made; images come out channel-last
(C, H, W, D').  Backward gradients of centres/conics/abs-centres share one
(C, N, 8) record per Gaussian (centre xy, conic a b c, opacity, |centre| xy)
so a wavefront's atomics for one Gaussian land in one 32-byte row.
"""

from dataclasses import dataclass
import ctypes

import torch
from torch import Tensor

from ..runtime import abi, native

RECORD = 8  # floats per Gaussian in the gradient record


@dataclass(slots=True)
class RenderedPixels:
    features: Tensor       # (C, H, W, D') channel-last
    transmittance: Tensor  # (C, H, W)
    contributors: Tensor   # (C, H, W) int32


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


@torch.no_grad()
def render_views(ranges: Tensor, ids: Tensor, centers: Tensor, conics: Tensor, features: Tensor,
                 width: int, height: int, *, extra: Tensor | None = None, background: Tensor | None = None,
                 one_tail: bool = True) -> RenderedPixels:
    views, n = centers.shape[0], centers.shape[1]
    device = centers.device
    keep = []
    a, channels = _args(width, height, views, n, ranges, ids, centers, conics, features, extra, background,
                        one_tail, keep)
    out = RenderedPixels(
        torch.empty((views, height, width, channels), dtype=torch.float32, device=device),
        torch.empty((views, height, width), dtype=torch.float32, device=device),
        torch.empty((views, height, width), dtype=torch.int32, device=device),
    )
    a.image, a.final_t, a.contributors = (native.ptr(out.features), native.ptr(out.transmittance),
                                          native.ptr(out.contributors))
    native.call("gs3d_render_fwd", ctypes.byref(a), native.stream(device))
    return out


@torch.no_grad()
def backward_views(ranges: Tensor, ids: Tensor, centers: Tensor, conics: Tensor, features: Tensor,
                   final_t: Tensor, contributors: Tensor, upstream: Tensor, width: int, height: int, *,
                   extra: Tensor | None = None, background: Tensor | None = None, one_tail: bool = True,
                   absgrad: bool = False, need_features: bool = True, need_extra: bool = True):
    """Returns (record (C,N,8), grad_features like features or None,
    grad_extra like extra or None)."""
    views, n = centers.shape[0], centers.shape[1]
    device = centers.device
    keep = []
    a, channels = _args(width, height, views, n, ranges, ids, centers, conics, features, extra, background,
                        one_tail, keep)
    final_t, contributors = final_t.contiguous(), contributors.contiguous()
    upstream = upstream.reshape(views, height, width, channels).contiguous()
    keep += [final_t, contributors, upstream]
    a.final_t, a.contributors = native.ptr(final_t), native.ptr(contributors)
    b = abi.RenderBwdArgs()
    b.fwd = a
    b.upstream = native.ptr(upstream)
    record = torch.zeros((views, n, RECORD), dtype=torch.float32, device=device)
    b.grad_centers, b.grad_centers_stride = native.ptr(record), RECORD
    b.grad_conics, b.grad_conics_stride = native.ptr(record, 2), RECORD
    if absgrad:
        b.abs_centers, b.abs_stride = native.ptr(record, 6), RECORD
    grad_features = grad_extra = None
    if need_features and features is not None:
        grad_features = torch.zeros(features.shape, dtype=torch.float32, device=device)
        b.grad_features = native.ptr(grad_features)
        b.grad_feat_stride = features.shape[-1]
        b.grad_feat_view_stride = n * features.shape[-1] if features.ndim == 3 else 0
    if need_extra and extra is not None:
        grad_extra = torch.zeros(extra.shape, dtype=torch.float32, device=device)
        b.grad_extra = native.ptr(grad_extra)
        b.grad_extra_stride = extra.shape[-1]
        b.grad_extra_view_stride = n * extra.shape[-1] if extra.ndim == 3 else 0
    native.call("gs3d_render_bwd", ctypes.byref(b), native.stream(device))
    return record, grad_features, grad_extra
