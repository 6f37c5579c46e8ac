"""First-order autograd bridge for float32 SH0-3 on the HIP kernels
(primitives/spherical_harmonics.py:18-159 of the reference)."""

from numbers import Integral
from typing import Any

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from ..runtime import native


class _SphericalHarmonics(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, coefficients: Tensor, directions: Tensor, radii: Tensor | None, degree: int,
                grad_enabled: bool) -> Tensor:
        n = len(coefficients)
        needs = (ctx.needs_input_grad[0], degree > 0 and ctx.needs_input_grad[1])
        save = grad_enabled and any(needs)
        coefficients = coefficients.contiguous()
        directions = directions.contiguous()
        colors = coefficients.new_empty((n, 3))
        active = torch.empty((n if save else 0, 3), dtype=torch.uint8, device=coefficients.device)
        if n:
            native.call("gs3d_sh_fwd", native.ptr(coefficients), coefficients.shape[1], native.ptr(directions),
                        native.ptr(radii), n, degree, native.ptr(colors), native.ptr(active) if save else None,
                        native.stream(coefficients.device))
        if save:
            ctx.save_for_backward(coefficients, directions, radii, active)
            ctx.degree, ctx.needs = degree, needs
        ctx.set_materialize_grads(False)
        return colors

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, gradient: Tensor | None) -> tuple[Tensor | None, ...]:
        if gradient is None:
            return (None,) * 5
        coefficients, directions, radii, active = ctx.saved_tensors
        n = len(coefficients)
        need_coefficients, need_directions = ctx.needs
        gradient = gradient.contiguous()
        grad_coefficients = torch.empty_like(coefficients) if need_coefficients else None
        grad_directions = torch.empty((n, 3), dtype=torch.float32, device=coefficients.device) if need_directions else None
        if n:
            native.call("gs3d_sh_bwd", native.ptr(coefficients), coefficients.shape[1], native.ptr(directions),
                        native.ptr(radii), native.ptr(active), native.ptr(gradient), n, ctx.degree,
                        native.ptr(grad_coefficients), native.ptr(grad_directions),
                        native.stream(coefficients.device))
        return grad_coefficients, grad_directions, None, None, None


def _check(coefficients, directions, radii, degree) -> None:
    """ValueError for anything the SH kernels cannot take (messages of
    primitives/spherical_harmonics.py:104-159 of the reference)."""
    if isinstance(degree, bool) or not isinstance(degree, Integral) or not 0 <= degree <= 3:
        raise ValueError("SH degree must be an integer in [0,3]")
    c = coefficients
    if not (isinstance(c, Tensor) and c.is_cuda and c.dtype == torch.float32 and c.ndim == 3 and c.shape[2] == 3
            and c.shape[1] >= (degree + 1) ** 2):
        raise ValueError("SH coefficients must be CUDA float32 (N,K,3) with enough coefficients")
    d = directions
    if not (isinstance(d, Tensor) and d.dtype == torch.float32 and d.device == c.device
            and tuple(d.shape) == (c.shape[0], 3)):
        raise ValueError("SH directions must be float32 (N,3) on the coefficients' device")
    if radii is not None and not (radii.dtype == torch.int32 and radii.device == c.device
                                  and tuple(radii.shape) == (c.shape[0],)):
        raise ValueError("SH radii must be int32 (N,) on the coefficients' device")


def spherical_harmonics(coefficients: Tensor, directions: Tensor, degree: int, *, radii: Tensor | None = None,
                        bindings=None) -> Tensor:
    """max(sum_k Y_k(unit direction) c_k + 0.5, 0) per Gaussian, zero where
    radii <= 0; coefficients (N,K,3) and directions (N,3) are device float32.
    Differentiable in both (degree 0 ignores the directions)."""
    _check(coefficients, directions, radii, degree)
    if degree == 0:
        directions = directions.detach()
    return _SphericalHarmonics.apply(coefficients, directions, radii, int(degree), torch.is_grad_enabled())
