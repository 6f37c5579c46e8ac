"""Destination of one camera's absolute screen gradients (the role of
runtime/gradients.py:8-16 of the reference): a (N, 2) slice of
``means2d.absgrad`` for dense metadata, or the packed rows of that camera
together with the Gaussian index of each row."""

from dataclasses import dataclass

import torch
from torch import Tensor


@dataclass(slots=True)
class AbsGradientTarget:
    target: Tensor
    gaussian_ids: Tensor | None = None

    @torch.no_grad()
    def write(self, gradient: Tensor) -> None:
        """Store the camera's (N, 2) absolute centre gradients."""
        if self.gaussian_ids is not None:
            gradient = gradient.index_select(0, self.gaussian_ids)
        self.target.copy_(gradient)
