"""Gaussian parameter container (reference: src/gaussian_splats/splats/splats.py:13-84)."""

from __future__ import annotations

from dataclasses import dataclass
from functools import cached_property
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import nn
from typing_extensions import Self

from .utils import rgb_to_sh


@dataclass(frozen=True)
class ProjectedGaussianSplat:
    """Screen-space Gaussians (splats.py:13-23): means (u, v, depth), 2x2 covariances."""

    mean: torch.Tensor  # N x 3
    covariance: torch.Tensor  # N x 2 x 2
    color: torch.Tensor  # N x 3
    opacity: torch.Tensor  # N x 1
    normals: torch.Tensor | None = None

    @cached_property
    def inverse_covariance(self) -> torch.Tensor:  # N x 2 x 2
        return torch.linalg.inv(self.covariance)


class GaussianSplat(nn.Module):
    """Learnable Gaussians: ``mean`` N x 3, ``rotation`` N x 4 (w, x, y, z, not
    necessarily normalised), ``scale`` N x 3 (log sigma), ``opacity`` N x 1 (logit),
    ``color`` N x (degree + 1)^2 x 3 (SH coefficients, RGB innermost) and
    ``normals`` N x 3 (carried, not rendered).  Initialisation follows
    splats.py:34-44."""

    mean: torch.Tensor
    rotation: torch.Tensor
    scale: torch.Tensor
    opacity: torch.Tensor
    color: torch.Tensor
    normals: torch.Tensor

    def __init__(self, num_points: int, sh_degree: int = 3):
        super().__init__()
        self.sh_degree = sh_degree
        self.mean = nn.Parameter(torch.randn(num_points, 3))
        self.rotation = nn.Parameter(F.normalize(torch.randn(num_points, 4)))
        self.scale = nn.Parameter(torch.randn(num_points, 3))
        self.opacity = nn.Parameter(torch.randn(num_points, 1))
        color = torch.zeros(num_points, (sh_degree + 1) ** 2, 3)
        color[:, 0, :] = rgb_to_sh(torch.rand(num_points, 3))
        self.color = nn.Parameter(color)
        self.normals = nn.Parameter(torch.zeros_like(self.mean))

    def save_checkpoint(self, path: str | Path) -> None:
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        torch.save(self.state_dict(), path)

    @classmethod
    def from_checkpoint(cls, checkpoint: str | Path) -> Self:
        state = torch.load(checkpoint, map_location="cpu", weights_only=True)
        splats = cls(len(state["mean"]), int(state["color"].shape[1] ** 0.5) - 1)
        splats.load_state_dict(state)
        return splats

    @classmethod
    def from_tensors(
        cls,
        mean: torch.Tensor,
        rotation: torch.Tensor,
        scale: torch.Tensor,
        opacity: torch.Tensor,
        color: torch.Tensor,
        normals: torch.Tensor | None = None,
    ) -> Self:
        splats = cls(0, int(color.shape[1] ** 0.5) - 1)
        with torch.no_grad():
            splats.mean = nn.Parameter(mean)
            splats.rotation = nn.Parameter(rotation)
            splats.scale = nn.Parameter(scale)
            splats.opacity = nn.Parameter(opacity)
            splats.color = nn.Parameter(color)
            splats.normals = nn.Parameter(
                normals if normals is not None else torch.zeros_like(mean)
            )
        return splats

    @property
    def num_points(self) -> int:
        return len(self.mean)
