"""Backend dispatcher (reference: src/gaussian_splats/splats/rasterize.py:12-43).

The only backend of this build is ``"hip"``: the hand-written gfx950 kernels
behind ``torch.ops.gaussian_splats.rasterize``.  The reference's other
backends ("torch", "triton", "gsplat") are not part of it and raise.
"""

from __future__ import annotations

from typing import Literal

import torch

from ..kernels.rasterize.interface import rasterize as hip_rasterize
from ..kernels.rasterize.views import rasterize_views
from .camera import Camera
from .splats import GaussianSplat


def rasterize(
    splats: GaussianSplat,
    camera: Camera,
    tile_size: int = 4,
    opacity_threshold: float = 0.999,
    near: float = 0.2,
    far: float = 100.0,
    rendering_mode: Literal["gaussian", "ellipsoid"] = "gaussian",
    confidence: float = 0.95,
    indices: torch.Tensor | None = None,
    backend: Literal["hip"] = "hip",
) -> torch.Tensor:
    match backend:
        case "hip":
            render = hip_rasterize
        case _:
            raise ValueError(f"Unknown rasterization backend: {backend} (available: 'hip')")
    return render(
        splats,
        camera,
        tile_size,
        opacity_threshold,
        near,
        far,
        rendering_mode,
        confidence,
        indices,
    )


__all__ = ["rasterize", "rasterize_views"]
