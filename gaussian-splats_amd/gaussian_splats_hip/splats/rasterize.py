"""Backend dispatcher (reference: src/gaussian_splats/splats/rasterize.py:12-43).

The backend of this build is ``"hip"``: the hand-written gfx950 kernels behind
``torch.ops.gaussian_splats_hip.rasterize``.  The reference's two GPU backend
names, ``"triton"`` and ``"gsplat"``, select the same kernels, so a caller that
passes the reference's module constant (``training/train.py:27,49``:
``BACKEND = "gsplat"`` on a GPU) runs unchanged.  ``"torch"`` names the
reference's CPU path, which this build does not ship: it raises, as an unknown
name does (``rasterize.py:31-32``).
"""

from __future__ import annotations

from typing import Literal

import torch

from ..kernels.rasterize.interface import rasterize as hip_rasterize
from ..kernels.rasterize.views import rasterize_views
from .camera import Camera
from .splats import GaussianSplat

#: Backend names that select the HIP kernels.
GPU_BACKENDS = ("hip", "triton", "gsplat")


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
    backend: Literal["hip", "triton", "gsplat"] = "hip",
) -> torch.Tensor:
    match backend:
        case "hip" | "triton" | "gsplat":
            render = hip_rasterize
        case "torch":
            raise ValueError(
                "Rasterization backend 'torch' is the reference's CPU path, which this "
                "build does not ship; use 'hip' on a ROCm device"
            )
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


__all__ = ["rasterize", "rasterize_views", "GPU_BACKENDS"]
