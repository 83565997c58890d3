"""Render entry of the splat viewer (reference:
src/gaussian_splats/visualize/gaussian/backend.py:19-90 and
visualize/__init__.py:7-21).

``render_gaussians`` is what the viewer's page calls per frame: the image is
rendered at the tile-rounded size with the principal point at the centre of
the requested size and cropped back, ``num_splats`` Gaussians spread evenly
over the scene are drawn through ``indices``, the rasterizer options come
from the page's settings, and the stage timings are collected when
``GAUSSIAN_SPLATS_PROFILE`` is set.  ``GaussianViewer`` holds a loaded scene
and the optional ``torch.compile``-d rasterizer (``compile_render`` = "1").
The web server, pages and camera controller are not part of this package.
"""

from __future__ import annotations

import math
import os
from contextlib import nullcontext
from dataclasses import dataclass, field, replace
from pathlib import Path

import torch

from .splats.camera import PinholeCamera
from .splats.rasterize import rasterize
from .splats.splats import GaussianSplat
from .timing import record_timings


@dataclass
class Frame:
    image: torch.Tensor
    timings: dict[str, float] = field(default_factory=dict)
    metadata: dict[str, str] = field(default_factory=dict)


def default_device() -> str:
    """``VISUALIZE_DEVICE``, else the ROCm GPU when present, else the CPU."""
    return os.getenv("VISUALIZE_DEVICE") or ("cuda" if torch.cuda.is_available() else "cpu")


def render_gaussians(splats, camera, settings, width, height, rasterizer=rasterize) -> Frame:
    """One viewer frame of ``width`` x ``height`` pixels (backend.py:19-57).
    The backend defaults to "hip", this build's rasterizer."""
    if splats.num_points == 0:
        return Frame(splats.mean.new_zeros((height, width, 3)), metadata={"X-Total-Splats": "0"})
    tile = int(settings.get("tile_size", 8))
    image_size = ((width + tile - 1) // tile * tile, (height + tile - 1) // tile * tile)
    camera = replace(camera, image_size=image_size, principal_point=(width / 2, height / 2))
    count = min(max(1, int(settings.get("num_splats") or 10_000)), splats.num_points)
    options = {
        "backend": settings.get("backend", "hip"),
        "tile_size": tile,
        "opacity_threshold": float(settings.get("opacity_threshold", 0.999)),
        "near": float(settings.get("near", 0.1)),
        "far": float(settings.get("far", 100)),
        "rendering_mode": settings.get("rendering_mode", "gaussian"),
        "confidence": float(settings.get("confidence", 0.95)),
        # Spread the drawn subset over the whole scene, not its first rows.
        "indices": torch.linspace(0, splats.num_points - 1, count, device=splats.mean.device)
        .round()
        .long(),
    }
    timing = (
        record_timings(splats.mean.device)
        if os.getenv("GAUSSIAN_SPLATS_PROFILE", "0") != "0"
        else nullcontext({})
    )
    with torch.no_grad(), timing as groups:
        image = rasterizer(splats, camera, **options)
    timings = {
        f"{group}/{name}": value for group, entries in groups.items() for name, value in entries.items()
    }
    return Frame(image[:height, :width], timings, {"X-Total-Splats": str(splats.num_points)})


@dataclass
class GaussianViewer:
    """A loaded scene and its camera (backend.py:60-90)."""

    splats: GaussianSplat | None = None
    camera: PinholeCamera | None = None
    checkpoint_name: str = ""
    compiled_rasterizer: object | None = None

    def load_checkpoint(self, path: str | Path, filename: str | None = None) -> None:
        """Loads a ``.pt`` checkpoint (or a ``.ply`` scene) and fits a camera
        pitched down by 45 degrees to its points (backend.py:68-75)."""
        device = self.splats.mean.device if self.splats is not None else default_device()
        path = Path(path)
        if path.suffix.lower() == ".ply":
            from .splats.ply import load_ply

            splats = GaussianSplat.from_tensors(**load_ply(path, device=device))
        else:
            splats = GaussianSplat.from_checkpoint(path).to(device)
        splats = splats.eval()
        rotation = splats.mean.new_tensor([math.cos(math.pi / 8), -math.sin(math.pi / 8), 0.0, 0.0])
        self.camera = PinholeCamera(rotation=rotation).fit_to_points(splats.mean)
        self.splats = splats
        self.checkpoint_name = filename or path.name

    def render(self, settings, width, height) -> Frame | None:
        if self.splats is None:
            return None
        if settings.get("compile_render") == "1" and self.compiled_rasterizer is None:
            self.compiled_rasterizer = torch.compile(rasterize, dynamic=True)
        rasterizer = self.compiled_rasterizer or rasterize
        frame = render_gaussians(self.splats, self.camera, settings, width, height, rasterizer)
        frame.metadata["X-Checkpoint-Name"] = self.checkpoint_name
        return frame
