"""Seeded synthetic scenes: the benchmark configurations and test scenes.

Draw order is fixed (means -> log-scales -> quaternions -> opacity logits -> SH
band 0 -> higher SH bands -> loss target) from a CPU ``torch.Generator`` seeded
with ``seed``, so the GPU run and the CPU checker see identical tensors.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .splats.camera import PinholeCamera
from .splats.utils import rgb_to_sh


@dataclass
class Scene:
    name: str
    mean: torch.Tensor
    rotation: torch.Tensor
    scale: torch.Tensor
    opacity: torch.Tensor
    color: torch.Tensor
    cameras: list[PinholeCamera]
    near: float = 0.2
    far: float = 100.0
    tile_size: int = 16
    backward: bool = False
    target: torch.Tensor | None = None
    notes: dict = field(default_factory=dict)

    @property
    def num_points(self) -> int:
        return self.mean.shape[0]

    def params(self) -> tuple[torch.Tensor, ...]:
        return self.mean, self.rotation, self.scale, self.opacity, self.color

    def to(self, device) -> "Scene":
        moved = Scene(
            self.name, *(t.to(device) for t in self.params()), self.cameras, self.near, self.far,
            self.tile_size, self.backward,
            None if self.target is None else self.target.to(device), dict(self.notes),
        )
        return moved


def _quats(n: int, g: torch.Generator) -> torch.Tensor:
    q = torch.randn(n, 4, generator=g)
    return q / q.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def _sh3(n: int, g: torch.Generator, dc_std: float = 0.5, rest_std: float = 0.05) -> torch.Tensor:
    dc = torch.randn(n, 1, 3, generator=g) * dc_std
    rest = torch.randn(n, 15, 3, generator=g) * rest_std
    return torch.cat((dc, rest), 1)


def config1(seed: int = 0, n: int = 10_000) -> Scene:
    """CPU plumbing case: 10k Gaussians, SH0, 256x256, forward only.

    Means U[-1, 1]^3, camera at (0, 0, -3) looking at the origin, fx = fy = 256,
    near 0.01, log-scales N(-3, 0.5), normalised N(0, I4) quaternions, opacity
    logits N(0, 1), colours U(0, 1) stored as the DC coefficient (rgb_to_sh).
    """
    g = torch.Generator().manual_seed(seed)
    mean = torch.rand(n, 3, generator=g) * 2 - 1
    scale = torch.randn(n, 3, generator=g) * 0.5 - 3
    rotation = _quats(n, g)
    opacity = torch.randn(n, 1, generator=g)
    color = rgb_to_sh(torch.rand(n, 1, 3, generator=g))
    cam = PinholeCamera.look_at(
        (0.0, 0.0, -3.0), image_size=(256, 256), focal_length=(256.0, 256.0),
        principal_point=(128.0, 128.0),
    )
    return Scene("config1", mean, rotation, scale, opacity, color, [cam], near=0.01)


def _config2_body(n: int, g: torch.Generator):
    mean = torch.randn(n, 3, generator=g) * torch.tensor([2.0, 1.0, 2.0])
    scale = torch.randn(n, 3, generator=g) * 0.7 - 4
    rotation = _quats(n, g)
    opacity = torch.randn(n, 1, generator=g) * 1.5
    color = _sh3(n, g)
    return mean, rotation, scale, opacity, color


def _camera_1080p() -> PinholeCamera:
    return PinholeCamera.look_at(
        (0.0, 0.0, 6.0), (0.0, 0.0, 0.0), image_size=(1920, 1080), focal_length=(1500.0, 1500.0),
        principal_point=(960.0, 540.0),
    )


def config2(seed: int = 0, n: int = 200_000) -> Scene:
    """Forward only, SH3: 200k Gaussians, means N(0, diag(4, 1, 4)), 1920x1080,
    fx = fy = 1500, camera at distance 6, log-scales N(-4, 0.7), opacity logits
    N(0, 1.5), SH band 0 N(0, 0.5), higher bands N(0, 0.05), near 0.2."""
    g = torch.Generator().manual_seed(seed)
    body = _config2_body(n, g)
    return Scene("config2", *body, [_camera_1080p()])


def config3(seed: int = 0, n: int = 1_000_000) -> Scene:
    """Training step: config 2's distributions with 1M Gaussians, forward +
    backward of mean |image - target| with target U(0, 1) (no clamp)."""
    g = torch.Generator().manual_seed(seed)
    body = _config2_body(n, g)
    target = torch.rand(1080, 1920, 3, generator=g)
    return Scene("config3", *body, [_camera_1080p()], backward=True, target=target,
                 notes={"loss": "mean |image - target|, image not clamped"})


def config4(seed: int = 0, n: int = 4_000_000, distance: float = 3.0, focal: float = 1600.0) -> Scene:
    """Depth-complexity stress: 4M Gaussians in a 0.5-unit cube in front of a
    1600x1600 camera (distance 3, fx = fy = 1600 chosen here), log-scales
    N(-3.5, 0.5), opacity logits N(-1, 1), SH3 as config 2."""
    g = torch.Generator().manual_seed(seed)
    mean = torch.rand(n, 3, generator=g) * 0.5 - 0.25
    scale = torch.randn(n, 3, generator=g) * 0.5 - 3.5
    rotation = _quats(n, g)
    opacity = torch.randn(n, 1, generator=g) - 1
    color = _sh3(n, g)
    target = torch.rand(1600, 1600, 3, generator=g)
    cam = PinholeCamera.look_at(
        (0.0, 0.0, distance), image_size=(1600, 1600), focal_length=(focal, focal),
        principal_point=(800.0, 800.0),
    )
    return Scene("config4", mean, rotation, scale, opacity, color, [cam], backward=True,
                 target=target, notes={"distance": distance, "focal": focal})


def config5(
    seed: int = 0, n: int = 500_000, views: int = 16, size: int = 800, focal: float = 1000.0
) -> Scene:
    """Baked-mesh-style flat splats: 500k on the unit sphere, two log-scales
    N(-4, 0.3) and a third of -9.2, the thin axis turned to a random normal,
    opacity logits N(0, 1.5), SH3 as config 2; 16 cameras on a radius-3 ring in
    the XZ plane looking at the origin, 800x800, fx = fy = 1000 (``size`` and
    ``focal`` shrink the images for parity tests)."""
    g = torch.Generator().manual_seed(seed)
    mean = torch.randn(n, 3, generator=g)
    mean = mean / mean.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    scale = torch.randn(n, 3, generator=g) * 0.3 - 4
    scale[:, 2] = -9.2
    normal = torch.randn(n, 3, generator=g)
    normal = normal / normal.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    # Shortest-arc rotation taking +z to the normal: (1 + z, -y, x, 0) normalised.
    x, y, z = normal.unbind(-1)
    rotation = torch.stack((1 + z, -y, x, torch.zeros_like(z)), -1)
    flip = rotation.norm(dim=-1) < 1e-6
    rotation[flip] = torch.tensor([0.0, 1.0, 0.0, 0.0])
    rotation = rotation / rotation.norm(dim=-1, keepdim=True)
    opacity = torch.randn(n, 1, generator=g) * 1.5
    color = _sh3(n, g)
    cams = []
    for k in range(views):
        angle = 2 * math.pi * k / views
        cams.append(
            PinholeCamera.look_at(
                (3 * math.sin(angle), 0.0, 3 * math.cos(angle)), image_size=(size, size),
                focal_length=(focal, focal), principal_point=(size / 2, size / 2),
            )
        )
    target = torch.rand(views, size, size, 3, generator=g)
    return Scene("config5", mean, rotation, scale, opacity, color, cams, backward=True, target=target)


CONFIGS = {"config1": config1, "config2": config2, "config3": config3, "config4": config4, "config5": config5}


def edge_case_scene(
    n: int = 1000,
    sh_degree: int = 3,
    image_size: tuple[int, int] = (96, 80),
    seed: int = 42,
    near: float = 0.1,
    far: float = 100.0,
) -> Scene:
    """Parity scene with the edge cases of the reference's test scene
    (kernels/rasterize/tests/common.py:19-50) placed in front of the camera
    (the reference's scene sits behind it): 5% each of near-plane, far-plane,
    off-screen and large Gaussians.  The camera is the identity pose looking
    down -Z with fx = fy = 0.75 * width."""
    g = torch.Generator().manual_seed(seed)
    m = max(1, n // 20)
    mean = torch.empty(n, 3)
    mean[:, :2] = torch.rand(n, 2, generator=g) * 5 - 2.5
    mean[:, 2] = -(torch.rand(n, generator=g) * 7 + 1)
    mean[:m, 2] = -(torch.rand(m, generator=g) * (near - 0.03) + 0.03)
    mean[m:2 * m, 2] = -(torch.rand(m, generator=g) * 20 + far)
    mean[2 * m:3 * m, :2] = torch.rand(m, 2, generator=g) * 12 + 8
    scale = torch.rand(n, 3, generator=g) * 2 - 3
    scale[3 * m:4 * m] = torch.rand(m, 3, generator=g) * 0.75 - 0.5
    rotation = torch.randn(n, 4, generator=g)
    opacity = torch.rand(n, 1, generator=g) * 6 - 3
    k = (sh_degree + 1) ** 2
    color = torch.randn(n, k, 3, generator=g) * 0.5
    w, h = image_size
    cam = PinholeCamera(
        image_size=image_size, focal_length=(0.75 * w, 0.75 * w), principal_point=(w / 2, h / 2)
    )
    return Scene("edge_cases", mean, rotation, scale, opacity, color, [cam], near=near, far=far)


def from_file(
    path: str,
    image_size: tuple[int, int] = (1920, 1080),
    seed: int = 0,
    near: float = 0.2,
    far: float = 100.0,
) -> Scene:
    """A scene stored on disk — a GaussianSplat checkpoint (``.pt``, what the
    reference's baking and training write) or a PLY file — viewed as the
    viewer opens one: a camera pitched 45 degrees down, fitted to the points
    (visualize/gaussian/backend.py:68-75), with fx = fy = 0.75 * width.  The
    loss target is seeded U(0, 1)."""
    from pathlib import Path

    from .splats.ply import load_ply
    from .splats.splats import GaussianSplat

    path = Path(path)
    if path.suffix.lower() == ".ply":
        state = load_ply(path)
    else:
        state = GaussianSplat.from_checkpoint(path).state_dict()
    mean, rotation, scale, opacity, color = (
        state[k].detach().float().contiguous() for k in ("mean", "rotation", "scale", "opacity", "color")
    )
    w, h = image_size
    q = torch.tensor([math.cos(math.pi / 8), -math.sin(math.pi / 8), 0.0, 0.0])
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)  # fit_to_points samples 10k points of large scenes
        cam = PinholeCamera(
            rotation=q, image_size=image_size, focal_length=(0.75 * w, 0.75 * w),
            principal_point=(w / 2, h / 2),
        ).fit_to_points(mean)
    g = torch.Generator().manual_seed(seed)
    target = torch.rand(h, w, 3, generator=g)
    return Scene(path.name, mean, rotation, scale, opacity, color, [cam], near=near, far=far,
                 backward=True, target=target, notes={"source": str(path)})
