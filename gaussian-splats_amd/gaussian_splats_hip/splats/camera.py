"""Camera conventions (reference: src/gaussian_splats/splats/camera.py:14-144).

World-to-camera rotation stored as a (w, x, y, z) quaternion plus a translation,
so a world point X maps to camera space as R X + t.  The camera looks down -Z
with +Y up; image y grows downwards: u = fx x / (-z) + cx, v = -fy y / (-z) + cy.
Projection itself runs inside the HIP rasterizer (gs_project_and_count).
"""

from __future__ import annotations

import math
from abc import ABC
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F
from typing_extensions import Self

from .utils import quaternion_to_rotation_matrix, rotation_matrix_to_quaternion


@dataclass(kw_only=True)
class Camera(ABC):
    rotation: torch.Tensor = field(default_factory=lambda: torch.tensor([1.0, 0.0, 0.0, 0.0]))
    translation: torch.Tensor = field(default_factory=lambda: torch.zeros(3))
    image_size: tuple[int, int] = (640, 480)

    @property
    def rotation_matrix(self) -> torch.Tensor:
        return quaternion_to_rotation_matrix(F.normalize(self.rotation, dim=-1))

    @property
    def position(self) -> torch.Tensor:
        return -(self.rotation_matrix.T @ self.translation)

    def to(self, device: torch.device | str) -> Self:
        self.rotation = self.rotation.to(device)
        self.translation = self.translation.to(device)
        return self

    @property
    def device(self) -> torch.device:
        return self.translation.device

    @property
    def dtype(self) -> torch.dtype:
        return self.translation.dtype


@dataclass(kw_only=True)
class PinholeCamera(Camera):
    """OpenGL/Blender-style pinhole camera (camera.py:55-144)."""

    focal_length: tuple[float, float] = (500.0, 500.0)
    principal_point: tuple[float, float] = (320.0, 240.0)
    intrinsics: torch.Tensor = field(init=False, repr=False)

    def __post_init__(self) -> None:
        fx, fy = self.focal_length
        cx, cy = self.principal_point
        # Homogeneous map (x, y, z) -> (fx x - cx z, -fy y - cy z, -z) (camera.py:63-74).
        self.intrinsics = torch.tensor(
            [[fx, 0, -cx], [0, -fy, -cy], [0, 0, -1]], dtype=self.dtype, device=self.device
        )

    def to(self, device: torch.device | str) -> Self:
        super().to(device)
        self.intrinsics = self.intrinsics.to(device)
        return self

    @torch.no_grad()
    def fit_to_points(self, points: torch.Tensor) -> Self:
        """Moves the camera back along its viewing axis until the points' bounding
        sphere fits the narrower field of view (camera.py:126-144)."""
        self.to(points.device)
        if len(points) > 10_000:
            points = points[torch.randint(len(points), (10_000,), device=points.device)]
        lower, upper = torch.aminmax(points, dim=0)
        center = 0.5 * (lower + upper)
        radius = 0.5 * (upper - lower).norm().clamp_min(1e-3)
        fx, fy = self.focal_length
        width, height = self.image_size
        tan_half_fov = min(width / (2 * fx), height / (2 * fy))
        distance = 1.1 * radius / math.sin(math.atan(tan_half_fov))
        rotation = self.rotation_matrix
        position = center + distance * rotation[2]
        self.translation = -(rotation @ position)
        return self

    @classmethod
    def look_at(
        cls,
        position: tuple[float, float, float] | torch.Tensor,
        target: tuple[float, float, float] | torch.Tensor = (0.0, 0.0, 0.0),
        up: tuple[float, float, float] | torch.Tensor = (0.0, 1.0, 0.0),
        **kwargs,
    ) -> Self:
        """Camera at ``position`` facing ``target``: rotation rows are (right, up,
        -forward), as the viewer's controller builds them (visualize/camera.py:73-78),
        and t = -R position."""
        pos = torch.as_tensor(position, dtype=torch.float64)
        tgt = torch.as_tensor(target, dtype=torch.float64)
        upv = torch.as_tensor(up, dtype=torch.float64)
        forward = F.normalize(tgt - pos, dim=0)
        right = torch.linalg.cross(forward, upv)
        if right.norm() < 1e-9:
            right = torch.linalg.cross(forward, torch.tensor([0.0, 0.0, 1.0], dtype=torch.float64))
        right = F.normalize(right, dim=0)
        cam_up = torch.linalg.cross(right, forward)
        rotation = torch.stack((right, cam_up, -forward))
        quaternion = rotation_matrix_to_quaternion(rotation)
        translation = -(rotation @ pos)
        return cls(
            rotation=quaternion.float(), translation=translation.float(), **kwargs
        )


@torch.compiler.disable  # host arithmetic: runs as it is under torch.compile
def host_extrinsics(camera: Camera) -> tuple[torch.Tensor, torch.Tensor]:
    """The world-to-camera rotation matrix [3, 3] and translation [3] as
    float32 tensors in host memory (the rasterizer passes them to its kernels
    as arguments).  For a float32 quaternion the matrix is built from numpy
    float32 scalars with the operations of ``camera.rotation_matrix`` in the
    same order (F.normalize: sequential sum of squares, sqrt, clamp at 1e-12,
    divide; then utils.py:8-25), so the values are the same, without the ~25
    small tensor operations (~0.3 ms of host time per call) of the torch
    path; other dtypes take the torch path."""
    q = camera.rotation.detach()
    t = camera.translation.detach()
    if q.dtype != torch.float32 or q.numel() != 4:
        return (camera.rotation_matrix.detach().to(device="cpu", dtype=torch.float32),
                t.to(device="cpu", dtype=torch.float32).reshape(3))
    # One device-to-host copy for a camera on the GPU.
    host = torch.cat((q.reshape(4), t.reshape(3).to(torch.float32))).cpu()
    t = host[4:].clone()
    w, x, y, z = (np.float32(v) for v in host[:4].tolist())
    norm = max(np.sqrt(((w * w + x * x) + y * y) + z * z), np.float32(1e-12))
    w, x, y, z = w / norm, x / norm, y / norm, z / norm
    one, two = np.float32(1), np.float32(2)
    xx, yy, zz = x * x, y * y, z * z
    rows = [
        [one - two * (yy + zz), two * (x * y - w * z), two * (x * z + w * y)],
        [two * (x * y + w * z), one - two * (xx + zz), two * (y * z - w * x)],
        [two * (x * z - w * y), two * (y * z + w * x), one - two * (xx + yy)],
    ]
    return torch.from_numpy(np.array(rows, dtype=np.float32)), t
