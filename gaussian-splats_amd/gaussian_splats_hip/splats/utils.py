"""Small math helpers of the splat API (reference: src/gaussian_splats/splats/utils.py)."""

from __future__ import annotations

import torch

# Degree-0 real SH normalisation, 1 / (2 sqrt(pi)) (utils.py:5).
SH_C0 = 0.28209479177387814


def quaternion_to_rotation_matrix(quaternion: torch.Tensor) -> torch.Tensor:
    """Rotation matrix of a unit quaternion stored as (w, x, y, z) (utils.py:8-25)."""
    w, x, y, z = quaternion.unbind(dim=-1)
    xx, yy, zz = x * x, y * y, z * z
    rows = (
        (1 - 2 * (yy + zz), 2 * (x * y - w * z), 2 * (x * z + w * y)),
        (2 * (x * y + w * z), 1 - 2 * (xx + zz), 2 * (y * z - w * x)),
        (2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (xx + yy)),
    )
    return torch.stack([torch.stack(r, dim=-1) for r in rows], dim=-2)


def rgb_to_sh(rgb: torch.Tensor) -> torch.Tensor:
    """Degree-0 coefficient whose evaluation (c * SH_C0 + 0.5) is ``rgb`` (utils.py:28-29)."""
    return (rgb - 0.5) / SH_C0


def rotation_matrix_to_quaternion(matrix: torch.Tensor) -> torch.Tensor:
    """(w, x, y, z) unit quaternion of a 3x3 rotation matrix (Shepperd's method)."""
    m = matrix.double()
    trace = m[0, 0] + m[1, 1] + m[2, 2]
    candidates = torch.stack((trace, m[0, 0], m[1, 1], m[2, 2]))
    i = int(torch.argmax(candidates))
    if i == 0:
        s = torch.sqrt(trace + 1.0) * 2
        q = (0.25 * s, (m[2, 1] - m[1, 2]) / s, (m[0, 2] - m[2, 0]) / s, (m[1, 0] - m[0, 1]) / s)
    elif i == 1:
        s = torch.sqrt(1.0 + m[0, 0] - m[1, 1] - m[2, 2]) * 2
        q = ((m[2, 1] - m[1, 2]) / s, 0.25 * s, (m[0, 1] + m[1, 0]) / s, (m[0, 2] + m[2, 0]) / s)
    elif i == 2:
        s = torch.sqrt(1.0 + m[1, 1] - m[0, 0] - m[2, 2]) * 2
        q = ((m[0, 2] - m[2, 0]) / s, (m[0, 1] + m[1, 0]) / s, 0.25 * s, (m[1, 2] + m[2, 1]) / s)
    else:
        s = torch.sqrt(1.0 + m[2, 2] - m[0, 0] - m[1, 1]) * 2
        q = ((m[1, 0] - m[0, 1]) / s, (m[0, 2] + m[2, 0]) / s, (m[1, 2] + m[2, 1]) / s, 0.25 * s)
    out = torch.stack(q)
    if out[0] < 0:
        out = -out
    return (out / out.norm()).to(matrix.dtype)
