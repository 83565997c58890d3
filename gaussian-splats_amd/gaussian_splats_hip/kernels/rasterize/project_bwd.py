"""Projection backward (HIP: gs_project_bwd).

Same launcher contract as the reference's
src/gaussian_splats/kernels/rasterize/project_bwd.py:337-381.
"""

from __future__ import annotations

from ctypes import c_void_p

import torch

from . import _native as nat


def project_bwd(
    mean: torch.Tensor,
    rotation: torch.Tensor,
    scale: torch.Tensor,
    opacity: torch.Tensor,
    color: torch.Tensor,
    camera_rotation: torch.Tensor,
    camera_translation: torch.Tensor,
    inverse_covariance: torch.Tensor,
    grad_projected: torch.Tensor,
    counts: torch.Tensor,
    fx: float,
    fy: float,
    image_width: int,
    image_height: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns ``(grad_mean, grad_rotation, grad_scale, grad_opacity, grad_color)``."""
    if color.shape[1] > 16:
        raise NotImplementedError(
            f"SH degrees above 3 are not implemented. Got {color.shape[1]} coefficients."
        )
    device = nat.require_gpu(mean, rotation, scale, opacity, color, grad_projected, counts)
    mean, rotation, scale, opacity, color, inverse_covariance, grad_projected = (
        nat.prepare(t)
        for t in (mean, rotation, scale, opacity, color, inverse_covariance, grad_projected)
    )
    counts = nat.prepare(counts, torch.int32)
    camera_rotation = nat.host_floats(camera_rotation, 9, "camera_rotation")
    camera_translation = nat.host_floats(camera_translation, 3, "camera_translation")
    grad_mean = torch.empty_like(mean)
    grad_rotation = torch.empty_like(rotation)
    grad_scale = torch.empty_like(scale)
    grad_opacity = torch.empty_like(opacity)
    grad_color = torch.empty_like(color)
    n = mean.shape[0]
    if n == 0:
        return grad_mean, grad_rotation, grad_scale, grad_opacity, grad_color
    view = nat.make_view(fx, fy, 0.0, 0.0, image_width, image_height)
    nat.check(
        nat.library().gs_project_bwd(
            nat.ptr(mean), nat.ptr(rotation), nat.ptr(scale), nat.ptr(opacity), nat.ptr(color),
            n, color.shape[1], c_void_p(camera_rotation.data_ptr()), c_void_p(camera_translation.data_ptr()), view,
            nat.ptr(inverse_covariance), nat.ptr(grad_projected), nat.ptr(counts),
            nat.ptr(grad_mean), nat.ptr(grad_rotation), nat.ptr(grad_scale),
            nat.ptr(grad_opacity), nat.ptr(grad_color), nat.stream(device),
        ),
        "project_bwd",
    )
    return grad_mean, grad_rotation, grad_scale, grad_opacity, grad_color
