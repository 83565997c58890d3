"""Projection and tile-count stage (HIP: gs_project_and_count).

Same launcher contract as the reference's
src/gaussian_splats/kernels/rasterize/project.py:256-345.
"""

from __future__ import annotations

from ctypes import c_void_p

import torch

from . import _native as nat


def _check_tile(tile_size: int) -> None:
    if not (tile_size > 0 and tile_size & (tile_size - 1) == 0):
        raise ValueError(f"tile_size must be a positive power of two, got {tile_size}")


def project_and_count(
    mean: torch.Tensor,
    rotation: torch.Tensor,
    scale: torch.Tensor,
    opacity: torch.Tensor,
    color: torch.Tensor,
    camera_rotation: torch.Tensor,
    camera_translation: torch.Tensor,
    fx: float,
    fy: float,
    cx: float,
    cy: float,
    image_width: int,
    image_height: int,
    tile_size: int,
    near: float,
    far: float,
    rendering_mode: str,
    confidence: float,
    *,
    covariance_epsilon: float = 0.03,
    records: torch.Tensor | None = None,
    depth_keys: torch.Tensor | None = None,
    tile_rects: torch.Tensor | None = None,
    bounds: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor | None, torch.Tensor]:
    """Projects Gaussians and counts their tiles without compacting.

    Returns ``(projected_mean[N,3], inverse_covariance[N,2,2], projected_color[N,3],
    projected_opacity[N,1], bounds[N,2,2] int32, counts[N] int32)`` in the original
    Gaussian order; culled Gaussians keep their slot with ``count == 0``.
    ``records`` (N x 12 float32), ``depth_keys`` (N int32) and ``tile_rects``
    (N int32, the packed rectangles ``bin_tiles`` reads) are optional extra
    outputs used by the fused op, which also skips ``bounds`` (``bounds=False``
    returns None in its place; it needs ``tile_rects``).
    """
    _check_tile(tile_size)
    if color.shape[1] > 16:
        raise NotImplementedError(
            f"SH degrees above 3 are not implemented. Got {color.shape[1]} coefficients."
        )
    device = nat.require_gpu(mean, rotation, scale, opacity, color)
    mean, rotation, scale, opacity, color = (
        nat.prepare(t) for t in (mean, rotation, scale, opacity, color)
    )
    camera_rotation = nat.host_floats(camera_rotation, 9, "camera_rotation")
    camera_translation = nat.host_floats(camera_translation, 3, "camera_translation")

    n = mean.shape[0]
    projected_mean = mean.new_empty((n, 3))
    inverse_covariance = mean.new_empty((n, 2, 2))
    projected_color = mean.new_empty((n, 3))
    projected_opacity = mean.new_empty((n, 1))
    if not bounds and tile_rects is None:
        raise ValueError("bounds=False needs tile_rects")
    if tile_rects is not None and (
        tile_rects.device != device or tile_rects.dtype != torch.int32
        or tile_rects.numel() != mean.shape[0] or not tile_rects.is_contiguous()
    ):
        raise ValueError("tile_rects must be a contiguous int32 tensor of N elements on the "
                         "Gaussians' device")
    bounds = torch.empty((n, 2, 2), dtype=torch.int32, device=device) if bounds else None
    counts = torch.empty(n, dtype=torch.int32, device=device)
    if n == 0:
        return projected_mean, inverse_covariance, projected_color, projected_opacity, bounds, counts

    view = nat.make_view(
        fx, fy, cx, cy, image_width, image_height, tile_size, near, far, rendering_mode,
        confidence, covariance_epsilon=covariance_epsilon,
    )
    lib = nat.library()
    nat.check(
        nat.launch("project", lambda: lib.gs_project_and_count(
            nat.ptr(mean), nat.ptr(rotation), nat.ptr(scale), nat.ptr(opacity), nat.ptr(color),
            n, color.shape[1], c_void_p(camera_rotation.data_ptr()),
            c_void_p(camera_translation.data_ptr()), view,
            nat.ptr(projected_mean), nat.ptr(inverse_covariance), nat.ptr(projected_color),
            nat.ptr(projected_opacity), nat.ptr(bounds), nat.ptr(counts), nat.ptr(records),
            nat.ptr(depth_keys), nat.ptr(tile_rects), nat.stream(device),
        )),
        "project_and_count",
    )
    return projected_mean, inverse_covariance, projected_color, projected_opacity, bounds, counts


def pack_records(
    projected_mean: torch.Tensor,
    inverse_covariance: torch.Tensor,
    projected_color: torch.Tensor,
    projected_opacity: torch.Tensor,
    rendering_mode: str = "gaussian",
    confidence: float = 0.95,
) -> torch.Tensor:
    """Packs the 48-byte compositing records (N x 12 float32) from projected outputs."""
    device = nat.require_gpu(projected_mean, inverse_covariance, projected_color, projected_opacity)
    tensors = [nat.prepare(t) for t in (projected_mean, inverse_covariance, projected_color, projected_opacity)]
    n = tensors[0].shape[0]
    records = torch.empty((n, 12), dtype=torch.float32, device=device)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, 1, 1, 16, rendering_mode=rendering_mode, confidence=confidence)
    nat.check(
        nat.library().gs_pack_records(*(nat.ptr(t) for t in tensors), n, view, nat.ptr(records), nat.stream(device)),
        "pack_records",
    )
    return records
