"""Backward tile compositing (HIP: gs_composite_bwd).

Same launcher contract as the reference's
src/gaussian_splats/kernels/rasterize/composite_bwd.py:207-277: returns the
per-Gaussian gradient [N, 9] with columns (u, v, inv00, inv01, inv11, r, g, b,
opacity), and with ``return_absolute`` also the [N, 2] sums of the absolute
per-pixel terms of the (u, v) gradient.  Accumulation is always atomic (one
add per tile and Gaussian), so ``atomic`` is accepted for compatibility and
ignored.
"""

from __future__ import annotations

import torch

from . import _native as nat
from .composite import walk_key
from .project import _check_tile


def composite_bwd(
    projected_mean: torch.Tensor,
    inverse_covariance: torch.Tensor,
    projected_color: torch.Tensor,
    projected_opacity: torch.Tensor,
    gaussian_ids: torch.Tensor,
    ranges: torch.Tensor,
    grad_image: torch.Tensor,
    final_transmittance: torch.Tensor,
    n_contributors: torch.Tensor,
    image_width: int,
    image_height: int,
    tile_size: int,
    opacity_threshold: float,
    rendering_mode: str,
    atomic: bool = False,
    return_absolute: bool = False,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``out`` (optional, zero-filled [N, 9] float32) receives the gradient;
    returns ``(grad, absolute)`` when ``return_absolute``.

    A pure function of its arguments, as the reference's is.  When they are
    exactly those of an earlier ``composite`` call and its outputs (same
    tensors, unmodified), the walk skips the entries that call's hit masks
    leave out and starts long lists at its checkpoints.  Otherwise it walks
    every entry from the end of each list."""
    if rendering_mode != "gaussian":
        raise AssertionError("Backward gradients are only supported for Gaussian rendering.")
    _check_tile(tile_size)
    device = nat.require_gpu(projected_mean, gaussian_ids, ranges, grad_image)
    checkpoints, hits = nat.walk_buffers(n_contributors, walk_key(
        image_width, image_height, tile_size, opacity_threshold, rendering_mode, projected_mean,
        inverse_covariance, projected_color, projected_opacity, gaussian_ids, ranges,
        final_transmittance, n_contributors))
    projected_mean, inverse_covariance, projected_color, projected_opacity = (
        nat.prepare(t) for t in (projected_mean, inverse_covariance, projected_color, projected_opacity)
    )
    grad_image = nat.prepare(grad_image.float() if grad_image.dtype != torch.float32 else grad_image)
    final_transmittance = nat.prepare(final_transmittance)
    n_contributors = nat.prepare(n_contributors, torch.int32)
    active = nat.active_tiles(ranges)
    ranges = nat.prepare(ranges, torch.int64)
    gaussian_ids = nat.prepare(gaussian_ids, torch.int32)
    n = projected_mean.shape[0]
    if out is None:
        out = torch.zeros((n, 9), dtype=torch.float32, device=device)
    elif out.shape != (n, 9) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous zero-filled float32 tensor of shape [N, 9]")
    view = nat.make_view(
        1.0, 1.0, 0.0, 0.0, image_width, image_height, tile_size,
        opacity_threshold=opacity_threshold, active_tiles=active,
    )
    absolute = torch.zeros((n, 2), dtype=torch.float32, device=device) if return_absolute else None
    lib = nat.library()
    order = nat.dispatch_plan(view, ranges.shape[0], device, ranges=ranges,
                              n_contributors=n_contributors)
    nat.check(
        nat.launch(
            "composite_bwd",
            lambda: lib.gs_composite_bwd(
                nat.ptr(projected_mean), nat.ptr(inverse_covariance), nat.ptr(projected_color),
                nat.ptr(projected_opacity), n, nat.ptr(gaussian_ids), nat.ptr(ranges),
                nat.ptr(grad_image), nat.ptr(final_transmittance), nat.ptr(n_contributors),
                nat.ptr(order), view, nat.ptr(out), nat.ptr(absolute), nat.ptr(checkpoints),
                nat.buffer_bytes(checkpoints), gaussian_ids.numel(), nat.ptr(hits),
                nat.buffer_bytes(hits), nat.stream(device),
            ),
        ),
        "composite_bwd",
    )
    return (out, absolute) if return_absolute else out
