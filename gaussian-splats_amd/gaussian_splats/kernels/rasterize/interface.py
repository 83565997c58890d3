"""``torch.ops.gaussian_splats.rasterize``: the autograd unit of the HIP rasterizer.

Schema, outputs and autograd contract follow the reference's custom op
(src/gaussian_splats/kernels/rasterize/interface.py:17-244): 19 inputs, 10
outputs, gradients for the first five inputs.  Differences: ``ranges`` is int64
in both the real and the fake implementation, images need not be multiples of
the tile size, and the backward is the exact gradient of the forward.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Literal

import torch

from . import _native as nat
from .composite import composite
from .composite_bwd import composite_bwd
from .intersections import MAX_BUCKET_TILES, bin_gaussians, bin_tiles, emit_tiles, sort_tiles
from .project import _check_tile, project_and_count
from .project_bwd import project_bwd

if TYPE_CHECKING:  # the splat API imports this module, so only for annotations
    from ...splats.camera import Camera
    from ...splats.splats import GaussianSplat


def forward_pipeline(
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
    opacity_threshold: float,
    near: float,
    far: float,
    rendering_mode: str,
    confidence: float,
    timer=None,
) -> tuple[torch.Tensor, ...]:
    """Runs project -> bin -> emit -> sort -> composite; ``timer(name)`` (optional)
    is called between stages for per-stage event timing (with row/column
    bucketing, "bin" ends after the plan, "emit" after the row pass and "sort"
    after the column pass)."""
    _check_tile(tile_size)
    device = nat.require_gpu(mean, rotation, scale, opacity, color)
    n = mean.shape[0]
    tiles_w, tiles_h = nat.tiles(image_width, image_height, tile_size)
    mark = timer or (lambda name: None)

    records = torch.empty((n, 12), dtype=torch.float32, device=device)
    depth_keys = torch.empty(n, dtype=torch.int32, device=device)
    mark("start")
    projected_mean, inverse_covariance, projected_color, projected_opacity, bounds, counts = (
        project_and_count(
            mean, rotation, scale, opacity, color, camera_rotation, camera_translation,
            fx, fy, cx, cy, image_width, image_height, tile_size, near, far, rendering_mode,
            confidence, records=records, depth_keys=depth_keys,
        )
    )
    mark("project")
    if tiles_w <= MAX_BUCKET_TILES and tiles_h <= MAX_BUCKET_TILES:
        gaussian_ids, ranges = bin_tiles(depth_keys, bounds, counts, tiles_w, tiles_h, timer=mark)
    else:
        order, offsets = bin_gaussians(depth_keys, counts)
        mark("bin")
        # The one device-to-host read of the path: the intersection total sizes
        # the id buffers (the reference reads counts.sum() at intersections.py:51).
        total = int(offsets[n].item()) if n else 0
        tile_keys, ids = emit_tiles(bounds, order, offsets, total, tiles_w)
        mark("emit")
        gaussian_ids, ranges = sort_tiles(tile_keys, ids, tiles_w * tiles_h)
    mark("sort")
    image, final_transmittance, n_contributors = composite(
        projected_mean, inverse_covariance, projected_color, projected_opacity, gaussian_ids,
        ranges, image_width, image_height, tile_size, opacity_threshold, rendering_mode,
        confidence, records=records,
    )
    mark("composite")
    return (
        image,
        final_transmittance,
        n_contributors,
        projected_mean,
        inverse_covariance,
        projected_color,
        projected_opacity,
        gaussian_ids,
        ranges,
        counts,
    )


@torch.library.custom_op("gaussian_splats::rasterize", mutates_args=())
def _rasterize(
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
    opacity_threshold: float,
    near: float,
    far: float,
    rendering_mode: str,
    confidence: float,
) -> tuple[
    torch.Tensor,  # image
    torch.Tensor,  # final_transmittance
    torch.Tensor,  # n_contributors
    torch.Tensor,  # projected_mean
    torch.Tensor,  # inverse_covariance
    torch.Tensor,  # projected_color
    torch.Tensor,  # projected_opacity
    torch.Tensor,  # gaussian_ids
    torch.Tensor,  # ranges
    torch.Tensor,  # counts
]:
    return forward_pipeline(
        mean, rotation, scale, opacity, color, camera_rotation, camera_translation, fx, fy, cx,
        cy, image_width, image_height, tile_size, opacity_threshold, near, far, rendering_mode,
        confidence,
    )


@_rasterize.register_fake
def _rasterize_fake(
    mean, rotation, scale, opacity, color, camera_rotation, camera_translation, fx, fy, cx, cy,
    image_width, image_height, tile_size, opacity_threshold, near, far, rendering_mode,
    confidence,
):
    dynamic = torch.library.get_ctx().new_dynamic_size()
    tiles_w, tiles_h = nat.tiles(image_width, image_height, tile_size)
    n = mean.shape[0]
    return (
        mean.new_empty((image_height, image_width, 3)),
        mean.new_empty((image_height, image_width)),
        torch.empty((image_height, image_width), dtype=torch.int32, device=mean.device),
        mean.new_empty((n, 3)),
        mean.new_empty((n, 2, 2)),
        mean.new_empty((n, 3)),
        mean.new_empty((n, 1)),
        torch.empty((dynamic,), dtype=torch.int32, device=mean.device),
        torch.empty((tiles_w * tiles_h, 2), dtype=torch.int64, device=mean.device),
        torch.empty((n,), dtype=torch.int32, device=mean.device),
    )


def _setup_context(ctx, inputs, output) -> None:
    # The backward reads only the image gradient; unused outputs get None
    # instead of zero-filled gradient tensors.
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(*inputs[:7], *output[1:])
    (
        ctx.fx,
        ctx.fy,
        ctx.cx,
        ctx.cy,
        ctx.image_width,
        ctx.image_height,
        ctx.tile_size,
        ctx.opacity_threshold,
        ctx.near,
        ctx.far,
        ctx.rendering_mode,
        ctx.confidence,
    ) = inputs[7:]


def _backward(ctx, *grad_outputs):
    """composite_bwd -> project_bwd; gradients for the first five inputs."""
    if ctx.rendering_mode != "gaussian":
        raise AssertionError("Backward gradients are only supported for Gaussian rendering.")
    grad_image = grad_outputs[0]
    mean, rotation, scale, opacity, color, camera_rotation, camera_translation = ctx.saved_tensors[:7]
    (
        final_transmittance,
        n_contributors,
        projected_mean,
        inverse_covariance,
        projected_color,
        projected_opacity,
        gaussian_ids,
        ranges,
        counts,
    ) = ctx.saved_tensors[7:]
    if grad_image is None:
        grad_image = torch.zeros(
            (ctx.image_height, ctx.image_width, 3), dtype=mean.dtype, device=mean.device
        )
    grad_projected = composite_bwd(
        projected_mean, inverse_covariance, projected_color, projected_opacity, gaussian_ids,
        ranges, grad_image, final_transmittance, n_contributors, ctx.image_width,
        ctx.image_height, ctx.tile_size, ctx.opacity_threshold, ctx.rendering_mode,
    )
    gradients = project_bwd(
        mean, rotation, scale, opacity, color, camera_rotation, camera_translation,
        inverse_covariance, grad_projected, counts, ctx.fx, ctx.fy, ctx.image_width,
        ctx.image_height,
    )
    return (*gradients, *(None,) * (19 - len(gradients)))


torch.library.register_autograd(
    "gaussian_splats::rasterize", _backward, setup_context=_setup_context
)


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
) -> torch.Tensor:
    """Renders ``splats`` seen by ``camera`` into an [H, W, 3] image (interface.py:247-303)."""
    fx, fy = camera.focal_length
    cx, cy = camera.principal_point
    image_width, image_height = camera.image_size
    _check_tile(tile_size)
    if rendering_mode not in ("gaussian", "ellipsoid"):
        raise ValueError(f"Invalid rendering mode: {rendering_mode}")

    mean, rotation, scale, opacity, color = (
        splats.mean,
        splats.rotation,
        splats.scale,
        splats.opacity,
        splats.color,
    )
    if indices is not None:
        mean, rotation, scale, opacity, color = (
            mean[indices],
            rotation[indices],
            scale[indices],
            opacity[indices],
            color[indices],
        )
    device = mean.device
    return _rasterize(
        mean,
        rotation,
        scale,
        opacity,
        color,
        # Extrinsics stay in host memory: the kernels take them as arguments.
        camera.rotation_matrix.detach().to(device="cpu", dtype=torch.float32),
        camera.translation.detach().to(device="cpu", dtype=torch.float32),
        float(fx),
        float(fy),
        float(cx),
        float(cy),
        int(image_width),
        int(image_height),
        int(tile_size),
        float(opacity_threshold),
        float(near),
        float(far),
        rendering_mode,
        float(confidence),
    )[0]
