"""``torch.ops.gaussian_splats_hip.rasterize``: the autograd unit of the HIP rasterizer.

Schema, outputs and autograd contract follow the reference's custom op
(src/gaussian_splats/kernels/rasterize/interface.py:17-244): 19 inputs, 10
outputs, gradients for the first five inputs.  Differences: ``ranges`` is int64
in both the real and the fake implementation, images need not be multiples of
the tile size, and the backward is the exact gradient of the forward.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Literal

import torch

from ...timing import stage_timer
from . import _native as nat
from .composite import composite
from .intersections import (
    bin_gaussians,
    bin_tiles,
    bucketing_fits,
    depth_key_range,
    emit_tiles,
    sort_tiles,
)
from .project import _check_tile, project_and_count

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
    record_hits: bool = True,
) -> tuple[torch.Tensor, ...]:
    """Runs project -> bin -> emit -> sort -> composite; ``timer(name)`` (optional)
    is called between stages for per-stage event timing (with row/column
    bucketing, "bin" ends after the plan, "emit" after the row pass and "sort"
    after the column pass).  ``record_hits``: the compositing forward records
    the hit masks its backward walks (off when no gradient will follow)."""
    _check_tile(tile_size)
    device = nat.require_gpu(mean, rotation, scale, opacity, color)
    n = mean.shape[0]
    tiles_w, tiles_h = nat.tiles(image_width, image_height, tile_size)
    mark = timer or (lambda name: None)

    records = torch.empty((n, 12), dtype=torch.float32, device=device)
    depth_keys = torch.empty(n, dtype=torch.int32, device=device)
    # Row/column bucketing reads the projection's packed tile rectangles (the
    # int32 bounds are then not written); the other binning reads bounds.
    bucketing = bucketing_fits(n, tiles_w, tiles_h)
    tile_rects = torch.empty(n, dtype=torch.int32, device=device) if bucketing else None
    mark("start")
    projected_mean, inverse_covariance, projected_color, projected_opacity, bounds, counts = (
        project_and_count(
            mean, rotation, scale, opacity, color, camera_rotation, camera_translation,
            fx, fy, cx, cy, image_width, image_height, tile_size, near, far, rendering_mode,
            confidence, records=records, depth_keys=depth_keys, tile_rects=tile_rects,
            bounds=not bucketing,
        )
    )
    mark("project")
    # The backward's [N, 9] gradient accumulator, zeroed beside the depth
    # sort (on the binning's side stream) instead of on the stream later.
    accumulator = (torch.empty((n, 9), dtype=torch.float32, device=device)
                   if bucketing and record_hits and rendering_mode == "gaussian" else None)
    if bucketing:
        gaussian_ids, ranges = bin_tiles(depth_keys, None, None, tiles_w, tiles_h, timer=mark,
                                         tile_rects=tile_rects, clear=accumulator,
                                         key_range=depth_key_range(near, far))
    else:
        order, offsets = bin_gaussians(depth_keys, counts)
        mark("bin")
        # The one device-to-host read of the path: the intersection total sizes
        # the id buffers (the reference reads counts.sum() at intersections.py:51).
        total = int(offsets[n].item()) if n else 0
        nat.check_device_errors(device)  # the depth sort and scan, now that the stream is idle
        tile_keys, ids = emit_tiles(bounds, order, offsets, total, tiles_w)
        mark("emit")
        gaussian_ids, ranges = sort_tiles(tile_keys, ids, tiles_w * tiles_h)
    mark("sort")
    # With a backward to follow, the compositing walks write its dispatch
    # plan's keys (the backward's gs_tile_order then skips its key kernel).
    tile_keys = (nat.workspace(nat.library().gs_tile_order_workspace_bytes(ranges.shape[0]),
                               device)
                 if record_hits and rendering_mode == "gaussian" else None)
    image, final_transmittance, n_contributors = composite(
        projected_mean, inverse_covariance, projected_color, projected_opacity, gaussian_ids,
        ranges, image_width, image_height, tile_size, opacity_threshold, rendering_mode,
        confidence, records=records, record_hits=record_hits, tile_keys=tile_keys,
    )
    mark("composite")
    if accumulator is not None:
        nat.set_forward_buffer(n_contributors, "grad_accumulator", accumulator)
    if tile_keys is not None:
        nat.set_forward_buffer(n_contributors, "tile_keys", tile_keys)
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


@torch.library.custom_op("gaussian_splats_hip::rasterize", mutates_args=())
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
        confidence, timer=stage_timer(),
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
    # Prepared here, while the GPU still runs the forward, so the backward
    # launches its kernels without host work in front of them: the zeroed
    # [N, 9] gradient buffer the compositing backward accumulates into, the
    # camera extrinsics in host memory and the two views.
    mean = inputs[0]
    if mean.is_cuda and ctx.rendering_mode == "gaussian":
        ctx.grad_projected = nat.take_forward_buffer(output[2], "grad_accumulator")
        if ctx.grad_projected is None:
            ctx.grad_projected = torch.zeros((mean.shape[0], 9), dtype=torch.float32,
                                             device=mean.device)
        ctx.camera_host = (
            nat.host_floats(inputs[5], 9, "camera_rotation"),
            nat.host_floats(inputs[6], 3, "camera_translation"),
        )
        ctx.view_composite = nat.make_view(
            1.0, 1.0, 0.0, 0.0, ctx.image_width, ctx.image_height, ctx.tile_size,
            opacity_threshold=ctx.opacity_threshold, active_tiles=nat.active_tiles(output[8]),
        )
        ctx.view_project = nat.make_view(ctx.fx, ctx.fy, 0.0, 0.0, ctx.image_width, ctx.image_height)
        ctx.checkpoints, ctx.hit_masks = nat.walk_buffers(output[2])
        num_tiles = output[8].shape[0]
        lib = nat.library()
        order = torch.empty(lib.gs_tile_order_items(ctx.view_composite, 1), dtype=torch.int32,
                            device=mean.device)
        # The forward's walks wrote the plan's keys into this workspace, when
        # they ran as whole tiles (gs_tile_order checks).
        order_ws = nat.take_forward_buffer(output[2], "tile_keys")
        keys_ready = order_ws is not None
        if order_ws is None:
            order_ws = nat.workspace(lib.gs_tile_order_workspace_bytes(num_tiles), mean.device)
        # The backward's dispatch plan depends only on the forward's lists and
        # contributor counts, so it is computed now, behind the forward on the
        # stream: the backward then starts with the compositing kernel.
        _launch_backward_plan(output[8], output[2], ctx.view_composite, order, order_ws,
                              keys_ready)
        ctx.tile_order = order
    else:
        ctx.grad_projected = None


@torch.compiler.disable
def _launch_backward_plan(ranges, n_contributors, view, order, order_ws, keys_ready) -> None:
    """gs_tile_order for the backward, run eagerly (also under torch.compile,
    which cannot trace the C-ABI call)."""
    nat.check(
        nat.library().gs_tile_order(
            nat.ptr(ranges), nat.ptr(n_contributors), view, nat.ptr(order), nat.ptr(order_ws),
            order_ws.numel(), 1 if keys_ready else 0, nat.stream(ranges.device),
        ),
        "tile_order",
    )


def _contiguous(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous()


def _backward(ctx, *grad_outputs):
    """composite_bwd -> project_bwd; gradients for the first five inputs.

    Calls the C-ABI directly: every tensor but the incoming image gradient was
    produced (contiguous, aligned, on the device) by the forward."""
    if ctx.rendering_mode != "gaussian":
        raise AssertionError("Backward gradients are only supported for Gaussian rendering.")
    saved = ctx.saved_tensors
    mean, rotation, scale, opacity, color = (_contiguous(t) for t in saved[:5])
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
    ) = saved[7:]
    device = mean.device
    n = mean.shape[0]
    grad_image = grad_outputs[0]
    if grad_image is None:
        grad_image = torch.zeros(
            (ctx.image_height, ctx.image_width, 3), dtype=torch.float32, device=device
        )
    elif grad_image.dtype != torch.float32:
        grad_image = grad_image.float().contiguous()
    else:
        grad_image = _contiguous(grad_image)
    grad_projected = ctx.grad_projected
    if grad_projected is None:  # a second backward through the same graph
        grad_projected = torch.zeros((n, 9), dtype=torch.float32, device=device)
    ctx.grad_projected = None
    lib = nat.library()
    stream = nat.stream(device)
    ptr = nat.ptr
    order = ctx.tile_order
    checkpoints = ctx.checkpoints
    hits = ctx.hit_masks
    nat.check(
        nat.launch(
            "composite_bwd",
            lambda: lib.gs_composite_bwd(
                ptr(projected_mean), ptr(inverse_covariance), ptr(projected_color),
                ptr(projected_opacity), projected_mean.shape[0], ptr(gaussian_ids), ptr(ranges),
                ptr(grad_image), ptr(final_transmittance), ptr(n_contributors), ptr(order),
                ctx.view_composite, ptr(grad_projected), None, ptr(checkpoints),
                nat.buffer_bytes(checkpoints), gaussian_ids.numel(), ptr(hits),
                nat.buffer_bytes(hits), stream,
            ),
        ),
        "composite_bwd",
    )
    grads = tuple(torch.empty_like(t) for t in (mean, rotation, scale, opacity, color))
    if n:
        cam_r, cam_t = ctx.camera_host
        nat.check(
            nat.launch("project_bwd", lambda: lib.gs_project_bwd(
                ptr(mean), ptr(rotation), ptr(scale), ptr(opacity), ptr(color), n,
                color.shape[1], ptr(cam_r), ptr(cam_t), ctx.view_project, ptr(inverse_covariance),
                ptr(grad_projected), ptr(counts), *(ptr(g) for g in grads), stream,
            )),
            "project_bwd",
        )
    return (*grads, *(None,) * 14)


torch.library.register_autograd(
    "gaussian_splats_hip::rasterize", _backward, setup_context=_setup_context
)


class _RasterizeFunction(torch.autograd.Function):
    """The op's forward and backward as an autograd.Function, for eager
    calls: the same two functions, without the dispatcher's per-call work
    for a 19-argument custom op (default filling, schema checks), which
    costs tens of microseconds of host time per step.  Traced code
    (torch.compile, export) calls the registered op instead."""

    @staticmethod
    def forward(ctx, *inputs):
        output = forward_pipeline(*inputs, timer=stage_timer())
        _setup_context(ctx, inputs, output)
        return output

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, *grad_outputs):
        return _backward(ctx, *grad_outputs)


def rasterize_outputs(*inputs) -> tuple[torch.Tensor, ...]:
    """The op's ten outputs for its 19 inputs: the registered op when traced,
    the equivalent autograd.Function when a gradient will be needed, else the
    forward alone."""
    if torch.compiler.is_compiling():
        return _rasterize(*inputs)
    if torch.is_grad_enabled() and any(t.requires_grad for t in inputs[:5]):
        return _RasterizeFunction.apply(*inputs)
    return forward_pipeline(*inputs, timer=stage_timer(), record_hits=False)


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
    # Extrinsics stay in host memory: the kernels take them as arguments.
    from ...splats.camera import host_extrinsics  # the splat API imports this module

    camera_rotation, camera_translation = host_extrinsics(camera)
    return rasterize_outputs(
        mean,
        rotation,
        scale,
        opacity,
        color,
        camera_rotation,
        camera_translation,
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
