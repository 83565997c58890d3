"""``torch.ops.gaussian_splats_hip.rasterize_views``: several cameras in one pass.

No counterpart in the reference, which renders one camera per call of
``rasterize`` (src/gaussian_splats/kernels/rasterize/interface.py:247-303) and
leaves multi-view batches to a Python loop over views (training/train.py:128-147
steps one view at a time).  Here the V views of one image size are rendered as
a single mosaic: their tile grids are laid side by side, ``cols`` per row, and
every stage runs once over all of them:

* ``gs_project_views`` projects each Gaussian for every camera (parameters
  read once per 16 cameras) into [V, N] arrays, view v's Gaussian i at the
  virtual index v * N + i, with tile rectangles in mosaic coordinates;
* binning sorts the V * N virtual Gaussians over the mosaic's tiles; each tile
  belongs to one view and lists only that view's Gaussians, in the (depth,
  index) order of the single-view op;
* compositing and its backward run over the mosaic's tiles, writing and
  reading [V, H, W] images;
* ``gs_project_bwd_views`` sums the views' gradients per Gaussian.

Per view, the image, lists and transmittance equal those of ``rasterize`` with
that camera; the gradients equal the sum of the single-view gradients up to
the order of floating-point additions.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Literal, Sequence

import torch

from ...timing import stage_timer
from . import _native as nat
from .intersections import (
    MAX_BUCKET_TILES,
    bin_gaussians,
    bin_tiles,
    bucketing_fits,
    depth_key_range,
    emit_tiles,
    sort_tiles,
)
from .interface import _contiguous
from .project import _check_tile

if TYPE_CHECKING:
    from ...splats.camera import Camera
    from ...splats.splats import GaussianSplat


def mosaic_columns(views: int, tiles_w: int, tiles_h: int) -> int:
    """Views per mosaic row: the most nearly square layout whose tile grid fits
    ``MAX_BUCKET_TILES`` per axis (row/column bucketing), else the most nearly
    square one."""
    if views <= 1:
        return 1
    best, best_key = 1, None
    for cols in range(1, views + 1):
        rows = -(-views // cols)
        w, h = cols * tiles_w, rows * tiles_h
        fits = w <= MAX_BUCKET_TILES and h <= MAX_BUCKET_TILES
        # Fitting layouts first, then the squarest, then the fewest empty slots.
        key = (not fits, max(w, h), rows * cols - views)
        if best_key is None or key < best_key:
            best, best_key = cols, key
    return best


def _mosaic_view(
    image_width: int, image_height: int, tile_size: int, views: int, cols: int, **kwargs
) -> nat.GsView:
    return nat.make_view(
        1.0, 1.0, 0.0, 0.0, image_width, image_height, tile_size, views=views, mosaic_cols=cols,
        **kwargs,
    )


def _camera_arrays(
    camera_rotations: torch.Tensor, camera_translations: torch.Tensor, intrinsics: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]:
    views = camera_rotations.shape[0]
    r = nat.host_floats(camera_rotations, 9 * views, "camera_rotations")
    t = nat.host_floats(camera_translations, 3 * views, "camera_translations")
    k = nat.host_floats(intrinsics, 4 * views, "intrinsics")
    return r, t, k, views


def forward_views(
    mean: torch.Tensor,
    rotation: torch.Tensor,
    scale: torch.Tensor,
    opacity: torch.Tensor,
    color: torch.Tensor,
    camera_rotations: torch.Tensor,
    camera_translations: torch.Tensor,
    intrinsics: torch.Tensor,
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
    """project (all views) -> bin (mosaic) -> composite (mosaic); ``timer(name)``
    marks the stages and ``record_hits`` selects the hit masks as
    ``forward_pipeline`` does."""
    _check_tile(tile_size)
    if color.shape[1] > 16:
        raise NotImplementedError(
            f"SH degrees above 3 are not implemented. Got {color.shape[1]} coefficients."
        )
    device = nat.require_gpu(mean, rotation, scale, opacity, color)
    mark = timer or (lambda name: None)
    mean, rotation, scale, opacity, color = (
        nat.prepare(t) for t in (mean, rotation, scale, opacity, color)
    )
    cam_r, cam_t, intr, views = _camera_arrays(camera_rotations, camera_translations, intrinsics)
    if views < 1:
        raise ValueError("rasterize_views needs at least one camera")
    n = mean.shape[0]
    tw, th = nat.tiles(image_width, image_height, tile_size)
    cols = mosaic_columns(views, tw, th)
    rows = -(-views // cols)
    canvas_w, canvas_h = cols * tw, rows * th
    vn = views * n

    projected_mean = mean.new_empty((views, n, 3))
    inverse_covariance = mean.new_empty((views, n, 2, 2))
    projected_color = mean.new_empty((views, n, 3))
    projected_opacity = mean.new_empty((views, n, 1))
    # Row/column bucketing reads the projection's packed tile rectangles (the
    # int32 bounds are then not written); the other binning reads bounds.
    bucketing = bucketing_fits(vn, canvas_w, canvas_h)
    bounds = (None if bucketing
              else torch.empty((views, n, 2, 2), dtype=torch.int32, device=device))
    tile_rects = torch.empty(vn, dtype=torch.int32, device=device) if bucketing else None
    counts = torch.empty((views, n), dtype=torch.int32, device=device)
    records = torch.empty((vn, 12), dtype=torch.float32, device=device)
    depth_keys = torch.empty(vn, dtype=torch.int32, device=device)
    lib = nat.library()
    stream = nat.stream(device)
    ptr = nat.ptr
    project_view = nat.make_view(
        0.0, 0.0, 0.0, 0.0, image_width, image_height, tile_size, near, far, rendering_mode,
        confidence, views=views, mosaic_cols=cols,
    )
    mark("start")
    nat.check(
        lib.gs_project_views(
            ptr(mean), ptr(rotation), ptr(scale), ptr(opacity), ptr(color), n, color.shape[1],
            ptr(cam_r), ptr(cam_t), ptr(intr), project_view,
            ptr(projected_mean), ptr(inverse_covariance), ptr(projected_color),
            ptr(projected_opacity), ptr(bounds), ptr(counts), ptr(records), ptr(depth_keys),
            ptr(tile_rects), stream,
        ),
        "project_views",
    )
    mark("project")
    flat_counts = counts.view(vn)
    # The backward's [V N, 9] gradient accumulator, zeroed beside the depth
    # sort (on the binning's side stream) instead of on the stream later.
    accumulator = (torch.empty((vn, 9), dtype=torch.float32, device=device)
                   if bucketing and record_hits and rendering_mode == "gaussian" else None)
    if bucketing:
        gaussian_ids, ranges = bin_tiles(
            depth_keys, None, None, canvas_w, canvas_h, timer=mark, tile_rects=tile_rects,
            clear=accumulator, key_range=depth_key_range(near, far),
        )
    else:
        flat_bounds = bounds.view(vn, 2, 2)
        order, offsets = bin_gaussians(depth_keys, flat_counts)
        mark("bin")
        total = int(offsets[vn].item()) if vn else 0
        nat.check_device_errors(device)  # the depth sort and scan, now that the stream is idle
        tile_keys, ids = emit_tiles(flat_bounds, order, offsets, total, canvas_w)
        mark("emit")
        gaussian_ids, ranges = sort_tiles(tile_keys, ids, canvas_w * canvas_h)
    mark("sort")
    image = torch.empty((views, image_height, image_width, 3), dtype=torch.float32, device=device)
    final_transmittance = torch.empty(
        (views, image_height, image_width), dtype=torch.float32, device=device
    )
    n_contributors = torch.empty((views, image_height, image_width), dtype=torch.int32, device=device)
    view = _mosaic_view(
        image_width, image_height, tile_size, views, cols, rendering_mode=rendering_mode,
        confidence=confidence, opacity_threshold=opacity_threshold,
        active_tiles=nat.active_tiles(ranges),
    )
    checkpoints = nat.checkpoint_buffer(view, gaussian_ids.numel(), nat.longest_list(ranges),
                                        device)
    # With long lists the longest walks start first (as composite does).
    plan = (nat.dispatch_plan(view, ranges.shape[0], device, ranges=ranges)
            if checkpoints is not None else None)
    hits = (nat.hit_mask_buffer(view, gaussian_ids.numel(), device)
            if record_hits and rendering_mode == "gaussian" else None)
    nat.check(
        lib.gs_composite(
            ptr(records), records.shape[0], ptr(gaussian_ids), gaussian_ids.numel(), ptr(ranges),
            ptr(plan), view, ptr(image), ptr(final_transmittance), ptr(n_contributors),
            ptr(checkpoints), nat.buffer_bytes(checkpoints), ptr(hits), nat.buffer_bytes(hits),
            None, 0, stream,
        ),
        "composite",
    )
    nat.set_walk_state(n_contributors, None, checkpoints, hits)
    if accumulator is not None:
        nat.set_forward_buffer(n_contributors, "grad_accumulator", accumulator)
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


@torch.library.custom_op("gaussian_splats_hip::rasterize_views", mutates_args=())
def _rasterize_views(
    mean: torch.Tensor,
    rotation: torch.Tensor,
    scale: torch.Tensor,
    opacity: torch.Tensor,
    color: torch.Tensor,
    camera_rotations: torch.Tensor,
    camera_translations: torch.Tensor,
    intrinsics: torch.Tensor,
    image_width: int,
    image_height: int,
    tile_size: int,
    opacity_threshold: float,
    near: float,
    far: float,
    rendering_mode: str,
    confidence: float,
) -> tuple[
    torch.Tensor,  # image [V, H, W, 3]
    torch.Tensor,  # final_transmittance [V, H, W]
    torch.Tensor,  # n_contributors [V, H, W]
    torch.Tensor,  # projected_mean [V, N, 3]
    torch.Tensor,  # inverse_covariance [V, N, 2, 2]
    torch.Tensor,  # projected_color [V, N, 3]
    torch.Tensor,  # projected_opacity [V, N, 1]
    torch.Tensor,  # gaussian_ids (virtual indices v * N + i)
    torch.Tensor,  # ranges [mosaic tiles, 2]
    torch.Tensor,  # counts [V, N]
]:
    return forward_views(
        mean, rotation, scale, opacity, color, camera_rotations, camera_translations, intrinsics,
        image_width, image_height, tile_size, opacity_threshold, near, far, rendering_mode,
        confidence, timer=stage_timer(),
    )


@_rasterize_views.register_fake
def _rasterize_views_fake(
    mean, rotation, scale, opacity, color, camera_rotations, camera_translations, intrinsics,
    image_width, image_height, tile_size, opacity_threshold, near, far, rendering_mode,
    confidence,
):
    dynamic = torch.library.get_ctx().new_dynamic_size()
    views = camera_rotations.shape[0]
    tw, th = nat.tiles(image_width, image_height, tile_size)
    cols = mosaic_columns(views, tw, th)
    rows = -(-views // cols)
    n = mean.shape[0]
    dev = mean.device
    return (
        mean.new_empty((views, image_height, image_width, 3)),
        mean.new_empty((views, image_height, image_width)),
        torch.empty((views, image_height, image_width), dtype=torch.int32, device=dev),
        mean.new_empty((views, n, 3)),
        mean.new_empty((views, n, 2, 2)),
        mean.new_empty((views, n, 3)),
        mean.new_empty((views, n, 1)),
        torch.empty((dynamic,), dtype=torch.int32, device=dev),
        torch.empty((cols * tw * rows * th, 2), dtype=torch.int64, device=dev),
        torch.empty((views, n), dtype=torch.int32, device=dev),
    )


@torch.compiler.disable
def _backward_plan(view, ranges, n_contributors) -> torch.Tensor:
    """The backward's dispatch plan, computed eagerly (also under
    torch.compile, which cannot trace the C-ABI call)."""
    return nat.dispatch_plan(view, ranges.shape[0], ranges.device, ranges=ranges,
                             n_contributors=n_contributors)


def _setup_context(ctx, inputs, output) -> None:
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(*inputs[:5], *output[1:])
    (
        ctx.camera_rotations,
        ctx.camera_translations,
        ctx.intrinsics,
    ) = inputs[5:8]
    (
        ctx.image_width,
        ctx.image_height,
        ctx.tile_size,
        ctx.opacity_threshold,
        ctx.near,
        ctx.far,
        ctx.rendering_mode,
        ctx.confidence,
    ) = inputs[8:]
    ctx.active_tiles = nat.active_tiles(output[8])
    ctx.checkpoints, ctx.hit_masks = nat.walk_buffers(output[2])
    ctx.order = None
    if inputs[0].is_cuda and ctx.rendering_mode == "gaussian":
        # The backward's dispatch plan depends only on the forward's lists and
        # contributor counts: computed now, behind the forward on the stream.
        views = inputs[5].shape[0]
        tw, th = nat.tiles(ctx.image_width, ctx.image_height, ctx.tile_size)
        cols = mosaic_columns(views, tw, th)
        view = _mosaic_view(ctx.image_width, ctx.image_height, ctx.tile_size, views, cols,
                            opacity_threshold=ctx.opacity_threshold,
                            active_tiles=ctx.active_tiles)
        ctx.order = _backward_plan(view, output[8], output[2])


def backward_views(
    mean: torch.Tensor,
    rotation: torch.Tensor,
    scale: torch.Tensor,
    opacity: torch.Tensor,
    color: torch.Tensor,
    camera_rotations: torch.Tensor,
    camera_translations: torch.Tensor,
    intrinsics: torch.Tensor,
    image_width: int,
    image_height: int,
    tile_size: int,
    opacity_threshold: float,
    saved: Sequence[torch.Tensor],
    grad_image: torch.Tensor | None,
    timer=None,
    active_tiles: int | None = None,
    checkpoints: torch.Tensor | None = None,
    order: torch.Tensor | None = None,
    hit_masks: torch.Tensor | None = None,
) -> tuple[torch.Tensor, ...]:
    """composite_bwd over the mosaic -> project_bwd summed over the views.

    ``saved`` holds the forward's outputs 1..9 (transmittance through counts);
    returns the gradients of the five parameter tensors.  ``timer(name)``
    marks "composite_bwd" and "project_bwd".  ``active_tiles``: tiles with a
    non-empty list, ``checkpoints``: the forward's checkpoint buffer, and
    ``hit_masks``: its hit masks (defaults: those the forward recorded on its
    ``n_contributors`` output); ``order``: the dispatch plan of these lists and contributor
    counts (default: computed here)."""
    mark = timer or (lambda name: None)
    if active_tiles is None:
        active_tiles = nat.active_tiles(saved[7])
    if checkpoints is None and hit_masks is None:
        checkpoints, hit_masks = nat.walk_buffers(saved[1])
    mean, rotation, scale, opacity, color = (
        _contiguous(t) for t in (mean, rotation, scale, opacity, color)
    )
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
    ) = saved
    device = mean.device
    n = mean.shape[0]
    cam_r, cam_t, intr, views = _camera_arrays(camera_rotations, camera_translations, intrinsics)
    w, h, tile = image_width, image_height, tile_size
    tw, th = nat.tiles(w, h, tile)
    cols = mosaic_columns(views, tw, th)
    if grad_image is None:
        grad_image = torch.zeros((views, h, w, 3), dtype=torch.float32, device=device)
    else:
        grad_image = _contiguous(grad_image.float())
    lib = nat.library()
    stream = nat.stream(device)
    ptr = nat.ptr
    view = _mosaic_view(w, h, tile, views, cols, opacity_threshold=opacity_threshold,
                        active_tiles=active_tiles)
    grad_projected = nat.take_forward_buffer(saved[1], "grad_accumulator")
    if grad_projected is None:
        grad_projected = torch.zeros((views * n, 9), dtype=torch.float32, device=device)
    if order is None:
        order = nat.dispatch_plan(view, ranges.shape[0], device, ranges=ranges,
                                  n_contributors=n_contributors)
    nat.check(
        nat.launch(
            "composite_bwd",
            lambda: lib.gs_composite_bwd(
                ptr(projected_mean), ptr(inverse_covariance), ptr(projected_color),
                ptr(projected_opacity), projected_mean.numel() // 3, ptr(gaussian_ids),
                ptr(ranges), ptr(grad_image), ptr(final_transmittance), ptr(n_contributors),
                ptr(order), view, ptr(grad_projected), None, ptr(checkpoints),
                nat.buffer_bytes(checkpoints), gaussian_ids.numel(), ptr(hit_masks),
                nat.buffer_bytes(hit_masks), stream,
            ),
        ),
        "composite_bwd",
    )
    mark("composite_bwd")
    grads = tuple(torch.empty_like(t) for t in (mean, rotation, scale, opacity, color))
    if n:
        project_view = nat.make_view(0.0, 0.0, 0.0, 0.0, w, h, tile, views=views, mosaic_cols=cols)
        nat.check(
            lib.gs_project_bwd_views(
                ptr(mean), ptr(rotation), ptr(scale), ptr(opacity), ptr(color), n,
                color.shape[1], ptr(cam_r), ptr(cam_t), ptr(intr), project_view,
                ptr(inverse_covariance), ptr(grad_projected), ptr(counts),
                *(ptr(g) for g in grads), stream,
            ),
            "project_bwd_views",
        )
    mark("project_bwd")
    return grads


def _backward(ctx, *grad_outputs):
    if ctx.rendering_mode != "gaussian":
        raise AssertionError("Backward gradients are only supported for Gaussian rendering.")
    saved = ctx.saved_tensors
    grads = backward_views(
        *saved[:5], ctx.camera_rotations, ctx.camera_translations, ctx.intrinsics,
        ctx.image_width, ctx.image_height, ctx.tile_size, ctx.opacity_threshold, saved[5:],
        grad_outputs[0], active_tiles=ctx.active_tiles, checkpoints=ctx.checkpoints,
        order=ctx.order, hit_masks=ctx.hit_masks,
    )
    return (*grads, *(None,) * 11)


torch.library.register_autograd(
    "gaussian_splats_hip::rasterize_views", _backward, setup_context=_setup_context
)


class _RasterizeViewsFunction(torch.autograd.Function):
    """The multi-view op's forward and backward as an autograd.Function for
    eager calls (see _RasterizeFunction in interface.py)."""

    @staticmethod
    def forward(ctx, *inputs):
        output = forward_views(*inputs, timer=stage_timer())
        _setup_context(ctx, inputs, output)
        return output

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, *grad_outputs):
        return _backward(ctx, *grad_outputs)


def rasterize_views_outputs(*inputs) -> tuple[torch.Tensor, ...]:
    """The multi-view op's ten outputs for its 16 inputs: the registered op
    when traced, the equivalent autograd.Function when a gradient will be
    needed, else the forward alone."""
    if torch.compiler.is_compiling():
        return _rasterize_views(*inputs)
    if torch.is_grad_enabled() and any(t.requires_grad for t in inputs[:5]):
        return _RasterizeViewsFunction.apply(*inputs)
    return forward_views(*inputs, timer=stage_timer(), record_hits=False)


def camera_tensors(cameras: Sequence[Camera]) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int, int]:
    """Host-side camera arrays of ``rasterize_views``: rotations [V, 3, 3],
    translations [V, 3], intrinsics [V, 4] = (fx, fy, cx, cy), and the shared
    image size."""
    if not cameras:
        raise ValueError("rasterize_views needs at least one camera")
    sizes = {tuple(int(s) for s in cam.image_size) for cam in cameras}
    if len(sizes) != 1:
        raise ValueError(f"all cameras must share one image size, got {sorted(sizes)}")
    (width, height), = sizes
    from ...splats.camera import host_extrinsics  # the splat API imports this module

    extrinsics = [host_extrinsics(cam) for cam in cameras]
    rotations = torch.stack([r for r, _ in extrinsics])
    translations = torch.stack([t for _, t in extrinsics])
    intrinsics = torch.tensor(
        [[float(c) for c in (*cam.focal_length, *cam.principal_point)] for cam in cameras],
        dtype=torch.float32,
    )
    return rotations, translations, intrinsics, width, height


def rasterize_views(
    splats: GaussianSplat,
    cameras: Sequence[Camera],
    tile_size: int = 16,
    opacity_threshold: float = 0.999,
    near: float = 0.2,
    far: float = 100.0,
    rendering_mode: Literal["gaussian", "ellipsoid"] = "gaussian",
    confidence: float = 0.95,
    indices: torch.Tensor | None = None,
) -> torch.Tensor:
    """Renders ``splats`` seen by each of ``cameras`` (one image size) into a
    [V, H, W, 3] batch; the arguments are those of ``rasterize``."""
    _check_tile(tile_size)
    if rendering_mode not in ("gaussian", "ellipsoid"):
        raise ValueError(f"Invalid rendering mode: {rendering_mode}")
    rotations, translations, intrinsics, width, height = camera_tensors(cameras)
    params = (splats.mean, splats.rotation, splats.scale, splats.opacity, splats.color)
    if indices is not None:
        params = tuple(p[indices] for p in params)
    return rasterize_views_outputs(
        *params,
        rotations,
        translations,
        intrinsics,
        width,
        height,
        int(tile_size),
        float(opacity_threshold),
        float(near),
        float(far),
        rendering_mode,
        float(confidence),
    )[0]
