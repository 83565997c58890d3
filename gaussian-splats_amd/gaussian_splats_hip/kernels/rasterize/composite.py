"""Forward tile compositing (HIP: gs_composite).

Same launcher contract as the reference's
src/gaussian_splats/kernels/rasterize/composite.py:110-162, except that image
sizes need not be multiples of the tile size (edge tiles are masked).
"""

from __future__ import annotations

import torch

from . import _native as nat
from .project import _check_tile, pack_records


def tile_order(
    ranges: torch.Tensor | None,
    n_contributors: torch.Tensor | None,
    image_width: int,
    image_height: int,
    tile_size: int,
    active_tiles: int = 0,
) -> torch.Tensor:
    """Dispatch plan of the compositing kernels (gs_tile_order) for one view:
    work items (``tile << 7`` for a whole tile, ``tile << 7 | 0x20 | q`` for
    quarter ``q`` of its pixel bands, ``tile << 7 | 0x40 | s`` for segment
    ``s`` of a backward walk, -1 unused) that keep each XCD's region of tiles
    and start the longest expected work first.  The estimate is the list length from ``ranges``
    (the forward) or the largest contributor count per tile from
    ``n_contributors`` (the backward).  ``active_tiles`` must be the value the
    compositing call's view carries."""
    source = n_contributors if n_contributors is not None else ranges
    if source is None:
        raise ValueError("tile_order needs ranges or n_contributors")
    device = nat.require_gpu(source)
    tiles_w, tiles_h = nat.tiles(image_width, image_height, tile_size)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, image_width, image_height, tile_size,
                         active_tiles=active_tiles)
    return nat.dispatch_plan(view, tiles_w * tiles_h, device, ranges=ranges,
                             n_contributors=n_contributors)


def composite(
    mean: torch.Tensor,
    inverse_covariance: torch.Tensor,
    color: torch.Tensor,
    opacity: torch.Tensor,
    gaussian_ids: torch.Tensor,
    ranges: torch.Tensor,
    image_width: int,
    image_height: int,
    tile_size: int,
    opacity_threshold: float,
    rendering_mode: str,
    confidence: float,
    *,
    records: torch.Tensor | None = None,
    order: torch.Tensor | None = None,
    record_hits: bool = True,
    tile_keys: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Composites the sorted per-tile lists; returns ``(image[H,W,3],
    final_transmittance[H,W], n_contributors[H,W] int32)``.  The walk's
    checkpoints and (``record_hits``, Gaussian mode) hit masks (gs_composite)
    are recorded on the returned ``n_contributors`` with a fingerprint of
    this call's arguments; ``composite_bwd`` uses them only when its own
    arguments carry the same fingerprint.  ``tile_keys`` (optional, a
    gs_tile_order workspace) receives the backward plan's keys as the walks
    end (gs_composite's tile_keys)."""
    _check_tile(tile_size)
    device = nat.require_gpu(mean, gaussian_ids, ranges)
    if records is None:
        records = pack_records(mean, inverse_covariance, color, opacity, rendering_mode, confidence)
    tiles_w, tiles_h = nat.tiles(image_width, image_height, tile_size)
    if ranges.shape != (tiles_w * tiles_h, 2):
        raise ValueError(f"ranges must be [{tiles_w * tiles_h}, 2], got {tuple(ranges.shape)}")
    active = nat.active_tiles(ranges)
    ranges_in, gaussian_ids_in = ranges, gaussian_ids
    ranges = nat.prepare(ranges, torch.int64)
    gaussian_ids = nat.prepare(gaussian_ids, torch.int32)
    image = torch.empty((image_height, image_width, 3), dtype=torch.float32, device=device)
    final_transmittance = torch.empty((image_height, image_width), dtype=torch.float32, device=device)
    n_contributors = torch.empty((image_height, image_width), dtype=torch.int32, device=device)
    view = nat.make_view(
        1.0, 1.0, 0.0, 0.0, image_width, image_height, tile_size, rendering_mode=rendering_mode,
        confidence=confidence, opacity_threshold=opacity_threshold, active_tiles=active,
    )
    checkpoints = nat.checkpoint_buffer(view, gaussian_ids.numel(), nat.longest_list(ranges_in),
                                        device)
    if order is None and checkpoints is not None:
        # Long lists (above 8192 entries): more tiles than resident waves, and
        # the kernel's span is the longest walk, so the longest lists start
        # first (config 4: 0.90 -> 0.83 ms).
        order = nat.dispatch_plan(view, tiles_w * tiles_h, device, ranges=ranges)
    hits = (nat.hit_mask_buffer(view, gaussian_ids.numel(), device)
            if record_hits and rendering_mode == "gaussian" else None)
    nat.check(
        nat.launch("composite", lambda: nat.library().gs_composite(
            nat.ptr(records), records.shape[0], nat.ptr(gaussian_ids), gaussian_ids.numel(),
            nat.ptr(ranges), nat.ptr(order), view, nat.ptr(image), nat.ptr(final_transmittance),
            nat.ptr(n_contributors), nat.ptr(checkpoints), nat.buffer_bytes(checkpoints),
            nat.ptr(hits), nat.buffer_bytes(hits), nat.ptr(tile_keys),
            nat.buffer_bytes(tile_keys), nat.stream(device),
        )),
        "composite",
    )
    # The backward of this walk starts its segment walks at the checkpoints
    # and walks the entries the hit masks mark.
    nat.set_walk_state(
        n_contributors,
        walk_key(image_width, image_height, tile_size, opacity_threshold, rendering_mode,
                 mean, inverse_covariance, color, opacity, gaussian_ids_in, ranges_in,
                 final_transmittance, n_contributors),
        checkpoints, hits,
    )
    return image, final_transmittance, n_contributors


def walk_key(image_width, image_height, tile_size, opacity_threshold, rendering_mode, mean,
             inverse_covariance, color, opacity, gaussian_ids, ranges, final_transmittance,
             n_contributors) -> tuple:
    """The fingerprint shared by ``composite`` and ``composite_bwd``."""
    return nat.walk_fingerprint(
        (int(image_width), int(image_height), int(tile_size), float(opacity_threshold),
         str(rendering_mode)),
        mean, inverse_covariance, color, opacity, gaussian_ids, ranges, final_transmittance,
        n_contributors,
    )
