"""Tile-intersection emission and ordering (HIP).

``emit_intersections`` / ``sort_intersections`` keep the contract of the
reference's src/gaussian_splats/kernels/rasterize/intersections.py:44-88
(64-bit keys ``tile_id << 32 | depth bits`` in Gaussian order, then a sort and
half-open per-tile ranges), with the sort made stable so depth ties keep
ascending Gaussian index.  ``bin_gaussians`` / ``emit_tiles`` / ``sort_tiles``
are the fused variant: Gaussians are ordered by (depth bits, index) once,
intersections are emitted in that order with 32-bit tile keys, and a stable
sort on the tile bits alone yields the same ids and ranges.  ``bin_tiles`` is
what the op uses for grids of at most 256 x 256 tiles: the same ids and ranges
with the row and column buckets filled straight from the tile rectangles.
"""

from __future__ import annotations

from ctypes import c_void_p

import numpy as np
import torch

from . import _native as nat


def emit_intersections(
    bounds: torch.Tensor,
    depths: torch.Tensor,
    counts: torch.Tensor,
    tiles_w: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Emits packed ``(tile ID, depth)`` keys and their Gaussian IDs, Gaussian-major."""
    device = nat.require_gpu(bounds, depths, counts)
    if depths.dtype != torch.float32:
        raise TypeError(f"depths must be float32, got {depths.dtype}")
    bounds = nat.prepare(bounds, torch.int32)
    counts = nat.prepare(counts, torch.int32)
    n = counts.shape[0]
    if depths.dim() != 1:
        raise ValueError("depths must be one-dimensional")
    if depths.stride(0) < 1 or depths.data_ptr() % 4:
        depths = depths.contiguous()
    lib = nat.library()
    offsets = torch.empty(n + 1, dtype=torch.int64, device=device)
    ws = nat.workspace(lib.gs_scan_workspace_bytes(n), device)
    s = nat.stream(device)
    nat.check(lib.gs_scan_counts(nat.ptr(counts), n, nat.ptr(offsets), nat.ptr(ws), ws.numel(), s), "scan_counts")
    total = int(offsets[n].item())
    nat.check_device_errors(device)  # the scan's look-back, now that the stream is idle
    keys = torch.empty(total, dtype=torch.int64, device=device)
    gaussian_ids = torch.empty(total, dtype=torch.int32, device=device)
    if n and total:
        nat.check(
            lib.gs_emit_intersections(
                nat.ptr(bounds), nat.ptr(depths), depths.stride(0), nat.ptr(offsets), n, total, tiles_w,
                nat.ptr(keys), nat.ptr(gaussian_ids), s,
            ),
            "emit_intersections",
        )
    return keys, gaussian_ids


def sort_intersections(
    keys: torch.Tensor, gaussian_ids: torch.Tensor, num_tiles: int
) -> tuple[torch.Tensor, torch.Tensor]:
    """Stable sort by key; returns the sorted Gaussian IDs and int64 ranges [T, 2]."""
    device = nat.require_gpu(keys, gaussian_ids)
    keys = nat.prepare(keys, torch.int64).clone()
    ids = nat.prepare(gaussian_ids, torch.int32).clone()
    total = keys.shape[0]
    lib = nat.library()
    sorted_ids = torch.empty(total, dtype=torch.int32, device=device)
    ranges = torch.empty((num_tiles, 2), dtype=torch.int64, device=device)
    ws = nat.workspace(lib.gs_sort_workspace_bytes(total, num_tiles), device)
    nat.check(
        lib.gs_sort_intersections(
            nat.ptr(keys), nat.ptr(ids), total, num_tiles, nat.ptr(sorted_ids), nat.ptr(ranges),
            nat.ptr(ws), ws.numel(), nat.stream(device),
        ),
        "sort_intersections",
    )
    return sorted_ids, ranges


def bin_gaussians(
    depth_keys: torch.Tensor, counts: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Orders Gaussians by (depth bits, index) and scans their counts in that order.

    ``depth_keys`` (int32 view of the u32 keys written by the projection) is consumed.
    Returns ``(order[N] int32, offsets[N + 1] int64)``; ``offsets[N]`` is the total.
    """
    device = nat.require_gpu(depth_keys, counts)
    n = counts.shape[0]
    lib = nat.library()
    order = torch.empty(n, dtype=torch.int32, device=device)
    offsets = torch.empty(n + 1, dtype=torch.int64, device=device)
    ws = nat.workspace(lib.gs_bin_workspace_bytes(n), device)
    nat.check(
        lib.gs_bin_gaussians(
            nat.ptr(depth_keys), nat.ptr(counts), n, nat.ptr(order), nat.ptr(offsets), nat.ptr(ws),
            ws.numel(), nat.stream(device),
        ),
        "bin_gaussians",
    )
    return order, offsets


def emit_tiles(
    bounds: torch.Tensor, order: torch.Tensor, offsets: torch.Tensor, total: int, tiles_w: int
) -> tuple[torch.Tensor, torch.Tensor]:
    """Emits (tile key, Gaussian id) pairs in depth order."""
    device = nat.require_gpu(bounds, order, offsets)
    n = order.shape[0]
    tile_keys = torch.empty(total, dtype=torch.int32, device=device)
    ids = torch.empty(total, dtype=torch.int32, device=device)
    if n and total:
        nat.check(
            nat.library().gs_emit_tiles(
                nat.ptr(bounds), nat.ptr(order), nat.ptr(offsets), n, total, tiles_w, nat.ptr(tile_keys),
                nat.ptr(ids), nat.stream(device),
            ),
            "emit_tiles",
        )
    return tile_keys, ids


def sort_tiles(
    tile_keys: torch.Tensor, ids: torch.Tensor, num_tiles: int
) -> tuple[torch.Tensor, torch.Tensor]:
    """Stable sort of depth-ordered pairs by tile; consumes both inputs."""
    device = nat.require_gpu(tile_keys, ids)
    total = tile_keys.shape[0]
    lib = nat.library()
    sorted_ids = torch.empty(total, dtype=torch.int32, device=device)
    ranges = torch.empty((num_tiles, 2), dtype=torch.int64, device=device)
    ws = nat.workspace(lib.gs_sort_workspace_bytes(total, num_tiles), device)
    nat.check(
        lib.gs_sort_tiles(
            nat.ptr(tile_keys), nat.ptr(ids), total, num_tiles, nat.ptr(sorted_ids), nat.ptr(ranges),
            nat.ptr(ws), ws.numel(), nat.stream(device),
        ),
        "sort_tiles",
    )
    return sorted_ids, ranges


MAX_BUCKET_TILES = 256
# Row/column bucketing takes fewer Gaussians than this (the row pass's
# look-back packs a row's entry count into 26 bits).
MAX_BUCKET_GAUSSIANS = 1 << 26


def bucketing_fits(n: int, tiles_w: int, tiles_h: int) -> bool:
    """Whether bin_tiles takes n Gaussians on a tiles_w x tiles_h grid."""
    return tiles_w <= MAX_BUCKET_TILES and tiles_h <= MAX_BUCKET_TILES and n < MAX_BUCKET_GAUSSIANS


def depth_key_range(near: float, far: float) -> tuple[int, int]:
    """(key_base, key_bits) of gs_bin_tiles_plan for depth keys of the
    projection with these clipping planes: every counted Gaussian's depth d
    satisfies near < d < far (float32), so its key (the bits of d) minus the
    bits of near lies in [1, bits(far) - bits(near)), below 2^key_bits - 1,
    the value culled keys map to.  (0, 32) (the keys' own 32 bits) unless
    0 < near < far < inf."""
    n32, f32 = np.float32(near), np.float32(far)
    if not (0.0 < n32 < f32 < np.inf):
        return 0, 32
    base = int(n32.view(np.uint32))
    span = int(f32.view(np.uint32)) - base
    bits = span.bit_length()
    return (base, bits) if bits < 32 else (0, 32)


def bin_tiles(
    depth_keys: torch.Tensor,
    bounds: torch.Tensor | None,
    counts: torch.Tensor | None,
    tiles_w: int,
    tiles_h: int,
    timer=None,
    *,
    tile_rects: torch.Tensor | None = None,
    clear: torch.Tensor | None = None,
    key_range: tuple[int, int] = (0, 32),
) -> tuple[torch.Tensor, torch.Tensor]:
    """Sorted Gaussian ids and int64 ranges [T, 2] by row/column bucketing.

    Equivalent to ``bin_gaussians`` + ``emit_tiles`` + ``sort_tiles`` for grids of
    at most ``MAX_BUCKET_TILES`` tiles per axis and fewer than
    ``MAX_BUCKET_GAUSSIANS`` Gaussians (``bucketing_fits``); ``depth_keys`` is
    consumed.  The rectangles come from ``tile_rects`` (the projection's packed
    rectangles, as the op passes them; ``bounds`` and ``counts`` are then
    unused) or are packed here from ``bounds`` and ``counts``.  ``clear``
    (optional, a contiguous float32 or int32 tensor on the device) is zeroed
    beside the depth sort, on the side stream, before the call returns (the
    op's gradient accumulator).  ``key_range`` = (key_base, key_bits) of the
    depth sort (``depth_key_range``; the default sorts the keys' 32 bits).
    ``timer(name)`` (optional) marks the end of the plan ("bin") and of the
    bucketing passes ("emit").
    """
    mark = timer or (lambda name: None)
    lib = nat.library()
    if tile_rects is None:
        device = nat.require_gpu(depth_keys, bounds, counts)
        n = counts.shape[0]
        bounds = nat.prepare(bounds, torch.int32)
        counts = nat.prepare(counts, torch.int32)
        tile_rects = torch.empty(n, dtype=torch.int32, device=device)
        nat.check(
            lib.gs_pack_tile_rects(nat.ptr(bounds), nat.ptr(counts), n, tiles_w, tiles_h,
                                   nat.ptr(tile_rects), nat.stream(device)),
            "pack_tile_rects",
        )
    else:
        device = nat.require_gpu(depth_keys, tile_rects)
        n = tile_rects.shape[0]
    s = nat.stream(device)
    plan = nat.workspace(lib.gs_bin_tiles_plan_bytes(n, tiles_w, tiles_h), device)
    ranges = torch.empty((tiles_w * tiles_h, 2), dtype=torch.int64, device=device)
    totals = torch.empty(4, dtype=torch.int64, device=device)
    # The one device-to-host read of the path: the totals size the id buffer
    # (the reference reads counts.sum() at intersections.py:51).  The call
    # returns once they are in host_totals, while the depth sort still runs;
    # the fifth word's low half is the device's sticky check-failure word.
    host_totals = torch.zeros(5, dtype=torch.int64, pin_memory=True)
    nat.check(
        lib.gs_bin_tiles_plan(
            nat.ptr(depth_keys), nat.ptr(tile_rects), n, int(key_range[0]), int(key_range[1]),
            tiles_w, tiles_h,
            nat.ptr(ranges), nat.ptr(totals), c_void_p(host_totals.data_ptr()), nat.ptr(plan),
            plan.numel(), nat.ptr(clear), nat.buffer_bytes(clear), s,
        ),
        "bin_tiles_plan",
    )
    mark("bin")
    total, row_entries, blocks, tiles_word, flags = host_totals.tolist()
    if flags:
        nat.device_errors(device, clear=True)  # report each failure once
        nat.raise_device_flags(flags, "bin_tiles")
    # Tiles with a non-empty list (low half) and the longest list (high half).
    nat.set_active_tiles(ranges, tiles_word & 0xFFFFFFFF)
    nat.set_longest_list(ranges, tiles_word >> 32)
    sorted_ids = torch.empty(total, dtype=torch.int32, device=device)
    if total:
        ws = nat.workspace(
            lib.gs_bin_tiles_emit_bytes(n, total, row_entries, blocks, tiles_w, tiles_h), device
        )
        nat.check(
            lib.gs_bin_tiles_emit(
                n, tiles_w, tiles_h, nat.ptr(totals), total,
                row_entries, blocks, nat.ptr(plan), plan.numel(), nat.ptr(ranges),
                nat.ptr(sorted_ids), nat.ptr(ws), ws.numel(), s,
            ),
            "bin_tiles_emit",
        )
    mark("emit")
    return sorted_ids, ranges
