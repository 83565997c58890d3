"""Shared helpers of the parity tests: oracle adapters and flip-aware comparisons.

A "flip" is a discrete decision (alpha >= 1/255, 1 - T < threshold, o*G <= 0.99,
floor at a tile edge) that an ulp-level difference between two fp32 evaluations
can turn the other way.  The CPU oracle reports, per pixel, the relative
distance of every such decision from its threshold; pixels closer than
``MARGIN`` are compared against a looser bound and counted, everything else is
compared at the stated tolerance.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import rasterizer as orc

MARGIN = 1e-4  # relative distance below which a decision may legitimately flip


def oracle_camera(cam) -> orc.Camera:
    """The oracle's camera with the extrinsics the rasterizer passes its
    kernels (host_extrinsics: the values of cam.rotation_matrix)."""
    from gaussian_splats_hip.splats.camera import host_extrinsics

    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    r, t = host_extrinsics(cam)
    return orc.Camera(r, t, float(fx), float(fy), float(cx), float(cy), int(w), int(h))


def assert_close_flip_aware(actual, expected, margin, atol, rtol=0.0, loose=None, max_flagged=0.01, what=""):
    """|actual - expected| <= atol + rtol |expected| wherever ``margin >= MARGIN``;
    elsewhere (at most ``max_flagged`` of the pixels) only ``loose`` is enforced."""
    a = torch.as_tensor(actual).detach().double().cpu()
    e = torch.as_tensor(expected).detach().double().cpu()
    m = torch.as_tensor(margin).double().cpu()
    while m.dim() < a.dim():
        m = m[..., None]
    m = m.expand_as(a)
    ok = m >= MARGIN
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    bad = ok & (err > bound)
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {int(ok.sum())} well-conditioned values exceed "
        f"atol={atol} rtol={rtol}; max err {float(err[ok].max()):.3e} at "
        f"{np.unravel_index(int(torch.where(ok, err, 0).argmax()), a.shape)}"
    )
    flagged = float((~ok).double().mean())
    assert flagged <= max_flagged, f"{what}: {flagged:.4%} of values ill-conditioned"
    if loose is not None and bool((~ok).any()):
        worst = float(err[~ok].max())
        assert worst <= loose, f"{what}: ill-conditioned value off by {worst}"
    return {"max_err": float(err[ok].max()) if bool(ok.any()) else 0.0, "flagged": flagged}


def rect_flip_tolerant_equal(actual_bounds, expected_bounds, projected, tile_size, extent):
    """Bounds must match exactly except where the oracle's (u -/+ r) / tile lies
    within 1e-5 (relative) of an integer, i.e. where an ulp decides the floor."""
    a = np.asarray(actual_bounds)
    e = np.asarray(expected_bounds)
    diff = np.any(a != e, axis=(1, 2))
    if not diff.any():
        return 0
    u = projected.mean[:, 0].detach().double().numpy()
    v = projected.mean[:, 1].detach().double().numpy()
    rx = extent * np.sqrt(projected.covariance[:, 0, 0].detach().double().numpy())
    ry = extent * np.sqrt(projected.covariance[:, 1, 1].detach().double().numpy())
    edges = np.stack(((u - rx) / tile_size, (u + rx) / tile_size, (v - ry) / tile_size, (v + ry) / tile_size), -1)
    dist = np.abs(edges - np.round(edges)) / np.maximum(np.abs(edges), 1.0)
    near_edge = np.min(dist, axis=-1) < 1e-5
    unexplained = diff & ~near_edge
    assert not unexplained.any(), f"{int(unexplained.sum())} tile rectangles differ away from a tile edge: {np.nonzero(unexplained)[0][:10]}"
    return int(diff.sum())


# Gradient tolerance of the north star: 1e-4 relative, 1e-6 absolute.  The
# absolute term is 1e-6 * min(1, largest |gradient| of the column): never
# looser than 1e-6, and proportionally tighter for columns whose gradients are
# all small (mean losses over megapixel images).
GRAD_RTOL = 1e-4
GRAD_ATOL = 1e-6
# Relative distance from a threshold within which two float32 evaluations of
# the same alpha (different operation order, a few ulps apart) may decide the
# alpha cut or the 0.99 clamp differently.
DECISION_WINDOW = 4e-6


def assert_gradients_close(actual, expected, what, explained=None, max_explained=0.01):
    """Every row (Gaussian) of ``actual`` within GRAD_RTOL |e| + GRAD_ATOL
    min(1, max|e| of the column) of ``expected``.  Rows that fail must be
    ``explained`` (a bool [rows]: a cut or clamp decision of theirs, or of a
    pixel they reach, lies within DECISION_WINDOW of its threshold) and at
    most ``max_explained`` of the rows.  Returns statistics."""
    a = torch.as_tensor(actual).detach().double().cpu()
    e = torch.as_tensor(expected).detach().double().cpu()
    a2 = a.reshape(a.shape[0], -1)
    e2 = e.reshape(e.shape[0], -1)
    colmax = e2.abs().amax(0)
    bound = GRAD_RTOL * e2.abs() + GRAD_ATOL * colmax.clamp(max=1.0)
    excess = (a2 - e2).abs() / bound.clamp_min(1e-300)
    bad = (excess > 1).any(1)
    stats = {
        "rows": int(a2.shape[0]),
        "failing": int(bad.sum()),
        "worst_excess": float(excess.max()) if excess.numel() else 0.0,
        "median_rel": float(((a2 - e2).abs() / e2.abs().clamp_min(1e-30)).median()) if e2.numel() else 0.0,
    }
    if explained is None:
        assert not bool(bad.any()), (
            f"{what}: {int(bad.sum())} of {a2.shape[0]} rows off; worst {stats['worst_excess']:.2f}x "
            f"the bound at row {int(excess.amax(1).argmax())}"
        )
    else:
        ex = torch.as_tensor(explained).bool().cpu()
        unexplained = bad & ~ex
        assert not bool(unexplained.any()), (
            f"{what}: {int(unexplained.sum())} rows off with no decision near a threshold; worst "
            f"{float(excess[unexplained].max()):.2f}x at row {int(torch.nonzero(unexplained)[0])}"
        )
        frac = float(bad.double().mean()) if bad.numel() else 0.0
        assert frac <= max_explained, f"{what}: {frac:.3%} of rows off (all near a threshold)"
    return stats


def assert_lists_exact(gids, ranges, bounds, counts, depth, tiles_w, chunk=1 << 26):
    """Proves on the GPU (torch used as the checker) that ``gids``/``ranges`` are
    exactly the stable (tile, depth bits, index) sort of the intersections of
    the rectangles ``bounds`` [N, 2, 2] of the Gaussians with ``counts`` > 0:

    * per-tile lengths equal a 2-D histogram of those rectangles and ranges
      partition [0, I);
    * every entry's Gaussian is counted and its rectangle contains the tile;
    * within a tile, (depth bits, index) strictly increases.

    Strict increase rules out repeats, so each tile lists a subset of its
    covering Gaussians as large as the whole set: that set, in sorted order.
    Works at any size (the oracle's numpy sort of 5e8 keys would not)."""
    dev = gids.device
    n = counts.shape[0]
    num_tiles = ranges.shape[0]
    tiles_h = num_tiles // tiles_w
    b = bounds.reshape(n, 4).long()
    x0, x1, y0, y1 = b.unbind(1)
    on = counts > 0
    diff = torch.zeros((tiles_h + 1) * (tiles_w + 1), dtype=torch.int64, device=dev)
    stride = tiles_w + 1
    for yy, xx, sign in ((y0, x0, 1), (y0, x1, -1), (y1, x0, -1), (y1, x1, 1)):
        diff.index_add_(0, (yy * stride + xx)[on], torch.full_like(xx[on], sign))
    hist = diff.view(tiles_h + 1, tiles_w + 1).cumsum(0).cumsum(1)[:tiles_h, :tiles_w].reshape(-1)
    lengths = ranges[:, 1] - ranges[:, 0]
    assert torch.equal(lengths, hist), "per-tile list lengths differ from the rectangles' histogram"
    assert int(ranges[0, 0]) == 0 and int(ranges[-1, 1]) == gids.numel()
    assert torch.equal(ranges[1:, 0], ranges[:-1, 1]), "ranges do not partition the entries"
    bits = depth.contiguous().view(torch.int32).long()
    assert bool((bits[on] >= 0).all()), "counted Gaussians must have positive depths"
    total = gids.numel()
    ends = ranges[:, 1].contiguous()
    prev_key = prev_tile = None
    for s0 in range(0, total, chunk):
        e = torch.arange(s0, min(total, s0 + chunk), device=dev)
        tile = torch.searchsorted(ends, e, right=True)
        g = gids[s0:s0 + e.numel()].long()
        assert bool(((g >= 0) & (g < n)).all()), "Gaussian id out of range"
        assert bool(on[g].all()), "an uncounted Gaussian is listed"
        tx, ty = tile % tiles_w, tile // tiles_w
        inside = (x0[g] <= tx) & (tx < x1[g]) & (y0[g] <= ty) & (ty < y1[g])
        assert bool(inside.all()), "an entry's rectangle does not contain its tile"
        key = (bits[g] << 32) | g
        if prev_key is not None:
            key = torch.cat((prev_key, key))
            tile = torch.cat((prev_tile, tile))
        same = tile[1:] == tile[:-1]
        assert bool((key[1:][same] > key[:-1][same]).all()), "a tile's list is not strictly sorted"
        prev_key, prev_tile = key[-1:], tile[-1:]
    return {"intersections": int(total), "tiles": int(num_tiles)}


def sample_tiles(ranges, count=32, longest=4, seed=0):
    """The ``longest`` tiles with the longest lists plus seeded random other
    non-empty tiles, ``count`` in all, sorted."""
    r = np.asarray(ranges)
    lengths = r[:, 1] - r[:, 0]
    top = np.argsort(-lengths, kind="stable")[:longest]
    rest = np.setdiff1d(np.nonzero(lengths > 0)[0], top)
    rng = np.random.default_rng(seed)
    extra = rng.choice(rest, size=min(len(rest), count - len(top)), replace=False)
    return np.sort(np.concatenate((top, extra)))


def oracle_tile_lists(bounds, counts, depth32, tiles, tiles_w, num_tiles, limits=None):
    """The oracle's lists of ``tiles`` only (every other tile empty): the
    counted Gaussians whose rectangle contains the tile, by (depth bits,
    index), each cut at ``limits[tile]`` entries when given.  Returns (ids,
    ranges [num_tiles, 2])."""
    b = np.asarray(bounds)
    bits = np.ascontiguousarray(depth32, dtype=np.float32).view(np.uint32)
    on = np.asarray(counts) > 0
    ids, ranges, pos = [], np.zeros((num_tiles, 2), dtype=np.int64), 0
    for t in sorted(int(t) for t in tiles):
        tx, ty = t % tiles_w, t // tiles_w
        hit = on & (b[:, 0, 0] <= tx) & (tx < b[:, 0, 1]) & (b[:, 1, 0] <= ty) & (ty < b[:, 1, 1])
        idx = np.nonzero(hit)[0]
        idx = idx[np.lexsort((idx, bits[idx]))]
        if limits is not None:
            idx = idx[: int(limits[t])]
        ids.append(idx.astype(np.int32))
        ranges[t] = (pos, pos + len(idx))
        pos += len(idx)
    return (np.concatenate(ids) if ids else np.zeros(0, np.int32)), ranges


def restrict_lists(gids, ranges, tiles, limits=None):
    """The given lists (numpy) with every tile outside ``tiles`` emptied and
    each kept tile cut at ``limits[tile]`` entries; compacted."""
    gids = np.asarray(gids)
    r = np.asarray(ranges)
    out_ids, out = [], np.zeros_like(r)
    pos = 0
    for t in sorted(int(t) for t in tiles):
        s, e = int(r[t, 0]), int(r[t, 1])
        if limits is not None:
            e = min(e, s + int(limits[t]))
        out_ids.append(gids[s:e])
        out[t] = (pos, pos + e - s)
        pos += e - s
    return (np.concatenate(out_ids) if out_ids else np.zeros(0, np.int32)), out


def tile_pixel_mask(tiles, tiles_w, tile_size, width, height):
    """[H, W] bool: pixels of the given tiles."""
    m = np.zeros((-(-height // tile_size) * tile_size, tiles_w * tile_size), dtype=bool)
    for t in tiles:
        tx, ty = int(t) % tiles_w, int(t) // tiles_w
        m[ty * tile_size:(ty + 1) * tile_size, tx * tile_size:(tx + 1) * tile_size] = True
    return m[:height, :width]


def tile_max(values_hw, tiles, tiles_w, tile_size):
    """Per tile, the largest value of an [H, W] array over the tile's pixels
    (dict tile -> int)."""
    v = np.asarray(values_hw)
    out = {}
    for t in tiles:
        tx, ty = int(t) % tiles_w, int(t) // tiles_w
        out[int(t)] = int(v[ty * tile_size:(ty + 1) * tile_size, tx * tile_size:(tx + 1) * tile_size].max())
    return out
