"""Shared helpers of the parity tests: oracle adapters and flip-aware comparisons.

A "flip" is a discrete decision (alpha >= 1/255, 1 - T < threshold, o*G <= 0.99,
floor at a tile edge) that an ulp-level difference between two fp32 evaluations
can turn the other way.  The CPU oracle reports, per pixel, the relative
distance of every such decision from its threshold; pixels closer than
``MARGIN`` are compared against a looser bound and counted, everything else is
compared at the stated tolerance.
"""

from __future__ import annotations

import math

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


def assert_forward_every_pixel(image, final_t, ncon, cols32, ids, ranges, width, height,
                               tile_size, mask=None, threshold=0.999, atol=1e-5, t_rtol=1e-4,
                               tile_chunk=64, max_multi=0.005, rendering_mode="gaussian",
                               confidence=0.95, what=""):
    """Bounds every pixel of a GPU forward, those near a decision included.

    The float64 oracle composites the GPU's own projected values ``cols32``
    (u, v, inv00, inv01, inv11, rgb [N, 3], alpha0) along the GPU's lists with
    the GPU's activity decisions (``ncon``) and the float32 oracle's cut and
    clamp decisions (run A).  The GPU image must match run A within ``atol``
    (transmittance: + ``t_rtol`` relative) on every pixel of ``mask``.

    The exception is an entry whose alpha-cut decision lies within
    orc.CUT_NEAR of 1/255 (ellipsoid mode: also the indicator D <= cutoff).
    The GPU may keep or drop it differently from the float32 oracle.  Run B
    flips every such (entry, pixel) decision of run A.  A pixel with one
    such entry must match run A or run B at the same tolerance.  A pixel with
    several (at most ``max_multi`` of the pixels) is bounded by run A plus
    their count times the most one entry changes: keeping or dropping an
    entry of alpha a changes the pixel by a * (T rgb + colour after it) <= 2 a
    max(rgb) and the transmittance by a * T <= a, with a = 1/255 at the cut
    (ellipsoid: a <= min(max alpha0, 0.99)).  Returns statistics."""
    cols32 = [torch.as_tensor(c).detach().float().cpu() for c in cols32]
    ids = np.asarray(ids)
    ranges = np.asarray(ranges)
    ncon = np.asarray(torch.as_tensor(ncon).cpu())
    run32 = orc.composite(*cols32, ids, ranges, width, height, tile_size, threshold,
                          rendering_mode, confidence, tile_chunk=tile_chunk)
    cols64 = [c.double() for c in cols32]

    def run64(decisions):
        return orc.composite(*cols64, ids, ranges, width, height, tile_size, threshold,
                             rendering_mode, confidence, tile_chunk=tile_chunk,
                             decisions=decisions, active_counts=ncon)

    run_a = run64(run32.decisions)
    flipped = {t0: (keep ^ run_a.near_pairs[t0], clamped)
               for t0, (keep, clamped) in run32.decisions.items()}
    run_b = run64(flipped)
    m = (torch.ones(height, width, dtype=torch.bool) if mask is None
         else torch.as_tensor(mask).bool().cpu())
    near = run_a.cut_near
    img = torch.as_tensor(image).detach().double().cpu()
    t = torch.as_tensor(final_t).detach().double().cpu()

    def errors(run):
        e_img = (img - run.image.double()).abs().amax(-1)
        t64 = run.final_transmittance.double()
        e_t = (t - t64).abs()
        return e_img, e_t, atol + t_rtol * t64.abs()

    ea, ta, tba = errors(run_a)
    eb, tb, tbb = errors(run_b)
    fits_a = (ea <= atol) & (ta <= tba)
    fits_b = (eb <= atol) & (tb <= tbb)
    single = near <= 1
    bad = m & single & ~(fits_a | (fits_b & (near == 1)))
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {int(m.sum())} pixels match neither decision; worst image "
        f"error {float(torch.where(bad, torch.minimum(ea, eb), 0).max()):.3e} at "
        f"{np.unravel_index(int(torch.where(bad, torch.minimum(ea, eb), 0).argmax()), ea.shape)}")
    multi = m & ~single
    max_rgb = float(cols32[5].abs().max()) if cols32[5].numel() else 0.0
    if rendering_mode == "ellipsoid":
        flip = min(float(cols32[6].max()) if cols32[6].numel() else 0.0, orc.MAX_ALPHA)
    else:
        flip = orc.MIN_ALPHA
    flip *= 1 + 1e-5
    k = near.double()
    loose_bad = multi & ((ea > atol + k * 2 * max_rgb * flip) | (ta > tba + k * flip))
    assert not bool(loose_bad.any()), f"{what}: {int(loose_bad.sum())} pixels exceed their bound"
    frac = float(multi.double().sum() / max(int(m.sum()), 1))
    assert frac <= max_multi, f"{what}: {frac:.3%} of pixels have several cut decisions near 1/255"
    took_b = m & single & ~fits_a
    stats = {
        "pixels": int(m.sum()),
        "one_near_cut": int((m & (near == 1)).sum()),
        "matched_flipped": int(took_b.sum()),
        "several_near_cuts": int(multi.sum()),
        "max_err": float(torch.where(m & single & fits_a, ea, 0).max()),
        "max_err_several": float(ea[multi].max()) if bool(multi.any()) else 0.0,
    }
    print(f"[{what}] every pixel: {stats}", flush=True)
    return stats


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


def _rows(x):
    x = torch.as_tensor(x).detach().double().cpu()
    return x.reshape(x.shape[0], -1)


# A row may instead be within FLOAT32_FACTOR times the float32 restatement's
# error scale on that row: the largest error of FLOAT32_SAMPLES float32
# evaluations (the plain one and ones with every input moved by one ulp in a
# random direction; the last half of the compositing ones form the
# transmittance as a float32 product, as a float32 implementation does).  If
# the kernel's error had the distribution of one such evaluation's, a row
# would exceed 8x the largest of 12 with probability far below 1e-5, while a
# dropped term or a wrong sign, off by the size of the term, still fails.
# The tests print, per comparison, how many rows used this clause and the
# largest factor any of them needed ("float32_factor_needed").
FLOAT32_FACTOR = 8.0
FLOAT32_SAMPLES = 12
# Compositing gradients add WALK_SAMPLES float32 evaluations of the
# reference's back-to-front backward (orc.composite_backward_walk).
WALK_SAMPLES = 4


def ulp_perturbed(tensors, sample, seed=1234):
    """Sample 0: the float32 inputs as given; sample k > 0: every element
    moved one ulp up or down (seeded random direction)."""
    out = []
    for i, t in enumerate(tensors):
        t = torch.as_tensor(t).detach().float().cpu()
        if sample == 0:
            out.append(t)
            continue
        g = torch.Generator().manual_seed(seed + 7919 * sample + i)
        up = torch.rand(t.shape, generator=g) < 0.5
        inf = torch.full_like(t, math.inf)
        out.append(torch.where(up, torch.nextafter(t, inf), torch.nextafter(t, -inf)))
    return out


def _float32_error(reference32, e2):
    refs = reference32 if isinstance(reference32, (list, tuple)) else [reference32]
    return torch.stack([(_rows(r) - e2).abs().amax(1) for r in refs]).amax(0)[:, None]


def assert_gradients_close(actual, expected, what, explained=None, max_explained=0.01,
                           reference32=None):
    """Every row (Gaussian) of ``actual`` within GRAD_RTOL |e| + GRAD_ATOL
    min(1, max|e| of the column) of ``expected`` (float64 truth).

    ``reference32``: the same gradients computed by the float32 restatement of
    the reference (the oracle in float32, same decisions), or a list of such
    evaluations (FLOAT32_SAMPLES, from ulp_perturbed inputs).  Where float32
    arithmetic itself cannot reach the tolerance (cancellation among large
    terms, ill-conditioned 2x2 covariances) a row may instead lie within
    FLOAT32_FACTOR times the largest of their errors on the row: the kernel
    is then as accurate as the reference's own numerics.

    Rows that still fail must be ``explained`` (a bool [rows]: a cut or clamp
    decision of theirs, or of a pixel they reach, lies within DECISION_WINDOW
    of its threshold) and at most ``max_explained`` of the rows.  Returns
    statistics."""
    a2, e2 = _rows(actual), _rows(expected)
    colmax = e2.abs().amax(0)
    strict = GRAD_RTOL * e2.abs() + GRAD_ATOL * colmax.clamp(max=1.0)
    bound = strict
    if reference32 is not None:
        bound = torch.maximum(strict, FLOAT32_FACTOR * _float32_error(reference32, e2))
    err = (a2 - e2).abs()
    excess = err / bound.clamp_min(1e-300)
    bad = (excess > 1).any(1)
    stats = {
        "rows": int(a2.shape[0]),
        "failing": int(bad.sum()),
        "at_float32_accuracy": int(((err > strict).any(1) & ~bad).sum()),
        "worst_excess": float(excess.max()) if excess.numel() else 0.0,
    }
    if reference32 is not None:
        # The factor the rows beyond the strict bound needed: their error in
        # units of the float32 evaluations' largest error on the row.
        over = err > strict
        if bool(over.any()):
            f32 = _float32_error(reference32, e2).expand_as(err)
            stats["float32_factor_needed"] = float((err[over] / f32[over].clamp_min(1e-300)).max())
        else:
            stats["float32_factor_needed"] = 0.0
    if bool(bad.any()):
        r, c = divmod(int(excess.argmax()), excess.shape[1])
        refs = reference32 if isinstance(reference32, (list, tuple)) else [reference32]
        f32 = (float(_float32_error([_rows(x)[r:r + 1] for x in refs], e2[r:r + 1])[0, 0])
               if reference32 is not None else float("nan"))
        stats["worst"] = (f"row {r} column {c}: actual {float(a2[r, c]):.9g} expected "
                          f"{float(e2[r, c]):.9g} bound {float(bound[r, c]):.3g} strict "
                          f"{float(strict[r, c]):.3g} float32 row error {f32:.3g}; row {e2[r].tolist()}")
        print(f"[{what}] {stats['worst']}", flush=True)
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


def assert_close_to_truth(actual, truth, reference32, rtol, atol, what, rows=None):
    """|actual - truth| <= atol + rtol |truth| per element, or within
    FLOAT32_FACTOR times the float32 restatement's error scale on the same
    row (``reference32``: one evaluation or a list; ``rows``: optional bool
    mask of the rows to compare)."""
    a2, e2 = _rows(actual), _rows(truth)
    refs = reference32 if isinstance(reference32, (list, tuple)) else [reference32]
    refs = [_rows(r) for r in refs]
    if rows is not None:
        m = torch.as_tensor(rows).bool()
        a2, e2, refs = a2[m], e2[m], [r[m] for r in refs]
    strict = atol + rtol * e2.abs()
    f32 = _float32_error(refs, e2)
    bound = torch.maximum(strict, FLOAT32_FACTOR * f32)
    err = (a2 - e2).abs()
    bad = (err > bound).any(1)
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {a2.shape[0]} rows off; worst "
        f"{float((err / bound.clamp_min(1e-300)).max()):.2f}x the bound"
    )
    over = err > strict
    needed = (float((err[over] / f32.expand_as(err)[over].clamp_min(1e-300)).max())
              if bool(over.any()) else 0.0)
    return {"rows": int(a2.shape[0]), "at_float32_accuracy": int(over.any(1).sum()),
            "float32_factor_needed": needed}


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


def _form(sample, samples):
    """Transmittance form of float32 sample k: the reference's log-space sum
    for the first half, the float32 product for the rest."""
    return "log" if sample < (samples + 1) // 2 else "product"


def _entry_grads(leaves):
    du, dv, da, db, dc, drgb, dop = (x.grad for x in leaves)
    # The oracle's inv01 leaf enters the quadratic form twice (both
    # off-diagonal entries); the kernels' column is per matrix entry.
    return torch.stack((du, dv, da, db / 2, dc, drgb[:, 0], drgb[:, 1], drgb[:, 2], dop), -1)


def fixed_decision_composite_grads(cols32, ids, ranges, width, height, tile_size, ncon, weights,
                                   tile_chunk=64, threshold=0.999, probe=False,
                                   samples=FLOAT32_SAMPLES):
    """Gradients [N, 9] of sum(composite * weights) along the given lists, in
    float64 (truth) and float32 (the reference's numerics: ``samples``
    evaluations on ulp_perturbed inputs by autograd of the forward, and
    WALK_SAMPLES by the Triton backward's back-to-front walk), all with the
    cut/clamp decisions of
    the float32 oracle on ``cols32`` (u, v, inv00, inv01, inv11, rgb [N, 3],
    alpha0: float32) and the activity test fixed by ``ncon``.  Returns
    (grad64, [grad32 ...], cut_margin[N], absolute64 [N, 2] or None)."""
    cols32 = [c.detach().float().cpu() for c in cols32]
    run32 = orc.composite(*cols32, ids, ranges, width, height, tile_size, threshold,
                          tile_chunk=tile_chunk)
    weights = torch.as_tensor(weights).cpu()

    def grads(cols, dt, probe_list=None, form="log"):
        leaves = [c.to(dt).clone().requires_grad_(True) for c in cols]
        run = orc.composite(*leaves, ids, ranges, width, height, tile_size, threshold,
                            tile_chunk=tile_chunk, probe=probe_list, decisions=run32.decisions,
                            active_counts=ncon, transmittance=form)
        (run.image * weights.to(dt)).sum().backward()
        return _entry_grads(leaves)

    pr = [] if probe else None
    g64 = grads(cols32, torch.float64, pr)
    absolute = orc.absolute_mean_gradients(pr, cols32[0].shape[0]) if probe else None
    g32 = [grads(ulp_perturbed(cols32, k), torch.float32, form=_form(k, samples))
           for k in range(samples)]
    # The reference's Triton backward walks each list back to front in
    # float32; its rounding grows with the walk's length, unlike autograd's
    # of the forward above.  A few float32 evaluations of that algorithm join
    # the error scale.
    g32 += [orc.composite_backward_walk(*ulp_perturbed(cols32, k), ids, ranges, width, height,
                                        tile_size, weights.float(), run32.decisions, ncon,
                                        tile_chunk=tile_chunk)
            for k in range(WALK_SAMPLES)]
    return g64, g32, run32.gaussian_cut_margin, absolute


def fixed_decision_rasterize_grads(params, cam, tile_size, near, far, lists, cols32, ncon, weights,
                                   tile_chunk=64, threshold=0.999, gather=None,
                                   samples=FLOAT32_SAMPLES):
    """Parameter gradients of sum(rasterize * weights) through the oracle's
    projection and compositing along ``lists`` (the GPU's), in float64 and in
    float32, with decisions fixed as in fixed_decision_composite_grads
    (``cols32``: the GPU's projected values, whose float32 compositing fixes
    the cut/clamp decisions).  ``gather``: indices applied to the parameters
    before projection (the op's ``indices``).  Returns (grads64, per-parameter
    lists of ``samples`` float32 gradients on ulp_perturbed parameters,
    cut_margin) for mean, rotation, scale, opacity, color."""
    cols32 = [c.detach().float().cpu() for c in cols32]
    ids, ranges = lists
    run32 = orc.composite(*cols32, ids, ranges, cam.width, cam.height, tile_size, threshold,
                          tile_chunk=tile_chunk)
    weights = torch.as_tensor(weights).cpu()

    def grads(ps, dt, form="log"):
        p = [x.detach().to(dt).clone().requires_grad_(True) for x in ps]
        q = p if gather is None else [x[gather] for x in p]
        ref = orc.rasterize(*q, cam, tile_size=tile_size, opacity_threshold=threshold, near=near,
                            far=far, tile_chunk=tile_chunk, lists=lists,
                            decisions=run32.decisions, active_counts=ncon, transmittance=form)
        (ref.image * weights.to(dt)).sum().backward()
        return [x.grad for x in p]

    g64 = grads(params, torch.float64)
    runs = [grads(ulp_perturbed(params, k), torch.float32, form=_form(k, samples))
            for k in range(samples)]
    g32 = [list(per) for per in zip(*runs)]
    return g64, g32, run32.gaussian_cut_margin


def segmented_scene(entries, width=64, height=64, tile_size=8):
    """Projected splats whose lists cross the forward's checkpoints: every
    entry is listed in tiles (0, 0) and (0, 1), an eighth of them also in
    (1, 0) and (1, 1).  The first two lists are longer than the checkpoint
    minimum (8192 entries) and walk ~1300 entries until T ~ 1e-3; the other
    two walk their whole lists of 1125 or 1500.  The splats are wide (sigma >=
    2000 px, alpha 0.0045-0.006), so no pixel sits near a discrete decision.
    Returns (pmean, pinv, pcol, pop, sorted ids, ranges)."""
    g = torch.Generator().manual_seed(entries + 1)
    u = torch.rand(entries, generator=g) * 20 - 2
    v = torch.rand(entries, generator=g) * 20 - 2
    depth = torch.rand(entries, generator=g) * 5 + 1
    pmean = torch.stack((u, v, depth), -1)
    sigma = torch.rand(entries, generator=g) * 2000 + 2000
    rho = (torch.rand(entries, generator=g) * 2 - 1) * 0.5
    cov = torch.stack((sigma ** 2, rho * sigma ** 2, rho * sigma ** 2, sigma ** 2), -1).view(-1, 2, 2)
    pinv = torch.linalg.inv(cov.double()).float()
    pcol = torch.rand(entries, 3, generator=g)
    pop = torch.rand(entries, 1, generator=g) * 0.0015 + 0.0045
    tw = -(-width // tile_size)
    th = -(-height // tile_size)
    bounds = np.zeros((entries, 2, 2), dtype=np.int32)
    bounds[:, 0, 1] = 1
    bounds[: entries // 8, 0, 1] = 2
    bounds[:, 1, 1] = 2
    counts = ((bounds[:, 0, 1] - bounds[:, 0, 0]) * (bounds[:, 1, 1] - bounds[:, 1, 0])).astype(np.int32)
    keys, ids = orc.emit_intersections(bounds, depth.numpy(), counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
    return pmean, pinv, pcol, pop, sid, ranges


# ---------------------------------------------------------------------------
# Dispatch plan of the compositing kernels (gs_tile_order).
# ---------------------------------------------------------------------------

PLAN_WAVES = 4            # items per compositing workgroup
PLAN_SPLIT_TILES = 4096   # fewer tiles with work than this: every tile split in quarters
PLAN_SEGMENT_SPARE = 4    # spare slots per region (backward plans), in units of its tiles
PLAN_SORT_MAX = 8192      # larger regions keep index order
CHECKPOINT_ENTRIES = 1024  # forward checkpoints at multiples of this intersection index
CHECKPOINT_MAX = 63        # per tile
CHECKPOINT_MIN_LIST = 8192  # lists of at most this many entries record none


def plan_chunk(num_tiles, waves=PLAN_WAVES):
    """Tiles per chunk dealt to the regions: about num_tiles / 64, a multiple
    of the workgroup's waves, between one workgroup's tiles and 64."""
    k = -(-num_tiles // 64)
    return waves if k < waves else 64 if k > 64 else -(-k // waves) * waves


def plan_regions(num_tiles, waves=PLAN_WAVES):
    """Tiles of the eight XCD regions, in region order: chunk c of
    plan_chunk(num_tiles) consecutive tiles belongs to region c % 8."""
    k = plan_chunk(num_tiles, waves)
    tiles = np.arange(num_tiles)
    chunk = tiles // k
    return [tiles[chunk % 8 == r] for r in range(8)]


def plan_slots(num_tiles, tile_size, active=0, backward=False):
    """(item slots per region, tiles walked back in segments, every tile split)."""
    live = active if 0 < active < num_tiles else num_tiles
    split_all = tile_size >= 16 and live < PLAN_SPLIT_TILES
    segments = backward and not split_all
    k = plan_chunk(num_tiles)
    t_max = -(-(-(-num_tiles // k)) // 8) * k  # tiles of the largest region (region 0)
    cap = 4 * t_max if split_all else (1 + PLAN_SEGMENT_SPARE) * t_max if segments else t_max
    blocks = -(-cap // PLAN_WAVES) if cap > PLAN_WAVES else 1
    return PLAN_WAVES * blocks, segments, split_all


def checkpoint_crossings(start, max_n, list_len):
    """Checkpoints a walk of max_n entries of a list of list_len entries
    starting at intersection index `start` crosses: the multiples P of
    CHECKPOINT_ENTRIES at least 64 past start whose 64-entry batch starts
    below max_n (at most CHECKPOINT_MAX; none for lists of at most
    CHECKPOINT_MIN_LIST entries), as positions in the walk (the batch
    starts)."""
    if list_len <= CHECKPOINT_MIN_LIST:
        return []
    first = -(-(start + 64) // CHECKPOINT_ENTRIES) * CHECKPOINT_ENTRIES
    out = []
    p = first
    while len(out) < CHECKPOINT_MAX:
        b = (p - start) // 64 * 64
        if b >= max_n:
            break
        out.append(b)
        p += CHECKPOINT_ENTRIES
    return out


def expected_plan(keys, tile_size, active=0, backward=False, crossings=None):
    """The work items gs_tile_order writes for per-tile work keys (list
    lengths, or largest contributor counts for a backward plan): per region
    (plan_regions, tiles in ascending index), a
    stable sort by the key's eight most significant bits (relative to the
    region's largest key, keys capped at 2^16 - 1), largest first; each tile
    as its four quarters (tile << 7 | 0x20 | q) when every tile is split, as
    1 + c segments (tile << 7 | 0x40 | s, c = its checkpoint crossings) in a
    backward plan while the region's spare slots last (a tile whose segments
    do not fit stays whole), else whole (tile << 7); -1 fills the region's
    unused slots."""
    keys = np.minimum(np.maximum(np.asarray(keys, dtype=np.int64), 0), 0xFFFF)
    num_tiles = keys.size
    if crossings is None:
        crossings = np.zeros(num_tiles, dtype=np.int64)
    slots, segments, split_all = plan_slots(num_tiles, tile_size, active, backward)
    items = np.full(8 * slots, -1, dtype=np.int64)
    for r, region in enumerate(plan_regions(num_tiles)):
        n = region.size
        out = items[r * slots:(r + 1) * slots]
        if n == 0:
            continue
        if n > PLAN_SORT_MAX:
            if split_all:
                t = region[np.arange(4 * n) // 4]
                out[:4 * n] = t << 7 | 0x20 | (np.arange(4 * n) & 3)
            else:
                out[:n] = region << 7
            continue
        k = keys[region]
        shift = max(0, int(k.max() | 1).bit_length() - 8)
        order = np.lexsort((np.arange(n), -(k >> shift)))
        extra = np.array([3 if split_all else (min(int(crossings[region[e]]), CHECKPOINT_MAX)
                                                if segments else 0) for e in order],
                         dtype=np.int64)
        # Thread-blocked greedy of the library: blocks of 8 sorted tiles; a
        # tile keeps its extras if the original extras before its block plus
        # the kept extras before it in the block, plus its own, fit.
        spare = slots - n
        kept = extra.copy()
        for b0 in range(0, n, 8):
            before = int(extra[:b0].sum())
            for i in range(b0, min(b0 + 8, n)):
                if before + kept[i] > spare:
                    kept[i] = 0
                before += kept[i]
        pos = 0
        for p, e in enumerate(order):
            t = int(region[e])
            x = int(kept[p])
            if x == 0:
                out[pos] = t << 7
            else:
                code = 0x20 if split_all else 0x40
                out[pos:pos + x + 1] = t << 7 | code | np.arange(x + 1)
            pos += 1 + x
    return items.astype(np.int32)


def plan_tile_keys(ranges=None, ncon=None, width=0, height=0, tile_size=16):
    """Per-tile work keys of the plan: list lengths, or (given ncon, one
    view [H, W]) the largest contributor count of each tile's pixels."""
    if ncon is None:
        r = np.asarray(ranges)
        return r[:, 1] - r[:, 0]
    tw, th = -(-width // tile_size), -(-height // tile_size)
    padded = np.zeros((th * tile_size, tw * tile_size), dtype=np.int64)
    padded[:height, :width] = ncon
    return padded.reshape(th, tile_size, tw, tile_size).max(axis=(1, 3)).reshape(-1)


def plan_crossings(ranges, walks):
    """Checkpoint crossings per tile for the backward plan (tile starts from
    ranges, walks = largest contributor counts)."""
    r = np.asarray(ranges)
    return np.array([len(checkpoint_crossings(int(r[t, 0]), int(walks[t]),
                                              int(r[t, 1] - r[t, 0])))
                     for t in range(r.shape[0])], dtype=np.int64)
