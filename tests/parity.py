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
    from gaussian_splats.splats.camera import host_extrinsics

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
