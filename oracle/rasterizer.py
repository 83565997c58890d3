"""CPU restatement of the reference rasterizer — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker / CPU baseline.
The product path (``gaussian-splats_amd/``) never calls it.

It restates the reference's *torch* backend
(src/gaussian_splats/kernels/rasterize/torch.py:21-247 with
src/gaussian_splats/splats/camera.py:81-124 and splats/utils.py:8-99) plus the
outputs only the Triton path defines (original-index bounds/counts,
project.py:234-253; keys, intersections.py:10-88; final transmittance and
contributor counts, composite.py:44-107), with three stated conventions:

* index space: culled Gaussians keep their slot with ``count == 0`` (Triton)
  instead of being removed (torch.py:62-73);
* ties: the (tile, depth) sort is stable, so equal depths keep ascending index;
* tiles: partial tiles at the right/bottom edge (ceil), so e.g. 1080 rows work.

Everything is written with elementwise torch ops so that (a) it runs in float32
(reference numerics) or float64 ("truth") from the same code, (b) autograd
gives the reference's gradients, and (c) the camera-space point, pixel
coordinates and depth are computed in the same operation order as the HIP
projection, so depth bits (and hence keys) agree bit for bit.

Every function here is pinned by tests/test_oracle_*.py against closed forms, brute force, finite
differences or independent libraries (scipy).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

SH_C0 = 0.28209479177387814
MIN_ALPHA = 1.0 / 255.0
MAX_ALPHA = 0.99
# Relative distance from the alpha cut, in units of alpha's float32 rounding
# sensitivity, within which Composite.cut_near counts a decision.
CUT_NEAR = 1e-5

# Closed-form real SH constants (degree <= 3), band-major, m = -l..l.  These are
# the normalisations the recurrence of utils.py:32-66 produces; the equality is
# asserted by tests/test_oracle_math.py.
_C1 = 0.4886025119029199
_C2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792,
       0.5462742152960396)
_C3 = (-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154,
       -0.4570457994644658, 1.445305721320277, -0.5900435899266435)


def sh_basis(directions: torch.Tensor, num_coefficients: int) -> torch.Tensor:
    """Real SH basis [N, K] at unit directions [N, 3] (utils.py:32-66), K <= 16."""
    if num_coefficients not in (1, 4, 9, 16):
        raise ValueError(f"unsupported SH coefficient count {num_coefficients}")
    x, y, z = directions.unbind(-1)
    out = [torch.full_like(x, SH_C0)]
    if num_coefficients > 1:
        out += [-_C1 * y, _C1 * z, -_C1 * x]
    if num_coefficients > 4:
        xx, yy, zz = x * x, y * y, z * z
        out += [
            _C2[0] * (x * y),
            _C2[1] * (y * z),
            _C2[2] * (2.0 * zz - xx - yy),
            _C2[3] * (x * z),
            _C2[4] * (xx - yy),
        ]
        if num_coefficients > 9:
            out += [
                _C3[0] * y * (3.0 * xx - yy),
                _C3[1] * (x * y) * z,
                _C3[2] * y * (4.0 * zz - xx - yy),
                _C3[3] * z * (2.0 * zz - 3.0 * xx - 3.0 * yy),
                _C3[4] * x * (4.0 * zz - xx - yy),
                _C3[5] * z * (xx - yy),
                _C3[6] * x * (xx - 3.0 * yy),
            ]
    return torch.stack(out, dim=-1)


def quaternion_to_rotation(q: torch.Tensor) -> torch.Tensor:
    """[N, 3, 3] rotation of unit (w, x, y, z) quaternions (utils.py:8-25)."""
    w, x, y, z = q.unbind(-1)
    return torch.stack(
        (
            1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
            2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
            2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y),
        ),
        dim=-1,
    ).reshape(*q.shape[:-1], 3, 3)


def _normalize(v: torch.Tensor) -> torch.Tensor:
    """F.normalize: v / max(|v|, 1e-12)."""
    return v / v.norm(dim=-1, keepdim=True).clamp_min(1e-12)


@dataclass
class Camera:
    rotation: torch.Tensor  # [3, 3] world -> camera
    translation: torch.Tensor  # [3]
    fx: float
    fy: float
    cx: float
    cy: float
    width: int
    height: int


@dataclass
class Projected:
    mean: torch.Tensor  # [N, 3] (u, v, clamped depth)
    covariance: torch.Tensor  # [N, 2, 2]
    inverse: torch.Tensor  # [N, 2, 2]
    color: torch.Tensor  # [N, 3]
    opacity: torch.Tensor  # [N, 1]


def project(
    mean: torch.Tensor,
    rotation: torch.Tensor,
    scale: torch.Tensor,
    opacity: torch.Tensor,
    color: torch.Tensor,
    cam: Camera,
    covariance_epsilon: float = 0.03,
) -> Projected:
    """EWA projection, SH colour and sigmoid opacity (camera.py:81-124, torch.py:165-203)."""
    dt = mean.dtype
    R = cam.rotation.to(dt)
    t = cam.translation.to(dt)
    mx, my, mz = mean.unbind(-1)
    # p = R mu + t, summed left to right (camera.py:94).
    px = R[0, 0] * mx + R[0, 1] * my + R[0, 2] * mz + t[0]
    py = R[1, 0] * mx + R[1, 1] * my + R[1, 2] * mz + t[1]
    pz = R[2, 0] * mx + R[2, 1] * my + R[2, 2] * mz + t[2]
    d = -pz
    dc = torch.where(d.abs() >= 1e-4, d, torch.where(d >= 0, 1e-4, -1e-4).to(dt))
    # Homogeneous divide with the unclamped depth (camera.py:101-102).
    u = cam.fx * px / d + cam.cx
    v = -cam.fy * py / d + cam.cy
    lim_x = 1.3 * (cam.width / (2 * cam.fx))
    lim_y = 1.3 * (cam.height / (2 * cam.fy))
    j00 = cam.fx / dc
    j02 = cam.fx * (px / dc).clamp(-lim_x, lim_x) / dc
    j11 = -cam.fy / dc
    j12 = -cam.fy * (py / dc).clamp(-lim_y, lim_y) / dc
    zero = torch.zeros_like(j00)
    J = torch.stack((j00, zero, j02, zero, j11, j12), -1).reshape(-1, 2, 3)
    Rq = quaternion_to_rotation(_normalize(rotation))
    M = (J @ R) @ Rq * scale.exp()[:, None, :]
    cov = M @ M.transpose(-1, -2)
    eye = torch.eye(2, dtype=dt)
    cov = cov + covariance_epsilon * eye
    a, b, c = cov[:, 0, 0], cov[:, 0, 1], cov[:, 1, 1]
    det = a * c - b * b
    inv = torch.stack((c / det, -b / det, -b / det, a / det), -1).reshape(-1, 2, 2)
    campos = -(R.T @ t)
    direction = _normalize(campos - mean)
    basis = sh_basis(direction, color.shape[1])
    rgb = ((basis.unsqueeze(1) @ color).squeeze(1) + 0.5).clamp_min(0)
    alpha0 = opacity.sigmoid()
    return Projected(torch.stack((u, v, dc), -1), cov, inv, rgb, alpha0)


def tile_counts(
    projected: Projected,
    tile_size: int,
    tiles_w: int,
    tiles_h: int,
    near: float,
    far: float,
    rendering_mode: str = "gaussian",
    confidence: float = 0.95,
) -> tuple[np.ndarray, np.ndarray]:
    """Tile rectangles [N, 2, 2] (x/y, min/max, half-open) and culled counts
    (torch.py:62-73, 233-252; project.py:234-253)."""
    with torch.no_grad():
        u = projected.mean[:, 0]
        v = projected.mean[:, 1]
        depth = projected.mean[:, 2]
        alpha0 = projected.opacity[:, 0]
        if rendering_mode == "gaussian":
            extent = 2 * torch.log(alpha0 * 255).sqrt()
        elif rendering_mode == "ellipsoid":
            extent = torch.full_like(u, math.sqrt(-2 * math.log1p(-confidence)))
        else:
            raise ValueError(f"Invalid rendering mode: {rendering_mode}")
        rx = extent * projected.covariance[:, 0, 0].sqrt()
        ry = extent * projected.covariance[:, 1, 1].sqrt()

        def clampf(x, hi):  # NaN -> lower bound, as fmaxf/fminf do
            return torch.fmin(torch.fmax(x, torch.zeros_like(x)), torch.full_like(x, hi))

        x0 = clampf(torch.floor((u - rx) / tile_size), tiles_w)
        x1 = clampf(torch.floor((u + rx) / tile_size) + 1, tiles_w)
        y0 = clampf(torch.floor((v - ry) / tile_size), tiles_h)
        y1 = clampf(torch.floor((v + ry) / tile_size) + 1, tiles_h)
        bounds = torch.stack((torch.stack((x0, x1), -1), torch.stack((y0, y1), -1)), -2)
        bounds = bounds.numpy().astype(np.int32)
        visible = ((depth > near) & (depth < far)).numpy()
        size = bounds[:, :, 1] - bounds[:, :, 0]
        counts = np.where(visible, size[:, 0] * size[:, 1], 0).astype(np.int32)
    return bounds, counts


def emit_intersections(
    bounds: np.ndarray, depths: np.ndarray, counts: np.ndarray, tiles_w: int
) -> tuple[np.ndarray, np.ndarray]:
    """Keys (tile << 32 | depth bits) and ids, Gaussian-major, row-major tiles
    (intersections.py:10-74, torch.py:254-277)."""
    counts = counts.astype(np.int64)
    ids = np.repeat(np.arange(len(counts), dtype=np.int32), counts)
    starts = np.cumsum(counts) - counts
    local = np.arange(counts.sum(), dtype=np.int64) - np.repeat(starts, counts)
    width = (bounds[:, 0, 1] - bounds[:, 0, 0]).astype(np.int64)[ids]
    tile = (bounds[ids, 1, 0].astype(np.int64) + local // np.maximum(width, 1)) * tiles_w + (
        bounds[ids, 0, 0].astype(np.int64) + local % np.maximum(width, 1)
    )
    bits = np.ascontiguousarray(depths, dtype=np.float32).view(np.uint32).astype(np.int64)
    keys = (tile << 32) | bits[ids]
    return keys, ids


def sort_intersections(
    keys: np.ndarray, ids: np.ndarray, num_tiles: int
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Stable key sort, ids and half-open ranges [T, 2] (intersections.py:77-88)."""
    order = np.argsort(keys.view(np.uint64) if keys.dtype == np.int64 else keys, kind="stable")
    sorted_keys = keys[order]
    sorted_ids = ids[order]
    tiles = (sorted_keys >> 32).astype(np.int64)
    edges = np.searchsorted(tiles, np.arange(num_tiles + 1), side="left")
    ranges = np.stack((edges[:-1], edges[1:]), -1).astype(np.int64)
    return sorted_ids, ranges, sorted_keys


@dataclass
class Composite:
    image: torch.Tensor  # [H, W, 3]
    final_transmittance: torch.Tensor  # [H, W]
    n_contributors: torch.Tensor  # [H, W] int32
    margin: torch.Tensor  # [H, W] smallest relative distance of a discrete decision
    clamp_margin: torch.Tensor  # [H, W] smallest relative distance of o*G from 0.99
    gaussian_margin: torch.Tensor  # [N] smallest margin over the pixels a Gaussian reaches
    # [N] as gaussian_margin, counting only the alpha cut and the 0.99 clamp
    # (the decisions a float32 run fixes for a replay; the activity test is
    # fixed separately by active_counts), each relative distance divided by
    # 1 + the quadratic form with absolute terms (|a| dx^2 + 2|b dx dy| +
    # |c| dy^2): alpha's float32 rounding error grows with it, and with
    # cancellation in the form (near-degenerate covariances).
    gaussian_cut_margin: torch.Tensor
    # Per chunk start tile: (keep, clamped) booleans [entries, pixels] of the
    # alpha cut (alpha >= 1/255 after the clamp) and of the 0.99 clamp.
    decisions: dict
    # [H, W]: the number of entries processed while active (or the first
    # inactive one) whose alpha-cut decision lies within CUT_NEAR of 1/255, in
    # units of alpha's rounding sensitivity (the relative distance divided by
    # 1 + the quadratic form with absolute terms).  Two float32 evaluations of
    # such an entry's alpha may keep or drop it differently.
    cut_near: torch.Tensor
    # Per chunk start tile: the [entries, pixels] pairs counted by cut_near,
    # in the layout of ``decisions``.
    near_pairs: dict


def composite(
    u: torch.Tensor,
    v: torch.Tensor,
    inv00: torch.Tensor,
    inv01: torch.Tensor,
    inv11: torch.Tensor,
    rgb: torch.Tensor,
    alpha0: torch.Tensor,
    ids: np.ndarray,
    ranges: np.ndarray,
    width: int,
    height: int,
    tile_size: int,
    opacity_threshold: float = 0.999,
    rendering_mode: str = "gaussian",
    confidence: float = 0.95,
    tile_chunk: int = 64,
    probe: list | None = None,
    decisions: dict | None = None,
    active_counts: np.ndarray | None = None,
    transmittance: str = "log",
    diagnostics: bool = True,
) -> Composite:
    """Dense per-(entry, pixel) compositing of each tile list (torch.py:172-225).

    ``diagnostics=False`` computes the image only, as torch.py:172-225 does
    (the CPU baseline's timing); the other fields keep their initial values.

    ``transmittance``: "log" (the reference's torch backend, torch.py:209-212:
    exp of a float64 cumulative sum of log1p(-alpha)) or "product" (the
    exclusive cumulative product of 1 - alpha in the working dtype, as a plain
    float32 implementation such as the reference's Triton kernels forms it,
    composite.py:97-98); the two agree to rounding.

    Fixed decisions: ``decisions`` (the ``decisions`` of an earlier call over
    the same lists and ``tile_chunk``, e.g. a float32 run) replaces the alpha
    cut and the 0.99 clamp of every (entry, pixel) by that run's outcome, and
    ``active_counts`` ([H, W], e.g. another implementation's n_contributors)
    makes entry k of a pixel's list active iff k < active_counts[pixel].  The
    result is then the exact-arithmetic value (in float64) of a compositor
    that took those discrete decisions, differentiable as before: with both,
    a float64 run's gradients are what a float32 implementation deciding like
    that should produce up to its rounding.  In ellipsoid mode the kept
    entries' indicator D <= cutoff is taken as decided (alpha = alpha0, or
    0.99 where clamped).

    With ``probe`` (a list), every chunk appends ``(g, du, dv)``: zero leaves
    of shape [entries, pixels] added to the means inside the quadratic form, so
    that after a backward ``du.grad[e, p]`` is pixel p's term of dL/du for the
    Gaussian of entry e (composite_bwd.py:180-185 sums their absolute values).

    Transmittance is exp of the float64 exclusive cumulative sum of log1p(-alpha)
    (torch.py:209-212), cast to the working dtype; ``(1 - T) < threshold`` masks
    the weights (torch.py:214).  n_contributors counts the entries processed
    while active; final_transmittance is T after the last active entry.
    Differentiable w.r.t. the per-Gaussian tensors.  ``inv01`` enters the
    quadratic form twice (the off-diagonal pair), so its gradient is twice the
    per-entry gradient.
    """
    dt = u.dtype
    tiles_w = -(-width // tile_size)
    tiles_h = -(-height // tile_size)
    num_tiles = tiles_w * tiles_h
    P = tile_size * tile_size
    image = torch.zeros(num_tiles, P, 3, dtype=dt)
    final_t = torch.ones(num_tiles, P, dtype=dt)
    ncon = torch.zeros(num_tiles, P, dtype=torch.int64)
    margin = torch.full((num_tiles, P), math.inf, dtype=torch.float64)
    cmargin = torch.full((num_tiles, P), math.inf, dtype=torch.float64)
    local_y, local_x = np.divmod(np.arange(P), tile_size)
    ids_t = torch.as_tensor(ids, dtype=torch.int64)
    cutoff = -2 * math.log1p(-confidence)
    gmargin = torch.full((u.shape[0],), math.inf, dtype=torch.float64)
    gcmargin = torch.full((u.shape[0],), math.inf, dtype=torch.float64)
    near_count = torch.zeros(num_tiles, P, dtype=torch.int64)
    if active_counts is not None:
        ac = np.zeros((tiles_h * tile_size, tiles_w * tile_size), dtype=np.int64)
        ac[:height, :width] = np.asarray(active_counts)
        ac = ac.reshape(tiles_h, tile_size, tiles_w, tile_size).transpose(0, 2, 1, 3)
        active_tiles = torch.as_tensor(ac.reshape(num_tiles, P))
    recorded = {}
    near_pairs = {}
    parts = []
    for t0 in range(0, num_tiles, tile_chunk):
        t1 = min(num_tiles, t0 + tile_chunk)
        counts = ranges[t0:t1, 1] - ranges[t0:t1, 0]
        total = int(counts.sum())
        if total == 0:
            continue
        # Entry indices of the chunk's tiles (ranges need not be contiguous).
        starts = np.repeat(ranges[t0:t1, 0], counts)
        entry = starts + np.arange(total) - np.repeat(np.cumsum(counts) - counts, counts)
        lo, hi = 0, total
        tile_of = torch.as_tensor(np.repeat(np.arange(t0, t1), counts), dtype=torch.int64)
        g = ids_t[torch.as_tensor(entry, dtype=torch.int64)]
        ox = torch.as_tensor((tile_of.numpy() % tiles_w) * tile_size, dtype=dt)
        oy = torch.as_tensor((tile_of.numpy() // tiles_w) * tile_size, dtype=dt)
        px = ox[:, None] + torch.as_tensor(local_x, dtype=dt)[None]
        py = oy[:, None] + torch.as_tensor(local_y, dtype=dt)[None]
        dx = px - u[g][:, None]
        dy = py - v[g][:, None]
        if probe is not None:
            du = torch.zeros(dx.shape, dtype=dt, requires_grad=True)
            dv = torch.zeros(dy.shape, dtype=dt, requires_grad=True)
            probe.append((g, du, dv))
            dx = dx - du
            dy = dy - dv
        D = inv00[g][:, None] * dx * dx + 2 * inv01[g][:, None] * dx * dy + inv11[g][:, None] * dy * dy
        if rendering_mode == "ellipsoid":
            prob = (D <= cutoff).to(dt)
        else:
            prob = torch.exp(-0.5 * D)
        raw = alpha0[g][:, None] * prob
        if decisions is not None:
            keep, clamped = decisions[t0]
            # Ellipsoid mode: a kept entry's indicator (D <= cutoff) was 1.
            base = alpha0[g][:, None].expand_as(raw) if rendering_mode == "ellipsoid" else raw
            alpha = torch.where(clamped, torch.full_like(raw, MAX_ALPHA), base)
            alpha = torch.where(keep, alpha, torch.zeros_like(alpha))
        else:
            alpha = raw.clamp_max(MAX_ALPHA)
            alpha = torch.where(alpha >= MIN_ALPHA, alpha, torch.zeros_like(alpha))
            if diagnostics:
                with torch.no_grad():
                    recorded[t0] = (alpha > 0, raw > MAX_ALPHA)
        seg_start = torch.as_tensor(np.repeat(np.cumsum(counts) - counts, counts), dtype=torch.int64)
        if transmittance == "log":
            log_survival = torch.log1p(-alpha)
            # Segmented exclusive sum per tile, in float64 (torch.py:209-212).
            cums = log_survival.to(torch.float64).cumsum(0) - log_survival.to(torch.float64)
            cums = cums - cums[seg_start]
            T = torch.exp(cums).to(dt)
        elif transmittance == "product":
            # Segmented exclusive product per tile, in the working dtype.
            survival = 1 - alpha
            segs, pos0 = [], 0
            for cnt in counts:
                cnt = int(cnt)
                if cnt:
                    ones = torch.ones_like(survival[:1])
                    segs.append(torch.cumprod(torch.cat((ones, survival[pos0:pos0 + cnt - 1])), 0))
                pos0 += cnt
            T = torch.cat(segs)
        else:
            raise ValueError(f"unknown transmittance form {transmittance!r}")
        rel = tile_of - t0
        if active_counts is not None:
            pos_in_tile = torch.arange(hi - lo) - seg_start
            active = pos_in_tile[:, None] < active_tiles[tile_of]
        else:
            active = (1 - T) < opacity_threshold
        weights = T * alpha * active
        contrib = weights[..., None] * rgb[g][:, None, :]
        parts.append((t0, t1, torch.zeros(t1 - t0, P, 3, dtype=dt).index_add(0, rel, contrib)))
        if diagnostics:
            with torch.no_grad():
                n_active = torch.zeros(t1 - t0, P, dtype=torch.int64).index_add(0, rel, active.long())
                ncon[t0:t1] = n_active
                # T after the last active entry: T_i * (1 - alpha_i) at position n - 1.
                after = (T * (1 - alpha)).detach()
                pos = torch.arange(hi - lo) - seg_start
                last = active & (pos[:, None] == (n_active[rel] - 1))
                ft = torch.ones(t1 - t0, P, dtype=dt)
                sel = last.nonzero(as_tuple=True)
                ft[rel[sel[0]], sel[1]] = after[sel]
                final_t[t0:t1] = ft
                # Decision margins over entries up to and including the first inactive one.
                considered = pos[:, None] <= n_active[rel]
                a64 = raw.detach().to(torch.float64).clamp_max(MAX_ALPHA)
                m_cut = ((a64 - MIN_ALPHA).abs() / MIN_ALPHA)
                if rendering_mode == "ellipsoid":
                    m_cut = torch.minimum(m_cut, (D.detach().to(torch.float64) - cutoff).abs() / cutoff)
                T64 = T.detach().to(torch.float64)
                m_thr = ((1 - T64) - opacity_threshold).abs() / T64.clamp_min(1e-30)
                m = torch.minimum(m_cut, m_thr)
                m = torch.where(considered, m, torch.full_like(m, math.inf))
                mm = torch.full((t1 - t0, P), math.inf, dtype=torch.float64)
                mm.index_reduce_(0, rel, m, "amin")
                margin[t0:t1] = torch.minimum(margin[t0:t1], mm)
                r64 = raw.detach().to(torch.float64)
                m_cl = (r64 - MAX_ALPHA).abs() / MAX_ALPHA
                m_cl = torch.where(considered & (alpha.detach() > 0), m_cl, torch.full_like(m_cl, math.inf))
                cm = torch.full((t1 - t0, P), math.inf, dtype=torch.float64)
                cm.index_reduce_(0, rel, m_cl, "amin")
                cmargin[t0:t1] = torch.minimum(cmargin[t0:t1], cm)
                # Per Gaussian: worst pixel margin among the pixels it reaches, and
                # its own clamp margin there.
                reach = considered & (alpha.detach() > 0)
                per_entry = torch.where(reach, torch.minimum(mm[rel], m_cl), torch.full_like(m_cl, math.inf))
                gmargin.index_reduce_(0, g, per_entry.amin(1), "amin")
                # The same with the cut and clamp decisions only, in units of
                # alpha's rounding sensitivity.
                ddx, ddy = dx.detach().to(torch.float64), dy.detach().to(torch.float64)
                d_abs = (inv00[g].detach().to(torch.float64).abs()[:, None] * ddx * ddx
                         + 2 * (inv01[g].detach().to(torch.float64).abs()[:, None] * (ddx * ddy).abs())
                         + inv11[g].detach().to(torch.float64).abs()[:, None] * ddy * ddy)
                sens = 1 + d_abs
                m_cc = torch.where(considered, torch.minimum(m_cut, m_cl) / sens,
                                   torch.full_like(m_cl, math.inf))
                pc = torch.full((t1 - t0, P), math.inf, dtype=torch.float64)
                pc.index_reduce_(0, rel, m_cc, "amin")
                near_cut = considered & (m_cut / sens < CUT_NEAR)
                near_pairs[t0] = near_cut
                near_count[t0:t1] += torch.zeros(t1 - t0, P, dtype=torch.int64).index_add(
                    0, rel, near_cut.long())
                per_entry = torch.where(reach, torch.minimum(pc[rel], m_cl / sens),
                                        torch.full_like(m_cl, math.inf))
                gcmargin.index_reduce_(0, g, per_entry.amin(1), "amin")
    for t0, t1, img in parts:
        image = image.index_add(0, torch.arange(t0, t1), img)

    def to_image(x):
        x = x.reshape(tiles_h, tiles_w, tile_size, tile_size, *x.shape[2:])
        x = x.transpose(1, 2).reshape(tiles_h * tile_size, tiles_w * tile_size, *x.shape[4:])
        return x[:height, :width]

    return Composite(
        to_image(image),
        to_image(final_t),
        to_image(ncon).to(torch.int32),
        to_image(margin),
        to_image(cmargin),
        gmargin,
        gcmargin,
        decisions if decisions is not None else recorded,
        to_image(near_count),
        near_pairs,
    )


def composite_backward_walk(
    u: torch.Tensor,
    v: torch.Tensor,
    inv00: torch.Tensor,
    inv01: torch.Tensor,
    inv11: torch.Tensor,
    rgb: torch.Tensor,
    alpha0: torch.Tensor,
    ids: np.ndarray,
    ranges: np.ndarray,
    width: int,
    height: int,
    tile_size: int,
    grad_image: torch.Tensor,
    decisions: dict,
    active_counts: np.ndarray,
    tile_chunk: int = 64,
) -> torch.Tensor:
    """Gradients [N, 9] (u, v, inv00, inv01 per matrix entry, inv11, r, g, b,
    alpha0) of sum(composite * grad_image), by the algorithm of the
    reference's Triton backward (kernels/rasterize/composite_bwd.py:100-160),
    in the inputs' dtype.

    Each tile's list is walked from its last active entry to its first.  The
    suffix transmittance and suffix colour (the colour composited after an
    entry, relative to the transmittance there) are accumulated from the back.
    T_i = final_T / (suffix_T (1 - alpha_i)) and dL/dalpha_i = T_i g . (c_i -
    S_i).  final_T is the forward's product of (1 - alpha) in the same dtype.
    The Triton kernel floors the denominator at 1e-4, which makes its gradient
    inexact for T_i below that; this restatement has no floor, so in float64
    it equals autograd of :func:`composite`.  The discrete decisions are
    fixed: ``decisions`` (the cut and clamp of a :func:`composite` call with
    the same lists and ``tile_chunk``) and ``active_counts`` (entry k of a
    pixel's list is active iff k < active_counts).  Gaussian mode.  Used as a
    float32 evaluation of the reference's numerics along a back-to-front walk,
    whose rounding grows with the walk's length."""
    dt = u.dtype
    tiles_w = -(-width // tile_size)
    tiles_h = -(-height // tile_size)
    num_tiles = tiles_w * tiles_h
    P = tile_size * tile_size
    ranges = np.asarray(ranges)
    ids = np.asarray(ids)
    ac = np.zeros((tiles_h * tile_size, tiles_w * tile_size), dtype=np.int64)
    ac[:height, :width] = np.asarray(active_counts)
    ac = torch.as_tensor(ac.reshape(tiles_h, tile_size, tiles_w, tile_size)
                         .transpose(0, 2, 1, 3).reshape(num_tiles, P))
    gi = torch.zeros(tiles_h * tile_size, tiles_w * tile_size, 3, dtype=dt)
    gi[:height, :width] = torch.as_tensor(grad_image).to(dt)
    gi = gi.reshape(tiles_h, tile_size, tiles_w, tile_size, 3).permute(0, 2, 1, 3, 4)
    gi = gi.reshape(num_tiles, P, 3)
    local_y, local_x = np.divmod(np.arange(P), tile_size)
    lengths = ranges[:, 1] - ranges[:, 0]
    # Decisions of (tile, k): each chunk holds its tiles' lists in tile order
    # (composite's layout), so the chunks in order hold every list in tile
    # order and (tile, k) is entry first[tile] + k.
    chunks = [decisions[t0] for t0 in range(0, num_tiles, tile_chunk) if t0 in decisions]
    keep_all = torch.cat([c[0] for c in chunks]) if chunks else torch.zeros(0, P, dtype=torch.bool)
    clamp_all = torch.cat([c[1] for c in chunks]) if chunks else keep_all
    first = np.cumsum(lengths) - lengths
    walk = np.minimum(lengths, ac.amax(1).numpy())
    tiles = np.nonzero(walk > 0)[0]
    out = torch.zeros(u.shape[0], 9, dtype=dt)
    if tiles.size == 0:
        return out
    tt = torch.as_tensor(tiles)
    ox = torch.as_tensor((tiles % tiles_w) * tile_size, dtype=dt)[:, None]
    oy = torch.as_tensor((tiles // tiles_w) * tile_size, dtype=dt)[:, None]
    px = ox + torch.as_tensor(local_x, dtype=dt)[None]
    py = oy + torch.as_tensor(local_y, dtype=dt)[None]
    act = ac[tt]
    g = gi[tt]
    L = int(walk[tiles].max())

    def entry(k):
        """Per sampled tile: the Gaussian at position k (or -1) and its
        alpha, raw alpha, probability and offsets at the tile's pixels."""
        has = torch.as_tensor(k < walk[tiles])
        pos = torch.as_tensor(np.where(k < walk[tiles], ranges[tiles, 0] + k, 0))
        gid = torch.where(has, torch.as_tensor(ids)[pos].long(), torch.zeros_like(pos))
        dx = px - u[gid][:, None]
        dy = py - v[gid][:, None]
        D = (inv00[gid][:, None] * dx * dx + 2 * inv01[gid][:, None] * dx * dy
             + inv11[gid][:, None] * dy * dy)
        prob = torch.exp(-0.5 * D)
        raw = alpha0[gid][:, None] * prob
        slot = torch.as_tensor(np.where(k < walk[tiles], first[tiles] + k, 0))
        keep, clamped = keep_all[slot], clamp_all[slot]
        on = has[:, None] & keep & (k < act)
        alpha = torch.where(on, torch.where(clamped, torch.full_like(raw, MAX_ALPHA), raw),
                            torch.zeros_like(raw))
        return gid, has, dx, dy, prob, alpha, on & ~clamped

    # The forward's final transmittance, in the working dtype.
    final_t = torch.ones(len(tiles), P, dtype=dt)
    for k in range(L):
        final_t = final_t * (1 - entry(k)[5])
    suffix_t = torch.ones(len(tiles), P, dtype=dt)
    suffix_c = torch.zeros(len(tiles), P, 3, dtype=dt)
    for k in range(L - 1, -1, -1):
        gid, has, dx, dy, prob, alpha, free = entry(k)
        c = rgb[gid][:, None, :]
        t_i = final_t / (suffix_t * (1 - alpha))
        grad_alpha = torch.where(free, t_i * (g * (c - suffix_c)).sum(-1), torch.zeros_like(alpha))
        grad_d = grad_alpha * (-0.5 * alpha0[gid][:, None] * prob)
        a, b, cc = inv00[gid][:, None], inv01[gid][:, None], inv11[gid][:, None]
        rows = torch.stack((
            (-2 * grad_d * (a * dx + b * dy)).sum(1),
            (-2 * grad_d * (b * dx + cc * dy)).sum(1),
            (grad_d * dx * dx).sum(1),
            (grad_d * dx * dy).sum(1),
            (grad_d * dy * dy).sum(1),
            ((t_i * alpha)[..., None] * g).sum(1)[:, 0],
            ((t_i * alpha)[..., None] * g).sum(1)[:, 1],
            ((t_i * alpha)[..., None] * g).sum(1)[:, 2],
            (grad_alpha * prob).sum(1),
        ), -1)
        rows = torch.where(has[:, None], rows, torch.zeros_like(rows))
        out.index_add_(0, gid, rows)
        suffix_c = alpha[..., None] * c + (1 - alpha)[..., None] * suffix_c
        suffix_t = suffix_t * (1 - alpha)
    return out


@dataclass
class Render:
    image: torch.Tensor
    projected: Projected
    bounds: np.ndarray
    counts: np.ndarray
    gaussian_ids: np.ndarray
    ranges: np.ndarray
    sorted_keys: np.ndarray
    composite: Composite


def rasterize(
    mean: torch.Tensor,
    rotation: torch.Tensor,
    scale: torch.Tensor,
    opacity: torch.Tensor,
    color: torch.Tensor,
    cam: Camera,
    tile_size: int = 16,
    opacity_threshold: float = 0.999,
    near: float = 0.2,
    far: float = 100.0,
    rendering_mode: str = "gaussian",
    confidence: float = 0.95,
    covariance_epsilon: float = 0.03,
    tile_chunk: int = 64,
    lists: tuple[np.ndarray, np.ndarray] | None = None,
    decisions: dict | None = None,
    active_counts: np.ndarray | None = None,
    transmittance: str = "log",
    diagnostics: bool = True,
) -> Render:
    """project -> cull/rect -> emit -> stable sort -> composite (torch.py:228-247).

    ``lists`` = (sorted ids, ranges) composites those lists instead of the
    ones binned here (sorted_keys is then None); ``decisions``,
    ``active_counts``, ``transmittance`` and ``diagnostics`` are passed to
    :func:`composite`."""
    proj = project(mean, rotation, scale, opacity, color, cam, covariance_epsilon)
    tiles_w = -(-cam.width // tile_size)
    tiles_h = -(-cam.height // tile_size)
    bounds, counts = tile_counts(proj, tile_size, tiles_w, tiles_h, near, far, rendering_mode, confidence)
    if lists is None:
        depth32 = proj.mean[:, 2].detach().to(torch.float32).numpy()
        keys, ids = emit_intersections(bounds, depth32, counts, tiles_w)
        sorted_ids, ranges, sorted_keys = sort_intersections(keys, ids, tiles_w * tiles_h)
    else:
        sorted_ids, ranges = (np.asarray(x) for x in lists)
        sorted_keys = None
    comp = composite(
        proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0], proj.inverse[:, 0, 1],
        proj.inverse[:, 1, 1], proj.color, proj.opacity[:, 0], sorted_ids, ranges, cam.width,
        cam.height, tile_size, opacity_threshold, rendering_mode, confidence, tile_chunk,
        decisions=decisions, active_counts=active_counts, transmittance=transmittance,
        diagnostics=diagnostics,
    )
    return Render(comp.image, proj, bounds, counts, sorted_ids, ranges, sorted_keys, comp)


def absolute_mean_gradients(probe: list, n: int) -> torch.Tensor:
    """[n, 2] sums over (tile, pixel) of |dL/du| and |dL/dv| terms from a
    ``composite(..., probe=...)`` whose output has been back-propagated."""
    out = torch.zeros(n, 2, dtype=torch.float64)
    for g, du, dv in probe:
        out[:, 0].index_add_(0, g, du.grad.to(torch.float64).abs().sum(1))
        out[:, 1].index_add_(0, g, dv.grad.to(torch.float64).abs().sum(1))
    return out
