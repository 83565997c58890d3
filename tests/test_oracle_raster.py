"""Pins the oracle's binning and compositing: brute-force emission, numpy
lexsort, rectangle conservativeness, a per-pixel pure-Python compositor over
Gaussians sorted by (depth, index), tile-size independence, the weight/
transmittance identity, a single-Gaussian known answer and float64 finite
differences of the whole rasterizer.  CPU only."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import rasterizer as orc


def _scene(n=30, seed=5, k=4, w=40, h=28, spread=0.6, log_scale=-2.2):
    g = torch.Generator().manual_seed(seed)
    mean = torch.randn(n, 3, generator=g, dtype=torch.float64) * spread
    rot = torch.randn(n, 4, generator=g, dtype=torch.float64)
    scale = torch.randn(n, 3, generator=g, dtype=torch.float64) * 0.3 + log_scale
    op = torch.randn(n, 1, generator=g, dtype=torch.float64) * 1.5
    col = torch.randn(n, k, 3, generator=g, dtype=torch.float64) * 0.4
    cam = orc.Camera(torch.eye(3, dtype=torch.float64), torch.tensor([0.0, 0.0, -4.0], dtype=torch.float64),
                     0.9 * w, 0.9 * w, w / 2, h / 2, w, h)
    return (mean, rot, scale, op, col), cam


def test_emit_matches_brute_force():
    rng = np.random.default_rng(0)
    n, tw, th = 200, 9, 7
    x = np.sort(rng.integers(0, tw + 1, size=(n, 2)), 1)
    y = np.sort(rng.integers(0, th + 1, size=(n, 2)), 1)
    bounds = np.stack((x, y), 1).astype(np.int32)
    counts = ((x[:, 1] - x[:, 0]) * (y[:, 1] - y[:, 0])).astype(np.int32)
    counts[rng.random(n) < 0.2] = 0
    depths = rng.random(n).astype(np.float32) * 5 + 0.1
    keys, ids = orc.emit_intersections(bounds, depths, counts, tw)
    exp_k, exp_i = [], []
    for gi in range(n):
        if counts[gi] == 0:
            continue
        for ty in range(y[gi, 0], y[gi, 1]):
            for tx in range(x[gi, 0], x[gi, 1]):
                exp_k.append(((ty * tw + tx) << 32) | int(depths[gi:gi + 1].view(np.uint32)[0]))
                exp_i.append(gi)
    assert keys.tolist() == exp_k and ids.tolist() == exp_i


def test_sort_matches_lexsort_and_invariants():
    rng = np.random.default_rng(1)
    n, tw, th = 500, 11, 6
    x = np.sort(rng.integers(0, tw + 1, size=(n, 2)), 1)
    y = np.sort(rng.integers(0, th + 1, size=(n, 2)), 1)
    bounds = np.stack((x, y), 1).astype(np.int32)
    counts = ((x[:, 1] - x[:, 0]) * (y[:, 1] - y[:, 0])).astype(np.int32)
    depths = (rng.integers(1, 20, size=n) / 4).astype(np.float32)  # many ties
    keys, ids = orc.emit_intersections(bounds, depths, counts, tw)
    sid, ranges, skeys = orc.sort_intersections(keys, ids, tw * th)
    tile = keys >> 32
    order = np.lexsort((ids, depths[ids].view(np.uint32), tile))
    assert np.array_equal(sid, ids[order])
    assert ranges[0, 0] == 0 and ranges[-1, 1] == len(ids) and np.all(ranges[1:, 0] == ranges[:-1, 1])
    assert np.array_equal(np.diff(ranges, axis=1)[:, 0], np.bincount(tile, minlength=tw * th))
    assert np.all(np.diff(skeys) >= 0)


def test_rectangles_are_conservative():
    """Every pixel with alpha >= 1/255 lies inside the Gaussian's tile rectangle."""
    params, cam = _scene(n=60, w=64, h=48, log_scale=-1.8)
    proj = orc.project(*params, cam)
    ts = 8
    tw, th = 8, 6
    bounds, counts = orc.tile_counts(proj, ts, tw, th, 0.1, 100.0)
    ys, xs = np.mgrid[0:48, 0:64]
    for gi in range(60):
        u, v = proj.mean[gi, :2].numpy()
        inv = proj.inverse[gi].numpy()
        dx, dy = xs - u, ys - v
        D = inv[0, 0] * dx * dx + 2 * inv[0, 1] * dx * dy + inv[1, 1] * dy * dy
        alpha = np.minimum(proj.opacity[gi, 0].item() * np.exp(-0.5 * D), 0.99)
        hit = alpha >= 1 / 255
        if not hit.any() or counts[gi] == 0:
            assert counts[gi] == 0 or not hit.any() or proj.mean[gi, 2] <= 0.1
            continue
        tx, ty = xs[hit] // ts, ys[hit] // ts
        assert tx.min() >= bounds[gi, 0, 0] and tx.max() < bounds[gi, 0, 1]
        assert ty.min() >= bounds[gi, 1, 0] and ty.max() < bounds[gi, 1, 1]


def _hand_projected(rows):
    """Projected splats built directly from (u, v, depth, var_x, var_y, alpha0)
    rows: isotropic or axis-aligned screen covariances of chosen size."""
    t = torch.tensor(rows, dtype=torch.float64)
    n = len(rows)
    cov = torch.zeros(n, 2, 2, dtype=torch.float64)
    cov[:, 0, 0], cov[:, 1, 1] = t[:, 3], t[:, 4]
    inv = torch.zeros_like(cov)
    inv[:, 0, 0], inv[:, 1, 1] = 1 / t[:, 3], 1 / t[:, 4]
    return orc.Projected(t[:, :3].clone(), cov, inv, torch.zeros(n, 3, dtype=torch.float64),
                         t[:, 5:6].clone())


# alpha0 with ln(255 alpha0) = 4, so the gaussian-mode extent 2 sqrt(ln(255 alpha0)) is 4.
ALPHA_EXT4 = math.exp(4.0) / 255.0


def test_rectangles_closed_form():
    """Hand-computed tile rectangles (reference torch.py:89-108): extent
    2 sqrt(ln(255 alpha)) times the screen standard deviation, floor of
    (u -/+ r) / tile, +1 on the upper bound, clamps at 0 and the grid size,
    the empty rectangle of alpha < 1/255 (NaN extent) and the ellipsoid
    extent sqrt(-2 ln(1 - confidence)).  Tile 16 on a 10 x 8 grid."""
    ts, tw, th = 16, 10, 8
    rows = [
        # u, v, depth, var_x, var_y, alpha0      -> r = 4 * sqrt(var)
        (40.0, 40.0, 2.0, 4.0, 4.0, ALPHA_EXT4),    # r = 8: x [32, 48] -> tiles [2, 3+1)
        (40.0, 40.0, 2.0, 3.9, 3.9, ALPHA_EXT4),    # r < 8: 47.9 -> tile 2, upper bound 3
        (60.0, 100.0, 2.0, 25.0, 1.0, ALPHA_EXT4),  # r = (20, 4): x [40, 80] -> [2, 6), y [96, 104] -> [6, 7)
        (-5.0, 20.0, 2.0, 4.0, 4.0, ALPHA_EXT4),    # floor(-13/16) = -1 clamps to 0
        (158.0, 124.0, 2.0, 4.0, 4.0, ALPHA_EXT4),  # floor(166/16) + 1 = 11 clamps to 10; y 8 -> 8
        (-100.0, 20.0, 2.0, 4.0, 4.0, ALPHA_EXT4),  # entirely left: [0, 0)
        (40.0, 40.0, 2.0, 4.0, 4.0, 0.9 / 255.0),   # alpha < 1/255: NaN extent -> empty
        (40.0, 40.0, 2.0, 4.0, 4.0, 1.0 / 255.0),   # alpha = 1/255: extent 0, the pixel's tile
        (40.0, 40.0, 0.1, 4.0, 4.0, ALPHA_EXT4),    # culled (depth <= near): count 0
    ]
    bounds, counts = orc.tile_counts(_hand_projected(rows), ts, tw, th, 0.2, 100.0)
    expected = [
        ((2, 4), (2, 4)),
        ((2, 3), (2, 3)),
        ((2, 6), (6, 7)),
        ((0, 1), (0, 2)),
        ((9, 10), (7, 8)),
        ((0, 0), (0, 2)),
        ((0, 0), (0, 0)),
        ((2, 3), (2, 3)),
        ((2, 4), (2, 4)),
    ]
    assert bounds.tolist() == [[list(x), list(y)] for x, y in expected]
    assert counts.tolist() == [4, 1, 4, 2, 1, 0, 0, 1, 0]

    # Ellipsoid mode: extent sqrt(-2 ln(1 - 0.95)) = 2.4477..., var 25 -> r = 12.24.
    rows = [(40.0, 40.0, 2.0, 25.0, 25.0, 0.5), (64.0, 64.0, 2.0, 25.0, 25.0, 0.001)]
    bounds, counts = orc.tile_counts(_hand_projected(rows), ts, tw, th, 0.2, 100.0, "ellipsoid", 0.95)
    # 40 -/+ 12.24 = 27.76, 52.24 -> tiles [1, 4); 64 -/+ 12.24 -> [3, 5) (opacity ignored)
    assert bounds.tolist() == [[[1, 4], [1, 4]], [[3, 5], [3, 5]]]
    assert counts.tolist() == [9, 4]
    # confidence 0.5: extent sqrt(2 ln 2) = 1.1774, r = 5.89 -> 40 +/- 5.89 -> [2, 3)
    bounds, _ = orc.tile_counts(_hand_projected(rows[:1]), ts, tw, th, 0.2, 100.0, "ellipsoid", 0.5)
    assert bounds.tolist() == [[[2, 3], [2, 3]]]


def test_rectangles_equal_the_tile_box_of_the_extent_ellipse():
    """Tightness: for random anisotropic screen covariances the rectangle is
    exactly the tile bounding box of the ellipse {d : d^T cov^-1 d <= e^2},
    e = 2 sqrt(ln(255 alpha)), found by sampling its boundary densely (no
    use of the closed-form half-widths); edge cases within 1e-3 px of a tile
    boundary are skipped.  A wrong extent constant moves some boxes."""
    rng = np.random.default_rng(3)
    n, ts, tw, th = 400, 8, 40, 30
    u = rng.uniform(-20, 340, n)
    v = rng.uniform(-20, 260, n)
    sx, sy = np.exp(rng.uniform(0.0, 3.0, n)), np.exp(rng.uniform(0.0, 3.0, n))
    rho = rng.uniform(-0.9, 0.9, n)
    alpha0 = rng.uniform(1.2 / 255, 0.99, n)
    cov = np.stack((sx * sx, rho * sx * sy, rho * sx * sy, sy * sy), -1).reshape(n, 2, 2)
    proj = orc.Projected(
        torch.tensor(np.stack((u, v, np.full(n, 2.0)), -1)), torch.tensor(cov),
        torch.tensor(np.linalg.inv(cov)), torch.zeros(n, 3, dtype=torch.float64),
        torch.tensor(alpha0[:, None]),
    )
    bounds, counts = orc.tile_counts(proj, ts, tw, th, 0.2, 100.0)
    theta = np.linspace(0, 2 * np.pi, 200_001)
    circle = np.stack((np.cos(theta), np.sin(theta)))
    checked = 0
    for i in range(n):
        e = 2 * math.sqrt(math.log(255 * alpha0[i]))
        pts = e * np.linalg.cholesky(cov[i]) @ circle
        lo = np.array([u[i], v[i]]) + pts.min(1)
        hi = np.array([u[i], v[i]]) + pts.max(1)
        edges = np.concatenate((lo, hi)) / ts
        if np.min(np.abs(edges - np.round(edges))) * ts < 1e-3:
            continue
        checked += 1
        box = np.stack((np.floor(lo / ts), np.floor(hi / ts) + 1), -1)
        box = np.clip(box, 0, np.array([[tw], [th]]))
        assert bounds[i].tolist() == box.astype(int).tolist(), i
        size = box[:, 1] - box[:, 0]
        assert counts[i] == size[0] * size[1]
    assert checked > 350


def _brute_force(proj, w, h, near, far, thr=0.999):
    """Per pixel, every visible Gaussian in (depth bits, index) order, float64."""
    depth = proj.mean[:, 2].numpy()
    order = sorted((i for i in range(len(depth)) if near < depth[i] < far),
                   key=lambda i: (np.float32(depth[i]).view(np.uint32), i))
    img = np.zeros((h, w, 3))
    T = np.ones((h, w))
    for py in range(h):
        for px in range(w):
            t = 1.0
            c = np.zeros(3)
            for i in order:
                if not (1 - t) < thr:
                    break
                u, v = proj.mean[i, :2].numpy()
                inv = proj.inverse[i].numpy()
                dx, dy = px - u, py - v
                D = inv[0, 0] * dx * dx + 2 * inv[0, 1] * dx * dy + inv[1, 1] * dy * dy
                a = min(proj.opacity[i, 0].item() * math.exp(-0.5 * D), 0.99)
                if a < 1 / 255:
                    continue
                c += t * a * proj.color[i].numpy()
                t *= 1 - a
            img[py, px] = c
            T[py, px] = t
    return img, T


@pytest.mark.parametrize("tile_size", (4, 8, 16))
def test_composite_matches_brute_force(tile_size):
    params, cam = _scene(n=25, w=30, h=22)
    r = orc.rasterize(*params, cam, tile_size=tile_size, near=0.1)
    img, T = _brute_force(r.projected, cam.width, cam.height, 0.1, 100.0)
    np.testing.assert_allclose(r.image.detach().numpy(), img, atol=1e-12)
    np.testing.assert_allclose(r.composite.final_transmittance.numpy(), T, atol=1e-12)


def test_image_independent_of_tile_size():
    params, cam = _scene(n=80, w=48, h=40, spread=0.8)
    imgs = [orc.rasterize(*params, cam, tile_size=t, near=0.1).image.detach() for t in (4, 8, 16, 32)]
    for im in imgs[1:]:
        torch.testing.assert_close(im, imgs[0], atol=1e-12, rtol=0)


def test_image_without_diagnostics_is_identical():
    """diagnostics=False (the CPU baseline's timing) leaves the image and its
    gradients bit for bit unchanged."""
    params, cam = _scene(n=60, w=40, h=32)
    leaves = [p.clone().requires_grad_(True) for p in params]
    a = orc.rasterize(*leaves, cam, tile_size=8, near=0.1)
    a.image.sum().backward()
    ga = [p.grad.clone() for p in leaves]
    for p in leaves:
        p.grad = None
    b = orc.rasterize(*leaves, cam, tile_size=8, near=0.1, diagnostics=False)
    b.image.sum().backward()
    assert torch.equal(a.image, b.image)
    assert all(torch.equal(x, p.grad) for x, p in zip(ga, leaves))


def test_weights_sum_to_one_minus_transmittance():
    params, cam = _scene(n=60, w=40, h=32)
    mean, rot, scale, op, col = params
    white = torch.zeros_like(col)
    white[:, 0] = (1 - 0.5) / orc.SH_C0  # rgb = 1 everywhere
    r = orc.rasterize(mean, rot, scale, op, white, cam, tile_size=8, near=0.1)
    torch.testing.assert_close(
        r.image.detach(), (1 - r.composite.final_transmittance)[..., None].expand_as(r.image), atol=1e-12, rtol=0
    )


def test_single_gaussian_known_answer():
    cam = orc.Camera(torch.eye(3, dtype=torch.float64), torch.zeros(3, dtype=torch.float64),
                     50.0, 50.0, 16.0, 16.0, 32, 32)
    mean = torch.tensor([[0.0, 0.0, -2.0]], dtype=torch.float64)
    s = math.log(0.05)
    scale = torch.tensor([[s, s, s]], dtype=torch.float64)
    op = torch.tensor([[0.0]], dtype=torch.float64)  # sigmoid -> 0.5
    col = torch.zeros(1, 1, 3, dtype=torch.float64)
    col[0, 0] = torch.tensor([0.5, 0.0, -0.5], dtype=torch.float64) / orc.SH_C0  # rgb = (1, 0.5, 0)
    r = orc.rasterize(mean, torch.tensor([[1.0, 0, 0, 0]], dtype=torch.float64), scale, op, col, cam,
                      tile_size=8, near=0.1)
    var = (50.0 / 2.0 * 0.05) ** 2 + 0.03  # fx/d * sigma, squared, + epsilon
    ys, xs = np.mgrid[0:32, 0:32]
    alpha = 0.5 * np.exp(-0.5 * ((xs - 16.0) ** 2 + (ys - 16.0) ** 2) / var)
    alpha = np.where(alpha >= 1 / 255, np.minimum(alpha, 0.99), 0)
    expected = alpha[..., None] * np.array([1.0, 0.5, 0.0])
    np.testing.assert_allclose(r.image.detach().numpy(), expected, atol=1e-12)
    assert int(r.composite.n_contributors[16, 16]) == 1


def test_empty_scene_is_black():
    params, cam = _scene(n=5)
    mean = params[0].clone()
    mean[:, 2] = 10.0  # behind the camera
    r = orc.rasterize(mean, *params[1:], cam, tile_size=8, near=0.1)
    assert float(r.image.abs().max()) == 0.0
    assert len(r.gaussian_ids) == 0


def test_gradients_match_finite_differences():
    """float64 autograd of the oracle = central differences of its forward."""
    params, cam = _scene(n=12, w=24, h=20, seed=9)
    params = [p.clone().requires_grad_(True) for p in params]
    g = torch.Generator().manual_seed(2)
    weight = torch.rand(20, 24, 3, generator=g, dtype=torch.float64)

    def loss(ps):
        return (orc.rasterize(*ps, cam, tile_size=8, near=0.1).image * weight).sum()

    loss(params).backward()
    eps = 1e-6
    rng = np.random.default_rng(0)
    for pi, p in enumerate(params):
        flat = p.detach().reshape(-1)
        for idx in rng.choice(flat.numel(), size=min(12, flat.numel()), replace=False):
            plus = [q.detach().clone() for q in params]
            minus = [q.detach().clone() for q in params]
            plus[pi].view(-1)[idx] += eps
            minus[pi].view(-1)[idx] -= eps
            fd = (loss(plus) - loss(minus)).item() / (2 * eps)
            an = p.grad.reshape(-1)[idx].item()
            assert abs(fd - an) <= 1e-5 * max(1.0, abs(an)), (pi, idx, fd, an)


def _probe_composite(proj, w, h, tile_size, gimg):
    """Composite with per-pixel mean probes; back-propagates sum(image * gimg)."""
    bounds, counts = orc.tile_counts(proj, tile_size, -(-w // tile_size), -(-h // tile_size), 0.1, 100.0)
    tw = -(-w // tile_size)
    keys, ids = orc.emit_intersections(bounds, proj.mean[:, 2].numpy(), counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * -(-h // tile_size))
    leaves = [x.detach().clone().requires_grad_(True) for x in (
        proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0], proj.inverse[:, 0, 1],
        proj.inverse[:, 1, 1], proj.color, proj.opacity[:, 0])]
    probe = []
    out = orc.composite(*leaves, sid, ranges, w, h, tile_size, probe=probe)
    (out.image * gimg).sum().backward()
    return leaves, probe


def test_absolute_mean_gradient_terms_sum_to_the_gradient():
    """The probed per-pixel terms add up to autograd's mean gradient (so their
    absolute sums are those of composite_bwd.py:180-185) and their absolute
    sums do not depend on the tile size."""
    params, cam = _scene(n=30, w=40, h=28)
    proj = orc.project(*params, cam)
    w, h = cam.width, cam.height
    gimg = torch.randn(h, w, 3, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    absolute = []
    for ts in (4, 16):
        leaves, probe = _probe_composite(proj, w, h, ts, gimg)
        n = proj.mean.shape[0]
        signed = torch.zeros(n, 2, dtype=torch.float64)
        for g, du, dv in probe:
            signed[:, 0].index_add_(0, g, du.grad.sum(1))
            signed[:, 1].index_add_(0, g, dv.grad.sum(1))
        torch.testing.assert_close(signed[:, 0], leaves[0].grad, rtol=1e-12, atol=1e-15)
        torch.testing.assert_close(signed[:, 1], leaves[1].grad, rtol=1e-12, atol=1e-15)
        a = orc.absolute_mean_gradients(probe, n)
        assert torch.all(a[:, 0] >= signed[:, 0].abs() - 1e-15)
        assert torch.all(a[:, 1] >= signed[:, 1].abs() - 1e-15)
        absolute.append(a)
    # Per-pixel terms: summed over tiles, independent of the tile size.
    torch.testing.assert_close(absolute[0], absolute[1], rtol=1e-12, atol=1e-15)
    assert float(absolute[0].sum()) > float(
        torch.stack((leaves[0].grad, leaves[1].grad), 1).abs().sum()) * (1 + 1e-6)


def _lists(proj, ts, tw, th, near=0.1, far=100.0):
    bounds, counts = orc.tile_counts(proj, ts, tw, th, near, far)
    keys, ids = orc.emit_intersections(bounds, proj.mean[:, 2].float().numpy(), counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
    return sid, ranges


def test_fixed_decisions_replay():
    """Replaying a run's own cut/clamp decisions and activity counts gives the
    same image and gradients; float64 with float32's decisions equals float64
    wherever their decisions agree; a wrong activity count changes the image."""
    params, cam = _scene(n=80, w=48, h=32, log_scale=-1.6)
    proj = orc.project(*params, cam)
    ts, tw, th = 8, 6, 4
    sid, ranges = _lists(proj, ts, tw, th)
    g = torch.Generator().manual_seed(3)
    w_img = torch.rand(32, 48, 3, generator=g, dtype=torch.float64)

    def run(dt, **kw):
        leaves = [x.detach().to(dt).clone().requires_grad_(True) for x in (
            proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0], proj.inverse[:, 0, 1],
            proj.inverse[:, 1, 1], proj.color, proj.opacity[:, 0])]
        c = orc.composite(*leaves, sid, ranges, 48, 32, ts, tile_chunk=3, **kw)
        (c.image * w_img.to(dt)).sum().backward()
        return c, [x.grad for x in leaves]

    c32, g32 = run(torch.float32)
    r32, h32 = run(torch.float32, decisions=c32.decisions, active_counts=c32.n_contributors.numpy())
    assert torch.equal(c32.image, r32.image) and torch.equal(c32.n_contributors, r32.n_contributors)
    assert all(torch.equal(a, b) for a, b in zip(g32, h32))

    c64, g64 = run(torch.float64)
    f64, k64 = run(torch.float64, decisions=c32.decisions, active_counts=c32.n_contributors.numpy())
    same = c64.gaussian_margin > 1e-5  # float32 and float64 decide alike there
    assert float(same.double().mean()) > 0.5
    pix = torch.as_tensor(c64.margin >= 1e-5)
    assert torch.allclose(c64.image[pix], f64.image[pix], rtol=0, atol=1e-12)
    for a, b in zip(g64, k64):
        assert torch.allclose(a[same], b[same], rtol=1e-10, atol=1e-12)

    fewer = np.maximum(c32.n_contributors.numpy() - 1, 0)
    bad, _ = run(torch.float64, decisions=c32.decisions, active_counts=fewer)
    assert float((bad.image - f64.image).detach().abs().max()) > 1e-3

    # Ellipsoid mode: replaying a float32 run's own decisions reproduces it;
    # float64 with them equals float64 wherever the indicators agree.
    cols = [x.detach() for x in (
        proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0], proj.inverse[:, 0, 1],
        proj.inverse[:, 1, 1], proj.color, proj.opacity[:, 0])]
    e32 = orc.composite(*(x.float() for x in cols), sid, ranges, 48, 32, ts,
                        rendering_mode="ellipsoid", tile_chunk=3)
    q32 = orc.composite(*(x.float() for x in cols), sid, ranges, 48, 32, ts,
                        rendering_mode="ellipsoid", tile_chunk=3, decisions=e32.decisions,
                        active_counts=e32.n_contributors.numpy())
    assert torch.equal(e32.image, q32.image)
    e64 = orc.composite(*cols, sid, ranges, 48, 32, ts, rendering_mode="ellipsoid", tile_chunk=3)
    q64 = orc.composite(*cols, sid, ranges, 48, 32, ts, rendering_mode="ellipsoid", tile_chunk=3,
                        decisions=e32.decisions, active_counts=e32.n_contributors.numpy())
    pix = torch.as_tensor(e64.margin >= 1e-5)
    assert float(pix.double().mean()) > 0.5
    assert torch.allclose(e64.image[pix], q64.image[pix], rtol=0, atol=1e-12)


@pytest.mark.parametrize("tile_size", (4, 16))
def test_backward_walk_equals_autograd(tile_size):
    """composite_backward_walk (the Triton backward's back-to-front algorithm,
    without its 1e-4 floor) equals float64 autograd of composite with the same
    fixed decisions, for every Gaussian and column; in float32 it stays
    within float32 rounding of that."""
    params, cam = _scene(n=120, w=40, h=28, log_scale=-1.7, spread=0.5)
    proj = orc.project(*params, cam)
    tw, th = -(-40 // tile_size), -(-28 // tile_size)
    sid, ranges = _lists(proj, tile_size, tw, th)
    cols = [proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0], proj.inverse[:, 0, 1],
            proj.inverse[:, 1, 1], proj.color, proj.opacity[:, 0]]
    cols = [c.detach() for c in cols]
    g = torch.rand(28, 40, 3, generator=torch.Generator().manual_seed(4), dtype=torch.float64) * 2 - 1
    run32 = orc.composite(*(c.float() for c in cols), sid, ranges, 40, 28, tile_size, tile_chunk=5)
    ncon = run32.n_contributors.numpy()
    assert int(ncon.max()) > 5 and float(run32.final_transmittance.min()) < 0.2
    leaves = [c.clone().requires_grad_(True) for c in cols]
    ref = orc.composite(*leaves, sid, ranges, 40, 28, tile_size, tile_chunk=5,
                        decisions=run32.decisions, active_counts=ncon)
    (ref.image * g).sum().backward()
    du, dv, da, db, dc, drgb, dop = (x.grad for x in leaves)
    expected = torch.stack((du, dv, da, db / 2, dc, drgb[:, 0], drgb[:, 1], drgb[:, 2], dop), -1)
    walk = orc.composite_backward_walk(*cols, sid, ranges, 40, 28, tile_size, g, run32.decisions,
                                       ncon, tile_chunk=5)
    scale = expected.abs().amax(0).clamp_min(1e-300)
    assert float(((walk - expected).abs() / scale).max()) < 1e-10
    walk32 = orc.composite_backward_walk(*(c.float() for c in cols), sid, ranges, 40, 28,
                                         tile_size, g.float(), run32.decisions, ncon, tile_chunk=5)
    assert float(((walk32.double() - expected).abs() / scale).max()) < 1e-4
