"""Stage-wise parity of the HIP kernels against the CPU oracle (cf. the
reference's kernels/rasterize/tests/test_project.py, test_intersections.py,
test_composite.py).  Each stage is fed identical inputs on both sides."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from gaussian_splats_hip import scenes
from gaussian_splats_hip.kernels.rasterize import (
    bin_gaussians,
    bin_tiles,
    composite,
    emit_intersections,
    emit_tiles,
    project_and_count,
    sort_intersections,
    sort_tiles,
)
from gaussian_splats_hip.kernels.rasterize import _native as nat
from oracle import rasterizer as orc
from parity import (
    FLOAT32_SAMPLES,
    assert_close_flip_aware,
    assert_close_to_truth,
    assert_forward_every_pixel,
    expected_plan,
    oracle_camera,
    plan_crossings,
    plan_slots,
    plan_tile_keys,
    rect_flip_tolerant_equal,
    ulp_perturbed,
)

pytestmark = pytest.mark.gpu

CONFIDENCE = 0.95
THRESHOLD = 0.999


def _project_both(scene, device, tile_size, mode="gaussian"):
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    params = [t.to(device) for t in scene.params()]
    gpu = project_and_count(
        *params, cam.rotation_matrix.to(device), cam.translation.to(device), fx, fy, cx, cy, w, h,
        tile_size, scene.near, scene.far, mode, CONFIDENCE,
    )
    ocam = oracle_camera(cam)
    proj = orc.project(*scene.params(), ocam)
    tw, th = nat.tiles(w, h, tile_size)
    bounds, counts = orc.tile_counts(proj, tile_size, tw, th, scene.near, scene.far, mode, CONFIDENCE)
    return gpu, proj, bounds, counts


@pytest.mark.parametrize("sh_degree", (0, 1, 2, 3))
@pytest.mark.parametrize("tile_size", (8, 16))
def test_project_matches_oracle(device, sh_degree, tile_size):
    scene = scenes.edge_case_scene(n=2000, sh_degree=sh_degree)
    gpu, proj, bounds, counts = _project_both(scene, device, tile_size)
    pmean, pinv, pcol, pop, gbounds, gcounts = (t.cpu() for t in gpu)
    torch.testing.assert_close(pmean, proj.mean.float(), rtol=2e-6, atol=1e-5)
    visible = torch.as_tensor(counts > 0)
    # The inverse against float64 (the kernel forms it in double precision),
    # or within the float32 restatement's error scale on ill-conditioned rows.
    ocam = oracle_camera(scene.cameras[0])
    truth = orc.project(*(p.double() for p in scene.params()), ocam).inverse.reshape(-1, 4)
    samples = [proj.inverse.reshape(-1, 4)] + [
        orc.project(*ulp_perturbed(scene.params(), k), ocam).inverse.reshape(-1, 4)
        for k in range(1, FLOAT32_SAMPLES)]
    stats = assert_close_to_truth(pinv.reshape(-1, 4), truth, samples, 1e-5, 1e-7,
                                  "inverse covariance", rows=visible)
    print("[project] inverse", stats, flush=True)
    torch.testing.assert_close(pcol, proj.color.float(), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(pop, proj.opacity.float(), rtol=1e-6, atol=1e-7)
    # Depth bits are bit-exact (same operation order, no transcendental).
    assert torch.equal(pmean[:, 2], proj.mean[:, 2].float())
    extent = 2 * np.sqrt(np.log(proj.opacity[:, 0].double().numpy() * 255))
    with np.errstate(invalid="ignore"):
        flips = rect_flip_tolerant_equal(gbounds.numpy(), bounds, proj, tile_size, extent)
    same_rect = np.all(gbounds.numpy() == bounds, axis=(1, 2))
    assert np.array_equal(gcounts.numpy()[same_rect], counts[same_rect])
    assert flips <= 2


def test_project_ellipsoid_mode(device):
    scene = scenes.edge_case_scene(n=500, sh_degree=1)
    gpu, proj, bounds, counts = _project_both(scene, device, 16, mode="ellipsoid")
    extent = np.full(500, math.sqrt(-2 * math.log1p(-CONFIDENCE)))
    rect_flip_tolerant_equal(gpu[4].cpu().numpy(), bounds, proj, 16, extent)


def test_launch_events_time_one_kernel(device):
    """A LaunchTimer's events ride on the projection kernel's launch: each
    pair is taken by exactly one launch, spans a positive time, and the
    outputs equal an untimed launch's; a call that launches no kernel (no
    Gaussians) takes none."""
    scene = scenes.edge_case_scene(n=2000, sh_degree=3)
    plain, _, _, _ = _project_both(scene, device, 16)
    with nat.LaunchTimer("project", capacity=4) as timer:
        timed = [_project_both(scene, device, 16)[0] for _ in range(3)]
        empty = [torch.empty((0,) + t.shape[1:], dtype=t.dtype, device=device)
                 for t in scene.params()]
        cam = scene.cameras[0]
        project_and_count(*empty, cam.rotation_matrix.to(device), cam.translation.to(device),
                          *cam.focal_length, *cam.principal_point, *cam.image_size, 16,
                          scene.near, scene.far, "gaussian", CONFIDENCE)
    assert len(timer.events) == 3
    times = [s.elapsed_time(e) for s, e in timer.events]
    print("[launch events] project ms", times, flush=True)
    assert all(0.0 < t < 100.0 for t in times)
    for out in timed:
        for a, b in zip(out, plain):
            assert torch.equal(a, b)
    lib = nat.library()
    assert lib.gs_disarm_launch_events() == 0


def _decode_rects(rects):
    """[x0, x1, y0, y1] of packed tile rectangles (numpy), decoded from the
    packing the header documents: x0 | (x1 - x0 - 1) << 8 | y0 << 16 |
    (y1 - y0 - 1) << 24."""
    r = rects.cpu().numpy().view(np.uint32).astype(np.int64)
    x0, y0 = r & 0xFF, (r >> 16) & 0xFF
    return np.stack([x0, x0 + ((r >> 8) & 0xFF) + 1, y0, y0 + (r >> 24) + 1], -1)


def _pack_from_bounds(bounds, counts, tw, th, device):
    rects = torch.empty(counts.numel(), dtype=torch.int32, device=device)
    nat.check(nat.library().gs_pack_tile_rects(
        nat.ptr(bounds), nat.ptr(counts), counts.numel(), tw, th, nat.ptr(rects),
        nat.stream(device)), "pack_tile_rects")
    return rects


@pytest.mark.parametrize("mode", ("gaussian", "ellipsoid"))
def test_projection_packs_tile_rects(device, mode):
    """The projection's packed rectangles decode to its bounds for every
    Gaussian with intersections and are 0xFFFFFFFF for the others; they equal
    gs_pack_tile_rects of the bounds and counts, and the projection writes the
    same ones without bounds (as the op calls it)."""
    scene = scenes.edge_case_scene(n=3000, sh_degree=1, image_size=(200, 120))
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    tw, th = nat.tiles(w, h, 16)
    params = [t.to(device) for t in scene.params()]
    args = (*params, cam.rotation_matrix, cam.translation, fx, fy, cx, cy, w, h, 16, scene.near,
            scene.far, mode, CONFIDENCE)
    rects = torch.empty(3000, dtype=torch.int32, device=device)
    out = project_and_count(*args, tile_rects=rects)
    bounds, counts = out[4], out[5]
    counted = counts.cpu().numpy() > 0
    assert 0 < counted.sum() < 3000
    raw = rects.cpu().numpy().view(np.uint32)
    assert (raw[~counted] == 0xFFFFFFFF).all()
    np.testing.assert_array_equal(_decode_rects(rects)[counted],
                                  bounds.cpu().numpy().reshape(-1, 4)[counted])
    assert torch.equal(rects, _pack_from_bounds(bounds, counts, tw, th, device))
    rects2 = torch.full_like(rects, 7)
    out2 = project_and_count(*args, tile_rects=rects2, bounds=False)
    assert out2[4] is None
    assert torch.equal(rects2, rects) and torch.equal(out2[5], counts)


def test_mosaic_projection_packs_shifted_tile_rects(device):
    """gs_project_views' packed rectangles are in the mosaic's tile grid: each
    view's bounds shifted to its tile origin, equal to gs_pack_tile_rects of
    the mosaic bounds."""
    from gaussian_splats_hip.kernels.rasterize.views import camera_tensors, mosaic_columns

    scene = scenes.config5(seed=3, n=2000, views=5, size=96, focal=120.0)
    rot, trans, intr, w, h = camera_tensors(scene.cameras)
    v, n = 5, 2000
    tw, th = nat.tiles(w, h, 16)
    cols = mosaic_columns(v, tw, th)
    rows = -(-v // cols)
    params = [t.to(device) for t in scene.params()]
    outs = [params[0].new_empty(s) for s in ((v, n, 3), (v, n, 2, 2), (v, n, 3), (v, n, 1))]
    bounds = torch.empty((v, n, 2, 2), dtype=torch.int32, device=device)
    counts = torch.empty((v, n), dtype=torch.int32, device=device)
    rects = torch.empty(v * n, dtype=torch.int32, device=device)
    view = nat.make_view(0.0, 0.0, 0.0, 0.0, w, h, 16, scene.near, scene.far, views=v,
                         mosaic_cols=cols)
    ptr = nat.ptr
    print(f"[mosaic rects] {v} views, {cols} columns", flush=True)
    nat.check(nat.library().gs_project_views(
        *(ptr(p) for p in params), n, params[4].shape[1], ptr(rot), ptr(trans), ptr(intr), view,
        *(ptr(o) for o in outs), ptr(bounds), ptr(counts), None, None, ptr(rects),
        nat.stream(device)), "project_views")
    flat_b = bounds.view(v * n, 2, 2)
    flat_c = counts.view(v * n)
    counted = flat_c.cpu().numpy() > 0
    decoded = _decode_rects(rects)
    np.testing.assert_array_equal(decoded[counted], flat_b.cpu().numpy().reshape(-1, 4)[counted])
    for k in range(v):  # each view's rectangles lie in its block of the mosaic
        d = decoded[k * n:(k + 1) * n][counted[k * n:(k + 1) * n]]
        ox, oy = (k % cols) * tw, (k // cols) * th
        assert len(d) and (d[:, 0] >= ox).all() and (d[:, 1] <= ox + tw).all()
        assert (d[:, 2] >= oy).all() and (d[:, 3] <= oy + th).all()
    assert torch.equal(rects, _pack_from_bounds(flat_b, flat_c, cols * tw, rows * th, device))


def test_project_rejects_sh4(device):
    scene = scenes.edge_case_scene(n=64, sh_degree=3)
    color = torch.zeros(64, 25, 3)
    cam = scene.cameras[0]
    with pytest.raises(NotImplementedError):
        project_and_count(
            scene.mean.to(device), scene.rotation.to(device), scene.scale.to(device),
            scene.opacity.to(device), color.to(device), cam.rotation_matrix.to(device),
            cam.translation.to(device), 72.0, 72.0, 48.0, 40.0, 96, 80, 16, 0.1, 100.0,
            "gaussian", 0.95,
        )


def _random_rects(n=4096, tiles_w=24, tiles_h=17, seed=42):
    """Random tile rectangles and depths (cf. test_intersections.py:8-18), with
    repeated depths to exercise the tie rule."""
    g = torch.Generator().manual_seed(seed)
    cx = torch.randint(0, tiles_w + 1, (n, 2), generator=g)
    cy = torch.randint(0, tiles_h + 1, (n, 2), generator=g)
    bounds = torch.stack(
        (torch.stack((cx.amin(1), cx.amax(1)), -1), torch.stack((cy.amin(1), cy.amax(1)), -1)), 1
    ).int()
    depths = torch.rand(n, generator=g) * 10 + 0.1
    depths[: n // 4] = depths[n // 4 : n // 2]  # ties
    counts = ((bounds[:, 0, 1] - bounds[:, 0, 0]) * (bounds[:, 1, 1] - bounds[:, 1, 0])).int()
    counts[torch.rand(n, generator=g) < 0.1] = 0  # culled
    return bounds, depths, counts


@pytest.mark.parametrize("shape", ((24, 17), (120, 68), (1, 1), (37, 1)))
def test_intersections_bit_exact(device, shape):
    tiles_w, tiles_h = shape
    bounds, depths, counts = _random_rects(tiles_w=tiles_w, tiles_h=tiles_h)
    keys_o, ids_o = orc.emit_intersections(bounds.numpy(), depths.numpy(), counts.numpy(), tiles_w)
    sid_o, ranges_o, skeys_o = orc.sort_intersections(keys_o, ids_o, tiles_w * tiles_h)

    keys, ids = emit_intersections(bounds.to(device), depths.to(device), counts.to(device), tiles_w)
    assert np.array_equal(keys.cpu().numpy(), keys_o)
    assert np.array_equal(ids.cpu().numpy(), ids_o)
    sid, ranges = sort_intersections(keys, ids, tiles_w * tiles_h)
    assert np.array_equal(sid.cpu().numpy(), sid_o)
    assert np.array_equal(ranges.cpu().numpy(), ranges_o)

    # Fused path: depth-ordered emission + tile-only sort gives the same lists.
    dkeys = depths.view(torch.int32).clone()
    dkeys[counts == 0] = -1
    order, offsets = bin_gaussians(dkeys.to(device), counts.to(device))
    total = int(offsets[-1].item())
    assert total == int(counts.sum())
    tk, tid = emit_tiles(bounds.to(device), order, offsets, total, tiles_w)
    sid2, ranges2 = sort_tiles(tk, tid, tiles_w * tiles_h)
    assert np.array_equal(sid2.cpu().numpy(), sid_o)
    assert np.array_equal(ranges2.cpu().numpy(), ranges_o)

    # Invariants: ranges partition [0, I); depth non-decreasing per tile,
    # ascending id on ties (test_intersections.py:36-38).
    r = ranges_o
    assert r[0, 0] == 0 and r[-1, 1] == len(sid_o) and np.all(r[1:, 0] == r[:-1, 1])
    d = depths.numpy()
    for s, e in r[:50]:
        seg = sid_o[s:e]
        assert np.all((d[seg][:-1] < d[seg][1:]) | ((d[seg][:-1] == d[seg][1:]) & (seg[:-1] < seg[1:])))


def _depth_keys(depths, counts):
    dkeys = depths.view(torch.int32).clone()
    dkeys[counts == 0] = -1
    return dkeys


@pytest.mark.parametrize(
    "shape,n",
    (
        ((24, 17), 4096),
        ((120, 68), 4096),
        ((256, 256), 768),
        ((1, 1), 4096),
        ((37, 1), 4096),
        ((1, 37), 4096),
        ((256, 2), 4096),
        ((3, 200), 4096),
    ),
)
def test_bucketed_binning_bit_exact(device, shape, n):
    """Row/column bucketing (the op's path) against the oracle's stable sort."""
    tiles_w, tiles_h = shape
    bounds, depths, counts = _random_rects(n=n, tiles_w=tiles_w, tiles_h=tiles_h, seed=7)
    keys_o, ids_o = orc.emit_intersections(bounds.numpy(), depths.numpy(), counts.numpy(), tiles_w)
    sid_o, ranges_o, _ = orc.sort_intersections(keys_o, ids_o, tiles_w * tiles_h)
    print(f"bucketed binning {shape} n={n} intersections={len(sid_o)}", flush=True)
    sid, ranges = bin_tiles(
        _depth_keys(depths, counts).to(device), bounds.to(device), counts.to(device), tiles_w, tiles_h
    )
    assert np.array_equal(ranges.cpu().numpy(), ranges_o)
    assert np.array_equal(sid.cpu().numpy(), sid_o)


@pytest.mark.parametrize(
    "near, far, n, shape",
    ((0.2, 100.0, 20000, (120, 68)), (0.01, 10.0, 4096, (24, 17)), (1.0, 1.5, 4096, (37, 1)),
     (0.2, 100.0, 0, (24, 17))),
    ids=("near0.2-far100", "near0.01-far10", "near1-far1.5", "empty"),
)
def test_bucketed_binning_remapped_depth_keys(device, near, far, n, shape):
    """The op's depth sort over min(key - bits(near), 2^k - 1) (near 0.2,
    far 100: k = 27, passes of 7, 7, 7 and 6 bits): the lists equal the
    oracle's stable (depth bits, index) sort, depths drawn between the planes
    with ties, culled Gaussians (key ~0) and depths just inside both
    planes."""
    from gaussian_splats_hip.kernels.rasterize import depth_key_range

    tiles_w, tiles_h = shape
    key_range = depth_key_range(near, far)
    assert key_range[1] < 32
    bounds, _, counts = _random_rects(n=max(n, 1), tiles_w=tiles_w, tiles_h=tiles_h, seed=n + 3)
    bounds, counts = bounds[:n], counts[:n]
    g = torch.Generator().manual_seed(n)
    lo, hi = np.float32(near), np.float32(far)
    depths = torch.exp(torch.rand(n, generator=g, dtype=torch.float64) * (math.log(hi) - math.log(lo))
                       + math.log(lo)).float()
    depths = torch.clamp(depths, float(np.nextafter(lo, hi)), float(np.nextafter(hi, lo)))
    if n >= 8:
        depths[: n // 8] = depths[n // 8 : n // 4]  # ties
        depths[n // 4] = float(np.nextafter(lo, hi))  # just inside the near plane
        depths[n // 4 + 1] = float(np.nextafter(hi, lo))  # just inside the far plane
    keys_o, ids_o = orc.emit_intersections(bounds.numpy(), depths.numpy(), counts.numpy(), tiles_w)
    sid_o, ranges_o, _ = orc.sort_intersections(keys_o, ids_o, tiles_w * tiles_h)
    print(f"remapped depth keys near={near} far={far} bits={key_range[1]} n={n} "
          f"intersections={len(sid_o)}", flush=True)
    sid, ranges = bin_tiles(_depth_keys(depths, counts).to(device), bounds.to(device),
                            counts.to(device), tiles_w, tiles_h, key_range=key_range)
    assert np.array_equal(ranges.cpu().numpy(), ranges_o)
    assert np.array_equal(sid.cpu().numpy(), sid_o)


def test_bucketed_binning_long_rows(device):
    """Rows holding many workgroups of intersections (full-width rectangles)
    and Gaussians spanning many rows, so both passes chain look-backs across
    several workgroups of one digit."""
    g = torch.Generator().manual_seed(11)
    n, tiles_w, tiles_h = 3000, 200, 40
    x0 = torch.randint(0, 20, (n,), generator=g)
    x1 = torch.randint(180, tiles_w + 1, (n,), generator=g)
    y0 = torch.randint(0, tiles_h, (n,), generator=g)
    y1 = torch.minimum(y0 + torch.randint(1, 30, (n,), generator=g), torch.tensor(tiles_h))
    bounds = torch.stack((torch.stack((x0, x1), -1), torch.stack((y0, y1), -1)), 1).int()
    depths = (torch.rand(n, generator=g) * 4).round() + 1.0  # many exact ties
    counts = ((x1 - x0) * (y1 - y0)).int()
    keys_o, ids_o = orc.emit_intersections(bounds.numpy(), depths.numpy(), counts.numpy(), tiles_w)
    sid_o, ranges_o, _ = orc.sort_intersections(keys_o, ids_o, tiles_w * tiles_h)
    print(f"long rows intersections={len(sid_o)}", flush=True)
    sid, ranges = bin_tiles(
        _depth_keys(depths, counts).to(device), bounds.to(device), counts.to(device), tiles_w, tiles_h
    )
    assert np.array_equal(ranges.cpu().numpy(), ranges_o)
    assert np.array_equal(sid.cpu().numpy(), sid_o)


def test_bucketed_binning_mosaic_windows(device):
    """A 200 x 200 grid (tables larger than LDS) whose Gaussians come in four
    groups confined to 100 x 100 blocks, as a multi-view mosaic's are: chunks
    inside one block accumulate their corners in an LDS window, chunks that
    straddle two blocks fall back to global atomics; both must give the
    oracle's lists."""
    g = torch.Generator().manual_seed(5)
    per, tiles_w, tiles_h = 20_000, 200, 200
    rects, depth_list = [], []
    for v in range(4):
        ox, oy = (v % 2) * 100, (v // 2) * 100
        x0 = torch.randint(0, 97, (per,), generator=g) + ox
        y0 = torch.randint(0, 97, (per,), generator=g) + oy
        x1 = x0 + torch.randint(1, 4, (per,), generator=g)
        y1 = y0 + torch.randint(1, 4, (per,), generator=g)
        rects.append(torch.stack((torch.stack((x0, x1), -1), torch.stack((y0, y1), -1)), 1))
        depth_list.append(torch.rand(per, generator=g) * 2 + 2.0)  # one exponent: shared digits
    bounds = torch.cat(rects).int()
    depths = torch.cat(depth_list)
    counts = ((bounds[:, 0, 1] - bounds[:, 0, 0]) * (bounds[:, 1, 1] - bounds[:, 1, 0])).int()
    counts[torch.rand(4 * per, generator=g) < 0.3] = 0  # culled
    keys_o, ids_o = orc.emit_intersections(bounds.numpy(), depths.numpy(), counts.numpy(), tiles_w)
    sid_o, ranges_o, _ = orc.sort_intersections(keys_o, ids_o, tiles_w * tiles_h)
    print(f"mosaic windows intersections={len(sid_o)}", flush=True)
    sid, ranges = bin_tiles(
        _depth_keys(depths, counts).to(device), bounds.to(device), counts.to(device), tiles_w, tiles_h
    )
    assert np.array_equal(ranges.cpu().numpy(), ranges_o)
    assert np.array_equal(sid.cpu().numpy(), sid_o)


def test_bucketed_binning_empty_and_deterministic(device):
    bounds = torch.zeros(5, 2, 2, dtype=torch.int32, device=device)
    counts = torch.zeros(5, dtype=torch.int32, device=device)
    sid, ranges = bin_tiles(torch.full((5,), -1, dtype=torch.int32, device=device), bounds, counts, 4, 3)
    assert sid.numel() == 0 and torch.equal(ranges.cpu(), torch.zeros(12, 2, dtype=torch.int64))
    sid, ranges = bin_tiles(
        torch.empty(0, dtype=torch.int32, device=device), bounds[:0], counts[:0], 4, 3
    )
    assert sid.numel() == 0 and torch.equal(ranges.cpu(), torch.zeros(12, 2, dtype=torch.int64))
    b, d, c = _random_rects(n=20000, tiles_w=120, tiles_h=68, seed=3)
    outs = [
        [t.cpu() for t in bin_tiles(_depth_keys(d, c).to(device), b.to(device), c.to(device), 120, 68)]
        for _ in range(2)
    ]
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("n, words", [(20000, 20000 * 9), (0, 4 * 9 + 1)])
def test_bucketed_binning_clears_the_given_buffer(device, n, words):
    """bin_tiles zeroes its `clear` buffer (the op's gradient accumulator) on
    the side stream before it returns; the lists are those of a call without
    it.  Word counts that are not a multiple of four take the tail path; with
    no Gaussians only the side stream's work runs."""
    b, d, c = _random_rects(n=max(n, 1), tiles_w=120, tiles_h=68, seed=5)
    b, d, c = b[:n], d[:n], c[:n]
    buf = torch.full((words,), 3.5, dtype=torch.float32, device=device)
    print(f"[clear] n={n} words={words}", flush=True)
    sid, rng = bin_tiles(_depth_keys(d, c).to(device), b.to(device), c.to(device), 120, 68,
                         clear=buf)
    assert not bool(buf.ne(0).any())
    sid2, rng2 = bin_tiles(_depth_keys(d, c).to(device), b.to(device), c.to(device), 120, 68)
    assert torch.equal(sid, sid2) and torch.equal(rng, rng2)


def test_intersections_empty(device):
    bounds = torch.zeros(5, 2, 2, dtype=torch.int32, device=device)
    counts = torch.zeros(5, dtype=torch.int32, device=device)
    keys, ids = emit_intersections(bounds, torch.ones(5, device=device), counts, 4)
    assert keys.numel() == 0
    sid, ranges = sort_intersections(keys, ids, 12)
    assert sid.numel() == 0 and torch.equal(ranges.cpu(), torch.zeros(12, 2, dtype=torch.int64))


def test_intersections_deterministic(device):
    bounds, depths, counts = _random_rects(n=20000, tiles_w=120, tiles_h=68, seed=3)
    outs = []
    for _ in range(2):
        dkeys = depths.view(torch.int32).clone().to(device)
        order, offsets = bin_gaussians(dkeys, counts.to(device))
        tk, tid = emit_tiles(bounds.to(device), order, offsets, int(offsets[-1]), 120)
        outs.append([t.cpu() for t in sort_tiles(tk, tid, 120 * 68)])
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def _oracle_lists(proj, bounds, counts, w, h, tile_size):
    tw, th = nat.tiles(w, h, tile_size)
    keys, ids = orc.emit_intersections(bounds, proj.mean[:, 2].float().numpy(), counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
    return sid, ranges


@pytest.mark.parametrize("tile_size", (4, 8, 16, 32))
@pytest.mark.parametrize("mode", ("gaussian", "ellipsoid"))
def test_composite_matches_oracle(device, tile_size, mode):
    scene = scenes.edge_case_scene(n=1500, sh_degree=1, image_size=(96, 80))
    cam = scene.cameras[0]
    w, h = cam.image_size
    proj = orc.project(*scene.params(), oracle_camera(cam))
    tw, th = nat.tiles(w, h, tile_size)
    bounds, counts = orc.tile_counts(proj, tile_size, tw, th, scene.near, scene.far, mode, CONFIDENCE)
    sid, ranges = _oracle_lists(proj, bounds, counts, w, h, tile_size)
    exp = orc.composite(
        proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0], proj.inverse[:, 0, 1],
        proj.inverse[:, 1, 1], proj.color, proj.opacity[:, 0], sid, ranges, w, h, tile_size,
        THRESHOLD, mode, CONFIDENCE,
    )
    image, final_t, ncon = composite(
        proj.mean.float().to(device), proj.inverse.float().to(device), proj.color.float().to(device),
        proj.opacity.float().to(device), torch.as_tensor(sid).to(device),
        torch.as_tensor(ranges).to(device), w, h, tile_size, THRESHOLD, mode, CONFIDENCE,
    )
    assert_close_flip_aware(image.cpu(), exp.image, exp.margin, atol=1e-5, what="image")
    assert_close_flip_aware(final_t.cpu(), exp.final_transmittance, exp.margin, atol=1e-5, rtol=1e-4,
                            what="final_transmittance")
    ok = exp.margin >= 1e-4
    assert torch.equal(ncon.cpu()[ok], exp.n_contributors[ok])
    cols = [proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0], proj.inverse[:, 0, 1],
            proj.inverse[:, 1, 1], proj.color, proj.opacity[:, 0]]
    assert_forward_every_pixel(image.cpu(), final_t.cpu(), ncon.cpu(), cols, sid, ranges, w, h,
                               tile_size, rendering_mode=mode, confidence=CONFIDENCE,
                               what=f"image {mode} tile {tile_size}")


def test_composite_empty_tiles(device):
    """Known answer: empty ranges give a black image (test_composite.py:19-25)."""
    n = 10
    z = torch.zeros(n, 3, device=device)
    inv = torch.eye(2, device=device).repeat(n, 1, 1)
    image, final_t, ncon = composite(
        z, inv, z, torch.ones(n, 1, device=device), torch.zeros(0, dtype=torch.int32, device=device),
        torch.zeros(6 * 5, 2, dtype=torch.int64, device=device), 90, 70, 16, THRESHOLD, "gaussian", 0.95,
    )
    assert torch.count_nonzero(image) == 0
    assert torch.all(final_t == 1) and torch.count_nonzero(ncon) == 0


@pytest.mark.parametrize("scene_kind, tile", [("edge96x64", 8), ("config2", 16), ("edge1040", 16),
                                              ("edge160x96", 32)])
def test_forward_writes_backward_plan_keys(device, scene_kind, tile):
    """The keys the forward's whole-tile walks write (gs_composite's
    tile_keys) equal the key kernel's, from the same n_contributors and
    ranges, and the backward plan made from them (keys_ready) equals the one
    made without.  When every tile ran as quarters (fewer than 4096 tiles
    with work, tiles of 16 and 32) the forward writes none and the plan
    recomputes them."""
    if scene_kind == "config2":
        scene = scenes.config2(n=40_000)
    else:
        size = {"edge96x64": (96, 64), "edge1040": (1040, 1040), "edge160x96": (160, 96)}[scene_kind]
        scene = scenes.edge_case_scene(n=3000, sh_degree=1, image_size=size)
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    params = [t.to(device) for t in scene.params()]
    pmean, pinv, pcol, pop, _, _ = project_and_count(
        *params, cam.rotation_matrix, cam.translation, fx, fy, cx, cy, w, h, tile, scene.near,
        scene.far, "gaussian", CONFIDENCE)
    tw, th = nat.tiles(w, h, tile)
    lib = nat.library()
    keys_fwd = nat.workspace(lib.gs_tile_order_workspace_bytes(tw * th), device)
    keys_fwd.fill_(0x5A)
    out = forward_lists(params, cam, scene, tile, device)
    sid, ranges = out
    active = nat.active_tiles(ranges)
    whole_tiles = tile not in (16, 32) or active >= 4096
    print(f"[plan keys] {scene_kind} tile {tile}: {active} active tiles, forward keys "
          f"{whole_tiles}", flush=True)
    if scene_kind == "config2":
        assert whole_tiles  # the case the forward's keys serve
    _, _, ncon = composite(pmean, pinv, pcol, pop, sid, ranges, w, h, tile, THRESHOLD, "gaussian",
                           CONFIDENCE, tile_keys=keys_fwd)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, tile, opacity_threshold=THRESHOLD,
                         active_tiles=nat.active_tiles(ranges))
    count = lib.gs_tile_order_items(view, 1)
    items = [torch.full((count,), -9, dtype=torch.int32, device=device) for _ in range(2)]
    keys_kernel = nat.workspace(lib.gs_tile_order_workspace_bytes(tw * th), device)
    s = nat.stream(device)
    nat.check(lib.gs_tile_order(nat.ptr(ranges), nat.ptr(ncon), view, nat.ptr(items[0]),
                                nat.ptr(keys_kernel), keys_kernel.numel(), 0, s), "tile_order")
    nat.check(lib.gs_tile_order(nat.ptr(ranges), nat.ptr(ncon), view, nat.ptr(items[1]),
                                nat.ptr(keys_fwd), keys_fwd.numel(), 1, s), "tile_order")
    torch.cuda.synchronize(device)
    assert torch.equal(items[0], items[1])
    nbytes = 2 * tw * th * 4  # both words of every tile
    assert torch.equal(keys_fwd[:nbytes], keys_kernel[:nbytes])


def forward_lists(params, cam, scene, tile, device):
    """Sorted ids and ranges of the op's binning for one camera."""
    from gaussian_splats_hip.kernels.rasterize.interface import forward_pipeline

    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    out = forward_pipeline(*params, cam.rotation_matrix, cam.translation, fx, fy, cx, cy, w, h,
                           tile, THRESHOLD, scene.near, scene.far, "gaussian", CONFIDENCE,
                           record_hits=False)
    return out[7], out[8]


@pytest.mark.parametrize(
    "shape", [(120, 68, 16, 0), (120, 68, 16, 3000), (7, 5, 8, 0), (1, 1, 16, 0), (33, 2, 4, 0),
              (100, 100, 16, 0), (60, 40, 32, 0)])
def test_dispatch_plan_matches_model(device, shape):
    """gs_tile_order's work items equal the plan's model (expected_plan) for
    both work estimates: list lengths (ranges, a forward plan) and the
    largest contributor count per tile with the ranges (a backward plan,
    which cuts the walks at the forward's checkpoints); every tile is covered
    exactly once: whole, as its four quarters in one workgroup's four slots,
    or as its segments 0..c in consecutive slots."""
    from gaussian_splats_hip.kernels.rasterize.composite import tile_order

    tw, th, tile, active = shape
    w, h = tw * tile - 3, th * tile - 1  # partial edge tiles
    tw, th = nat.tiles(w, h, tile)
    t = tw * th
    rng = np.random.default_rng(t + active)
    lengths = rng.integers(0, 3000, size=t)
    lengths[rng.random(t) < 0.1] = 0
    lengths[: min(3, t)] = 70000  # capped at 2^16 - 1: ties broken by index
    ranges = np.zeros((t, 2), dtype=np.int64)
    ranges[:, 1] = np.cumsum(lengths)
    ranges[1:, 0] = ranges[:-1, 1]

    def check_cover(items):
        used = items[items >= 0]
        tiles, code = used >> 7, used & 0x7F
        covered = np.bincount(tiles, minlength=t)
        assert np.all(covered >= 1)
        whole = code == 0
        assert np.all(covered[tiles[whole]] == 1)
        quarters = np.flatnonzero((items >= 0) & ((items & 0x60) == 0x20))
        assert np.all(items[quarters] & 3 == quarters % 4)  # quarter q in a workgroup's slot q
        segs = np.flatnonzero((items >= 0) & ((items & 0x40) != 0))
        first = segs - (items[segs] & 0x3F)  # a tile's segments fill consecutive slots
        assert np.all((items[first] >> 7 == items[segs] >> 7) & ((items[first] & 0x7F) == 0x40))

    items = tile_order(torch.as_tensor(ranges).to(device), None, w, h, tile,
                       active_tiles=active).cpu().numpy()
    np.testing.assert_array_equal(items, expected_plan(lengths, tile, active))
    check_cover(items)

    ncon = rng.integers(0, 500, size=(h, w)).astype(np.int32)
    ncon[:tile, :tile] = 20000  # a long walk: many checkpoint crossings
    ranges_d = torch.as_tensor(ranges).to(device)
    items = tile_order(ranges_d, torch.as_tensor(ncon).to(device), w, h, tile,
                       active_tiles=active).cpu().numpy()
    walks = plan_tile_keys(ncon=ncon, width=w, height=h, tile_size=tile)
    np.testing.assert_array_equal(
        items, expected_plan(walks, tile, active, backward=True,
                             crossings=plan_crossings(ranges, walks)))
    check_cover(items)
    if not plan_slots(t, tile, active, backward=True)[2]:
        assert np.any((items >= 0) & ((items & 0x40) != 0))  # some tile was segmented


@pytest.mark.parametrize("tile_size,image_size", [(8, (96, 80)), (16, (96, 80)),
                                                   (16, (1100, 1000))])
def test_compositing_results_do_not_depend_on_tile_order(device, tile_size, image_size):
    """The forward is bit-identical under every dispatch (index order, a plan
    with quarter items, every tile split); the backward equal up to the order
    of the float atomics."""
    scene = scenes.edge_case_scene(n=1500, sh_degree=1, image_size=image_size)
    cam = scene.cameras[0]
    w, h = cam.image_size
    proj = orc.project(*scene.params(), oracle_camera(cam))
    tw, th = nat.tiles(w, h, tile_size)
    bounds, counts = orc.tile_counts(proj, tile_size, tw, th, scene.near, scene.far, "gaussian", CONFIDENCE)
    sid, ranges = _oracle_lists(proj, bounds, counts, w, h, tile_size)
    args = [t.float().to(device) for t in (proj.mean, proj.inverse, proj.color, proj.opacity)]
    sid_d, ranges_d = torch.as_tensor(sid).to(device), torch.as_tensor(ranges).to(device)
    image, final_t, ncon = composite(*args, sid_d, ranges_d, w, h, tile_size, THRESHOLD, "gaussian",
                                     CONFIDENCE)
    # The same launch through the C ABI under other dispatches.
    from gaussian_splats_hip.kernels.rasterize import composite_bwd
    from gaussian_splats_hip.kernels.rasterize.composite import tile_order
    from gaussian_splats_hip.kernels.rasterize.project import pack_records

    records = pack_records(*args, "gaussian", CONFIDENCE)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, tile_size, opacity_threshold=THRESHOLD)

    def forward(order, v=view):
        img2 = torch.empty_like(image)
        ft2 = torch.empty_like(final_t)
        nc2 = torch.empty_like(ncon)
        nat.check(nat.library().gs_composite(
            nat.ptr(records), records.shape[0], nat.ptr(sid_d), sid_d.numel(), nat.ptr(ranges_d),
            nat.ptr(order), v, nat.ptr(img2), nat.ptr(ft2), nat.ptr(nc2), None, 0,
            None, 0, None, 0, nat.stream(device)), "composite")
        torch.cuda.synchronize()
        # The wrapper's walk records checkpoints, which sums each pixel's
        # colour in segments (rounding of the order of the sums).
        assert torch.equal(final_t, ft2) and torch.equal(ncon, nc2)
        assert float((image - img2).abs().max()) <= 1e-6

    # Tiles in index order, and a plan whose heaviest tiles run as quarters.
    forward(None)
    order = tile_order(ranges_d, None, w, h, tile_size)
    _, _, split_all = plan_slots(tw * th, tile_size)
    used = order.cpu().numpy()
    used = used[used >= 0]
    assert bool((used & 0x20).any()) == split_all
    forward(order)
    # Every tile split into quarters (few tiles with work).
    few = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, tile_size, opacity_threshold=THRESHOLD,
                        active_tiles=1)
    forward(None, few)
    forward(tile_order(ranges_d, None, w, h, tile_size, active_tiles=1), few)

    # Backward: the wrapper dispatches by contributor count (heavy tiles in
    # segments); the identity order gives the same gradient up to the order
    # of the atomic adds and the segments' recombination.
    g = torch.randn(h, w, 3, generator=torch.Generator().manual_seed(5)).to(device)
    grad = composite_bwd(*args, sid_d, ranges_d, g, final_t, ncon, w, h, tile_size, THRESHOLD,
                         "gaussian")
    grad2 = torch.zeros_like(grad)
    nat.check(nat.library().gs_composite_bwd(
        *(nat.ptr(t) for t in args), args[0].shape[0], nat.ptr(sid_d), nat.ptr(ranges_d), nat.ptr(g),
        nat.ptr(final_t), nat.ptr(ncon), None, view, nat.ptr(grad2), None, None, 0, 0,
        None, 0, nat.stream(device)), "composite_bwd")
    torch.cuda.synchronize()
    # Float atomics make both sums order-dependent: compare against the scale
    # of each gradient column (a skipped or repeated tile would be O(1) off).
    scale = grad2.abs().amax(dim=0, keepdim=True).clamp_min(1e-30)
    assert float(((grad - grad2).abs() / scale).max()) < 1e-4
    # The wrapper's backward walked the forward's hit masks; here a forward
    # whose tiles all ran as quarters (each band's wave stops at its own
    # pixels) writes them over a buffer of ones, and a backward of whole
    # tiles reads them: only the words each band's wave wrote may count.
    lib = nat.library()
    words = lib.gs_composite_hit_mask_bytes(few, sid_d.numel()) // 8
    hits = torch.full((words,), -1, dtype=torch.int64, device=device)
    img3, ft3, nc3 = torch.empty_like(image), torch.empty_like(final_t), torch.empty_like(ncon)
    nat.check(lib.gs_composite(
        nat.ptr(records), records.shape[0], nat.ptr(sid_d), sid_d.numel(), nat.ptr(ranges_d), None,
        few, nat.ptr(img3), nat.ptr(ft3), nat.ptr(nc3), None, 0, nat.ptr(hits), words * 8,
        None, 0, nat.stream(device)), "composite")
    grad3 = torch.zeros_like(grad)
    nat.check(lib.gs_composite_bwd(
        *(nat.ptr(t) for t in args), args[0].shape[0], nat.ptr(sid_d), nat.ptr(ranges_d), nat.ptr(g),
        nat.ptr(ft3), nat.ptr(nc3), None, view, nat.ptr(grad3), None, None, 0, sid_d.numel(),
        nat.ptr(hits), words * 8, nat.stream(device)), "composite_bwd")
    torch.cuda.synchronize()
    assert torch.equal(final_t, ft3) and torch.equal(ncon, nc3)
    assert float(((grad3 - grad2).abs() / scale).max()) < 1e-4


def test_device_check_failures_reach_the_host(device):
    """A binning pass handed sizes that differ from its plan's device totals
    (here one row-list entry too many) leaves every workgroup at once and
    sets the size-mismatch bit of the device's sticky check word (no kernel
    waits or reads out of bounds on that path: the row and column passes
    return before any other access, and the width scan in between clamps its
    reads and bounds its writes).  The bit reaches the host through
    gs_device_errors and through the next binning call's totals, which
    raises once; the call after that runs normally."""
    from ctypes import c_void_p

    lib = nat.library()
    assert nat.device_errors(device, clear=True) == 0, "an earlier test left a device check failure"
    b, d, c = _random_rects(n=3000, tiles_w=24, tiles_h=17, seed=9)
    bounds, counts = b.to(device), c.to(device)
    keys = _depth_keys(d, c).to(device)
    n, tw, th = 3000, 24, 17
    s = nat.stream(device)
    plan = nat.workspace(lib.gs_bin_tiles_plan_bytes(n, tw, th), device)
    ranges = torch.empty((tw * th, 2), dtype=torch.int64, device=device)
    totals = torch.empty(4, dtype=torch.int64, device=device)
    host = torch.zeros(5, dtype=torch.int64, pin_memory=True)
    rects = torch.empty(n, dtype=torch.int32, device=device)
    nat.check(lib.gs_pack_tile_rects(nat.ptr(bounds), nat.ptr(counts), n, tw, th, nat.ptr(rects),
                                     s), "pack")
    print("[device checks] plan", flush=True)
    nat.check(lib.gs_bin_tiles_plan(nat.ptr(keys), nat.ptr(rects), n, 0, 32, tw, th,
                                    nat.ptr(ranges), nat.ptr(totals), c_void_p(host.data_ptr()),
                                    nat.ptr(plan), plan.numel(), None, 0, s), "plan")
    total, rows, blocks, _, flags = host.tolist()
    assert flags == 0 and total > 0
    wrong_rows = rows + 1
    ws = nat.workspace(lib.gs_bin_tiles_emit_bytes(n, total, wrong_rows, blocks, tw, th), device)
    ids = torch.zeros(total, dtype=torch.int32, device=device)
    print("[device checks] emit with a wrong row-entry count", flush=True)
    nat.check(lib.gs_bin_tiles_emit(n, tw, th, nat.ptr(totals), total, wrong_rows, blocks,
                                    nat.ptr(plan), plan.numel(), nat.ptr(ranges), nat.ptr(ids),
                                    nat.ptr(ws), ws.numel(), s), "emit")
    assert nat.device_errors(device, clear=False) == 4  # GS_DEVICE_SIZE_MISMATCH
    # The next binning call sees the word beside its totals and raises once.
    keys2 = _depth_keys(d, c).to(device)
    with pytest.raises(RuntimeError, match="differ from the plan"):
        bin_tiles(keys2, bounds, counts, tw, th)
    assert nat.device_errors(device, clear=False) == 0
    sid, rng = bin_tiles(_depth_keys(d, c).to(device), bounds, counts, tw, th)
    ekeys, eids = orc.emit_intersections(b.numpy(), d.numpy(), c.numpy(), tw)
    esid, erng, _ = orc.sort_intersections(ekeys, eids, tw * th)
    assert np.array_equal(sid.cpu().numpy(), esid) and np.array_equal(rng.cpu().numpy(), erng)
    nat.check_device_errors(device)
