"""Parity at the benchmark workloads (configurations 2-5 of the north star) on
full-size scenes, against the CPU oracle (restating the reference's
kernels/rasterize/torch.py:228-247):

* projection of every Gaussian (floats to float32 rounding, depth bits exact)
  and its tile rectangle (exact away from a floor at a tile edge);
* the intersection lists of every tile, proved exact (per-tile lengths equal a
  2-D histogram of the rectangles, every entry covers its tile, strictly
  increasing (depth bits, index) keys), and for configurations 2 and 3 also
  compared with numpy's stable sort of the reference-format keys;
* image, transmittance and contributor counts on 32 seeded tiles including
  the 4 longest lists, against the oracle's own lists of those tiles;
* gradients of the mean-L1 loss restricted to those tiles against float64
  autograd of the oracle, every Gaussian compared (see tests/parity.py);
* configuration 5 through the multi-view op, per view against the oracle.

The oracle runs on the host; torch on the GPU is used only as a checker
(the list proof and the loss weights).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from gaussian_splats_hip import scenes
from gaussian_splats_hip.kernels.rasterize import _native as nat
from gaussian_splats_hip.kernels.rasterize import composite_bwd, project_and_count, project_bwd
from gaussian_splats_hip.kernels.rasterize.interface import forward_pipeline, rasterize_outputs
from gaussian_splats_hip.kernels.rasterize.views import (
    camera_tensors,
    mosaic_columns,
    rasterize_views_outputs,
)
from oracle import rasterizer as orc
from parity import (
    DECISION_WINDOW,
    FLOAT32_SAMPLES,
    assert_close_flip_aware,
    assert_close_to_truth,
    assert_forward_every_pixel,
    assert_gradients_close,
    fixed_decision_composite_grads,
    fixed_decision_rasterize_grads,
    assert_lists_exact,
    oracle_camera,
    oracle_tile_lists,
    rect_flip_tolerant_equal,
    restrict_lists,
    sample_tiles,
    tile_max,
    tile_pixel_mask,
    ulp_perturbed,
)

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

TILE = 16
THRESHOLD = 0.999
CHUNK = 4  # tiles per oracle compositing chunk (bounds its memory)
TRUNCATE_SLACK = 64  # entries kept past a tile's largest contributor count


def log(*args):
    print("[configs]", *args, flush=True)


_cache: dict = {}


def single_view(name, device):
    """GPU forward of a single-view configuration (the op's ten outputs and the
    projection's rectangles) and the float32 oracle's projection and
    rectangles; one configuration cached at a time."""
    if name in _cache:
        return _cache[name]
    _cache.clear()
    torch.cuda.empty_cache()
    log(name, "scene")
    scene = scenes.CONFIGS[name]()
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    params = [t.to(device) for t in scene.params()]
    args = (cam.rotation_matrix.to(device), cam.translation.to(device), fx, fy, cx, cy, w, h, TILE)
    log(name, "GPU forward")
    out = forward_pipeline(*params, *args, THRESHOLD, scene.near, scene.far, "gaussian", 0.95)
    bounds = project_and_count(*params, *args, scene.near, scene.far, "gaussian", 0.95)[4]
    torch.cuda.synchronize()
    nat.check_device_errors(device)
    log(name, "oracle projection")
    proj = orc.project(*scene.params(), oracle_camera(cam))
    tw, th = nat.tiles(w, h, TILE)
    obounds, ocounts = orc.tile_counts(proj, TILE, tw, th, scene.near, scene.far)
    r = dict(scene=scene, params=params, out=out, bounds=bounds, proj=proj, obounds=obounds,
             ocounts=ocounts, tw=tw, th=th, w=w, h=h, cam=cam)
    _cache[name] = r
    return r


def check_projection(pmean, pinv, pcol, pop, gbounds, gcounts, proj, obounds, ocounts, what,
                     params, cam):
    """Projected floats against the float64 oracle (2e-6 / 1e-5 relative, or
    within the float32 oracle's error scale on the Gaussian, see
    assert_close_to_truth: the 2x2 inversion loses the condition number's
    worth of digits in any float32 evaluation), depth bits exact against the
    float32 oracle (same operation order), rectangles exact away from tile
    edges, counts equal where the rectangles are."""
    n = pmean.shape[0]
    ocam = oracle_camera(cam)
    proj64 = orc.project(*(p.double() for p in params), ocam)
    samples = [proj] + [orc.project(*ulp_perturbed(params, k), ocam)
                        for k in range(1, FLOAT32_SAMPLES)]
    visible = torch.as_tensor(ocounts > 0)
    stats = {}
    stats["uv"] = assert_close_to_truth(pmean[:, :2], proj64.mean[:, :2],
                                        [q.mean[:, :2] for q in samples], 2e-6, 1e-5,
                                        f"{what} pixel means")
    stats["inverse"] = assert_close_to_truth(pinv.reshape(n, 4), proj64.inverse.reshape(n, 4),
                                             [q.inverse.reshape(n, 4) for q in samples], 1e-5,
                                             1e-7, f"{what} inverse covariance", rows=visible)
    stats["color"] = assert_close_to_truth(pcol, proj64.color, [q.color for q in samples], 1e-5,
                                           1e-6, f"{what} colour")
    stats["opacity"] = assert_close_to_truth(pop, proj64.opacity, [q.opacity for q in samples],
                                             1e-6, 1e-7, f"{what} opacity")
    log(what, "projection", stats)
    assert torch.equal(pmean[:, 2], proj.mean[:, 2].float()), f"{what}: depth bits differ"
    extent = 2 * np.sqrt(np.log(proj.opacity[:, 0].double().numpy() * 255))
    with np.errstate(invalid="ignore"):
        flips = rect_flip_tolerant_equal(gbounds, obounds, proj, TILE, extent)
    same = np.all(gbounds == obounds, axis=(1, 2))
    assert np.array_equal(gcounts[same], ocounts[same]), f"{what}: counts differ"
    n = len(ocounts)
    log(what, f"rectangle flips at tile edges: {flips} of {n}")
    assert flips <= max(4, n // 20000), f"{what}: {flips} edge flips"


@pytest.mark.parametrize("name", ("config2", "config3", "config4"))
def test_projection_matches_oracle(device, name):
    r = single_view(name, device)
    pmean, pinv, pcol, pop = (t.cpu() for t in r["out"][3:7])
    counts = r["out"][9].cpu().numpy()
    check_projection(pmean, pinv, pcol, pop, r["bounds"].cpu().numpy(), counts, r["proj"],
                     r["obounds"], r["ocounts"], name, r["scene"].params(), r["cam"])


@pytest.mark.parametrize("name", ("config2", "config3", "config4"))
def test_lists_exact(device, name):
    r = single_view(name, device)
    out = r["out"]
    gids, ranges, counts, pmean = out[7], out[8], out[9], out[3]
    log(name, f"list proof over {gids.numel()} intersections")
    stats = assert_lists_exact(gids, ranges, r["bounds"], counts, pmean[:, 2], r["tw"])
    log(name, stats)
    if name in ("config2", "config3"):
        # Also against numpy's stable sort of the reference-format keys
        # (tile << 32 | depth bits), emitted Gaussian-major as the reference does.
        keys, ids = orc.emit_intersections(r["bounds"].cpu().numpy(), pmean[:, 2].cpu().numpy(),
                                           counts.cpu().numpy(), r["tw"])
        sid, rng, _ = orc.sort_intersections(keys, ids, r["tw"] * r["th"])
        assert np.array_equal(gids.cpu().numpy(), sid)
        assert np.array_equal(ranges.cpu().numpy(), rng)


def _sampled_forward(r, name, seed=0):
    """The oracle's own lists of 32 sampled tiles (cut TRUNCATE_SLACK entries
    past the GPU's largest contributor count of each tile: the oracle must
    then stop earlier, which is asserted) composited in float32."""
    out = r["out"]
    ranges = out[8].cpu().numpy()
    ncon = out[2].cpu().numpy()
    tiles = sample_tiles(ranges, seed=seed)
    limits = {t: m + TRUNCATE_SLACK for t, m in tile_max(ncon, tiles, r["tw"], TILE).items()}
    proj = r["proj"]
    ids, rng = oracle_tile_lists(r["obounds"], r["ocounts"], proj.mean[:, 2].float().numpy(), tiles,
                                 r["tw"], r["tw"] * r["th"], limits)
    lengths = rng[:, 1] - rng[:, 0]
    log(name, f"oracle compositing {len(tiles)} tiles, {int(lengths.sum())} entries "
              f"(longest {int(lengths.max())})")
    comp = orc.composite(proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0],
                         proj.inverse[:, 0, 1], proj.inverse[:, 1, 1], proj.color,
                         proj.opacity[:, 0], ids, rng, r["w"], r["h"], TILE, THRESHOLD,
                         tile_chunk=CHUNK)
    onc = comp.n_contributors.numpy()
    full = np.asarray(out[8].cpu().numpy())
    for t in tiles:
        if limits[t] < full[t, 1] - full[t, 0]:  # cut: the oracle must have stopped before
            assert tile_max(onc, [t], r["tw"], TILE)[int(t)] < limits[t], f"tile {t} cut too early"
    return tiles, comp


@pytest.mark.parametrize("name", ("config2", "config3", "config4"))
def test_sampled_tiles_forward(device, name):
    r = single_view(name, device)
    tiles, comp = _sampled_forward(r, name)
    mask = torch.as_tensor(tile_pixel_mask(tiles, r["tw"], TILE, r["w"], r["h"]))
    image, final_t, ncon = (t.cpu() for t in r["out"][:3])
    margin = torch.where(mask, torch.as_tensor(comp.margin), torch.full_like(comp.margin, math.inf))
    stats = assert_close_flip_aware(image[mask], comp.image[mask], margin[mask], atol=1e-5,
                                    what=f"{name} image")
    log(name, "image", stats)
    assert_close_flip_aware(final_t[mask], comp.final_transmittance[mask], margin[mask], atol=1e-5,
                            rtol=1e-4, what=f"{name} transmittance")
    ok = mask & (torch.as_tensor(comp.margin) >= 1e-4)
    assert torch.equal(ncon[ok], comp.n_contributors[ok]), f"{name}: contributor counts differ"
    # Every pixel of those tiles, near a decision or not, against float64
    # along the GPU's own lists and decisions.
    out = r["out"]
    ids, rng = restrict_lists(out[7].cpu().numpy(), out[8].cpu().numpy(), tiles,
                              {t: m + TRUNCATE_SLACK for t, m in
                               tile_max(ncon.numpy(), tiles, r["tw"], TILE).items()})
    stats = assert_forward_every_pixel(image, final_t, ncon, _gpu_columns(out), ids, rng, r["w"],
                                       r["h"], TILE, mask=mask, tile_chunk=CHUNK,
                                       what=f"{name} image")
    log(name, "every pixel", stats)


def _gpu_columns(out, view=None):
    """The GPU's projected values as the oracle's compositing columns (u, v,
    inv00, inv01, inv11, rgb, alpha0), of one view for the multi-view op."""
    pm, pinv, pcol, pop = (t.detach().cpu() if view is None else t[view].detach().cpu()
                           for t in out[3:7])
    return [pm[:, 0], pm[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1], pcol, pop[:, 0]]


def _loss_weights(image, target, mask):
    """dL/dimage of L = mean |image - target| restricted to the masked pixels
    (the loss of configurations 3-5, summed over the sampled tiles only)."""
    g = torch.sign(image.detach() - target) / image.numel()
    return g * mask[..., None].to(g.device, g.dtype)


@pytest.mark.parametrize("name", ("config3", "config4"))
def test_sampled_tiles_composite_backward(device, name):
    """composite_bwd at full size with the loss restricted to the sampled
    tiles, on the GPU's own projected values and lists."""
    r = single_view(name, device)
    out = r["out"]
    image, final_t, ncon, pm, pinv, pcol, pop, gids, granges, counts = out
    tiles = sample_tiles(granges.cpu().numpy(), seed=1)
    mask = torch.as_tensor(tile_pixel_mask(tiles, r["tw"], TILE, r["w"], r["h"]))
    weights = _loss_weights(image, r["scene"].target.to(device), mask)
    grad = composite_bwd(pm, pinv, pcol, pop, gids, granges, weights.contiguous(), final_t, ncon,
                         r["w"], r["h"], TILE, THRESHOLD, "gaussian").cpu()
    ncon_h = ncon.cpu().numpy()
    limits = {t: m + 1 for t, m in tile_max(ncon_h, tiles, r["tw"], TILE).items()}
    ids, rng = restrict_lists(gids.cpu().numpy(), granges.cpu().numpy(), tiles, limits)
    log(name, f"float64 reference over {len(ids)} entries")
    pm, pinv, pcol, pop = (t.cpu() for t in (pm, pinv, pcol, pop))
    cols32 = (pm[:, 0], pm[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1], pcol, pop[:, 0])
    expected, expected32, cut_margin, _ = fixed_decision_composite_grads(
        cols32, ids, rng, r["w"], r["h"], TILE, ncon_h, weights.cpu(), tile_chunk=CHUNK)
    explained = cut_margin < DECISION_WINDOW
    stats = assert_gradients_close(grad, expected, f"{name} composite_bwd", explained=explained,
                                   reference32=expected32)
    log(name, "composite_bwd", stats, "explained", int(explained.sum()))
    touched = int((expected.abs().sum(1) > 0).sum())
    assert touched > 1000, touched


@pytest.mark.parametrize("name", ("config3", "config4"))
def test_op_backward(device, name):
    """The op end to end (projection, binning, compositing, both backward
    kernels; on config 4 with the long-list checkpoints and segment walks)
    with the mean-L1 loss restricted to the sampled tiles, against float64
    autograd of the oracle rasterizer along the GPU's lists with fixed
    decisions (reference interface.py:176-239)."""
    r = single_view(name, device)
    scene = r["scene"]
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    leaves = [p.clone().requires_grad_(True) for p in r["params"]]
    outs = rasterize_outputs(*leaves, cam.rotation_matrix.to(device), cam.translation.to(device),
                             fx, fy, cx, cy, r["w"], r["h"], TILE, THRESHOLD, scene.near, scene.far,
                             "gaussian", 0.95)
    image, _, ncon, pm, pinv, pcol, pop, gids, granges, _ = outs
    tiles = sample_tiles(granges.cpu().numpy(), seed=2)
    mask = torch.as_tensor(tile_pixel_mask(tiles, r["tw"], TILE, r["w"], r["h"]))
    weights = _loss_weights(image, scene.target.to(device), mask)
    (image * weights).sum().backward()
    actual = [p.grad.cpu() for p in leaves]
    ncon_h = ncon.cpu().numpy()
    limits = {t: m + 1 for t, m in tile_max(ncon_h, tiles, r["tw"], TILE).items()}
    ids, rng = restrict_lists(gids.cpu().numpy(), granges.cpu().numpy(), tiles, limits)
    log(f"{name} op: oracle projection of all Gaussians + compositing of", len(ids), "entries")
    cols32 = (pm[:, 0], pm[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1], pcol, pop[:, 0])
    g64, g32, margin = fixed_decision_rasterize_grads(
        scene.params(), oracle_camera(cam), TILE, scene.near, scene.far, (ids, rng), cols32, ncon_h,
        weights.cpu(), tile_chunk=CHUNK)
    explained = margin < DECISION_WINDOW
    for param, a, e, e32 in zip(("mean", "rotation", "scale", "opacity", "color"), actual, g64, g32):
        stats = assert_gradients_close(a, e, f"{name} grad {param}", explained=explained,
                                       reference32=e32)
        log(f"{name} op grad", param, stats)


def test_config3_project_bwd(device):
    """Projection backward of all 1M Gaussians for a seeded upstream gradient
    [N, 9] against float64 autograd of the oracle projection."""
    r = single_view("config3", device)
    scene = r["scene"]
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    out = r["out"]
    counts = out[9]
    n = counts.shape[0]
    g = torch.Generator().manual_seed(5)
    upstream = torch.randn(n, 9, generator=g) * torch.tensor([1, 1, 10, 10, 10, 1, 1, 1, 1.0])
    upstream[counts.cpu() == 0] = 0
    grads = project_bwd(*r["params"], cam.rotation_matrix.to(device), cam.translation.to(device),
                        out[4], upstream.to(device), counts, fx, fy, r["w"], r["h"])
    def oracle_grads(params, dt):
        p = [x.to(dt).clone().requires_grad_(True) for x in params]
        proj = orc.project(*p, oracle_camera(cam))
        u = upstream.to(dt)
        loss = (proj.mean[:, 0] * u[:, 0] + proj.mean[:, 1] * u[:, 1]
                + proj.inverse[:, 0, 0] * u[:, 2]
                + (proj.inverse[:, 0, 1] + proj.inverse[:, 1, 0]) * u[:, 3]
                + proj.inverse[:, 1, 1] * u[:, 4] + (proj.color * u[:, 5:8]).sum(1)
                + proj.opacity[:, 0] * u[:, 8]).sum()
        loss.backward()
        return [x.grad for x in p]

    g64 = oracle_grads(scene.params(), torch.float64)
    runs = [oracle_grads(ulp_perturbed(scene.params(), k), torch.float32)
            for k in range(FLOAT32_SAMPLES)]
    names = ("mean", "rotation", "scale", "opacity", "color")
    for name, a, e, e32 in zip(names, grads, g64, [list(x) for x in zip(*runs)]):
        stats = assert_gradients_close(a.cpu(), e, f"config3 project_bwd {name}", reference32=e32)
        log("config3 project_bwd", name, stats)


# --- configuration 5: 16 views through the multi-view op ---------------------

SAMPLED_VIEWS = (0, 5, 10)


def _views_project_bounds(params, cams, scene, device):
    """The mosaic rectangles [V, N, 2, 2] of gs_project_views (the op does not
    return them)."""
    rot, trans, intr, w, h = camera_tensors(cams)
    v = len(cams)
    n = params[0].shape[0]
    tw, th = nat.tiles(w, h, TILE)
    cols = mosaic_columns(v, tw, th)
    outs = [params[0].new_empty(s) for s in ((v, n, 3), (v, n, 2, 2), (v, n, 3), (v, n, 1))]
    bounds = torch.empty((v, n, 2, 2), dtype=torch.int32, device=device)
    counts = torch.empty((v, n), dtype=torch.int32, device=device)
    view = nat.make_view(0.0, 0.0, 0.0, 0.0, w, h, TILE, scene.near, scene.far, views=v,
                         mosaic_cols=cols)
    ptr = nat.ptr
    nat.check(nat.library().gs_project_views(
        *(ptr(p) for p in params), n, params[4].shape[1], ptr(rot), ptr(trans), ptr(intr), view, *(ptr(o) for o in outs), ptr(bounds),
        ptr(counts), None, None, None, nat.stream(device)), "project_views")
    return bounds, cols, tw, th


def _view_lists(gids, ranges, v, n, cols, tw, th):
    """View v's tile lists in its own tile grid with real Gaussian indices
    (numpy), from the mosaic's lists."""
    ox, oy = (v % cols) * tw, (v // cols) * th
    mosaic_w = cols * tw
    ty, tx = np.divmod(np.arange(tw * th), tw)
    mtile = (oy + ty) * mosaic_w + ox + tx
    r = ranges[mtile]
    lengths = r[:, 1] - r[:, 0]
    ids = np.concatenate([gids[s:e] for s, e in r]) - v * n if lengths.sum() else np.zeros(0, np.int32)
    ends = np.cumsum(lengths)
    local = np.stack((ends - lengths, ends), 1).astype(np.int64)
    return ids.astype(np.int32), local


@pytest.fixture(scope="module")
def config5(device):
    _cache.clear()
    torch.cuda.empty_cache()
    log("config5 scene")
    scene = scenes.config5()
    params = [t.to(device) for t in scene.params()]
    leaves = [p.clone().requires_grad_(True) for p in params]
    rot, trans, intr, w, h = camera_tensors(scene.cameras)
    log("config5 GPU forward (16 views)")
    outs = rasterize_views_outputs(*leaves, rot, trans, intr, w, h, TILE, THRESHOLD, scene.near,
                                   scene.far, "gaussian", 0.95)
    bounds, cols, tw, th = _views_project_bounds(params, scene.cameras, scene, device)
    torch.cuda.synchronize()
    nat.check_device_errors(device)
    yield dict(scene=scene, params=params, leaves=leaves, outs=outs, bounds=bounds, cols=cols,
               tw=tw, th=th, w=w, h=h)


def test_config5_projection_and_lists(device, config5):
    c = config5
    image, final_t, ncon, pm, pinv, pcol, pop, gids, ranges, counts = c["outs"]
    v_count, n = counts.shape
    log(f"config5 list proof over {gids.numel()} intersections")
    stats = assert_lists_exact(gids, ranges, c["bounds"].view(v_count * n, 2, 2),
                               counts.view(-1), pm.view(-1, 3)[:, 2].contiguous(), c["cols"] * c["tw"])
    log("config5", stats)
    for v in SAMPLED_VIEWS + (15,):
        cam = c["scene"].cameras[v]
        proj = orc.project(*c["scene"].params(), oracle_camera(cam))
        ob, oc = orc.tile_counts(proj, TILE, c["tw"], c["th"], c["scene"].near, c["scene"].far)
        ox, oy = (v % c["cols"]) * c["tw"], (v // c["cols"]) * c["th"]
        gb = c["bounds"][v].cpu().numpy() - np.array([[ox], [oy]], dtype=np.int32)
        gc = counts[v].cpu().numpy()
        # Rectangles of culled or off-view Gaussians only matter through their
        # count, which is compared below.
        live = (gc > 0) | (oc > 0)
        gb[~live] = ob[~live]
        check_projection(pm[v].detach().cpu(), pinv[v].detach().cpu(), pcol[v].detach().cpu(),
                         pop[v].detach().cpu(), gb, gc, proj, ob, oc, f"config5 view {v}",
                         c["scene"].params(), cam)


def test_config5_sampled_views_forward(device, config5):
    c = config5
    image, final_t, ncon, _, _, _, _, gids, ranges, counts = c["outs"]
    n = counts.shape[1]
    scene = c["scene"]
    for v in SAMPLED_VIEWS:
        ids_v, rng_v = _view_lists(gids.cpu().numpy(), ranges.cpu().numpy(), v, n, c["cols"],
                                   c["tw"], c["th"])
        tiles = sample_tiles(rng_v, count=8, longest=2, seed=v)
        ncon_v = ncon[v].cpu().numpy()
        limits = {t: m + TRUNCATE_SLACK for t, m in tile_max(ncon_v, tiles, c["tw"], TILE).items()}
        proj = orc.project(*scene.params(), oracle_camera(scene.cameras[v]))
        ob, oc = orc.tile_counts(proj, TILE, c["tw"], c["th"], scene.near, scene.far)
        ids, rng = oracle_tile_lists(ob, oc, proj.mean[:, 2].float().numpy(), tiles, c["tw"],
                                     c["tw"] * c["th"], limits)
        log(f"config5 view {v}: oracle compositing {len(ids)} entries")
        comp = orc.composite(proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0],
                             proj.inverse[:, 0, 1], proj.inverse[:, 1, 1], proj.color,
                             proj.opacity[:, 0], ids, rng, c["w"], c["h"], TILE, THRESHOLD,
                             tile_chunk=CHUNK)
        onc = comp.n_contributors.numpy()
        for t in tiles:
            if limits[int(t)] < rng_v[t, 1] - rng_v[t, 0]:
                assert tile_max(onc, [t], c["tw"], TILE)[int(t)] < limits[int(t)]
        mask = torch.as_tensor(tile_pixel_mask(tiles, c["tw"], TILE, c["w"], c["h"]))
        img = image[v].detach().cpu()
        margin = torch.as_tensor(comp.margin)
        # Flat splats put more pixels within 1e-4 of a decision (their alpha
        # falls from the peak to the cut within a pixel): up to 3% flagged.
        stats = assert_close_flip_aware(img[mask], comp.image[mask], margin[mask], atol=1e-5,
                                        what=f"config5 view {v} image", max_flagged=0.03)
        log(f"config5 view {v} image", stats)
        assert_close_flip_aware(final_t[v].cpu()[mask], comp.final_transmittance[mask],
                                margin[mask], atol=1e-5, rtol=1e-4, max_flagged=0.03,
                                what=f"config5 view {v} transmittance")
        ok = mask & (margin >= 1e-4)
        assert torch.equal(ncon[v].cpu()[ok], comp.n_contributors[ok])
        # Every pixel of the sampled tiles against float64 along the GPU's
        # own lists (virtual ids v * n + i in the mosaic) and decisions.
        gids_v, grng_v = _view_lists(gids.cpu().numpy(), ranges.cpu().numpy(), v, n, c["cols"],
                                     c["tw"], c["th"])
        ids_g, rng_g = restrict_lists(gids_v, grng_v, tiles, limits)
        stats = assert_forward_every_pixel(img, final_t[v].cpu(), ncon[v].cpu(),
                                           _gpu_columns(c["outs"], v), ids_g, rng_g, c["w"],
                                           c["h"], TILE, mask=mask, tile_chunk=CHUNK,
                                           what=f"config5 view {v} image")
        log(f"config5 view {v} every pixel", stats)


def test_config5_op_backward(device, config5):
    """Gradients of the multi-view op (mosaic compositing backward and the
    multi-view projection backward summed over views) for the mean-L1 loss on
    sampled tiles of three views, against float64 autograd of the oracle
    rasterizer per view along the GPU's lists with fixed decisions, summed."""
    c = config5
    scene = c["scene"]
    image, final_t, ncon, pm, pinv, pcol, pop, gids, ranges, counts = c["outs"]
    v_count, n = counts.shape
    target = scene.target.to(device)
    weights = torch.zeros_like(image)
    lists = {}
    for v in SAMPLED_VIEWS:
        ids_v, rng_v = _view_lists(gids.cpu().numpy(), ranges.cpu().numpy(), v, n, c["cols"],
                                   c["tw"], c["th"])
        tiles = sample_tiles(rng_v, count=8, longest=2, seed=10 + v)
        mask = torch.as_tensor(tile_pixel_mask(tiles, c["tw"], TILE, c["w"], c["h"]))
        weights[v] = _loss_weights(image[v], target[v], mask) * (image[v].numel() / image.numel())
        ncon_v = ncon[v].cpu().numpy()
        limits = {t: m + 1 for t, m in tile_max(ncon_v, tiles, c["tw"], TILE).items()}
        lists[v] = restrict_lists(ids_v, rng_v, tiles, limits) + (ncon_v,)
    (image * weights).sum().backward()
    actual = [p.grad.cpu() for p in c["leaves"]]
    g64 = g32 = None
    explained = torch.zeros(n, dtype=torch.bool)
    for v in SAMPLED_VIEWS:
        ids, rng, ncon_v = lists[v]
        log(f"config5 view {v}: oracle reference over {len(ids)} entries")
        cols32 = (pm[v, :, 0], pm[v, :, 1], pinv[v, :, 0, 0], pinv[v, :, 0, 1], pinv[v, :, 1, 1],
                  pcol[v], pop[v, :, 0])
        e64, e32, margin = fixed_decision_rasterize_grads(
            scene.params(), oracle_camera(scene.cameras[v]), TILE, scene.near, scene.far, (ids, rng),
            cols32, ncon_v, weights[v].cpu(), tile_chunk=CHUNK)
        g64 = e64 if g64 is None else [x + y for x, y in zip(g64, e64)]
        # Per parameter, the float32 samples of each view summed sample-wise.
        g32 = e32 if g32 is None else [[x + y for x, y in zip(xs, ys)] for xs, ys in zip(g32, e32)]
        explained |= margin < DECISION_WINDOW
    for name, a, e, e32 in zip(("mean", "rotation", "scale", "opacity", "color"), actual, g64, g32):
        stats = assert_gradients_close(a, e, f"config5 grad {name}", explained=explained,
                                       reference32=e32)
        log("config5 op grad", name, stats)
