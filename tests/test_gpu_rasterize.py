"""End-to-end parity of torch.ops.gaussian_splats_hip.rasterize (HIP) against the
CPU oracle: image, lists and gradients (cf. the reference's
kernels/rasterize/tests/test_rasterize.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splats_hip import scenes
from gaussian_splats_hip.kernels.rasterize import _native as nat
from gaussian_splats_hip.kernels.rasterize import composite, composite_bwd
from gaussian_splats_hip.kernels.rasterize.interface import forward_pipeline, rasterize_outputs
from oracle import rasterizer as orc
from parity import (
    DECISION_WINDOW,
    assert_close_flip_aware,
    assert_forward_every_pixel,
    assert_gradients_close,
    fixed_decision_composite_grads,
    fixed_decision_rasterize_grads,
    oracle_camera,
    segmented_scene,
)

pytestmark = pytest.mark.gpu

THRESHOLD = 0.999


def _op_inputs(scene, device, tile_size):
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    return (
        *(t.to(device) for t in scene.params()),
        cam.rotation_matrix.to(device), cam.translation.to(device), fx, fy, cx, cy, w, h,
        tile_size, THRESHOLD, scene.near, scene.far, "gaussian", 0.95,
    )


@pytest.mark.parametrize(
    "make, tile_size",
    [
        (lambda: scenes.config1(), 16),
        (lambda: scenes.edge_case_scene(n=3000, sh_degree=3, image_size=(200, 120)), 16),
        (lambda: scenes.edge_case_scene(n=3000, sh_degree=2, image_size=(200, 120)), 8),
        # More tiles than the band-split threshold: one wave per tile.
        (lambda: scenes.edge_case_scene(n=500, sh_degree=1, image_size=(1040, 1040)), 16),
        (lambda: scenes.edge_case_scene(n=400, sh_degree=1, image_size=(200, 120)), 32),
    ],
    ids=("config1", "edge_sh3_t16", "edge_sh2_t8", "edge_t16_one_wave_per_tile", "edge_t32"),
)
def test_forward_matches_oracle(device, make, tile_size):
    scene = make()
    out = forward_pipeline(*_op_inputs(scene, device, tile_size))
    image, final_t, ncon, pmean, pinv, pcol, pop, gids, ranges, counts = (t.cpu() for t in out)
    ref = orc.rasterize(*scene.params(), oracle_camera(scene.cameras[0]), tile_size=tile_size,
                        opacity_threshold=THRESHOLD, near=scene.near, far=scene.far)
    stats = assert_close_flip_aware(image, ref.image, ref.composite.margin, atol=1e-5, what="image")
    print("image", stats)
    assert image.dtype == torch.float32
    # Every pixel, near a decision or not, along the GPU's own lists.
    w, h = scene.cameras[0].image_size
    assert_forward_every_pixel(
        image, final_t, ncon, [pmean[:, 0], pmean[:, 1], pinv[:, 0, 0], pinv[:, 0, 1],
                               pinv[:, 1, 1], pcol, pop[:, 0]],
        gids.numpy(), ranges.numpy(), w, h, tile_size, what="image")

    # Lists: the oracle's binning of the GPU's own projected values is bit-exact.
    w, h = scene.cameras[0].image_size
    tw, th = nat.tiles(w, h, tile_size)
    bounds_gpu = None
    keys, ids = orc.emit_intersections(
        _bounds_from(out, scene, device, tile_size), pmean[:, 2].numpy(), counts.numpy(), tw
    )
    sid, rng, _ = orc.sort_intersections(keys, ids, tw * th)
    assert np.array_equal(gids.numpy(), sid)
    assert np.array_equal(ranges.numpy(), rng)
    del bounds_gpu


def _bounds_from(out, scene, device, tile_size):
    """Re-runs the projection stage to obtain the GPU's tile rectangles (the op
    does not return them, as the reference op does not)."""
    from gaussian_splats_hip.kernels.rasterize import project_and_count

    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    res = project_and_count(
        *(t.to(device) for t in scene.params()), cam.rotation_matrix.to(device),
        cam.translation.to(device), fx, fy, cx, cy, w, h, tile_size, scene.near, scene.far,
        "gaussian", 0.95,
    )
    return res[4].cpu().numpy()


@pytest.mark.parametrize(
    "n, size, ts",
    [
        (1200, (96, 80), 16),  # bands split over four waves per tile
        (300, (1040, 1040), 16),  # more tiles than the split threshold: one wave per tile
        (600, (96, 80), 32),
        (200, (2080, 2080), 32),
    ],
    ids=("t16_split", "t16_one_wave", "t32_split", "t32_one_wave"),
)
def test_composite_backward_matches_autograd(device, n, size, ts):
    """composite_bwd on identical inputs vs float64 autograd of the oracle
    composite with the discrete decisions fixed (the activity test by the
    GPU's contributor counts, the alpha cut and clamp by the float32 oracle):
    every Gaussian is compared."""
    print(f"[composite_bwd] n={n} size={size} tile={ts}", flush=True)
    scene = scenes.edge_case_scene(n=n, sh_degree=1, image_size=size)
    cam = scene.cameras[0]
    w, h = cam.image_size
    proj = orc.project(*scene.params(), oracle_camera(cam))
    tw, th = nat.tiles(w, h, ts)
    bounds, counts = orc.tile_counts(proj, ts, tw, th, scene.near, scene.far)
    keys, ids = orc.emit_intersections(bounds, proj.mean[:, 2].float().numpy(), counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
    g = torch.Generator().manual_seed(7)
    grad_image = torch.rand(h, w, 3, generator=g) * 2 - 1
    grad, absolute, expected, expected32, expected_abs, explained = _composite_bwd_case(
        device, proj.mean.float(), proj.inverse.float(), proj.color.float(), proj.opacity.float(),
        sid, ranges, grad_image, w, h, ts)
    stats = assert_gradients_close(grad, expected, "composite_bwd", explained=explained,
                                   reference32=expected32)
    print("composite_bwd", stats, "explained", int(explained.sum()), flush=True)
    stats = assert_gradients_close(absolute, expected_abs, "absolute mean gradients",
                                   explained=explained)
    print("absolute", stats, flush=True)


def _composite_bwd_case(device, pmean, pinv, pcol, pop, sid, ranges, grad_image, w, h, ts):
    """GPU composite + composite_bwd (with return_absolute) and the oracle's
    float64 and float32 gradients along the same lists with the decisions
    fixed (fixed_decision_composite_grads)."""
    f32 = lambda x: x.detach().float().contiguous().to(device)
    gids = torch.as_tensor(sid).to(device)
    granges = torch.as_tensor(ranges).to(device)
    image, final_t, ncon = composite(f32(pmean), f32(pinv), f32(pcol), f32(pop), gids, granges,
                                     w, h, ts, THRESHOLD, "gaussian", 0.95)
    grad, absolute = composite_bwd(f32(pmean), f32(pinv), f32(pcol), f32(pop), gids, granges,
                                   grad_image.to(device), final_t, ncon, w, h, ts, THRESHOLD,
                                   "gaussian", return_absolute=True)
    cols32 = [pmean[:, 0], pmean[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1], pcol, pop[:, 0]]
    g64, g32, margin, abs64 = fixed_decision_composite_grads(
        cols32, sid, ranges, w, h, ts, ncon.cpu().numpy(), grad_image, probe=True)
    explained = margin < DECISION_WINDOW
    return grad.cpu(), absolute.cpu(), g64, g32, abs64, explained


@pytest.mark.parametrize(
    "entries, alpha_range",
    [(3000, (0.0045, 0.006)), (7000, (0.0045, 0.03)), (1600, (0.0042, 0.0046))],
    ids=("3000_entries", "7000_entries", "1600_min_alpha"),
)
def test_composite_backward_long_lists(device, entries, alpha_range):
    """Lists of thousands of entries of small alpha, the longest of the
    benchmark scenes (config 3: up to 7031 entries per tile), whose pixels
    walk up to ~1600 blending entries before reaching T ~ 1e-3: the
    backward's transmittance, recovered entry by entry from the final one,
    stays within the gradient tolerance of float64 autograd.  The Gaussians
    are wide (sigma >= 2000 px), so alpha varies by < 0.03% over the image
    and no pixel sits at the 1/255 cut: the only discrete decision is the
    activity test, fixed by the GPU's contributor counts."""
    g = torch.Generator().manual_seed(entries)
    w = h = 32
    ts = 16
    u = torch.rand(entries, generator=g) * 40 - 4
    v = torch.rand(entries, generator=g) * 40 - 4
    depth = torch.rand(entries, generator=g) * 5 + 1
    pmean = torch.stack((u, v, depth), -1)
    sigma = torch.rand(entries, generator=g) * 2000 + 2000
    rho = (torch.rand(entries, generator=g) * 2 - 1) * 0.5
    cov = torch.stack((sigma ** 2, rho * sigma ** 2, rho * sigma ** 2, sigma ** 2), -1).view(-1, 2, 2)
    pinv = torch.linalg.inv(cov.double()).float()
    pcol = torch.rand(entries, 3, generator=g)
    lo, hi = alpha_range
    pop = (torch.rand(entries, 1, generator=g) * (hi - lo) + lo)
    tw, th = nat.tiles(w, h, ts)
    bounds = np.zeros((entries, 2, 2), dtype=np.int32)
    bounds[:, 0, 1] = tw
    bounds[:, 1, 1] = th
    counts = np.full(entries, tw * th, dtype=np.int32)
    keys, ids = orc.emit_intersections(bounds, depth.numpy(), counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
    grad_image = torch.rand(h, w, 3, generator=g) * 2 - 1
    grad, absolute, expected, expected32, _, explained = _composite_bwd_case(
        device, pmean, pinv, pcol, pop, sid, ranges, grad_image, w, h, ts)
    assert not bool(explained.any())  # no decision near a threshold by construction
    stats = assert_gradients_close(grad, expected, "long-list composite_bwd", reference32=expected32)
    print(f"[long lists] {entries} entries: {stats}", flush=True)
    # Against float64 the kernel is no less accurate than the float32 oracle.
    err = (grad.double() - expected).abs().max()
    err32 = max((e.double() - expected).abs().max() for e in expected32)
    print(f"[long lists] max error {float(err):.3e} (float32 oracle {float(err32):.3e})", flush=True)


@pytest.mark.parametrize("entries", (9000, 12000))
def test_composite_backward_segmented_walks(device, entries):
    """The backward's list segments: at tile 8 (no quarter split) the
    entries are listed only in four tiles of the image's corner, two of which
    hold lists of more than 8192 entries, walk ~1300 of them and cross forward
    checkpoints (intersection indices that are multiples of 1024).  Each segment starts its walk back from the
    checkpoint's record (T, colour after it): the gradients match float64
    autograd along the same lists with the decisions fixed, and the
    unsegmented backward (no plan, no checkpoints) up to rounding."""
    from gaussian_splats_hip.kernels.rasterize.composite import tile_order

    w = h = 64
    ts = 8
    pmean, pinv, pcol, pop, sid, ranges = segmented_scene(entries, w, h, ts)
    g = torch.Generator().manual_seed(entries + 2)
    grad_image = torch.rand(h, w, 3, generator=g) * 2 - 1
    print(f"[segmented walks] {entries} entries", flush=True)
    grad, absolute, expected, expected32, _, explained = _composite_bwd_case(
        device, pmean, pinv, pcol, pop, sid, ranges, grad_image, w, h, ts)
    assert not bool(explained.any())  # no decision near a threshold by construction
    # The backward plan walks tiles 0 and 8 in segments cut at the forward's
    # checkpoints (position 1024 of the list and its batch).
    f32 = lambda x: x.detach().float().contiguous().to(device)
    gids, granges = torch.as_tensor(sid).to(device), torch.as_tensor(ranges).to(device)
    image, final_t, ncon = composite(f32(pmean), f32(pinv), f32(pcol), f32(pop), gids, granges,
                                     w, h, ts, THRESHOLD, "gaussian", 0.95)
    # That forward took the long-list kernel (plan by list length, checkpoints,
    # records requested a batch ahead); the plain kernel in index order gives
    # the same transmittance and contributor counts, and the image up to the
    # order of the colour sums (the checkpoints sum each pixel's colour in
    # segments).
    from gaussian_splats_hip.kernels.rasterize.project import pack_records

    records = pack_records(f32(pmean), f32(pinv), f32(pcol), f32(pop), "gaussian", 0.95)
    img2, ft2, nc2 = torch.empty_like(image), torch.empty_like(final_t), torch.empty_like(ncon)
    plain = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, ts, opacity_threshold=THRESHOLD)
    ids32 = gids.to(torch.int32).contiguous()
    nat.check(nat.library().gs_composite(
        nat.ptr(records), records.shape[0], nat.ptr(ids32), ids32.numel(), nat.ptr(granges), None,
        plain, nat.ptr(img2), nat.ptr(ft2), nat.ptr(nc2), None, 0, None, 0, None, 0,
        nat.stream(device)),
        "composite")
    torch.cuda.synchronize()
    assert torch.equal(final_t, ft2) and torch.equal(ncon, nc2)
    assert float((image - img2).abs().max()) <= 1e-5
    plan = tile_order(granges, ncon, w, h, ts).cpu().numpy()
    segmented = set((plan[(plan >= 0) & ((plan & 0x40) != 0)] >> 7).tolist())
    assert {0, 8} <= segmented, segmented
    stats = assert_gradients_close(grad, expected, "segmented composite_bwd",
                                   reference32=expected32)
    print(f"[segmented walks] {stats}", flush=True)
    whole = torch.zeros_like(grad, device=device)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, ts, opacity_threshold=THRESHOLD)
    cols = [f32(pmean), f32(pinv), f32(pcol), f32(pop)]  # alive until the kernel has run
    g_dev = grad_image.to(device)
    nat.check(nat.library().gs_composite_bwd(
        *(nat.ptr(t) for t in cols), entries, nat.ptr(gids), nat.ptr(granges), nat.ptr(g_dev),
        nat.ptr(final_t), nat.ptr(ncon), None, view, nat.ptr(whole), None, None, 0, 0,
        None, 0, nat.stream(device)), "composite_bwd")
    torch.cuda.synchronize()
    scale = whole.abs().amax(dim=0, keepdim=True).clamp_min(1e-30).cpu()
    assert float(((grad - whole.cpu()).abs() / scale).max()) < 1e-5


def _op_case(device, scene, ts, loss, target):
    """The op's forward and backward on the GPU and the oracle's float64 and
    float32 parameter gradients along the GPU's lists with the decisions fixed
    (fixed_decision_rasterize_grads); the loss weights come from the GPU image,
    so the sign of |image - target| is one more fixed decision."""
    cam = scene.cameras[0]
    leaves = [p.detach().clone().to(device).requires_grad_(True) for p in scene.params()]
    inputs = _op_inputs(scene, device, ts)
    outs = rasterize_outputs(*leaves, *inputs[5:])
    image, _, ncon, pm, pinv, pcol, pop, gids, granges, _ = outs
    if loss == "sum":
        weights = target.to(device)
    else:
        weights = torch.sign(image.detach() - target.to(device)) / image.numel()
    (image * weights).sum().backward()
    actual = [p.grad.cpu() for p in leaves]
    cols32 = (pm[:, 0], pm[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1], pcol, pop[:, 0])
    g64, g32, margin = fixed_decision_rasterize_grads(
        scene.params(), oracle_camera(cam), ts, scene.near, scene.far,
        (gids.cpu().numpy(), granges.cpu().numpy()), cols32, ncon.cpu().numpy(), weights.cpu())
    return actual, g64, g32, margin < DECISION_WINDOW


@pytest.mark.parametrize("loss", ("sum", "mean_l1"))
def test_backward_matches_autograd(device, loss):
    """Full op backward vs float64 autograd of the oracle rasterizer, every
    Gaussian compared."""
    scene = scenes.edge_case_scene(n=800, sh_degree=3, image_size=(80, 64))
    g = torch.Generator().manual_seed(11)
    target = torch.rand(64, 80, 3, generator=g)
    actual, expected, expected32, explained = _op_case(device, scene, 16, loss, target)
    names = ("mean", "rotation", "scale", "opacity", "color")
    for name, a, e, e32 in zip(names, actual, expected, expected32):
        stats = assert_gradients_close(a, e, name, explained=explained, reference32=e32)
        print(loss, name, stats, flush=True)
