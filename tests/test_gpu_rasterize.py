"""End-to-end parity of torch.ops.gaussian_splats.rasterize (HIP) against the
CPU oracle: image, lists and gradients (cf. the reference's
kernels/rasterize/tests/test_rasterize.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splats import scenes
from gaussian_splats.kernels.rasterize import _native as nat
from gaussian_splats.kernels.rasterize import composite, composite_bwd
from gaussian_splats.kernels.rasterize.interface import forward_pipeline
from gaussian_splats.splats import GaussianSplat, rasterize
from oracle import rasterizer as orc
from parity import assert_close_flip_aware, oracle_camera

pytestmark = pytest.mark.gpu

THRESHOLD = 0.999
GRAD_MARGIN = 1e-5


def assert_grad_close(actual, expected, scale, what):
    err = (actual - expected).abs()
    bound = 1e-4 * expected.abs() + 1e-6 * scale
    bad = err > bound
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {bad.numel()} gradients off; worst excess "
        f"{float((err / bound).max()):.2f}x, max abs err {float(err.max()):.3e}, scale {scale:.3e}"
    )


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
    from gaussian_splats.kernels.rasterize import project_and_count

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
    "n, size, ts, min_good",
    [
        (1200, (96, 80), 16, 0.85),  # bands split over four waves per tile
        # More tiles than the split threshold: one wave per tile.  A Gaussian
        # covers many more pixels here, so more of them have some decision
        # near a threshold and are excluded.
        (300, (1040, 1040), 16, 0.4),
        (600, (96, 80), 32, 0.85),
        (200, (2080, 2080), 32, 0.4),
    ],
    ids=("t16_split", "t16_one_wave", "t32_split", "t32_one_wave"),
)
def test_composite_backward_matches_autograd(device, n, size, ts, min_good):
    """composite_bwd on identical inputs vs float64 autograd of the oracle composite."""
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

    leaves = [x.detach().double().clone().requires_grad_(True) for x in (
        proj.mean[:, 0], proj.mean[:, 1], proj.inverse[:, 0, 0], proj.inverse[:, 0, 1],
        proj.inverse[:, 1, 1], proj.color, proj.opacity[:, 0])]
    probe = []
    exp = orc.composite(*leaves, sid, ranges, w, h, ts, THRESHOLD, probe=probe)
    (exp.image * grad_image.double()).sum().backward()
    expected_abs = orc.absolute_mean_gradients(probe, leaves[0].shape[0])
    du, dv, da, db, dc, drgb, dop = (x.grad for x in leaves)
    expected = torch.stack((du, dv, da, db / 2, dc, drgb[:, 0], drgb[:, 1], drgb[:, 2], dop), -1)

    f32 = lambda x: x.detach().float().to(device)
    image, final_t, ncon = composite(
        f32(proj.mean), f32(proj.inverse), f32(proj.color), f32(proj.opacity),
        torch.as_tensor(sid).to(device), torch.as_tensor(ranges).to(device), w, h, ts, THRESHOLD,
        "gaussian", 0.95,
    )
    grad, absolute = composite_bwd(
        f32(proj.mean), f32(proj.inverse), f32(proj.color), f32(proj.opacity),
        torch.as_tensor(sid).to(device), torch.as_tensor(ranges).to(device),
        grad_image.to(device), final_t, ncon, w, h, ts, THRESHOLD, "gaussian",
        return_absolute=True,
    )
    grad, absolute = grad.cpu(), absolute.cpu()
    # Tolerance: 1e-4 relative, 1e-6 absolute in units of the column's largest
    # gradient.  Gaussians one of whose discrete decisions lies within 1e-5 of
    # its threshold are excluded: there any float32 evaluation (the reference's
    # own included) may decide differently from float64.
    good = exp.gaussian_margin >= GRAD_MARGIN
    assert float(good.double().mean()) > min_good, float(good.double().mean())
    for col in range(9):
        scale = float(expected[:, col].abs().max())
        assert_grad_close(grad.double()[good, col], expected[good, col], scale, f"column {col}")
    # Absolute per-pixel mean-gradient sums (return_absolute).
    for col in range(2):
        scale = float(expected_abs[:, col].abs().max())
        assert_grad_close(absolute.double()[good, col], expected_abs[good, col], scale,
                          f"absolute {col}")


@pytest.mark.parametrize("loss", ("sum", "mean_l1"))
def test_backward_matches_autograd(device, loss):
    """Full op backward vs float64 autograd of the oracle rasterizer."""
    scene = scenes.edge_case_scene(n=800, sh_degree=3, image_size=(80, 64))
    cam = scene.cameras[0]
    ts = 16
    g = torch.Generator().manual_seed(11)
    target = torch.rand(64, 80, 3, generator=g)

    params64 = [p.detach().double().clone().requires_grad_(True) for p in scene.params()]
    ref = orc.rasterize(*params64, oracle_camera(cam), tile_size=ts, opacity_threshold=THRESHOLD,
                        near=scene.near, far=scene.far)
    if loss == "sum":
        ref_loss = (ref.image * target.double()).sum()
    else:
        ref_loss = (ref.image - target.double()).abs().mean()
    ref_loss.backward()
    expected = [p.grad for p in params64]

    splats = GaussianSplat.from_tensors(*(p.detach().clone().to(device) for p in scene.params()))
    cam_gpu = cam
    image = rasterize(splats, cam_gpu, tile_size=ts, opacity_threshold=THRESHOLD, near=scene.near,
                      far=scene.far)
    tgt = target.to(device)
    out_loss = (image * tgt).sum() if loss == "sum" else (image - tgt).abs().mean()
    out_loss.backward()
    actual = [splats.mean.grad, splats.rotation.grad, splats.scale.grad, splats.opacity.grad,
              splats.color.grad]
    # Tolerance: 1e-4 relative, 1e-6 absolute in units of the parameter's
    # largest gradient, over the Gaussians whose decisions are well conditioned.
    good = ref.composite.gaussian_margin >= GRAD_MARGIN
    assert float(good.double().mean()) > 0.85, float(good.double().mean())
    names = ("mean", "rotation", "scale", "opacity", "color")
    for name, a, e in zip(names, actual, expected):
        a = a.detach().cpu().double()[good]
        e = e.detach()[good]
        assert_grad_close(a, e, float(e.abs().max()), name)
