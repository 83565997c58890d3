"""The compositing launch shape chosen from the tiles with work: binning
records how many tiles have a non-empty list, and with fewer than 4096 of
them the compositing kernels split each tile's bands over four waves even
when the image has more tiles.  Both shapes must give the same forward
outputs bit for bit; the forward and both shapes' gradients are checked
against the oracle (float64 autograd for the gradients, at the tolerance of
the other backward parity tests)."""

from __future__ import annotations

import pytest
import torch

from gaussian_splats_hip import scenes
from gaussian_splats_hip.kernels.rasterize import _native as nat
from gaussian_splats_hip.kernels.rasterize import composite, composite_bwd
from gaussian_splats_hip.kernels.rasterize.interface import forward_pipeline
from oracle import rasterizer as orc
from parity import (
    DECISION_WINDOW,
    assert_close_flip_aware,
    assert_forward_every_pixel,
    assert_gradients_close,
    fixed_decision_composite_grads,
    oracle_camera,
)

pytestmark = pytest.mark.gpu

THRESHOLD = 0.999


def _scene(clustered: bool):
    # Spread: the edge-case scene, 500 Gaussians (about 2e5 intersections,
    # which the float64 oracle differentiates in seconds).
    scene = scenes.edge_case_scene(n=3000 if clustered else 500, sh_degree=1,
                                   image_size=(1040, 1040))
    if clustered:  # small Gaussians around the optical axis: ~670 tiles with work
        g = torch.Generator().manual_seed(5)
        scene.mean[:, :2] = torch.randn(3000, 2, generator=g) * 0.4
        scene.mean[:, 2] = -(torch.rand(3000, generator=g) * 4 + 4)
        scene.scale[:] = torch.rand(3000, 3, generator=g) * 1.5 - 4.5
    return scene


@pytest.mark.parametrize("clustered", [True, False], ids=("clustered", "spread"))
def test_split_and_one_wave_shapes_agree(device, clustered):
    scene = _scene(clustered)
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    print(f"[split] clustered={clustered}", flush=True)
    out = forward_pipeline(
        *(t.to(device) for t in scene.params()), cam.rotation_matrix, cam.translation, fx, fy, cx,
        cy, w, h, 16, THRESHOLD, scene.near, scene.far, "gaussian", 0.95,
    )
    image, final_t, ncon, pmean, pinv, pcol, pop, gids, ranges, counts = out
    active = nat.active_tiles(ranges)
    assert active == int((ranges[:, 1] > ranges[:, 0]).sum())
    assert ranges.shape[0] == 65 * 65
    if clustered:
        assert 0 < active < 4096  # the op composited with the split shape

    split_ranges, one_wave_ranges = ranges.clone(), ranges.clone()
    nat.set_active_tiles(split_ranges, 1)  # forces four waves per tile
    # No recorded count: the image's 4225 tiles select one wave per tile.
    args = (pmean, pinv, pcol, pop, gids)
    a = composite(*args, split_ranges, w, h, 16, THRESHOLD, "gaussian", 0.95)
    b = composite(*args, one_wave_ranges, w, h, 16, THRESHOLD, "gaussian", 0.95)
    for x, y, op_out, name in zip(a, b, (image, final_t, ncon), ("image", "T", "n_contributors")):
        assert torch.equal(x, y), name
        assert torch.equal(x, op_out), name

    ref = orc.rasterize(*scene.params(), oracle_camera(cam), tile_size=16,
                        opacity_threshold=THRESHOLD, near=scene.near, far=scene.far)
    assert_close_flip_aware(a[0].cpu(), ref.image, ref.composite.margin, atol=1e-5, what="image")
    cols32 = [pmean[:, 0], pmean[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1], pcol,
              pop[:, 0]]
    ids_np, ranges_np = gids.cpu().numpy(), ranges.cpu().numpy()
    assert_forward_every_pixel(a[0].cpu(), a[1].cpu(), a[2].cpu(), [c.cpu() for c in cols32],
                               ids_np, ranges_np, w, h, 16, what="image")

    g = torch.Generator().manual_seed(3)
    grad_image = torch.rand(h, w, 3, generator=g) * 2 - 1
    # Each shape's backward takes its own forward's outputs (bit-identical to
    # the op's), so it walks with that forward's hit masks.
    ga = composite_bwd(*args, split_ranges, grad_image.to(device), a[1], a[2], w, h, 16,
                       THRESHOLD, "gaussian").cpu()
    gb = composite_bwd(*args, one_wave_ranges, grad_image.to(device), b[1], b[2], w, h, 16,
                       THRESHOLD, "gaussian").cpu()

    # float64 autograd of the oracle compositor on the GPU's own projected
    # values and lists with the GPU's activity decisions and the float32
    # oracle's cut/clamp decisions, every Gaussian compared.
    expected, expected32, margin, _ = fixed_decision_composite_grads(
        [c.cpu() for c in cols32], ids_np, ranges_np, w, h, 16, ncon.cpu().numpy(), grad_image)
    explained = margin < DECISION_WINDOW
    for name, got in (("split", ga), ("one wave", gb)):
        stats = assert_gradients_close(got, expected, f"{name} composite_bwd", explained=explained,
                                       reference32=expected32)
        print(f"[split] {name}: {stats}", flush=True)
