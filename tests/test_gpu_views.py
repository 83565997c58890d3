"""Parity of the multi-view op (torch.ops.gaussian_splats_hip.rasterize_views)
against the single-view op, which the other GPU tests pin to the CPU oracle.

Per view, the mosaic render must give bit-identical images, transmittance,
contributor counts, projections and per-tile lists (the lists as virtual
indices v * N + i); the gradients must equal the sum of the single-view
gradients up to the order of floating-point additions.
"""

from __future__ import annotations

import math

import pytest
import torch

from gaussian_splats_hip import scenes
from gaussian_splats_hip.kernels.rasterize import _native as nat
from gaussian_splats_hip.kernels.rasterize.interface import forward_pipeline
from gaussian_splats_hip.kernels.rasterize.views import camera_tensors, forward_views, mosaic_columns
from gaussian_splats_hip.splats import GaussianSplat, PinholeCamera, rasterize, rasterize_views

pytestmark = pytest.mark.gpu

THRESHOLD = 0.999


def _scene(n, views, size, vary_intrinsics=False):
    scene = scenes.config5(seed=3, n=n, views=views, size=size, focal=1.25 * size)
    if vary_intrinsics:
        # Per-view focal lengths and principal points (one image size).
        cams = []
        for k, cam in enumerate(scene.cameras):
            f = 1.25 * size * (1.0 + 0.1 * (k % 3))
            cams.append(
                PinholeCamera(
                    rotation=cam.rotation, translation=cam.translation, image_size=cam.image_size,
                    focal_length=(f, 0.9 * f), principal_point=(size / 2 + k, size / 2 - k),
                )
            )
        scene.cameras = cams
    return scene


def _single_forward(params, cam, tile, mode):
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    return forward_pipeline(
        *params, cam.rotation_matrix, cam.translation, float(fx), float(fy), float(cx), float(cy),
        int(w), int(h), tile, THRESHOLD, 0.2, 100.0, mode, 0.95,
    )


def _tile_lists(ranges, ids):
    """Per-tile lengths and the concatenated lists in tile order."""
    r = ranges.long()
    lengths = r[:, 1] - r[:, 0]
    starts = torch.repeat_interleave(r[:, 0], lengths)
    offsets = torch.arange(int(lengths.sum()), device=r.device) - torch.repeat_interleave(
        torch.cumsum(lengths, 0) - lengths, lengths
    )
    return lengths, ids.long()[starts + offsets]


@pytest.mark.parametrize(
    "n, views, size, tile, mode, vary",
    [
        (20_000, 4, 160, 16, "gaussian", False),
        (20_000, 5, 136, 16, "gaussian", True),  # 3 x 2 mosaic with an empty slot
        (8_000, 18, 64, 8, "gaussian", True),  # more than 16 cameras per launch
        (20_000, 3, 120, 16, "ellipsoid", False),
    ],
    ids=("4v_t16", "5v_empty_slot_intrinsics", "18v_t8_two_launches", "3v_ellipsoid"),
)
def test_views_forward_equals_single_views(device, n, views, size, tile, mode, vary):
    scene = _scene(n, views, size, vary)
    params = [t.to(device) for t in scene.params()]
    rotations, translations, intrinsics, w, h = camera_tensors(scene.cameras)
    (image, final_t, ncon, pmean, inv, pcolor, popacity, ids, ranges, counts) = forward_views(
        *params, rotations, translations, intrinsics, w, h, tile, THRESHOLD, 0.2, 100.0, mode, 0.95
    )
    torch.cuda.synchronize()
    tw, th = nat.tiles(w, h, tile)
    cols = mosaic_columns(views, tw, th)
    rows = math.ceil(views / cols)
    grid = ranges.view(rows * th, cols * tw, 2)
    covered = torch.zeros(rows * th, cols * tw, dtype=torch.bool, device=device)
    for v, cam in enumerate(scene.cameras):
        single = _single_forward(params, cam, tile, mode)
        what = f"view {v}"
        assert torch.equal(image[v], single[0]), what
        assert torch.equal(final_t[v], single[1]), what
        assert torch.equal(ncon[v], single[2]), what
        assert torch.equal(pmean[v], single[3]), what
        assert torch.equal(inv[v], single[4]), what
        assert torch.equal(pcolor[v], single[5]), what
        assert torch.equal(popacity[v], single[6]), what
        assert torch.equal(counts[v], single[9]), what
        vx, vy = v % cols, v // cols
        mine = grid[vy * th:(vy + 1) * th, vx * tw:(vx + 1) * tw].reshape(-1, 2)
        covered[vy * th:(vy + 1) * th, vx * tw:(vx + 1) * tw] = True
        lengths, lists = _tile_lists(mine, ids)
        s_lengths, s_lists = _tile_lists(single[8], single[7])
        assert torch.equal(lengths, s_lengths), what
        assert torch.equal(lists - v * n, s_lists), what
    # Tiles of empty mosaic slots list nothing.
    empty = grid[~covered]
    assert bool((empty[:, 1] == empty[:, 0]).all())
    assert int(ranges[-1, 1]) == ids.numel()


@pytest.mark.parametrize(
    "n, views, size, tile",
    [(20_000, 4, 160, 16), (8_000, 18, 64, 8)],
    ids=("4v_t16", "18v_t8_two_launches"),
)
def test_views_backward_equals_sum_of_single_views(device, n, views, size, tile):
    scene = _scene(n, views, size, vary_intrinsics=True)
    g = torch.Generator().manual_seed(11)
    weights = torch.randn(views, size, size, 3, generator=g).to(device)

    def make():
        return GaussianSplat.from_tensors(*(t.to(device).clone() for t in scene.params()))

    splats = make()
    images = rasterize_views(splats, scene.cameras, tile_size=tile)
    (images * weights).sum().backward()
    got = [p.grad for p in (splats.mean, splats.rotation, splats.scale, splats.opacity, splats.color)]

    total = None
    magnitude = None
    for v, cam in enumerate(scene.cameras):
        ref = make()
        image = rasterize(ref, cam, tile_size=tile)
        assert torch.equal(image.detach(), images[v].detach()), f"view {v}"
        (image * weights[v]).sum().backward()
        grads = [p.grad for p in (ref.mean, ref.rotation, ref.scale, ref.opacity, ref.color)]
        if total is None:
            total = [x.clone() for x in grads]
            magnitude = [x.abs() for x in grads]
        else:
            for a, m, x in zip(total, magnitude, grads):
                a += x
                m += x.abs()
    names = ("mean", "rotation", "scale", "opacity", "color")
    for name, a, e, m in zip(names, got, total, magnitude):
        # Relative to the magnitude of the summed per-view terms, with a floor
        # of 1e-4 of the column's largest: each per-view gradient is itself a
        # sum of per-pixel terms that the compositing backward accumulates with
        # atomics in a run-dependent order, so near-cancelled values differ by
        # the rounding of their terms (a missing or repeated view or tile
        # would be off by O(1) of the column).
        m2 = m.reshape(m.shape[0], -1)
        floor = m2.amax(dim=0, keepdim=True).reshape((1, *m.shape[1:]))
        bound = 1e-4 * m + 1e-4 * floor
        err = (a - e).abs()
        assert bool((err <= bound).all()), (
            f"{name}: {int((err > bound).sum())} of {err.numel()} off, worst "
            f"{float((err / bound).max()):.2f}x the bound"
        )
