"""Consumers of the op on the GPU: ``indices`` subsampling (the viewer's
path, interface.py:274-281 of the reference) with gradients scattered back,
the op under ``torch.compile(rasterize, dynamic=True)`` (the viewer's
compile path, visualize/gaussian/backend.py:80-81), the reference viewer's
frame call (backend.py:19-57) through the dispatcher, per-stage timings and
the trajectory benchmark.  Images and gradients are checked against the CPU
oracle; equalities with the HIP op itself are additional."""

from __future__ import annotations

import json
from dataclasses import replace

import pytest
import torch

from gaussian_splats_hip import scenes, timing
from gaussian_splats_hip.kernels.rasterize import benchmark as bm
from gaussian_splats_hip.kernels.rasterize.interface import rasterize_outputs
from gaussian_splats_hip.splats import GaussianSplat, rasterize
from oracle import rasterizer as orc
from parity import (
    DECISION_WINDOW,
    assert_close_flip_aware,
    assert_gradients_close,
    fixed_decision_rasterize_grads,
    oracle_camera,
)

pytestmark = pytest.mark.gpu


def _scene(device, n=3000):
    scene = scenes.edge_case_scene(n=n, sh_degree=3, image_size=(96, 80))
    splats = GaussianSplat.from_tensors(*(t.clone().to(device) for t in scene.params()))
    return scene, splats


def test_indices_forward_and_scattered_gradients(device):
    scene, splats = _scene(device)
    cam = scene.cameras[0]
    g = torch.Generator().manual_seed(0)
    idx = torch.randint(0, splats.num_points, (2500,), generator=g).to(device)  # with repeats
    print("indices fwd/bwd", flush=True)
    image = rasterize(splats, cam, tile_size=16, near=scene.near, far=scene.far, indices=idx)
    sub = GaussianSplat.from_tensors(*(p.detach()[idx].clone() for p in (
        splats.mean, splats.rotation, splats.scale, splats.opacity, splats.color)))
    ref = rasterize(sub, cam, tile_size=16, near=scene.near, far=scene.far)
    assert torch.equal(image, ref)
    idx_h = idx.cpu()
    gathered = [p[idx_h] for p in scene.params()]
    oracle = orc.rasterize(*gathered, oracle_camera(cam), tile_size=16, near=scene.near,
                           far=scene.far)
    assert_close_flip_aware(image.detach().cpu(), oracle.image, oracle.composite.margin, atol=1e-5,
                            what="indexed image")
    weight = torch.rand(image.shape, generator=g).to(device)
    (image * weight).sum().backward()
    (ref * weight).sum().backward()
    for name in ("mean", "rotation", "scale", "opacity", "color"):
        full = getattr(splats, name).grad.double()
        part = getattr(sub, name).grad.double()
        expected = torch.zeros_like(full).index_add_(0, idx, part)
        err = (full - expected).abs().max()
        scale = expected.abs().max().clamp_min(1e-30)
        assert float(err / scale) < 1e-5, name
        untouched = torch.ones(splats.num_points, dtype=torch.bool, device=device)
        untouched[idx] = False
        assert float(full[untouched].abs().max()) == 0.0, name
    # Against float64 autograd of the oracle through the same gather, along
    # the GPU's lists of the subset with its decisions fixed.
    cam_args = _inputs_after_params(scene, device)
    outs = rasterize_outputs(*(p.detach()[idx].clone() for p in (
        splats.mean, splats.rotation, splats.scale, splats.opacity, splats.color)), *cam_args)
    _, _, ncon, pm, pinv, pcol, pop, gids, granges, _ = outs
    cols32 = (pm[:, 0], pm[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1], pcol, pop[:, 0])
    g64, g32, margin = fixed_decision_rasterize_grads(
        scene.params(), oracle_camera(cam), 16, scene.near, scene.far,
        (gids.cpu().numpy(), granges.cpu().numpy()), cols32, ncon.cpu().numpy(), weight.cpu(),
        gather=idx_h)
    explained = torch.zeros(splats.num_points, dtype=torch.bool)
    explained[idx_h[margin < DECISION_WINDOW]] = True
    for name, e, e32 in zip(("mean", "rotation", "scale", "opacity", "color"), g64, g32):
        assert_gradients_close(getattr(splats, name).grad, e, f"indexed grad {name}",
                               explained=explained, reference32=e32)


def _inputs_after_params(scene, device, tile_size=16):
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    return (cam.rotation_matrix.to(device), cam.translation.to(device), fx, fy, cx, cy, w, h,
            tile_size, 0.999, scene.near, scene.far, "gaussian", 0.95)


@pytest.mark.timeout(300)
def test_torch_compile_path(device):
    """torch.compile(rasterize, dynamic=True): the op runs opaque inside the
    graph; images equal eager's bit for bit at two sizes (dynamic shapes),
    gradients up to the order of the atomic adds."""
    torch._dynamo.reset()
    compiled = torch.compile(rasterize, dynamic=True)
    for n in (3000, 2000):
        scene, splats = _scene(device, n)
        cam = scene.cameras[0]
        print(f"torch.compile n={n}", flush=True)
        out = compiled(splats, cam, 16, 0.999, scene.near, scene.far)
        eager_splats = GaussianSplat.from_tensors(*(p.detach().clone() for p in (
            splats.mean, splats.rotation, splats.scale, splats.opacity, splats.color)))
        ref = rasterize(eager_splats, cam, 16, 0.999, scene.near, scene.far)
        assert torch.equal(out, ref)
        oracle = orc.rasterize(*scene.params(), oracle_camera(cam), tile_size=16, near=scene.near,
                               far=scene.far)
        assert_close_flip_aware(out.detach().cpu(), oracle.image, oracle.composite.margin,
                                atol=1e-5, what=f"compiled image n={n}")
        out.square().mean().backward()
        ref.square().mean().backward()
        for name in ("mean", "rotation", "scale", "opacity", "color"):
            a, b = getattr(splats, name).grad, getattr(eager_splats, name).grad
            assert float((a - b).abs().max()) <= 1e-5 * float(b.abs().max()) + 1e-12, name


def test_stage_timings_are_recorded(device):
    scene, splats = _scene(device)
    cam = scene.cameras[0]
    with torch.no_grad(), timing.record_timings(device) as times:
        rasterize(splats, cam, tile_size=16, near=scene.near, far=scene.far)
    stages = times["default"]
    assert set(stages) == {"Project", "Bin", "Emit", "Sort", "Composite"}
    assert all(v >= 0 for v in stages.values()) and sum(stages.values()) > 0


def test_reference_viewer_frame_call(device):
    """The call the reference's viewer makes per frame
    (visualize/gaussian/backend.py:19-54) through this build's dispatcher:
    its default backend name "gsplat", the image rounded up to the tile size
    with the principal point at the requested size's centre, an evenly
    spread subset through ``indices``, then the crop.  Compared with the
    oracle on the gathered subset."""
    scene, splats = _scene(device)
    cam = scene.cameras[0]
    width, height, tile, count = 90, 70, 16, 1500
    size = ((width + tile - 1) // tile * tile, (height + tile - 1) // tile * tile)
    frame_cam = replace(cam, image_size=size, principal_point=(width / 2, height / 2))
    idx = torch.linspace(0, splats.num_points - 1, count, device=device).round().long()
    with torch.no_grad():
        image = rasterize(splats, frame_cam, tile_size=tile, opacity_threshold=0.999,
                          near=scene.near, far=100.0, rendering_mode="gaussian", confidence=0.95,
                          indices=idx, backend="gsplat")[:height, :width]
    assert image.shape == (height, width, 3)
    idx_h = idx.cpu()
    oracle = orc.rasterize(*(p[idx_h] for p in scene.params()), oracle_camera(frame_cam),
                           tile_size=tile, near=scene.near, far=100.0)
    assert_close_flip_aware(image.cpu(), oracle.image[:height, :width],
                            oracle.composite.margin[:height, :width], atol=1e-5, what="frame")


@pytest.mark.timeout(300)
def test_trajectory_benchmark_runs(tmp_path):
    torch._dynamo.reset()
    print("trajectory benchmark", flush=True)
    m = bm.run(checkpoint=None, output_dir=tmp_path, device="cuda", image_size=(128, 96),
               num_splats=2000, frames=6, repeats=1, seed=42, views_per_call=4)
    assert set(m["first_frame"]) == {"hip", "hip_compiled"}
    assert set(m["trajectory"]) == {"hip", "hip_compiled", "hip_views"}
    # Inductor also compiles the camera's quaternion -> matrix glue (host
    # code), whose float rounding differs from eager's by an ulp or so.
    assert m["max_abs_difference_vs_hip"]["hip_compiled"] <= 1e-4
    assert m["max_abs_difference_vs_hip"]["hip_views"] <= 1e-5
    (run_dir,) = list(tmp_path.iterdir())
    assert json.loads((run_dir / "measurements.json").read_text())["config"]["frames"] == 6
    assert (run_dir / "hip.gif").exists()
