"""Consumers of the op on the GPU: ``indices`` subsampling (the viewer's
path, interface.py:274-281 of the reference) with gradients scattered back,
the op under ``torch.compile(rasterize, dynamic=True)`` (the viewer's
compile path, visualize/gaussian/backend.py:80-81), per-stage timings,
the viewer's frame function and the trajectory benchmark."""

from __future__ import annotations

import json
from dataclasses import replace

import pytest
import torch

from gaussian_splats import scenes, timing
from gaussian_splats.kernels.rasterize import benchmark as bm
from gaussian_splats.splats import GaussianSplat, rasterize
from gaussian_splats.viewer import GaussianViewer, render_gaussians

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


def test_render_gaussians_on_gpu(device, monkeypatch):
    scene, splats = _scene(device)
    cam = scene.cameras[0]
    monkeypatch.setenv("GAUSSIAN_SPLATS_PROFILE", "1")
    settings = {"tile_size": "16", "num_splats": "1500", "near": str(scene.near)}
    frame = render_gaussians(splats, cam, settings, 90, 70)
    assert frame.image.shape == (70, 90, 3) and frame.image.is_cuda
    assert "default/Composite" in frame.timings
    idx = torch.linspace(0, splats.num_points - 1, 1500, device=device).round().long()
    cam2 = replace(cam, image_size=(96, 80), principal_point=(45.0, 35.0))
    with torch.no_grad():
        ref = rasterize(splats, cam2, tile_size=16, near=scene.near, far=100.0, indices=idx)
    assert torch.equal(frame.image, ref[:70, :90])


@pytest.mark.timeout(300)
def test_viewer_compiled_render(device, tmp_path):
    torch._dynamo.reset()
    _, splats = _scene(device)
    path = tmp_path / "scene.pt"
    splats.save_checkpoint(path)
    viewer = GaussianViewer()
    viewer.load_checkpoint(path)
    viewer.splats = viewer.splats.to(device)
    eager = viewer.render({"tile_size": "8"}, 64, 48)
    compiled = viewer.render({"tile_size": "8", "compile_render": "1"}, 64, 48)
    assert viewer.compiled_rasterizer is not None
    assert torch.equal(eager.image, compiled.image)


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
