"""Consumers of the op on the CPU: the trajectory benchmark's scene, subset
and camera path (kernels/rasterize/benchmark.py:26-90), the viewer's frame
settings (visualize/gaussian/backend.py:19-57) with a stand-in rasterizer,
and the timing API (timing.py).  No GPU."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from scipy.spatial.transform import Rotation

from gaussian_splats import timing
from gaussian_splats.kernels.rasterize import benchmark as bm
from gaussian_splats.splats import GaussianSplat, PinholeCamera
from gaussian_splats.viewer import GaussianViewer, render_gaussians


def test_random_scene_distribution():
    s = bm.random_scene(4000, seed=42, device="cpu")
    assert s.sh_degree == 1 and s.color.shape == (4000, 4, 3)
    z = s.mean.detach()[:, 2]
    assert float(z.min()) >= 2.0 and float(z.max()) <= 6.0
    assert abs(float(s.mean.detach()[:, :2].std()) - 0.5) < 0.03
    assert torch.equal(s.scale, torch.full_like(s.scale, -2.0))
    again = bm.random_scene(4000, seed=42, device="cpu")
    assert torch.equal(again.mean, s.mean) and torch.equal(again.color, s.color)


def test_select_splats_is_a_seeded_subset():
    s = bm.random_scene(500, seed=1, device="cpu")
    with torch.no_grad():
        s.normals.normal_()
    sub = bm.select_splats(s, 120, seed=7)
    torch.manual_seed(7)
    idx = torch.randperm(500)[:120]
    for name in ("mean", "rotation", "scale", "opacity", "color", "normals"):
        assert torch.equal(getattr(sub, name), getattr(s, name)[idx]), name
    assert bm.select_splats(s, None, 0) is s and bm.select_splats(s, 900, 0) is s


def test_trajectory_rotations_and_fit():
    """Frame f's world-to-camera rotation is R_x(-45 deg) R_y(360 f / F)
    (scipy), and every point of the scene lies inside the fitted view."""
    s = bm.random_scene(3000, seed=0, device="cpu")
    frames = 8
    cams = bm.generate_trajectory(s, (320, 240), frames)
    pts = s.mean.detach().double()
    for f, cam in enumerate(cams):
        expected = Rotation.from_euler("x", -45.0, degrees=True) * Rotation.from_euler(
            "y", 360.0 * f / frames, degrees=True)
        assert np.allclose(cam.rotation_matrix.double().numpy(), expected.as_matrix(), atol=1e-6)
        assert cam.focal_length == (240.0, 240.0) and cam.principal_point == (160.0, 120.0)
        r = cam.rotation_matrix.double()
        p = pts @ r.T + cam.translation.double()
        depth = -p[:, 2]
        assert float(depth.min()) > 0
        u = 240.0 * p[:, 0] / depth + 160.0
        v = -240.0 * p[:, 1] / depth + 120.0
        assert float(u.min()) >= 0 and float(u.max()) <= 320 and float(v.min()) >= 0 and float(v.max()) <= 240


def test_render_gaussians_settings():
    """Tile-rounded size, centred principal point, evenly spread subset,
    options from the settings, crop back to the requested size."""
    calls = {}

    def fake(splats, camera, **options):
        calls["camera"], calls["options"] = camera, options
        w, h = camera.image_size
        return torch.arange(h * w * 3, dtype=torch.float32).reshape(h, w, 3)

    s = GaussianSplat(1000, sh_degree=0)
    cam = PinholeCamera(image_size=(10, 10))
    frame = render_gaussians(s, cam, {"tile_size": "16", "num_splats": "7", "near": "0.5"}, 50, 30, fake)
    assert calls["camera"].image_size == (64, 32)
    assert calls["camera"].principal_point == (25.0, 15.0)
    opts = calls["options"]
    assert opts["backend"] == "hip" and opts["tile_size"] == 16 and opts["near"] == 0.5
    assert opts["far"] == 100.0 and opts["opacity_threshold"] == 0.999
    # float32 linspace: 832.5 is computed as 832.49997 and rounds down
    assert opts["indices"].tolist() == [0, 166, 333, 500, 666, 832, 999]
    assert frame.image.shape == (30, 50, 3)
    assert frame.metadata == {"X-Total-Splats": "1000"}
    empty = render_gaussians(GaussianSplat(0, sh_degree=0), cam, {}, 8, 4, fake)
    assert empty.image.shape == (4, 8, 3) and empty.metadata["X-Total-Splats"] == "0"
    frame = render_gaussians(s, cam, {"num_splats": "5000"}, 8, 8, fake)
    assert len(calls["options"]["indices"]) == 1000


def test_viewer_loads_checkpoints_and_ply(tmp_path):
    from gaussian_splats.splats.ply import save_ply

    torch.manual_seed(0)
    s = GaussianSplat(300, sh_degree=3)
    s.save_checkpoint(tmp_path / "scene.pt")
    save_ply(s.state_dict(), tmp_path / "scene.ply")
    for name in ("scene.pt", "scene.ply"):
        viewer = GaussianViewer()
        viewer.load_checkpoint(tmp_path / name)
        assert viewer.checkpoint_name == name
        assert torch.equal(viewer.splats.mean.cpu(), s.mean.detach())
        q = viewer.camera.rotation
        assert torch.allclose(q, torch.tensor([math.cos(math.pi / 8), -math.sin(math.pi / 8), 0, 0]))


def test_timing_api():
    with timing.record_timings("cpu") as times:
        with timing.timed("Step"):
            pass

        @timing.timed
        def project_points():
            return 3

        @timing.timed("Named", tag="extra")
        def other():
            return 4

        assert project_points() == 3 and other() == 4
        assert timing.stage_timer() is None  # no GPU recording on the CPU
    assert set(times) == {"default", "extra"}
    assert set(times["default"]) == {"Step", "Project Points"}
    assert "Named" in times["extra"]
    with timing.timed("Outside"):  # no active recording: a no-op
        pass


@pytest.mark.parametrize("frames", [2, 5])
def test_trajectory_frame_count(frames):
    s = bm.random_scene(100, seed=0, device="cpu")
    assert len(bm.generate_trajectory(s, (64, 48), frames)) == frames


def test_scene_from_file(tmp_path):
    """Checkpoints and PLY files load as the same benchmark scene."""
    from gaussian_splats import scenes
    from gaussian_splats.splats.ply import save_ply

    torch.manual_seed(3)
    s = GaussianSplat(20_000, sh_degree=3)
    s.save_checkpoint(tmp_path / "baked.pt")
    save_ply(s.state_dict(), tmp_path / "baked.ply")
    a = scenes.from_file(str(tmp_path / "baked.pt"), image_size=(320, 180))
    b = scenes.from_file(str(tmp_path / "baked.ply"), image_size=(320, 180))
    for x, y in zip(a.params(), b.params()):
        assert torch.equal(x, y)
    assert torch.equal(a.cameras[0].translation, b.cameras[0].translation)
    assert a.target.shape == (180, 320, 3) and a.cameras[0].image_size == (320, 180)


def test_host_extrinsics_equal_the_torch_rotation_matrix():
    """The rasterizer's host path gives exactly cam.rotation_matrix (float32
    quaternions of all magnitudes, unnormalised), and falls back to it for
    float64 quaternions."""
    from gaussian_splats.splats.camera import host_extrinsics

    g = torch.Generator().manual_seed(11)
    for i in range(3000):
        scale = 10.0 ** float(torch.randint(-4, 4, (1,), generator=g))
        cam = PinholeCamera(rotation=torch.randn(4, generator=g) * scale,
                            translation=torch.randn(3, generator=g))
        r, t = host_extrinsics(cam)
        assert r.dtype == torch.float32 and r.device.type == "cpu"
        assert torch.equal(r, cam.rotation_matrix.float()), i
        assert torch.equal(t, cam.translation.float())
    cam = PinholeCamera(rotation=torch.randn(4, dtype=torch.float64, generator=g),
                        translation=torch.randn(3, dtype=torch.float64, generator=g))
    r, t = host_extrinsics(cam)
    assert torch.equal(r, cam.rotation_matrix.float()) and t.dtype == torch.float32
