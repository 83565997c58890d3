"""Consumers of the op on the CPU: the trajectory benchmark's scene, subset
and camera path (kernels/rasterize/benchmark.py:26-90), the timing API
(timing.py), the dispatcher's backend names and the reference-side binding
(splats/rasterize.py:12-43).  No GPU."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from scipy.spatial.transform import Rotation

from gaussian_splats_hip import timing
from gaussian_splats_hip.kernels.rasterize import benchmark as bm
from gaussian_splats_hip.splats import GaussianSplat, PinholeCamera


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
    from gaussian_splats_hip import scenes
    from gaussian_splats_hip.splats.ply import save_ply

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
    from gaussian_splats_hip.splats.camera import host_extrinsics

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
