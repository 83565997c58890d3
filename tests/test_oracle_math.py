"""Pins the oracle's projection math against independent statements of it:
the reference's own SH recurrence (utils.py:32-66, a different formula from the
oracle's closed form), scipy's spherical harmonics and rotations, finite
differences of the projection, and the EWA covariance composed from scipy
rotations.  CPU only."""

from __future__ import annotations

import math

import numpy as np
import pytest
import scipy.special as sps
import torch
from scipy.spatial.transform import Rotation

from oracle import rasterizer as orc


def _dirs(n=64, seed=0):
    rng = np.random.default_rng(seed)
    d = rng.normal(size=(n, 3))
    return d / np.linalg.norm(d, axis=1, keepdims=True)


def _recurrence_basis(d: torch.Tensor, k: int) -> torch.Tensor:
    """Associated-Legendre recurrence over bands with the x + iy edge update, the
    algorithm of the reference's spherical_harmonics (utils.py:32-66)."""
    degree = math.isqrt(k) - 1
    x, y, z = d.unbind(-1)
    bands = [torch.full_like(z[:, None], orc.SH_C0)]
    prev = bands[0]
    older = torch.zeros_like(prev)
    re, im = prev[:, 0], torch.zeros_like(z)
    for l in range(1, degree + 1):
        m = torch.arange(1 - l, l, dtype=d.dtype)
        a = torch.sqrt((4 * l * l - 1) / (l * l - m * m))
        b = torch.sqrt(((l - 1) ** 2 - m * m) / (4 * (l - 1) ** 2 - 1)) if l > 1 else torch.zeros_like(m)
        interior = a * (z[:, None] * prev - b * older)
        edge = -math.sqrt(3 if l == 1 else (2 * l + 1) / (2 * l))
        re, im = edge * (x * re - y * im), edge * (x * im + y * re)
        cur = torch.cat((im[:, None], interior, re[:, None]), -1)
        bands.append(cur)
        older = torch.nn.functional.pad(prev, (1, 1))
        prev = cur
    return torch.cat(bands, -1)


@pytest.mark.parametrize("k", (1, 4, 9, 16))
def test_sh_closed_form_equals_recurrence(k):
    d = torch.tensor(_dirs(), dtype=torch.float64)
    torch.testing.assert_close(orc.sh_basis(d, k), _recurrence_basis(d, k), rtol=0, atol=1e-13)


def test_sh_matches_scipy():
    """Real SH from scipy's complex SH (Condon-Shortley phase included):
    sqrt(2) Im Y_l^|m| for m < 0, Y_l^0, sqrt(2) Re Y_l^m for m > 0."""
    d = _dirs()
    theta = np.arccos(d[:, 2])
    phi = np.arctan2(d[:, 1], d[:, 0])
    cols = []
    for l in range(4):
        for m in range(-l, l + 1):
            y = sps.sph_harm_y(l, abs(m), theta, phi)
            cols.append(y.real if m == 0 else math.sqrt(2) * (y.imag if m < 0 else y.real))
    expected = np.stack(cols, -1)
    got = orc.sh_basis(torch.tensor(d), 16).numpy()
    np.testing.assert_allclose(got, expected, rtol=0, atol=1e-12)


def test_sh_orthonormal():
    """Gauss-Legendre x uniform-phi quadrature of Y_i Y_j over the sphere = identity."""
    nodes, weights = np.polynomial.legendre.leggauss(16)
    phis = np.linspace(0, 2 * np.pi, 32, endpoint=False)
    ct, ph = np.meshgrid(nodes, phis, indexing="ij")
    st = np.sqrt(1 - ct**2)
    d = np.stack((st * np.cos(ph), st * np.sin(ph), ct), -1).reshape(-1, 3)
    w = (weights[:, None] * np.full(32, 2 * np.pi / 32)[None]).reshape(-1)
    b = orc.sh_basis(torch.tensor(d), 16).numpy()
    gram = (b * w[:, None]).T @ b
    np.testing.assert_allclose(gram, np.eye(16), atol=1e-12)


def test_quaternion_matches_scipy():
    rng = np.random.default_rng(1)
    q = rng.normal(size=(50, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    got = orc.quaternion_to_rotation(torch.tensor(q)).numpy()
    expected = Rotation.from_quat(q[:, [1, 2, 3, 0]]).as_matrix()  # scipy: scalar last
    np.testing.assert_allclose(got, expected, atol=1e-14)
    np.testing.assert_allclose(np.linalg.det(got), 1.0, atol=1e-12)


def _camera(fx=300.0, fy=280.0, w=320, h=240, seed=2):
    rng = np.random.default_rng(seed)
    R = Rotation.from_rotvec(rng.normal(size=3) * 0.3).as_matrix()
    t = rng.normal(size=3) * 0.2 + np.array([0, 0, -5.0])
    return orc.Camera(torch.tensor(R), torch.tensor(t), fx, fy, w / 2 + 3.0, h / 2 - 2.0, w, h)


def _scene(n=40, seed=3, k=16):
    g = torch.Generator().manual_seed(seed)
    mean = torch.randn(n, 3, generator=g, dtype=torch.float64) * 0.5
    rot = torch.randn(n, 4, generator=g, dtype=torch.float64)
    scale = torch.randn(n, 3, generator=g, dtype=torch.float64) * 0.3 - 2
    op = torch.randn(n, 1, generator=g, dtype=torch.float64)
    col = torch.randn(n, k, 3, generator=g, dtype=torch.float64) * 0.3
    return mean, rot, scale, op, col


def test_pixel_conventions():
    """Camera looks down -Z, +x right, +y up, image rows grow downwards, no +0.5."""
    cam = orc.Camera(torch.eye(3, dtype=torch.float64), torch.zeros(3, dtype=torch.float64),
                     100.0, 100.0, 50.0, 40.0, 100, 80)
    pts = torch.tensor([[0.0, 0.0, -2.0], [1.0, 0.0, -2.0], [0.0, 1.0, -2.0]], dtype=torch.float64)
    proj = orc.project(pts, torch.tensor([[1.0, 0, 0, 0]] * 3, dtype=torch.float64),
                       torch.zeros(3, 3, dtype=torch.float64), torch.zeros(3, 1, dtype=torch.float64),
                       torch.zeros(3, 1, 3, dtype=torch.float64), cam)
    np.testing.assert_allclose(proj.mean.numpy(), [[50, 40, 2], [100, 40, 2], [50, -10, 2]])


def test_jacobian_matches_finite_differences():
    """The EWA Jacobian equals the derivative of (u, v) w.r.t. the camera-space
    point (inside the 1.3 x FOV clamp), which pins its signs and scaling."""
    cam = _camera()
    mean, rot, scale, op, col = _scene()
    R, t = cam.rotation, cam.translation
    p = mean @ R.T + t
    eps = 1e-6

    def uv(pc):
        d = -pc[:, 2]
        return torch.stack((cam.fx * pc[:, 0] / d + cam.cx, -cam.fy * pc[:, 1] / d + cam.cy), -1)

    J_fd = torch.stack([(uv(p + eps * e) - uv(p - eps * e)) / (2 * eps) for e in torch.eye(3, dtype=torch.float64)], -1)
    # Oracle covariance with a point-like Gaussian of known shape: Sigma3 = I * s^2.
    s = 0.01
    proj = orc.project(mean, torch.tensor([[1.0, 0, 0, 0]] * len(mean), dtype=torch.float64),
                       torch.full_like(mean, math.log(s)), op, col, cam, covariance_epsilon=0.0)
    inside = ((p[:, 0] / -p[:, 2]).abs() < 1.3 * cam.width / (2 * cam.fx)) & (
        (p[:, 1] / -p[:, 2]).abs() < 1.3 * cam.height / (2 * cam.fy))
    expected = (J_fd @ R) @ (J_fd @ R).transpose(-1, -2) * s * s
    torch.testing.assert_close(proj.covariance[inside], expected[inside], rtol=1e-6, atol=1e-12)


def test_covariance_matches_scipy_composition():
    """Sigma = J W (Rq S^2 Rq^T) W^T J^T + 0.03 I with Rq from scipy."""
    cam = _camera()
    mean, rot, scale, op, col = _scene()
    proj = orc.project(mean, rot, scale, op, col, cam)
    q = (rot / rot.norm(dim=-1, keepdim=True)).numpy()
    Rq = torch.tensor(Rotation.from_quat(q[:, [1, 2, 3, 0]]).as_matrix())
    S2 = torch.diag_embed(torch.exp(2 * scale))
    sigma3 = Rq @ S2 @ Rq.transpose(-1, -2)
    R, t = cam.rotation, cam.translation
    p = mean @ R.T + t
    d = -p[:, 2]
    lx = 1.3 * cam.width / (2 * cam.fx)
    ly = 1.3 * cam.height / (2 * cam.fy)
    J = torch.zeros(len(mean), 2, 3, dtype=torch.float64)
    J[:, 0, 0] = cam.fx / d
    J[:, 0, 2] = cam.fx * (p[:, 0] / d).clamp(-lx, lx) / d
    J[:, 1, 1] = -cam.fy / d
    J[:, 1, 2] = -cam.fy * (p[:, 1] / d).clamp(-ly, ly) / d
    JW = J @ R
    expected = JW @ sigma3 @ JW.transpose(-1, -2) + 0.03 * torch.eye(2, dtype=torch.float64)
    torch.testing.assert_close(proj.covariance, expected, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(proj.covariance @ proj.inverse, torch.eye(2, dtype=torch.float64).expand(len(mean), 2, 2), atol=1e-10, rtol=0)


def test_sh_colour_uses_direction_towards_camera():
    """rgb = max(B(normalize(camera centre - mean)) . c + 0.5, 0) (torch.py:198,
    utils.py:75): a Gaussian on the optical axis in front of the camera sees the
    camera along +z of its own frame when the camera sits at +z."""
    cam = orc.Camera(torch.eye(3, dtype=torch.float64), torch.tensor([0, 0, -6.0], dtype=torch.float64),
                     100.0, 100.0, 50.0, 50.0, 100, 100)  # camera centre (0, 0, 6)
    col = torch.zeros(1, 4, 3, dtype=torch.float64)
    col[0, 2] = torch.tensor([1.0, -1.0, 0.25])  # band-1 z coefficient
    proj = orc.project(torch.zeros(1, 3, dtype=torch.float64), torch.tensor([[1.0, 0, 0, 0]], dtype=torch.float64),
                       torch.zeros(1, 3, dtype=torch.float64), torch.zeros(1, 1, dtype=torch.float64), col, cam)
    c1 = math.sqrt(3 / (4 * math.pi))
    np.testing.assert_allclose(proj.color.numpy()[0], [0.5 + c1, max(0.0, 0.5 - c1), 0.5 + 0.25 * c1])
