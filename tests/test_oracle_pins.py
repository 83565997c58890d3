"""Pins three oracle behaviours that random scenes never reach, against the
closed-form numbers of ``known_answers.py`` (CPU, float64):

* the 0.99 alpha ceiling and its zero gradient (reference
  src/gaussian_splats/kernels/rasterize/torch.py:205, composite_bwd.py:149);
* colour clamped below at 0 only (splats/utils.py:75);
* the 1.3 x tan(half-FOV) clamp of the EWA Jacobian, with no gradient
  through a clamped ratio (splats/camera.py:106-119).

Each of these oracle mutations fails at least one test here: MAX_ALPHA
0.99 -> 0.999, clamp_min(0) -> clamp(0, 1), the 1.3 factor -> 1.0, and the
clamp widened to 2x.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import known_answers as ka
from oracle import rasterizer as orc

F64 = torch.float64


def _peak_params():
    p = ka.PEAK
    mean = torch.tensor([p["mean"]], dtype=F64, requires_grad=True)
    rot = torch.tensor([p["rotation"]], dtype=F64, requires_grad=True)
    scale = torch.full((1, 3), p["log_scale"], dtype=F64, requires_grad=True)
    op = torch.tensor([[p["opacity_logit"]]], dtype=F64, requires_grad=True)
    col = torch.tensor([[p["dc"]]], dtype=F64, requires_grad=True)
    cam = orc.Camera(torch.eye(3, dtype=F64), torch.zeros(3, dtype=F64), p["fx"], p["fy"],
                     p["cx"], p["cy"], p["width"], p["height"])
    return (mean, rot, scale, op, col), cam


@pytest.mark.parametrize("tile_size", (4, 16))
def test_peak_forward_known_answer(tile_size):
    params, cam = _peak_params()
    r = orc.rasterize(*params, cam, tile_size=tile_size, near=0.1)
    # Colour: 1.7 stays 1.7, -0.3 becomes 0.
    np.testing.assert_allclose(r.projected.color.detach().numpy()[0], ka.PEAK_RGB, rtol=0, atol=1e-12)
    np.testing.assert_allclose(r.image.detach().numpy(), ka.peak_image(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(r.composite.final_transmittance.numpy(), ka.peak_transmittance(),
                               rtol=0, atol=1e-12)
    x, y = ka.PEAK["centre"]
    # The ceiling itself: alpha is exactly 0.99 at the centre, above 1 in red.
    np.testing.assert_allclose(r.image.detach().numpy()[y, x], [0.99 * 1.7, 0.99, 0.0], atol=1e-12)
    assert int(r.composite.n_contributors[y, x]) == 1


def _peak_grads(pixel):
    params, cam = _peak_params()
    r = orc.rasterize(*params, cam, tile_size=16, near=0.1)
    x, y = pixel
    r.image[y, x].sum().backward()
    return [p.grad.numpy() for p in params]


def test_peak_gradient_is_zero_through_the_ceiling():
    g_mean, g_rot, g_scale, g_op, g_col = _peak_grads(ka.PEAK["centre"])
    for g in (g_mean, g_rot, g_scale, g_op):
        np.testing.assert_array_equal(g, np.zeros_like(g))
    np.testing.assert_allclose(g_col[0, 0], ka.PEAK_CENTRE_GRAD_DC, rtol=1e-12, atol=0)


def test_peak_gradient_below_the_ceiling():
    x, y = ka.PEAK["centre"]
    g_mean, g_rot, g_scale, g_op, g_col = _peak_grads((x + 1, y))
    np.testing.assert_allclose(g_op[0, 0], ka.PEAK_RIGHT_GRAD_LOGIT, rtol=1e-10)
    np.testing.assert_allclose(g_mean[0], ka.PEAK_RIGHT_GRAD_MEAN, rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(g_scale[0], ka.PEAK_RIGHT_GRAD_LOG_SCALE, rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(g_col[0, 0], ka.PEAK_RIGHT_GRAD_DC, rtol=1e-12, atol=0)
    np.testing.assert_allclose(g_rot, 0.0, atol=1e-13)


def _jac_params():
    p = ka.JAC
    n = len(ka.JAC_MEANS)
    mean = torch.tensor(ka.JAC_MEANS, dtype=F64, requires_grad=True)
    rot = torch.tensor([[1.0, 0.0, 0.0, 0.0]] * n, dtype=F64, requires_grad=True)
    scale = torch.full((n, 3), p["log_scale"], dtype=F64, requires_grad=True)
    op = torch.zeros(n, 1, dtype=F64, requires_grad=True)
    col = torch.zeros(n, 1, 3, dtype=F64, requires_grad=True)
    cam = orc.Camera(torch.eye(3, dtype=F64), torch.zeros(3, dtype=F64), p["fx"], p["fy"],
                     p["cx"], p["cy"], p["width"], p["height"])
    return (mean, rot, scale, op, col), cam


def test_jacobian_clamp_covariance_known_answer():
    params, cam = _jac_params()
    proj = orc.project(*params, cam)
    np.testing.assert_allclose(proj.covariance.detach().numpy(), ka.jac_covariance(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(proj.inverse.detach().numpy(), ka.jac_inverse(), rtol=1e-12, atol=1e-15)
    # Pixel means use the unclamped ratio: (fx x/d + cx, -fy y/d + cy).
    m = ka.JAC_MEANS
    np.testing.assert_allclose(proj.mean.detach().numpy()[:, 0], 100 * m[:, 0] / 2 + 50, atol=1e-12)
    np.testing.assert_allclose(proj.mean.detach().numpy()[:, 1], -100 * m[:, 1] / 2 + 40, atol=1e-12)


@pytest.mark.parametrize("axis", (0, 1))
def test_jacobian_clamp_gradient_known_answer(axis):
    params, cam = _jac_params()
    proj = orc.project(*params, cam)
    expected = ka.jac_grad_inverse_diagonal(axis)
    proj.inverse[expected["rows"], axis, axis].sum().backward()
    mean, rot, scale = (p.grad.numpy() for p in params[:3])
    rows = expected["rows"]
    np.testing.assert_allclose(mean[rows], expected["mean"], rtol=1e-10, atol=1e-15)
    np.testing.assert_allclose(scale[rows], expected["log_scale"], rtol=1e-10, atol=1e-15)
    np.testing.assert_allclose(rot, 0.0, atol=1e-15)
