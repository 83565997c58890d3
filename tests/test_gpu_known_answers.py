"""The HIP kernels against the closed-form numbers of ``known_answers.py``:
the 0.99 alpha ceiling and its zero gradient, colour above 1 left unclamped,
and the 1.3 x half-FOV Jacobian clamp with no gradient through it (reference
src/gaussian_splats/kernels/rasterize/torch.py:205, splats/utils.py:75,
splats/camera.py:106-119).  The oracle is pinned to the same numbers by
``test_oracle_pins.py``, so these behaviours do not rest on the oracle and
the kernels sharing a constant."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import known_answers as ka
from gaussian_splats_hip.kernels.rasterize import project_and_count, project_bwd
from gaussian_splats_hip.kernels.rasterize.interface import rasterize_outputs

pytestmark = pytest.mark.gpu


def _peak_inputs(device, tile_size, requires_grad=False):
    p = ka.PEAK
    params = [
        torch.tensor([p["mean"]], dtype=torch.float32),
        torch.tensor([p["rotation"]], dtype=torch.float32),
        torch.full((1, 3), p["log_scale"], dtype=torch.float32),
        torch.tensor([[p["opacity_logit"]]], dtype=torch.float32),
        torch.tensor([[p["dc"]]], dtype=torch.float32),
    ]
    params = [t.to(device).requires_grad_(requires_grad) for t in params]
    return params, (
        *params, torch.eye(3), torch.zeros(3), p["fx"], p["fy"], p["cx"], p["cy"],
        p["width"], p["height"], tile_size, 0.999, 0.1, 100.0, "gaussian", 0.95,
    )


@pytest.mark.parametrize("tile_size", (4, 16))
def test_peak_forward_known_answer(device, tile_size):
    _, inputs = _peak_inputs(device, tile_size)
    image, final_t, ncon, _, _, pcol, *_ = rasterize_outputs(*inputs)
    np.testing.assert_allclose(pcol.cpu().numpy()[0], ka.PEAK_RGB, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(image.cpu().numpy(), ka.peak_image(), rtol=0, atol=1e-6)
    np.testing.assert_allclose(final_t.cpu().numpy(), ka.peak_transmittance(), rtol=0, atol=1e-6)
    x, y = ka.PEAK["centre"]
    # float32 min(alpha0, 0.99f): exactly 0.99f.
    assert image[y, x, 1].item() == np.float32(0.99) * np.float32(1.0)
    assert int(ncon[y, x]) == 1


def _peak_grads(device, pixel):
    params, inputs = _peak_inputs(device, 16, requires_grad=True)
    image = rasterize_outputs(*inputs)[0]
    x, y = pixel
    image[y, x].sum().backward()
    return [p.grad.cpu().numpy() for p in params]


def test_peak_gradient_is_zero_through_the_ceiling(device):
    g_mean, g_rot, g_scale, g_op, g_col = _peak_grads(device, ka.PEAK["centre"])
    for g in (g_mean, g_rot, g_scale, g_op):
        np.testing.assert_array_equal(g, np.zeros_like(g))
    np.testing.assert_allclose(g_col[0, 0], ka.PEAK_CENTRE_GRAD_DC, rtol=1e-6, atol=0)


def test_peak_gradient_below_the_ceiling(device):
    x, y = ka.PEAK["centre"]
    g_mean, g_rot, g_scale, g_op, g_col = _peak_grads(device, (x + 1, y))
    np.testing.assert_allclose(g_op[0, 0], ka.PEAK_RIGHT_GRAD_LOGIT, rtol=1e-4)
    np.testing.assert_allclose(g_mean[0], ka.PEAK_RIGHT_GRAD_MEAN, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(g_scale[0], ka.PEAK_RIGHT_GRAD_LOG_SCALE, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(g_col[0, 0], ka.PEAK_RIGHT_GRAD_DC, rtol=1e-5, atol=0)
    np.testing.assert_allclose(g_rot, 0.0, atol=1e-6)


def _jac_inputs(device):
    p = ka.JAC
    n = len(ka.JAC_MEANS)
    params = [
        torch.tensor(ka.JAC_MEANS, dtype=torch.float32),
        torch.tensor([[1.0, 0.0, 0.0, 0.0]] * n, dtype=torch.float32),
        torch.full((n, 3), p["log_scale"], dtype=torch.float32),
        torch.zeros(n, 1),
        torch.zeros(n, 1, 3),
    ]
    return [t.to(device) for t in params]


def test_jacobian_clamp_covariance_known_answer(device):
    p = ka.JAC
    params = _jac_inputs(device)
    pmean, pinv, *_ = project_and_count(
        *params, torch.eye(3), torch.zeros(3), p["fx"], p["fy"], p["cx"], p["cy"],
        p["width"], p["height"], 16, 0.1, 100.0, "gaussian", 0.95)
    np.testing.assert_allclose(pinv.cpu().numpy(), ka.jac_inverse(), rtol=2e-6, atol=1e-9)
    m = ka.JAC_MEANS
    np.testing.assert_allclose(pmean.cpu().numpy()[:, 0], 100 * m[:, 0] / 2 + 50, rtol=1e-6)
    np.testing.assert_allclose(pmean.cpu().numpy()[:, 1], -100 * m[:, 1] / 2 + 40, rtol=1e-6)


@pytest.mark.parametrize("axis", (0, 1))
def test_jacobian_clamp_gradient_known_answer(device, axis):
    """gs_project_bwd with dL/d inverse[i, axis, axis] = 1 on the rows with
    Sigma01 = 0.  counts are passed as ones: the stage zeroes the gradient of
    a Gaussian without intersections, and most of these lie off-screen."""
    p = ka.JAC
    params = _jac_inputs(device)
    n = params[0].shape[0]
    pmean, pinv, *_ = project_and_count(
        *params, torch.eye(3), torch.zeros(3), p["fx"], p["fy"], p["cx"], p["cy"],
        p["width"], p["height"], 16, 0.1, 100.0, "gaussian", 0.95)
    expected = ka.jac_grad_inverse_diagonal(axis)
    grad = torch.zeros(n, 9, device=device)
    grad[torch.as_tensor(expected["rows"], device=device), 2 if axis == 0 else 4] = 1.0
    counts = torch.ones(n, dtype=torch.int32, device=device)
    g_mean, g_rot, g_scale, g_op, g_col = (
        t.cpu().numpy() for t in project_bwd(
            *params, torch.eye(3), torch.zeros(3), pinv, grad, counts,
            p["fx"], p["fy"], p["width"], p["height"]))
    rows = expected["rows"]
    np.testing.assert_allclose(g_mean[rows], expected["mean"], rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(g_scale[rows], expected["log_scale"], rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(g_rot, 0.0, atol=1e-8)
    np.testing.assert_array_equal(g_op, np.zeros_like(g_op))
