"""The CPU restatement of the L1 loss term against torch's autograd of the
reference expression (training/train.py:137-138), in float64."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import losses


def _torch_l1(x: np.ndarray, t: np.ndarray, clamp: bool):
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    y = xt.clamp(0, 1) if clamp else xt
    loss = (y - torch.tensor(t, dtype=torch.float64)).abs().mean()
    loss.backward()
    return float(loss.detach()), xt.grad.numpy()


@pytest.mark.parametrize("clamp", [False, True])
@pytest.mark.parametrize("shape", [(7, 5, 3), (16, 9, 3), (1,)])
def test_l1_matches_torch_autograd(shape, clamp):
    rng = np.random.default_rng(sum(shape) + clamp)
    x = rng.uniform(-0.3, 1.3, size=shape)
    t = rng.uniform(0.0, 1.0, size=shape)
    flat_x, flat_t = x.reshape(-1), t.reshape(-1)
    # Exact clamp edges and zero differences, where the gradient rules matter.
    flat_x[:1] = 0.0
    if flat_x.size > 3:
        flat_x[1] = 1.0
        flat_x[2] = flat_t[2]
        flat_x[3] = -0.0
    loss, grad = losses.l1_loss(x, t, clamp)
    ref_loss, ref_grad = _torch_l1(x, t, clamp)
    assert loss == pytest.approx(ref_loss, rel=1e-14)
    np.testing.assert_array_equal(grad, ref_grad)


def test_l1_planted_mistakes_are_caught():
    """A dropped clamp mask or a wrong sign would differ from autograd."""
    rng = np.random.default_rng(3)
    x = rng.uniform(-0.5, 1.5, size=(64,))
    t = rng.uniform(0.0, 1.0, size=(64,))
    _, ref_grad = _torch_l1(x, t, True)
    _, unmasked = losses.l1_loss(x, t, False)  # gradient without the clamp's mask
    assert not np.array_equal(unmasked, ref_grad)
    _, grad = losses.l1_loss(x, t, True)
    assert not np.array_equal(-grad, ref_grad)


def test_l1_nan_and_empty():
    loss, grad = losses.l1_loss(np.array([np.nan, 0.5]), np.array([0.0, 0.0]), True)
    assert np.isnan(loss)
    assert grad[0] == 0.0 and grad[1] == 0.5
    loss, grad = losses.l1_loss(np.zeros(0), np.zeros(0))
    assert np.isnan(loss) and grad.size == 0


def _torch_ssim(x: np.ndarray, t: np.ndarray):
    """torchmetrics' algorithm written with torch conv2d (float64, autograd):
    reflect-pad by 5, 2-D Gaussian kernel (outer product), five moment maps,
    variances clamped at 0, crop by 5, mean."""
    import torch.nn.functional as F

    xt = torch.tensor(x, dtype=torch.float64).permute(2, 0, 1)[None].requires_grad_(True)
    tt = torch.tensor(t, dtype=torch.float64).permute(2, 0, 1)[None]
    c = xt.shape[1]
    g = torch.tensor(losses.ssim_window(), dtype=torch.float64)
    kernel = (g[:, None] @ g[None, :]).expand(c, 1, 11, 11)
    p = F.pad(xt, (5, 5, 5, 5), mode="reflect")
    q = F.pad(tt, (5, 5, 5, 5), mode="reflect")
    out = F.conv2d(torch.cat((p, q, p * p, q * q, p * q)), kernel, groups=c)
    mx, my, exx, eyy, exy = out.split(1)
    sxx = torch.clamp(exx - mx * mx, min=0.0)
    syy = torch.clamp(eyy - my * my, min=0.0)
    sxy = exy - mx * my
    s = ((2 * mx * my + losses.SSIM_C1) * (2 * sxy + losses.SSIM_C2)) / (
        (mx * mx + my * my + losses.SSIM_C1) * (sxx + syy + losses.SSIM_C2)
    )
    value = s[..., 5:-5, 5:-5].mean()
    value.backward()
    return float(value.detach()), xt.grad[0].permute(1, 2, 0).numpy()


def test_ssim_window_matches_scipy():
    from scipy import ndimage

    w = losses.ssim_window()
    assert w.size == 11 and abs(w.sum() - 1) < 1e-15
    impulse = np.zeros(11)
    impulse[5] = 1.0
    ref = ndimage.gaussian_filter1d(impulse, 1.5, truncate=5 / 1.5, mode="constant")
    np.testing.assert_allclose(w, ref[::-1], rtol=1e-12)


@pytest.mark.parametrize("shape", [(16, 17, 3), (31, 24, 3), (11, 11, 3)])
def test_ssim_matches_torch_conv_autograd(shape):
    rng = np.random.default_rng(shape[0])
    x = rng.random(shape)
    t = np.clip(x + rng.normal(0, 0.2, shape), 0, 1)
    value, grad = losses.ssim(x, t)
    ref_value, ref_grad = _torch_ssim(x, t)
    assert value == pytest.approx(ref_value, rel=1e-12)
    np.testing.assert_allclose(grad, ref_grad, rtol=1e-9, atol=1e-14)


def test_ssim_matches_scipy_moments():
    from scipy import ndimage

    rng = np.random.default_rng(9)
    x, t = rng.random((25, 30, 3)), rng.random((25, 30, 3))

    def f(a):
        return np.stack([ndimage.gaussian_filter(a[..., ch], 1.5, truncate=5 / 1.5) for ch in range(3)], -1)

    mx, my = f(x), f(t)
    sxx = np.maximum(f(x * x) - mx**2, 0)
    syy = np.maximum(f(t * t) - my**2, 0)
    sxy = f(x * t) - mx * my
    s = ((2 * mx * my + 1e-4) * (2 * sxy + 9e-4)) / ((mx**2 + my**2 + 1e-4) * (sxx + syy + 9e-4))
    assert losses.ssim(x, t)[0] == pytest.approx(s[5:-5, 5:-5].mean(), rel=1e-12)


def test_ssim_known_answers_and_planted_mistake(monkeypatch):
    rng = np.random.default_rng(4)
    x = rng.random((20, 20, 3))
    value, grad = losses.ssim(x, x)
    assert value == pytest.approx(1.0, abs=1e-12)
    assert np.abs(grad).max() < 1e-12  # the maximum: zero gradient
    # Constant images: s = (2ab + c1) / (a^2 + b^2 + c1) exactly.
    a, b = 0.3, 0.7
    value, _ = losses.ssim(np.full((15, 15, 3), a), np.full((15, 15, 3), b))
    assert value == pytest.approx((2 * a * b + 1e-4) / (a * a + b * b + 1e-4), rel=1e-12)
    # An unnormalised window (a plausible slip) moves the value: the conv2d
    # and scipy checks above would fail.
    t = rng.random((20, 20, 3))
    good = losses.ssim(x, t)[0]
    monkeypatch.setattr(losses, "ssim_window", lambda: np.exp(-((np.arange(11) - 5) / 1.5) ** 2 / 2))
    assert abs(losses.ssim(x, t)[0] - good) > 1e-3
