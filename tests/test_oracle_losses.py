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
