"""The CPU restatements of the optimiser step and the regularisers against
torch (float64) on the CPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import losses
from oracle import optim as oopt


@pytest.mark.parametrize("weight_decay", [0.0, 0.01])
def test_adam_step_matches_torch(weight_decay):
    rng = np.random.default_rng(2)
    p0 = rng.normal(size=(50, 3))
    grads = [rng.normal(size=(50, 3)) * 10 ** rng.uniform(-8, 0) for _ in range(6)]
    tp = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.Adam([tp], lr=0.01, eps=1e-15, weight_decay=weight_decay, foreach=False)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for step, g in enumerate(grads, start=1):
        lr = 0.01 * 0.9 ** step  # the position group's rate changes every step
        opt.param_groups[0]["lr"] = lr
        tp.grad = torch.tensor(g)
        opt.step()
        p, m, v = oopt.adam_step(p, g, m, v, step, lr, eps=1e-15, weight_decay=weight_decay)
        np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-13, atol=1e-16)
    state = opt.state[tp]
    np.testing.assert_allclose(m, state["exp_avg"].numpy(), rtol=1e-13)
    np.testing.assert_allclose(v, state["exp_avg_sq"].numpy(), rtol=1e-13)


def test_adam_planted_mistake():
    """Dropping the second-moment bias correction changes the first step."""
    p, g = np.ones(4), np.full(4, 0.5)
    good = oopt.adam_step(p, g, np.zeros(4), np.zeros(4), 1, 0.1)[0]
    np.testing.assert_allclose(good, p - 0.1, rtol=1e-7)  # first step: p - lr sign(g)
    assert not np.allclose(p - 0.1 / 0.1 * 0.05 / (np.sqrt(0.00025) + 1e-8), good)


def test_regularizers_match_torch_autograd():
    rng = np.random.default_rng(5)
    o, s = rng.normal(0, 2, size=(100, 1)), rng.normal(-4, 1, size=(100, 3))
    to = torch.tensor(o, requires_grad=True)
    ts = torch.tensor(s, requires_grad=True)
    a, b = to.sigmoid().mean(), ts.exp().mean()
    (a + 2 * b).backward()
    (va, vb), (ga, gb) = losses.splat_regularizers(o, s)
    assert va == pytest.approx(float(a.detach()), rel=1e-14)
    assert vb == pytest.approx(float(b.detach()), rel=1e-14)
    np.testing.assert_allclose(ga, to.grad.numpy(), rtol=1e-13)
    np.testing.assert_allclose(2 * gb, ts.grad.numpy(), rtol=1e-13)

