"""Training-step kernels on the GPU: the fused Adam step against
torch.optim.Adam (the GPU default, multi-tensor) and the CPU restatement, and
the fused regularisers against torch autograd (train.py:140-141, 151)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splats_hip.training import FusedAdam, splat_regularizers
from oracle import losses as olosses
from oracle import optim as oopt

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _params(seed, n=1001):
    g = torch.Generator().manual_seed(seed)
    shapes = [(n, 3), (n, 4), (n, 3), (n, 1), (n, 16, 3)]  # mean, rotation, scale, opacity, color
    return [torch.randn(s, generator=g) for s in shapes]


@pytest.mark.parametrize("weight_decay", [0.0, 0.01])
def test_fused_adam_matches_torch_adam(weight_decay):
    print(f"[adam] weight_decay={weight_decay}", flush=True)
    init = _params(0)
    ours = [torch.nn.Parameter(p.clone().to(DEV)) for p in init]
    ref = [torch.nn.Parameter(p.clone().to(DEV)) for p in init]
    lrs = [1.6e-4, 1e-3, 5e-3, 5e-2, 2.5e-3]
    groups = lambda ps: [{"params": [p], "lr": lr} for p, lr in zip(ps, lrs)]  # noqa: E731
    opt = FusedAdam(groups(ours), eps=1e-15, weight_decay=weight_decay)
    opt_ref = torch.optim.Adam(groups(ref), eps=1e-15, weight_decay=weight_decay)
    assert isinstance(opt, torch.optim.Adam)
    gen = torch.Generator().manual_seed(1)
    cpu = [p.double().numpy() for p in init]
    m = [np.zeros_like(c) for c in cpu]
    v = [np.zeros_like(c) for c in cpu]
    for step in range(1, 6):
        scale = 10.0 ** (-step)  # gradients over several magnitudes
        grads = [torch.randn(p.shape, generator=gen) * scale for p in init]
        for k, (a, b) in enumerate(zip(ours, ref)):
            a.grad = grads[k].to(DEV)
            b.grad = grads[k].to(DEV)
        lr0 = 1.6e-4 * 0.97**step  # the position group's rate changes every step
        opt.param_groups[0]["lr"] = lr0
        opt_ref.param_groups[0]["lr"] = lr0
        opt.step()
        opt_ref.step()
        for k in range(5):
            lr = lr0 if k == 0 else lrs[k]
            cpu[k], m[k], v[k] = oopt.adam_step(cpu[k], grads[k].double().numpy(), m[k], v[k], step,
                                                lr, eps=1e-15, weight_decay=weight_decay)
    torch.cuda.synchronize()
    for k, (a, b) in enumerate(zip(ours, ref)):
        # Against torch's float32 update: within a few float32 ulps of the parameter.
        torch.testing.assert_close(a.detach(), b.detach(), rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(a.detach().cpu().double().numpy(), cpu[k], rtol=1e-5, atol=1e-6)
        st, st_ref = opt.state[a], opt_ref.state[b]
        assert int(st["step"]) == int(st_ref["step"]) == 5
        # Moments near zero (sums of opposite terms) differ in the last bits.
        torch.testing.assert_close(st["exp_avg"], st_ref["exp_avg"], rtol=1e-5, atol=1e-9)
        torch.testing.assert_close(st["exp_avg_sq"], st_ref["exp_avg_sq"], rtol=1e-5, atol=1e-20)


def test_fused_adam_skips_parameters_without_grad():
    p = torch.nn.Parameter(torch.ones(10, device=DEV))
    q = torch.nn.Parameter(torch.ones(7, device=DEV))
    opt = FusedAdam([p, q], lr=0.1)
    p.grad = torch.full_like(p, 2.0)
    opt.step()
    torch.cuda.synchronize()
    assert torch.allclose(p.detach(), torch.full_like(p, 0.9))  # first step moves by lr
    assert torch.equal(q.detach(), torch.ones(7, device=DEV)) and len(opt.state[q]) == 0


def test_regularizers_match_torch():
    g = torch.Generator().manual_seed(3)
    o = (torch.randn(100_003, 1, generator=g) * 2).to(DEV).requires_grad_(True)
    s = (torch.randn(100_003, 3, generator=g) - 4).to(DEV).requires_grad_(True)
    out = splat_regularizers(o, s)
    (0.01 * out[0] + 0.02 * out[1]).backward()
    o2 = o.detach().clone().requires_grad_(True)
    s2 = s.detach().clone().requires_grad_(True)
    a, b = o2.sigmoid().mean(), s2.exp().mean()
    (0.01 * a + 0.02 * b).backward()
    torch.cuda.synchronize()
    torch.testing.assert_close(out.detach(), torch.stack([a, b]).detach(), rtol=1e-6, atol=0)
    torch.testing.assert_close(o.grad, o2.grad, rtol=1e-6, atol=0)
    torch.testing.assert_close(s.grad, s2.grad, rtol=1e-6, atol=0)
    (va, vb), (ga, gb) = olosses.splat_regularizers(o.detach().cpu().numpy(), s.detach().cpu().numpy())
    out = out.detach()
    assert abs(float(out[0]) - va) <= 1e-6 * va and abs(float(out[1]) - vb) <= 1e-6 * vb
    # float32's 1 - sigmoid(o) keeps few bits where sigmoid(o) is near 1
    # (torch's float32 formula shares this): absolute error against float64
    # relative to the largest gradient there.
    np.testing.assert_allclose(o.grad.cpu().numpy(), 0.01 * ga, rtol=1e-5,
                               atol=1e-6 * 0.01 * np.abs(ga).max())
    np.testing.assert_allclose(s.grad.cpu().numpy(), 0.02 * gb, rtol=1e-5)
