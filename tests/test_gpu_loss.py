"""Fused L1 loss (training/train.py:137-138) on the GPU against torch's
autograd of the same expression on the same device and against the CPU
restatement in float64."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gaussian_splats_hip.kernels.rasterize import _native as nat
from gaussian_splats_hip.training import l1_loss, l1_loss_backward, l1_loss_forward, ssim, ssim_forward
from oracle import losses as orc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _inputs(shape, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(shape, generator=g) * 1.4 - 0.2
    t = torch.rand(shape, generator=g)
    flat = x.view(-1)
    flat[0] = 0.0  # clamp edges pass the gradient
    if flat.numel() > 3:
        flat[1] = 1.0
        flat[2] = t.view(-1)[2]  # zero difference: zero gradient
        flat[3] = 1.5
    return x, t


def _torch_l1(x, t, clamp, scale):
    xg = x.detach().clone().requires_grad_(True)
    y = xg.clamp(0, 1) if clamp else xg
    loss = (y - t).abs().mean()
    (loss * scale).backward()
    return loss.detach(), xg.grad


@pytest.mark.parametrize("clamp", [False, True])
@pytest.mark.parametrize("shape", [(1080, 1920, 3), (37, 29, 3), (5,), (1,)])
def test_l1_loss_matches_torch(shape, clamp):
    print(f"[l1] shape={shape} clamp={clamp}", flush=True)
    x, t = _inputs(shape, seed=len(shape) + shape[0])
    xd, td = x.to(DEV), t.to(DEV)
    for scale in (1.0, 0.37):
        ref_loss, ref_grad = _torch_l1(xd, td, clamp, scale)
        xg = xd.clone().requires_grad_(True)
        loss = l1_loss(xg, td, clamp=clamp)
        (loss * scale).backward()
        loss = loss.detach()
        torch.cuda.synchronize()
        assert loss.shape == ()
        assert abs(float(loss) - float(ref_loss)) <= 1e-6 * max(1.0, abs(float(ref_loss)))
        # The gradient is autograd's product, bit for bit.
        assert torch.equal(xg.grad, ref_grad), float((xg.grad - ref_grad).abs().max())
    o_loss, o_grad = orc.l1_loss(x.double().numpy(), t.double().numpy(), clamp)
    assert abs(float(loss) - o_loss) <= 1e-6 * max(1.0, abs(o_loss))
    np.testing.assert_allclose(xg.grad.cpu().double().numpy(), 0.37 * o_grad, rtol=1e-6, atol=0)


def test_l1_loss_deterministic_and_empty():
    x, t = _inputs((256, 256, 3), seed=7)
    xd, td = x.to(DEV), t.to(DEV)
    a, ca = l1_loss_forward(xd, td, True)
    b, cb = l1_loss_forward(xd, td, True)
    assert torch.equal(a, b) and torch.equal(ca, cb)
    empty, code = l1_loss_forward(torch.zeros(0, 3, device=DEV), torch.zeros(0, 3, device=DEV))
    assert torch.isnan(empty) and code.numel() == 0
    assert l1_loss_backward(code, torch.ones((), device=DEV)).numel() == 0


def test_l1_loss_nan_pixel():
    x, t = _inputs((8, 8, 3), seed=3)
    x.view(-1)[5] = float("nan")
    loss, code = l1_loss_forward(x.to(DEV), t.to(DEV), True)
    assert torch.isnan(loss)
    assert int(code.view(-1)[5]) == 0


def test_l1_loss_unaligned_through_c_abi():
    """Scalar path: buffers that are not 16-byte aligned, odd element count."""
    numel = 1001
    x, t = _inputs((numel + 1,), seed=11)
    xd, td = x.to(DEV), t.to(DEV)
    code = torch.zeros(numel + 4, dtype=torch.int8, device=DEV)
    grad = torch.zeros(numel + 1, dtype=torch.float32, device=DEV)
    loss = torch.zeros((), device=DEV)
    lib = nat.library()
    ws_bytes = lib.gs_l1_loss_workspace_bytes(numel)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    s = nat.stream(DEV)
    off = lambda tensor, k: ctypes.c_void_p(tensor.data_ptr() + k * tensor.element_size())  # noqa: E731
    nat.check(lib.gs_l1_loss_fwd(off(xd, 1), off(td, 1), numel, 1, nat.ptr(loss), off(code, 1),
                                 nat.ptr(ws), ws_bytes, s), "fwd")
    one = torch.ones((), device=DEV)
    nat.check(lib.gs_l1_loss_bwd(off(code, 1), nat.ptr(one), numel, off(grad, 1), s), "bwd")
    ref_loss, ref_grad = _torch_l1(xd[1:], td[1:], True, 1.0)
    torch.cuda.synchronize()
    assert abs(float(loss) - float(ref_loss)) <= 1e-6
    assert torch.equal(grad[1:], ref_grad)
    assert int(code[0]) == 0 and int(code[numel + 1]) == 0 and float(grad[0]) == 0.0


def _torch_ssim_f32(x, t):
    """torchmetrics' algorithm in float32 with torch ops on the GPU (the plain
    PyTorch reference of the kernel): reflect pad, 2-D Gaussian conv2d of the
    five moment maps, clamped variances, crop, mean."""
    import torch.nn.functional as F

    from oracle import losses as olosses

    xt = x.permute(2, 0, 1)[None].detach().clone().requires_grad_(True)
    tt = t.permute(2, 0, 1)[None]
    g = torch.tensor(olosses.ssim_window(), dtype=torch.float32, device=x.device)
    kernel = (g[:, None] @ g[None, :]).expand(3, 1, 11, 11).contiguous()
    p = F.pad(xt, (5, 5, 5, 5), mode="reflect")
    q = F.pad(tt, (5, 5, 5, 5), mode="reflect")
    out = F.conv2d(torch.cat((p, q, p * p, q * q, p * q)), kernel, groups=3)
    mx, my, exx, eyy, exy = out.split(1)
    sxx = torch.clamp(exx - mx * mx, min=0.0)
    syy = torch.clamp(eyy - my * my, min=0.0)
    sxy = exy - mx * my
    s = ((2 * mx * my + 1e-4) * (2 * sxy + 9e-4)) / ((mx * mx + my * my + 1e-4) * (sxx + syy + 9e-4))
    value = s[..., 5:-5, 5:-5].mean()
    value.backward()
    return value.detach(), xt.grad[0].permute(1, 2, 0)


def _ssim_inputs(h, w, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(h, w, 3, generator=g)
    # A smooth region and a noisy one, as rendered images have.
    x[: h // 2] = x[: h // 2].mean()
    t = (x + 0.1 * torch.randn(h, w, 3, generator=g)).clamp(0, 1)
    return x, t


@pytest.mark.parametrize("shape", [(1080, 1920), (37, 29), (11, 11), (64, 80)])
def test_ssim_matches_torch_and_oracle(shape):
    h, w = shape
    print(f"[ssim] shape={shape}", flush=True)
    x, t = _ssim_inputs(h, w, seed=h + w)
    xd, td = x.to(DEV), t.to(DEV)
    xg = xd.clone().requires_grad_(True)
    value = ssim(xg, td)
    (0.7 * value).backward()
    torch.cuda.synchronize()
    ref_value, ref_grad = _torch_ssim_f32(xd, td)
    o_value, o_grad = orc.ssim(x.double().numpy(), t.double().numpy())
    value = value.detach()
    value_err = abs(float(value) - o_value)
    ref_value_err = abs(float(ref_value) - o_value)
    scale = np.abs(o_grad).max()
    err = np.abs(xg.grad.cpu().double().numpy() / 0.7 - o_grad).max() / scale
    ref_err = np.abs(ref_grad.cpu().double().numpy() - o_grad).max() / scale
    print(f"[ssim] value err {value_err:.2e} (torch float32 {ref_value_err:.2e}), "
          f"grad err {err:.2e} (torch float32 {ref_err:.2e})", flush=True)
    # Against float64: within 1e-5 for the value and 1e-4 of the largest
    # gradient, or no worse than 4x the float32 torch reference's own error.
    assert value_err <= max(1e-5, 4 * ref_value_err)
    assert err <= max(1e-4, 4 * ref_err)


def test_ssim_deterministic_and_checks():
    x, t = _ssim_inputs(96, 128, seed=1)
    xd, td = x.to(DEV), t.to(DEV)
    a, _ = ssim_forward(xd, td)
    b, _ = ssim_forward(xd, td)
    assert torch.equal(a, b)
    with pytest.raises(ValueError):
        ssim(torch.zeros(10, 30, 3, device=DEV), torch.zeros(10, 30, 3, device=DEV))
    with pytest.raises(ValueError):
        ssim(torch.zeros(30, 30, 4, device=DEV), torch.zeros(30, 30, 4, device=DEV))
