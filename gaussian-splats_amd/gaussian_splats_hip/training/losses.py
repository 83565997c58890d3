"""Photometric losses of the training step on the HIP library.

``l1_loss(image, target, clamp)`` is the term
``(image.clamp(0, 1) - target).abs().mean()`` of the reference's training step
(src/gaussian_splats/training/train.py:137-138; ``clamp=False`` drops the
clamp) as one autograd node: a forward kernel that reduces the absolute
differences and keeps a one-byte gradient sign per element, and a backward
kernel that expands it.  The gradient equals autograd's for the torch
expression bit for bit; the loss value is a deterministic fp32 sum that
matches torch's reduction to rounding.

``ssim(image, target)`` is the structural-similarity term of the same step
(train.py:139, training/utils.py:65-67): a forward kernel computes the
windowed moments, the mean SSIM and three per-pixel gradient maps; a backward
kernel filters those maps into the image gradient.
"""

from __future__ import annotations

import torch

from ..kernels.rasterize import _native as nat


def l1_loss_forward(
    image: torch.Tensor, target: torch.Tensor, clamp: bool = False
) -> tuple[torch.Tensor, torch.Tensor]:
    """Forward kernel: returns ``(loss, code)`` with ``code`` the int8 gradient
    sign per element that :func:`l1_loss_backward` expands."""
    device = nat.require_gpu(image, target)
    if image.shape != target.shape:
        raise ValueError(f"image {tuple(image.shape)} and target {tuple(target.shape)} differ")
    image = nat.prepare(image)
    target = nat.prepare(target)
    lib = nat.library()
    loss = torch.empty((), dtype=torch.float32, device=device)
    code = torch.empty(image.shape, dtype=torch.int8, device=device)
    numel = image.numel()
    ws_bytes = lib.gs_l1_loss_workspace_bytes(numel)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    nat.check(
        lib.gs_l1_loss_fwd(
            nat.ptr(image), nat.ptr(target), numel, int(bool(clamp)), nat.ptr(loss),
            nat.ptr(code), nat.ptr(ws), ws_bytes, nat.stream(device),
        ),
        "l1_loss",
    )
    return loss, code


def l1_loss_backward(code: torch.Tensor, grad_loss: torch.Tensor) -> torch.Tensor:
    """Backward kernel: gradient of the loss with respect to the image, for
    the upstream gradient ``grad_loss`` (a one-element device tensor)."""
    nat.require_gpu(code, grad_loss)
    grad_loss = nat.prepare(grad_loss.reshape(()))
    grad_image = torch.empty(code.shape, dtype=torch.float32, device=code.device)
    nat.check(
        nat.library().gs_l1_loss_bwd(
            nat.ptr(code), nat.ptr(grad_loss), code.numel(), nat.ptr(grad_image),
            nat.stream(code.device),
        ),
        "l1_loss backward",
    )
    return grad_image


class _L1Loss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, image: torch.Tensor, target: torch.Tensor, clamp: bool) -> torch.Tensor:
        loss, code = l1_loss_forward(image, target, clamp)
        ctx.save_for_backward(code)
        return loss

    @staticmethod
    def backward(ctx, grad_loss: torch.Tensor):
        (code,) = ctx.saved_tensors
        return l1_loss_backward(code, grad_loss), None, None


def l1_loss(image: torch.Tensor, target: torch.Tensor, clamp: bool = False) -> torch.Tensor:
    """Mean absolute difference of ``image`` (clamped to [0, 1] when ``clamp``)
    and ``target``; differentiable with respect to ``image`` only."""
    if target.requires_grad:
        raise ValueError("l1_loss does not propagate gradients to the target")
    if image.dtype != torch.float32 or target.dtype != torch.float32:
        raise TypeError("l1_loss expects float32 tensors")
    return _L1Loss.apply(image, target, clamp)


def ssim_forward(image: torch.Tensor, target: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Forward kernel: returns ``(ssim, workspace)``; the workspace holds what
    :func:`ssim_backward` needs."""
    device = nat.require_gpu(image, target)
    if image.shape != target.shape or image.dim() != 3 or image.shape[2] != 3:
        raise ValueError(
            f"ssim expects [H, W, 3] image and target, got {tuple(image.shape)} and {tuple(target.shape)}"
        )
    image = nat.prepare(image)
    target = nat.prepare(target)
    h, w = image.shape[0], image.shape[1]
    lib = nat.library()
    out = torch.empty((), dtype=torch.float32, device=device)
    ws_bytes = lib.gs_ssim_workspace_bytes(h, w)
    ws = nat.workspace(ws_bytes, device)
    nat.check(
        lib.gs_ssim_fwd(nat.ptr(image), nat.ptr(target), h, w, nat.ptr(out), nat.ptr(ws),
                        ws.numel(), nat.stream(device)),
        "ssim",
    )
    return out, ws


def ssim_backward(
    image: torch.Tensor, target: torch.Tensor, workspace: torch.Tensor, grad_ssim: torch.Tensor
) -> torch.Tensor:
    """Backward kernel: gradient of the SSIM with respect to the image for the
    upstream gradient ``grad_ssim`` (a one-element device tensor)."""
    device = nat.require_gpu(image, target, workspace, grad_ssim)
    image = nat.prepare(image)
    target = nat.prepare(target)
    grad_ssim = nat.prepare(grad_ssim.reshape(()))
    h, w = image.shape[0], image.shape[1]
    grad = torch.empty_like(image)
    nat.check(
        nat.library().gs_ssim_bwd(
            nat.ptr(image), nat.ptr(target), h, w, nat.ptr(grad_ssim), nat.ptr(workspace),
            workspace.numel(), nat.ptr(grad), nat.stream(device),
        ),
        "ssim backward",
    )
    return grad


class _Ssim(torch.autograd.Function):
    @staticmethod
    def forward(ctx, image: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        value, ws = ssim_forward(image, target)
        ctx.save_for_backward(image, target, ws)
        return value

    @staticmethod
    def backward(ctx, grad_ssim: torch.Tensor):
        image, target, ws = ctx.saved_tensors
        return ssim_backward(image, target, ws, grad_ssim), None


def ssim(image: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """Mean structural similarity of two [H, W, 3] images with data range 1,
    as the reference's training/utils.py:65-67 computes it with torchmetrics
    (11-tap Gaussian window, sigma 1.5, k1 = 0.01, k2 = 0.03, mean over the
    map cropped by 5 pixels and the channels); differentiable with respect to
    ``image`` only."""
    if target.requires_grad:
        raise ValueError("ssim does not propagate gradients to the target")
    if image.dtype != torch.float32 or target.dtype != torch.float32:
        raise TypeError("ssim expects float32 tensors")
    return _Ssim.apply(image, target)


class _Regularizers(torch.autograd.Function):
    @staticmethod
    def forward(ctx, opacity: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        device = nat.require_gpu(opacity, scale)
        n = opacity.shape[0]
        if opacity.numel() != n or scale.shape != (n, 3):
            raise ValueError(f"expected opacity [N, 1] and scale [N, 3], got {tuple(opacity.shape)} "
                             f"and {tuple(scale.shape)}")
        opacity, scale = nat.prepare(opacity), nat.prepare(scale)
        lib = nat.library()
        out = torch.empty(2, dtype=torch.float32, device=device)
        ws = nat.workspace(lib.gs_splat_regularizers_workspace_bytes(n), device)
        nat.check(lib.gs_splat_regularizers_fwd(nat.ptr(opacity), nat.ptr(scale), n, nat.ptr(out),
                                                nat.ptr(ws), ws.numel(), nat.stream(device)),
                  "regularizers")
        ctx.save_for_backward(opacity, scale)
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        opacity, scale = ctx.saved_tensors
        grad_out = nat.prepare(grad_out.contiguous())
        grad_opacity = torch.empty_like(opacity)
        grad_scale = torch.empty_like(scale)
        nat.check(nat.library().gs_splat_regularizers_bwd(
            nat.ptr(opacity), nat.ptr(scale), opacity.shape[0], nat.ptr(grad_out),
            nat.ptr(grad_opacity), nat.ptr(grad_scale), nat.stream(opacity.device)),
            "regularizers backward")
        return grad_opacity, grad_scale


def splat_regularizers(opacity: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``[opacity.sigmoid().mean(), scale.exp().mean()]`` in one kernel each way:
    the two regularisers of the training step before their weights
    (train.py:140-141)."""
    if opacity.dtype != torch.float32 or scale.dtype != torch.float32:
        raise TypeError("splat_regularizers expects float32 tensors")
    return _Regularizers.apply(opacity, scale)
