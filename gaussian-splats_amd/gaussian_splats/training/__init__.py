"""Training-step pieces that consume the rendered image."""

from .losses import l1_loss, l1_loss_backward, l1_loss_forward, ssim, ssim_backward, ssim_forward

__all__ = [
    "l1_loss",
    "l1_loss_backward",
    "l1_loss_forward",
    "ssim",
    "ssim_backward",
    "ssim_forward",
]
