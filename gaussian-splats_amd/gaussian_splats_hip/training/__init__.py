"""Training-step pieces that consume the rendered image: the loss terms of
the reference's training step and its optimiser, as HIP kernels."""

from .losses import (
    l1_loss,
    l1_loss_backward,
    l1_loss_forward,
    splat_regularizers,
    ssim,
    ssim_backward,
    ssim_forward,
)
from .optim import FusedAdam

__all__ = [
    "FusedAdam",
    "l1_loss",
    "l1_loss_backward",
    "l1_loss_forward",
    "splat_regularizers",
    "ssim",
    "ssim_backward",
    "ssim_forward",
]
