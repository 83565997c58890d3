"""CPU restatement of the training step's L1 term — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.

Restates src/gaussian_splats/training/train.py:137-138,
``(image.clamp(0, 1) - target).abs().mean()``, and the gradient autograd forms
for it: d loss / d image = sign(image' - target) / numel where the clamp passes
the gradient (0 <= image <= 1; torch's clamp backward) and 0 elsewhere, with
sign(0) = 0 (abs backward).  Pinned by tests/test_oracle_losses.py against
torch's autograd of the expression in float64.
"""

from __future__ import annotations

import numpy as np


def l1_loss(image: np.ndarray, target: np.ndarray, clamp: bool = False) -> tuple[float, np.ndarray]:
    """Returns (loss, gradient with respect to image), both in float64."""
    x = np.asarray(image, dtype=np.float64)
    t = np.asarray(target, dtype=np.float64)
    passes = np.ones(x.shape, dtype=bool)
    if clamp:
        passes = (x >= 0.0) & (x <= 1.0)
        x = np.where(np.isnan(x), x, np.clip(x, 0.0, 1.0))
    d = x - t
    loss = float(np.abs(d).sum() / d.size) if d.size else float("nan")
    grad = np.where(passes, np.sign(np.nan_to_num(d, nan=0.0)), 0.0) / max(d.size, 1)
    return loss, grad


SSIM_RADIUS = 5
SSIM_SIGMA = 1.5
SSIM_C1 = 0.01**2
SSIM_C2 = 0.03**2


def ssim_window() -> np.ndarray:
    """torchmetrics' 1-D Gaussian window for sigma = 1.5: 2 * int(3.5 * 1.5 + 0.5) + 1
    = 11 taps exp(-(d / sigma)^2 / 2), d = -5..5, normalised to sum 1."""
    taps = int(3.5 * SSIM_SIGMA + 0.5) * 2 + 1
    d = np.arange(taps, dtype=np.float64) - (taps - 1) / 2
    g = np.exp(-((d / SSIM_SIGMA) ** 2) / 2)
    return g / g.sum()


def _valid_filter(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Separable valid correlation of a [H, W, C] array with w along H and W."""
    k = w.size
    rows = np.lib.stride_tricks.sliding_window_view(a, k, axis=1) @ w  # [H, W-k+1, C]
    return np.lib.stride_tricks.sliding_window_view(rows, k, axis=0) @ w  # [H-k+1, W-k+1, C]


def _full_filter(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Adjoint of _valid_filter: scatters a [H-k+1, W-k+1, C] map back to [H, W, C]."""
    k = w.size
    r = k // 2
    padded = np.pad(a, ((2 * r, 2 * r), (2 * r, 2 * r), (0, 0)))
    return _valid_filter(padded, w[::-1])


def ssim(image: np.ndarray, target: np.ndarray) -> tuple[float, np.ndarray]:
    """Mean SSIM of [H, W, C] images (data range 1) and its gradient with respect
    to image, in float64: torchmetrics' structural_similarity_index_measure as
    training/utils.py:65-67 calls it (channels first, batch of one, Gaussian
    window, k1 = 0.01, k2 = 0.03, variances clamped at 0, map cropped by the
    window radius)."""
    x = np.asarray(image, dtype=np.float64)
    y = np.asarray(target, dtype=np.float64)
    w = ssim_window()
    mx, my = _valid_filter(x, w), _valid_filter(y, w)
    exx, eyy, exy = _valid_filter(x * x, w), _valid_filter(y * y, w), _valid_filter(x * y, w)
    vxx = exx - mx * mx
    pass_x = vxx >= 0
    sxx = np.maximum(vxx, 0.0)
    syy = np.maximum(eyy - my * my, 0.0)
    sxy = exy - mx * my
    a = 2 * mx * my + SSIM_C1
    b = 2 * sxy + SSIM_C2
    c = mx * mx + my * my + SSIM_C1
    d = sxx + syy + SSIM_C2
    s = a * b / (c * d)
    m = s.size
    gm = 2 * my * (b - a) / (c * d) - 2 * mx * s / c + np.where(pass_x, 2 * mx * s / d, 0.0)
    gxx = np.where(pass_x, -s / d, 0.0)
    gxy = 2 * a / (c * d)
    grad = (_full_filter(gm, w) + 2 * x * _full_filter(gxx, w) + y * _full_filter(gxy, w)) / m
    return float(s.mean()), grad


def splat_regularizers(opacity: np.ndarray, scale: np.ndarray):
    """The regularisers of train.py:140-141 before their weights:
    (mean sigmoid(opacity), mean exp(scale)) and their gradients, float64."""
    o = np.asarray(opacity, dtype=np.float64)
    s = np.asarray(scale, dtype=np.float64)
    y = 1 / (1 + np.exp(-o))
    e = np.exp(s)
    return (float(y.mean()), float(e.mean())), (y * (1 - y) / o.size, e / s.size)
