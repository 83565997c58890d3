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
