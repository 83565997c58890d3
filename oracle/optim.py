"""CPU restatement of the training step's optimiser update — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.

Restates the Adam update torch.optim.Adam applies in the reference's training
loop (src/gaussian_splats/training/train.py:115 builds it with eps = 1e-15;
train.py:151 steps it), for one tensor, in float64:
  g <- g + wd p;  m <- m + (1 - b1)(g - m);  v <- b2 v + (1 - b2) g^2;
  p <- p - lr / (1 - b1^t) * m / (sqrt(v) / sqrt(1 - b2^t) + eps).
Pinned by tests/test_oracle_optim.py against torch.optim.Adam in float64.
"""

from __future__ import annotations

import numpy as np


def adam_step(p, g, m, v, step, lr, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0):
    """One step at step count ``step`` (1-based, after incrementing); returns
    the new (p, m, v)."""
    p, g, m, v = (np.asarray(a, dtype=np.float64) for a in (p, g, m, v))
    if weight_decay:
        g = g + weight_decay * p
    m = m + (1 - beta1) * (g - m)
    v = beta2 * v + (1 - beta2) * g * g
    bc1 = 1 - beta1**step
    bc2 = 1 - beta2**step
    p = p - (lr / bc1) * m / (np.sqrt(v) / np.sqrt(bc2) + eps)
    return p, m, v
