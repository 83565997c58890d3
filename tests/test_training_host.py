"""Host-side checks of the training-step wrappers (no GPU): FusedAdam's
validation of the tensors its launch reads and writes."""

from __future__ import annotations

import pytest
import torch


def test_fused_adam_refuses_mismatched_state():
    """FusedAdam's launch reads p.numel() floats of the gradient and moments:
    a wrong size, dtype or device is refused on the host."""
    from gaussian_splats_hip.training.optim import check_adam_tensors

    p = torch.zeros(10)
    ok = torch.zeros(10)
    check_adam_tensors(p, ok, ok.clone(), ok.clone())
    with pytest.raises(ValueError, match="exp_avg has 9"):
        check_adam_tensors(p, ok, torch.zeros(9), ok)
    with pytest.raises(ValueError, match="grad has 11"):
        check_adam_tensors(p, torch.zeros(11), ok, ok)
    with pytest.raises(TypeError, match="exp_avg_sq is torch.float64"):
        check_adam_tensors(p, ok, ok, torch.zeros(10, dtype=torch.float64))
    with pytest.raises(ValueError, match="meta"):
        check_adam_tensors(p, ok, torch.zeros(10, device="meta"), ok)
    with pytest.raises(ValueError, match="contiguous"):
        check_adam_tensors(p, ok, torch.zeros(20)[::2], ok)
