"""Adam for the Gaussian parameters in one HIP launch per step.

:class:`FusedAdam` is a ``torch.optim.Adam`` (so code that checks
``isinstance(optimizer, torch.optim.Adam)`` and edits its ``state`` -- the
reference's relocation, training/utils.py:186-205 -- keeps working) whose
``step`` applies the update of torch's multi-tensor Adam to every parameter
with ``gs_adam_step``: each element is read and written once.  Supported:
float32 GPU parameters, per-group ``lr``/``betas``/``eps``/``weight_decay``;
``amsgrad``, ``maximize`` and sparse gradients are not.
"""

from __future__ import annotations

import ctypes

import torch

from ..kernels.rasterize import _native as nat


def check_adam_tensors(p: torch.Tensor, grad: torch.Tensor, exp_avg: torch.Tensor,
                       exp_avg_sq: torch.Tensor) -> None:
    """The kernel reads ``p.numel()`` float32 values of the gradient and of both
    moments and writes the moments: each must be a contiguous float32 tensor of
    that size on the parameter's device.  torch.optim.Adam raises on a
    mismatched state too (in its elementwise ops); here a mismatch would be an
    out-of-bounds device access, so it is refused before the launch."""
    for name, t in (("grad", grad), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        if t.dtype != torch.float32:
            raise TypeError(f"FusedAdam: {name} is {t.dtype}, expected torch.float32")
        if t.device != p.device:
            raise ValueError(f"FusedAdam: {name} is on {t.device}, the parameter on {p.device}")
        if t.numel() != p.numel():
            raise ValueError(
                f"FusedAdam: {name} has {t.numel()} elements, the parameter {p.numel()}"
            )
        if not t.is_contiguous():
            raise ValueError(f"FusedAdam: {name} is not contiguous")


class FusedAdam(torch.optim.Adam):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
                 amsgrad=False, *, maximize=False):
        if amsgrad or maximize:
            raise NotImplementedError("FusedAdam implements plain Adam (no amsgrad, no maximize)")
        super().__init__(params, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                         foreach=False)

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        # Tensors of every group that share betas, eps and weight decay go into
        # one launch (the learning rate is per tensor).
        batches: dict[tuple, list] = {}
        # Every tensor whose address a launch receives stays referenced until
        # all launches are enqueued (a contiguous copy of a gradient would
        # otherwise return to the caching allocator before the kernel runs).
        keep_alive: list[torch.Tensor] = []
        device = None
        for group in self.param_groups:
            beta1, beta2 = group["betas"]
            key = (float(beta1), float(beta2), float(group["eps"]), float(group["weight_decay"]))
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("FusedAdam does not support sparse gradients")
                if p.dtype != torch.float32 or not p.is_cuda:
                    raise TypeError("FusedAdam updates float32 parameters on a ROCm GPU")
                if not p.is_contiguous():
                    raise ValueError("FusedAdam needs contiguous parameters")
                if device is None:
                    device = nat.require_gpu(p)
                elif p.device != device:
                    raise ValueError(f"parameters on different devices: {device} and {p.device}")
                state = self.state[p]
                if len(state) == 0:
                    state["step"] = torch.tensor(0.0, dtype=torch.float32)
                    state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                grad = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
                for name in ("exp_avg", "exp_avg_sq"):
                    if not state[name].is_contiguous():
                        state[name] = state[name].contiguous()
                check_adam_tensors(p, grad, state["exp_avg"], state["exp_avg_sq"])
                state["step"] += 1
                keep_alive += (p, grad, state["exp_avg"], state["exp_avg_sq"])
                batches.setdefault(key, []).append(nat.GsAdamTensor(
                    p.data_ptr(), grad.data_ptr(), state["exp_avg"].data_ptr(),
                    state["exp_avg_sq"].data_ptr(), p.numel(), float(group["lr"]),
                    int(state["step"].item()),
                ))
        lib = nat.library()
        for (beta1, beta2, eps, weight_decay), entries in batches.items():
            for i in range(0, len(entries), nat.ADAM_MAX_TENSORS):
                chunk = entries[i:i + nat.ADAM_MAX_TENSORS]
                array = (nat.GsAdamTensor * len(chunk))(*chunk)
                nat.check(
                    lib.gs_adam_step(ctypes.cast(array, ctypes.c_void_p), len(chunk), beta1, beta2,
                                     eps, weight_decay, nat.stream(device)),
                    "adam_step",
                )
        del keep_alive  # the launches are enqueued; the stream orders any reuse
        return loss
