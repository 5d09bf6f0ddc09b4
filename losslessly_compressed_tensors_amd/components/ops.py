"""RMSNorm forward and backward for the compressed layers.

Same contract as ``LCT/components/ops.py:6-44``: ``rms_norm(x, gain)`` returns
``(y, rstd)`` over the last dimension, with the reciprocal RMS in FP32 and
``y`` in ``x``'s dtype; ``rms_norm_backward(grad, x, rstd, gain)`` returns
``(grad_x, grad_gain)`` (``grad_gain`` is ``None`` without a gain).  Both run
ATen's fused device kernels, so the dense regions around the codec need no
tracing compiler.  ``rms_norm`` is differentiable through ``rms_norm_backward``.
"""
from __future__ import annotations

import torch
from torch import Tensor


def _forward(x: Tensor, gain: Tensor | None) -> tuple[Tensor, Tensor]:
    return torch.ops.aten._fused_rms_norm.default(x, [x.shape[-1]], gain, None)


def rms_norm_backward(grad: Tensor, x: Tensor, rstd: Tensor,
                      gain: Tensor | None) -> tuple[Tensor, Tensor | None]:
    return torch.ops.aten._fused_rms_norm_backward.default(
        grad, x, [x.shape[-1]], rstd, gain, [True, gain is not None])


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gain):
        y, rstd = _forward(x, gain)
        ctx.save_for_backward(x, rstd, gain)
        ctx.mark_non_differentiable(rstd)
        return y, rstd

    @staticmethod
    def backward(ctx, grad, grad_rstd):
        x, rstd, gain = ctx.saved_tensors
        return rms_norm_backward(grad, x, rstd, gain)


def rms_norm(x: Tensor, gain: Tensor | None) -> tuple[Tensor, Tensor]:
    if torch.is_grad_enabled() and (x.requires_grad or (gain is not None and gain.requires_grad)):
        return _RMSNorm.apply(x, gain)
    return _forward(x, gain)
