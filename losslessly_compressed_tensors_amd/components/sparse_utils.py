"""Optimizers whose state (and optionally weights) stays compressed between steps.

Same classes, arguments and update rules as ``LCT/components/sparse_utils.py``:

* ``SparseSGDM`` (``:13-68``): momentum ``m <- 0.9 m + g`` and weight
  ``p <- p - lr m``.  Compressed, both are single-pass fused kernels on the
  compressed operands (``LCTTensor.mul_add_``, ``LCTTensor.add_comp_``), or,
  for a dense weight, one fused decode-and-update.
* ``SparseMuon`` (``:98-160``): BF16 momentum decoded and freed, the dense
  Newton-Schulz update, momentum compressed again; a compressed weight takes
  ``p <- decay p - lr u`` in one fused kernel.
* ``SparseAdamW`` (``:163-214``): dense moments by default; compressed BF16
  moments and compressed weights round-trip through the codec.

Scalars that the fused kernels read (``momentum``, ``neg_lr``, ``decay``) are
FP32 device tensors on the parameters' device, so a step issues no host
synchronisation.  The dense math runs eagerly (no tracing compiler).
"""
from __future__ import annotations

import math
from typing import Iterable

import torch
from torch import Tensor

from ..LCTensor import LCTTensor
from ..operations import a_compA_add_B
from ..tensor_buffer import TensorBuffer
from .dist_configs import momentum_dist, momentum_first_dist


def _device_of(params) -> torch.device:
    for p in params:
        return p.device
    return torch.device("cuda", torch.cuda.current_device())


def _scalar(value: float, device) -> Tensor:
    return torch.tensor([value], dtype=torch.float32, device=device)


class SparseSGDM:
    """SGD with momentum, the momentum held compressed (``compressed=True``)."""

    def __init__(self, params: Iterable[LCTTensor | Tensor], lr, momentum=0.9,
                 buffer: TensorBuffer | None = None, compressed=True):
        self.params = list(params)
        for p in self.params:
            assert isinstance(p, (LCTTensor, Tensor)), "params must be a list of LCTTensor or Tensor"
        device = _device_of(self.params)
        self.lr = lr
        self.momentum = torch.tensor(momentum, dtype=torch.float32, device=device)
        self.compressed = compressed
        self.buffer = buffer
        self.momentums: list[Tensor | LCTTensor | None] = [None] * len(self.params)
        self.neg_lr = _scalar(-self.lr, device)

    @torch.no_grad()
    def step(self):
        for i, p in enumerate(self.params):
            g = p.grad
            mom = self.momentums[i]
            if mom is None:
                # The first momentum is the gradient itself.
                mom = LCTTensor(g, buffer=self.buffer, dist=momentum_dist) if self.compressed else g
                self.momentums[i] = mom
            elif self.compressed:
                mom.mul_add_(self.momentum, g)
            else:
                torch.add(g, mom, alpha=0.9, out=mom)

            if not self.compressed:
                p.add_(mom * self.neg_lr)
            elif isinstance(p, LCTTensor):
                p.add_comp_(mom, self.neg_lr)
            else:
                # One fused decode of the momentum into the update of p.
                p.copy_(a_compA_add_B(mom.x, self.neg_lr, p))

    def zero_grad(self):
        for p in self.params:
            p.grad = None


def zeropower_via_newtonschulz5(G: Tensor, ns_iters: int) -> Tensor:
    """Approximate orthogonalisation of G by the cubic Newton-Schulz iteration
    ``X <- 2 X - 1.5 (X X^T) X + 0.5 (X X^T)^2 X`` in BF16, on the wide
    orientation of G after scaling it to unit Frobenius norm
    (``LCT/components/sparse_utils.py:71-86``)."""
    assert G.ndim >= 2
    tall = G.size(-2) > G.size(-1)
    X = G.bfloat16()
    if tall:
        X = X.mT
    X = X / (X.norm(dim=(-2, -1), keepdim=True) + 1e-7)
    a, b, c = 2, -1.5, 0.5
    for _ in range(ns_iters):
        A = X @ X.mT
        B = b * A + c * A @ A
        X = a * X + B @ X
    return X.mT if tall else X


def muon_update(grad, momentum, mu=0.95, nesterov=True, ns_iters=5):
    """Momentum ``lerp`` toward the gradient, the Nesterov blend, then the
    orthogonalised update scaled by ``sqrt(max(1, rows / cols))``
    (``LCT/components/sparse_utils.py:89-95``).  Updates ``momentum`` and, with
    ``nesterov``, ``grad`` in place."""
    momentum.lerp_(grad.to(momentum.dtype), 1 - mu)
    update = grad.lerp_(momentum.to(grad.dtype), mu) if nesterov else momentum
    update = zeropower_via_newtonschulz5(update, ns_iters)
    update *= max(1, grad.size(-2) / grad.size(-1)) ** 0.5
    return update


class SparseMuon:
    """Muon with BF16 momentum, compressed between steps (``compressed=True``)."""

    def __init__(self, params: Iterable[LCTTensor | Tensor], lr=0.02, weight_decay=0, mu=0.95,
                 buffer: TensorBuffer | None = None, compressed=True, distribution=None,
                 zero_first_step=False, ns_iters=5):
        self.params = list(params)
        for p in self.params:
            assert isinstance(p, (LCTTensor, Tensor)) and p.ndim >= 2, "Muon requires matrix parameters"
        device = _device_of(self.params)
        self.lr = lr
        self.weight_decay = weight_decay
        self.mu = mu
        self.distribution = distribution or momentum_dist
        self.decay = _scalar(1 - lr * weight_decay, device)
        self.compressed = compressed
        self.buffer = buffer
        self.momentums: list[Tensor | LCTTensor | None] = [None] * len(self.params)
        self.neg_lr = _scalar(-self.lr, device)
        self.first_step = zero_first_step
        self.ns_iters = ns_iters

    @torch.no_grad()
    def step(self):
        for i, p in enumerate(self.params):
            g = p.grad
            if g is None:
                continue
            mom = self.momentums[i]
            if mom is None:
                mom = torch.zeros_like(g, dtype=torch.bfloat16)
            elif self.compressed:
                mom = mom.decompress_free()
            self.momentums[i] = None

            update = muon_update(g, mom, mu=self.mu, ns_iters=self.ns_iters)
            if self.compressed:
                # The first step's momentum is mostly exact zeros.
                dist = momentum_first_dist if self.first_step else self.distribution
                mom = LCTTensor(mom, buffer=self.buffer, dist=dist)
            self.momentums[i] = mom
            del mom

            if isinstance(p, LCTTensor):
                p.mul_add_(self.decay, update, beta=self.neg_lr,
                           alpha_is_one=self.weight_decay == 0)
            else:
                p.mul_(1 - self.lr * self.weight_decay)
                p.add_(update, alpha=-self.lr)
            del update
        self.first_step = False

    def zero_grad(self):
        for p in self.params:
            p.grad = None


class SparseAdamW:
    """AdamW; BF16 moments optionally compressed between steps, compressed
    weights decoded for the update and encoded again."""

    def __init__(self, param_groups, *, betas=(0.8, 0.95), eps=1e-10,
                 weight_decay=0, compressed=True, buffer=None):
        self.param_groups = [dict(group, params=list(group["params"])) for group in param_groups]
        self.betas, self.eps, self.weight_decay = betas, eps, weight_decay
        self.compressed, self.buffer = compressed, buffer
        self.state = {}

    @torch.no_grad()
    def step(self):
        beta1, beta2 = self.betas
        for group in self.param_groups:
            lr = group["lr"]
            for p in group["params"]:
                grad = p.grad
                if grad is None:
                    continue
                state = self.state.setdefault(p, {"step": 0})
                state["step"] += 1
                t = state["step"]
                moments = []
                for key in ("exp_avg", "exp_avg_sq"):
                    value = state.pop(key, None)
                    if value is None:
                        value = torch.zeros_like(grad)
                    elif isinstance(value, LCTTensor):
                        value = value.decompress_free()
                    moments.append(value)
                avg, square_avg = moments
                avg.lerp_(grad, 1 - beta1)
                square_avg.mul_(beta2).addcmul_(grad, grad, value=1 - beta2)
                denom = square_avg.sqrt().div_(math.sqrt(1 - beta2 ** t)).add_(self.eps)
                weight = p.decompress() if isinstance(p, LCTTensor) else p
                weight.mul_(1 - lr * self.weight_decay)
                weight.addcdiv_(avg, denom, value=-lr / (1 - beta1 ** t))
                if isinstance(p, LCTTensor):
                    old = p.x
                    p.x = LCTTensor(weight, buffer=old.buffer, dist=old.distribution).x
                    old.free()
                for key, value in zip(("exp_avg", "exp_avg_sq"), moments):
                    keep = self.compressed and value.dtype == torch.bfloat16
                    state[key] = LCTTensor(value, buffer=self.buffer, dist=momentum_dist) if keep else value

    def zero_grad(self):
        for group in self.param_groups:
            for p in group["params"]:
                p.grad = None
