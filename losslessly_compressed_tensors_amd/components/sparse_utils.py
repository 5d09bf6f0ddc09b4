"""Optimizers that keep their per-parameter state -- and, for ``LCTTensor``
parameters, the parameters themselves -- LCT-compressed between steps.

Class names, constructor arguments and the state they expose (``momentums``,
``state``) are those of ``LCT/components/sparse_utils.py`` (``SparseSGDM``
:13-68, ``SparseMuon`` :98-160, ``SparseAdamW`` :163-214), which trainers bind
to.  The update rules are the published algorithms:

* heavy-ball SGD (Polyak 1964, dampening 0): ``v_1 = g_1``,
  ``v_t = mu v_{t-1} + g_t``, ``p_t = p_{t-1} - lr v_t``;
* Muon (K. Jordan et al., 2024): BF16 momentum ``m_t = m_{t-1} + (1 - mu)
  (g_t - m_{t-1})``, the Nesterov direction ``d_t = g_t + mu (m_t - g_t)``,
  its polar factor approximated by a Newton-Schulz iteration and scaled by
  ``sqrt(max(1, rows / cols))``; ``p_t = (1 - lr wd) p_{t-1} - lr O(d_t)``;
* AdamW (Loshchilov and Hutter, 2019) with bias-corrected moments.

How this build runs them on one MI355X:

* **Fused kernels for compressed state.**  A compressed SGD velocity is
  advanced in one pass over its compressed form and the dense gradient
  (``LCTTensor.mul_add_``), and a compressed weight takes ``p - lr v`` in one
  pass over two compressed operands (``LCTTensor.add_comp_``); a dense weight
  takes it in one decode-and-update pass.  A compressed Muon weight takes
  ``decay p - lr u`` in one pass.
* **Batched orthogonalisation.**  Muon groups its matrices by shape (tall
  ones transposed to wide) and runs one batched Newton-Schulz per group: three
  batched GEMMs per iteration for the group instead of three per matrix.  A
  GPT-2-small step's 72 block matrices form two groups (48 of 768x768, 24 of
  768x3072), so 12 iterations take 72 GEMM launches instead of 2592.
* **Multi-tensor AdamW.**  Parameters with the same dtype and step count are
  updated together with ``torch._foreach_*`` operations.
* **No host synchronisation.**  Scalars that the fused kernels read live on
  the parameters' device as FP32 tensors.

Dense and compressed modes share every floating-point operation, so (the codec
being lossless) a compressed run's state and dense weights equal the dense
run's bit for bit; only a compressed weight's fused update rounds once where
the dense update rounds after each operation.
"""
from __future__ import annotations

import math
from typing import Iterable

import torch
from torch import Tensor

from ..LCTensor import LCTTensor
from ..codec.decode import decode_batch
from ..operations import a_compA_add_B
from ..tensor_buffer import TensorBuffer
from .dist_configs import momentum_dist, momentum_first_dist

# Newton-Schulz polynomial p(s) = a s + b s^3 + c s^5 on the singular values:
# p(1) = 1 and p'(1) = 0, so unit singular values attract quadratically.
_NS_A, _NS_B, _NS_C = 2.0, -1.5, 0.5
_NS_EPS = 1e-7


def _device_of(params: list) -> torch.device:
    return params[0].device if params else torch.device("cuda", torch.cuda.current_device())


def _fp32(value: float, device: torch.device) -> Tensor:
    """A one-element FP32 device scalar, as the fused kernels read them."""
    return torch.full((1,), float(value), dtype=torch.float32, device=device)


def _dense(p) -> Tensor:
    return p.decompress() if isinstance(p, LCTTensor) else p


class _StateBank(list):
    """One optimizer state tensor per parameter (``None`` until first use),
    held dense or, for BF16 values of a compressed optimizer, as an
    ``LCTTensor`` in the shared buffer.  A step checks a value out dense and
    checks the new value back in."""

    def __init__(self, size: int, compressed: bool, buffer: TensorBuffer | None):
        super().__init__([None] * size)
        self.compressed = compressed
        self.buffer = buffer

    def check_out(self, index: int, like: Tensor | None = None) -> Tensor | None:
        """The slot's dense value, leaving the slot empty: a compressed value is
        decoded and its arena region released.  An empty slot gives BF16 zeros
        shaped like ``like`` (or None)."""
        value, self[index] = self[index], None
        if isinstance(value, LCTTensor):
            return value.decompress_free()
        if value is None and like is not None:
            return torch.zeros_like(like, dtype=torch.bfloat16)
        return value

    def check_out_many(self, indices, likes) -> list:
        """``check_out`` of several slots, the compressed values decoded with
        one launch per 16 (``decode_batch``)."""
        values = [self[i] for i in indices]
        for i in indices:
            self[i] = None
        packed = [k for k, v in enumerate(values) if isinstance(v, LCTTensor)]
        for k, dense in zip(packed, decode_batch([values[k].x for k in packed])):
            values[k].free()   # ordered after the decode on this stream
            values[k] = dense
        return [torch.zeros_like(like, dtype=torch.bfloat16) if v is None and like is not None
                else v for v, like in zip(values, likes)]

    def check_in(self, index: int, value: Tensor, distribution) -> None:
        if self.compressed and value.dtype == torch.bfloat16:
            value = LCTTensor(value, buffer=self.buffer, dist=distribution)
        self[index] = value

    def check_in_many(self, indices, values, distribution) -> None:
        """``check_in`` of several slots; with a buffer the BF16 values are
        compressed with one launch per 16 (``LCTTensor.compress_many``)."""
        if not (self.compressed and self.buffer is not None):
            for index, value in zip(indices, values):
                self.check_in(index, value, distribution)
            return
        packed = [k for k, v in enumerate(values) if v.dtype == torch.bfloat16]
        stored = list(values)
        for k, value in zip(packed, LCTTensor.compress_many([values[k] for k in packed],
                                                            self.buffer, distribution)):
            stored[k] = value
        for index, value in zip(indices, stored):
            self[index] = value


class SparseSGDM:
    """Heavy-ball SGD; the velocity stays compressed between steps
    (``compressed=True``)."""

    def __init__(self, params: Iterable[LCTTensor | Tensor], lr, momentum=0.9,
                 buffer: TensorBuffer | None = None, compressed=True):
        self.params = list(params)
        if not all(isinstance(p, (LCTTensor, Tensor)) for p in self.params):
            raise AssertionError("params must be a list of LCTTensor or Tensor")
        device = _device_of(self.params)
        self.lr = lr
        self.buffer = buffer
        self.compressed = compressed
        self.momentum = torch.tensor(momentum, dtype=torch.float32, device=device)
        self._mu = float(momentum)
        self._one = _fp32(1.0, device)
        self.neg_lr = _fp32(-lr, device)
        # The velocities (``momentums`` in the reference's naming).
        self.momentums = _StateBank(len(self.params), compressed, buffer)

    @torch.no_grad()
    def step(self):
        for index, param in enumerate(self.params):
            velocity = self._advance(index, param.grad)
            self._descend(param, velocity)

    def _advance(self, index: int, grad: Tensor):
        """v <- mu v + g (v <- g on the first step)."""
        velocity = self.momentums[index]
        if velocity is None:
            self.momentums.check_in(index, grad, momentum_dist)
        elif isinstance(velocity, LCTTensor):
            velocity.mul_add_(self.momentum, grad)   # one fused pass, one rounding
        else:
            torch.add(grad, velocity, alpha=self._mu, out=velocity)
        return self.momentums[index]

    def _descend(self, param, velocity) -> None:
        """p <- p - lr v."""
        if isinstance(param, LCTTensor) and isinstance(velocity, LCTTensor):
            param.add_comp_(velocity, self.neg_lr)   # one pass over two compressed operands
        elif isinstance(param, LCTTensor):
            param.mul_add_(self._one, velocity, beta=self.neg_lr, alpha_is_one=True)
        elif isinstance(velocity, LCTTensor):
            # The velocity is decoded inside the update of p.
            param.copy_(a_compA_add_B(velocity.x, self.neg_lr, param))
        else:
            param.add_(velocity * self.neg_lr)

    def zero_grad(self):
        for p in self.params:
            p.grad = None


def _orthogonalize_wide(batch: Tensor, steps: int) -> Tensor:
    """Newton-Schulz approximation of the polar factor of every matrix in a
    ``(k, r, c)`` batch with ``r <= c``: each is scaled to unit Frobenius norm,
    then ``X <- a X + (b A + c A^2) X`` with ``A = X X^T``, ``steps`` times, in
    BF16.  Every product is a batched GEMM on contiguous operands."""
    x = batch.to(torch.bfloat16)
    x = x / (x.norm(dim=(-2, -1), keepdim=True) + _NS_EPS)
    for _ in range(steps):
        gram = torch.bmm(x, x.transpose(-2, -1).contiguous())
        poly = torch.baddbmm(gram, gram, gram, beta=_NS_B, alpha=_NS_C)
        x = torch.baddbmm(x, poly, x, beta=_NS_A, alpha=1.0)
    return x


def zeropower_via_newtonschulz5(G: Tensor, ns_iters: int) -> Tensor:
    """The Newton-Schulz polar factor of ``G`` (a matrix, or a batch of them in
    its last two dimensions), in BF16 and in ``G``'s orientation: the iteration
    runs on the wide orientation (``LCT/components/sparse_utils.py:71-86`` for
    the name and contract)."""
    if G.ndim < 2:
        raise AssertionError("orthogonalisation needs a matrix")
    tall = G.size(-2) > G.size(-1)
    wide = G.transpose(-2, -1) if tall else G
    out = _orthogonalize_wide(wide.reshape(-1, *wide.shape[-2:]), ns_iters).reshape(wide.shape)
    return out.transpose(-2, -1) if tall else out


def _nesterov(grad: Tensor, momentum: Tensor, mu: float, nesterov: bool) -> Tensor:
    """Advance the BF16 momentum toward the gradient and return Muon's
    direction: the Nesterov look-ahead (computed in ``grad``'s storage) or the
    momentum itself."""
    momentum.lerp_(grad.to(momentum.dtype), 1 - mu)
    if not nesterov:
        return momentum
    return grad.lerp_(momentum.to(grad.dtype), mu)


def _aspect_scale(rows: int, cols: int) -> float:
    return math.sqrt(max(1.0, rows / cols))


def muon_update(grad, momentum, mu=0.95, nesterov=True, ns_iters=5):
    """One Muon direction for one matrix: updates ``momentum`` (and, with
    ``nesterov``, ``grad``) in place and returns the orthogonalised, scaled
    update (the contract of ``LCT/components/sparse_utils.py:89-95``).  A
    ``SparseMuon`` holding this one matrix computes the same values."""
    direction = _nesterov(grad, momentum, mu, nesterov)
    update = zeropower_via_newtonschulz5(direction, ns_iters)
    return update.mul_(_aspect_scale(grad.size(-2), grad.size(-1)))


class SparseMuon:
    """Muon with BF16 momentum, compressed between steps (``compressed=True``)."""

    def __init__(self, params: Iterable[LCTTensor | Tensor], lr=0.02, weight_decay=0, mu=0.95,
                 buffer: TensorBuffer | None = None, compressed=True, distribution=None,
                 zero_first_step=False, ns_iters=5):
        self.params = list(params)
        if not all(isinstance(p, (LCTTensor, Tensor)) and p.ndim >= 2 for p in self.params):
            raise AssertionError("Muon requires matrix parameters")
        device = _device_of(self.params)
        self.lr, self.weight_decay, self.mu = lr, weight_decay, mu
        self.buffer, self.compressed = buffer, compressed
        self.distribution = distribution or momentum_dist
        self.ns_iters = ns_iters
        # The first step's momentum (1 - mu) g of a zero momentum is stored with
        # the half-zero codebook when the caller asks for it.
        self.first_step = zero_first_step
        self.decay = _fp32(1 - lr * weight_decay, device)
        self.neg_lr = _fp32(-lr, device)
        self.momentums = _StateBank(len(self.params), compressed, buffer)

    @torch.no_grad()
    def step(self):
        dist = momentum_first_dist if self.first_step else self.distribution
        # Matrices grouped by wide shape: (rows, cols) with rows <= cols.
        groups: dict[tuple, list[tuple[int, Tensor, bool]]] = {}
        active = [(index, param.grad) for index, param in enumerate(self.params)
                  if param.grad is not None]
        # Momenta are checked out 16 at a time: one decode launch for the 16
        # (each is a few codec blocks, so its own decode would be bound by one
        # block's latency), and at most 16 dense momenta at once.
        for start in range(0, len(active), 16):
            part = active[start:start + 16]
            momenta = self.momentums.check_out_many([i for i, _ in part], [g for _, g in part])
            for (index, grad), momentum in zip(part, momenta):
                direction = _nesterov(grad, momentum, self.mu, nesterov=True)
                tall = direction.size(-2) > direction.size(-1)
                wide = direction.transpose(-2, -1) if tall else direction
                groups.setdefault(tuple(wide.shape), []).append((index, wide, tall))
            # The momenta go back (compressed, one launch for the 16) before
            # the GEMMs: only the directions stay dense.
            self.momentums.check_in_many([i for i, _ in part], momenta, dist)
            del momenta
        for shape, members in groups.items():
            stacked = torch.stack([wide.reshape(-1, *shape[-2:]) for _, wide, _ in members])
            polar = _orthogonalize_wide(stacked.reshape(-1, *shape[-2:]), self.ns_iters)
            polar = polar.reshape(len(members), *shape)
            params, updates = [], []
            for (index, _, tall), factor in zip(members, polar.unbind(0)):
                param = self.params[index]
                update = factor.transpose(-2, -1) if tall else factor
                params.append(param)
                updates.append(update.mul(_aspect_scale(param.size(-2), param.size(-1))))
            self._apply_many(params, updates)
        self.first_step = False

    def _apply_many(self, params, updates) -> None:
        """``_apply`` of each pair; the compressed weights with one fused-update
        launch of each kind per 8 (``LCTTensor.mul_add_many``: each weight is
        a few codec blocks)."""
        compressed = [(p, u) for p, u in zip(params, updates) if isinstance(p, LCTTensor)]
        for param, update in zip(params, updates):
            if not isinstance(param, LCTTensor):
                self._apply(param, update)
        if compressed:
            LCTTensor.mul_add_many([p for p, _ in compressed], self.decay,
                                   [u for _, u in compressed], beta=self.neg_lr,
                                   alpha_is_one=self.weight_decay == 0)

    def _apply(self, param, update: Tensor) -> None:
        """p <- (1 - lr wd) p - lr u."""
        if isinstance(param, LCTTensor):
            param.mul_add_(self.decay, update, beta=self.neg_lr,
                           alpha_is_one=self.weight_decay == 0)
        else:
            param.mul_(1 - self.lr * self.weight_decay).add_(update, alpha=-self.lr)

    def zero_grad(self):
        for p in self.params:
            p.grad = None


class SparseAdamW:
    """AdamW; BF16 moments optionally compressed between steps, compressed
    weights decoded for the update and encoded again."""

    _MOMENTS = ("exp_avg", "exp_avg_sq")

    def __init__(self, param_groups, *, betas=(0.8, 0.95), eps=1e-10,
                 weight_decay=0, compressed=True, buffer=None):
        self.param_groups = [dict(group, params=list(group["params"])) for group in param_groups]
        self.betas, self.eps, self.weight_decay = betas, eps, weight_decay
        self.compressed, self.buffer = compressed, buffer
        self.state: dict = {}

    def _moment(self, state: dict, key: str, like: Tensor) -> Tensor:
        value = state.pop(key, None)
        if isinstance(value, LCTTensor):
            return value.decompress_free()
        return torch.zeros_like(like) if value is None else value

    def _keep(self, state: dict, key: str, value: Tensor) -> None:
        if self.compressed and value.dtype == torch.bfloat16:
            value = LCTTensor(value, buffer=self.buffer, dist=momentum_dist)
        state[key] = value

    @torch.no_grad()
    def step(self):
        beta1, beta2 = self.betas
        for group in self.param_groups:
            lr = group["lr"]
            # Parameters updated together: same gradient dtype and step count.
            buckets: dict[tuple, list] = {}
            for p in group["params"]:
                if p.grad is None:
                    continue
                state = self.state.setdefault(p, {"step": 0})
                state["step"] += 1
                buckets.setdefault((p.grad.dtype, p.grad.device, state["step"]), []).append(p)
            for (_, _, step), params in buckets.items():
                grads = [p.grad for p in params]
                states = [self.state[p] for p in params]
                avgs = [self._moment(s, "exp_avg", g) for s, g in zip(states, grads)]
                squares = [self._moment(s, "exp_avg_sq", g) for s, g in zip(states, grads)]
                torch._foreach_lerp_(avgs, grads, 1 - beta1)
                torch._foreach_mul_(squares, beta2)
                torch._foreach_addcmul_(squares, grads, grads, value=1 - beta2)
                denoms = torch._foreach_sqrt(squares)
                torch._foreach_div_(denoms, math.sqrt(1 - beta2 ** step))
                torch._foreach_add_(denoms, self.eps)
                weights = [_dense(p) for p in params]
                torch._foreach_mul_(weights, 1 - lr * self.weight_decay)
                torch._foreach_addcdiv_(weights, avgs, denoms, value=-lr / (1 - beta1 ** step))
                for p, weight in zip(params, weights):
                    if isinstance(p, LCTTensor):
                        previous = p.x
                        p.x = LCTTensor(weight, buffer=previous.buffer,
                                        dist=previous.distribution).x
                        previous.free()
                for state, avg, square in zip(states, avgs, squares):
                    self._keep(state, "exp_avg", avg)
                    self._keep(state, "exp_avg_sq", square)

    def zero_grad(self):
        for group in self.param_groups:
            for p in group["params"]:
                p.grad = None
