"""``LCTTensor``: a BF16 tensor held compressed, with in-place fused updates.

Same behaviour as ``LCT/LCTensor.py:12-111``: every in-place update builds a
new ``CompressedTensor`` from the fused kernel's output and then frees the
previous one's arena reservation (stream order keeps that safe).
"""
from __future__ import annotations

import math

import torch
from torch import Tensor

from .comp_format import Distribution
from .comp_tensor import CompressedTensor
from .operations import (
    a_compA_add_B,
    a_compA_add_b_B,
    a_compA_add_b_B_batch,
    a_compA_add_compB,
    compA_add_B,
    compress,
    compress_batch,
    decompress,
)
from .tensor_buffer import TensorBuffer


class LCTTensor(Tensor):
    __torch_function__ = torch._C._disabled_torch_function_impl
    x: CompressedTensor

    @staticmethod
    def __new__(cls, x, buffer: TensorBuffer | None, dist: Distribution):
        assert x.dtype == torch.bfloat16
        assert x.device.type == "cuda", f"x.device={x.device}"
        return torch.Tensor._make_wrapper_subclass(
            cls, x.shape, dtype=x.dtype, device=x.device, requires_grad=x.requires_grad)

    def __init__(self, x: Tensor, buffer: TensorBuffer | None, dist: Distribution):
        self.x: CompressedTensor = compress(x, buffer=buffer, distribution=dist)

    @classmethod
    def compress_many(cls, tensors, buffer: TensorBuffer, dist: Distribution) -> list:
        """``LCTTensor(t, buffer, dist)`` of each tensor, compressed into
        ``buffer`` with one launch per 16 tensors (``compress_batch``)."""
        records = compress_batch(tensors, dist, buffer=buffer)
        out = []
        for tensor, record in zip(tensors, records):
            wrapper = cls.__new__(cls, tensor, buffer, dist)
            wrapper.x = record
            out.append(wrapper)
        return out

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func is torch.ops.aten.t.default or func is torch.ops.aten.permute.default:
            return decompress(args[0].x).T
        if func is torch.ops.aten.mm.default:
            a, b = args
            if isinstance(a, LCTTensor):
                a = decompress(a.x)
            if isinstance(b, LCTTensor):
                b = decompress(b.x)
            return a @ b
        raise NotImplementedError(f"{func} not implemented for LCTTensor")

    @property
    def nbytes(self):
        return self.x.memory_size()

    @property
    def dense_nbytes(self):
        return math.prod(self.x.shape) * 2

    @property
    def layout(self):
        return "LCT compressed"

    def __repr__(self):
        return f"LCTTensor({self.x})"

    def add_(self, update: Tensor):
        """In place ``x <- x + update``."""
        prev = self.x
        self.x = compA_add_B(prev, update, dense_output=False,
                             distribution=prev.distribution, buffer=prev.buffer)
        prev.free()

    def mul_add_(self, alpha: Tensor, update: Tensor, beta: Tensor | None = None, *,
                 alpha_is_one: bool = False):
        """In place ``x <- alpha * x + beta * update`` (beta defaults to 1)."""
        prev = self.x
        if beta is None:
            self.x = a_compA_add_B(prev, alpha, update, alpha_is_one=alpha_is_one,
                                   dense_output=False, distribution=prev.distribution,
                                   buffer=prev.buffer)
        else:
            self.x = a_compA_add_b_B(prev, alpha, update, beta, alpha_is_one=alpha_is_one,
                                     dense_output=False, distribution=prev.distribution,
                                     buffer=prev.buffer)
        prev.free()

    @staticmethod
    def mul_add_many(tensors, alpha: Tensor, updates, beta: Tensor | None = None, *,
                     alpha_is_one: bool = False) -> None:
        """``t.mul_add_(alpha, u, beta)`` for each pair: the tensors that share
        a buffer with one launch of each kind per 8 (``a_compA_add_b_B_batch``;
        a weight's update is a few codec blocks, so one launch per tensor
        would be bound by one block's latency), the others one by one."""
        tensors, updates = list(tensors), list(updates)
        if len(tensors) != len(updates):
            raise ValueError(f"one update per tensor: {len(tensors)} tensors, "
                             f"{len(updates)} updates")
        groups: dict[int, list] = {}
        for tensor, update in zip(tensors, updates):
            if tensor.x.buffer is None:
                tensor.mul_add_(alpha, update, beta, alpha_is_one=alpha_is_one)
            else:
                groups.setdefault(id(tensor.x.buffer), []).append((tensor, update))
        for members in groups.values():
            results = a_compA_add_b_B_batch(
                [t.x for t, _ in members], alpha, [u for _, u in members], beta,
                alpha_is_one=alpha_is_one, buffer=members[0][0].x.buffer)
            for (tensor, _), result in zip(members, results):
                prev, tensor.x = tensor.x, result
                prev.free()

    def add_comp_(self, update_comp: "LCTTensor", alpha: Tensor):
        """In place ``x <- x + alpha * update_comp`` with both compressed."""
        prev = self.x
        self.x = a_compA_add_compB(update_comp.x, alpha, prev, dense_output=False,
                                   buffer=prev.buffer, distribution=prev.distribution)
        prev.free()

    def decompress(self) -> Tensor:
        return decompress(self.x)

    def decompress_free(self) -> Tensor:
        """Decompress, then free the compressed representation."""
        dense = self.decompress()
        self.x.free()
        return dense

    def free(self):
        self.x.free()
