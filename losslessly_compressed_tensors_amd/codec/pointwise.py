"""Pointwise operations on compressed tensors.

Host logic of ``LCT/codec/pointwise.py:28-304``:

* ``pointwise_compressed_dense``: ``compA + B``, ``compA * B`` or
  ``alpha * compA + beta * B`` with one compressed and one dense operand;
* ``pointwise_scale_add_compressed``: ``alpha * compA + compB`` with both
  compressed (one fused launch when geometries and buffering modes agree,
  else decode B and use the dense path).

Dense output is BF16.  Compressed output re-encodes the fused kernel's split
components (side bytes in storage order + exponent bytes in logical order)
with a freshly sampled center, so it equals ``compress(result)``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

from ..comp_format import Distribution, StorageLayout
from ..comp_tensor import CompressedTensor
from ..compression.huffman_tables import get_distribution_tables
from ..kernels import dispatch, hip
from ..tensor_buffer import TensorBuffer
from .decode import decode as decode_dense
from .decode import overlay_of, shifted_decode_table, storage_of
from .encode import encode as compress_dense
from .encode import encode_components as compress_components
from .geometry import geometry

DENSE_OUTPUT = hip.LCT_DENSE_OUTPUT
COMPRESSED_OUTPUT = hip.LCT_COMPRESSED_OUTPUT


@dataclass(frozen=True)
class PointwiseOp:
    """An in-kernel operation code paired with its PyTorch meaning."""

    name: str
    code: int
    torch_fn: Callable


# compA + B elementwise.
ADD = PointwiseOp("add", hip.LCT_OP_ADD, torch.add)
# compA * B elementwise.
MULTIPLY = PointwiseOp("multiply", hip.LCT_OP_MULTIPLY, torch.mul)
# alpha * compA + B, or alpha * compA + beta * B.
SCALAR_MUL_ADD = PointwiseOp(
    "scalar_mul_add", hip.LCT_OP_SCALAR_MUL_ADD,
    lambda left, right, alpha=1.0: (left.float() * alpha + right.float()).to(torch.bfloat16),
)
POINTWISE_OPS = {op.name: op for op in (ADD, MULTIPLY, SCALAR_MUL_ADD)}


def _allocate_outputs(data: CompressedTensor, policy: int):
    device = data.data.device
    if policy == DENSE_OUTPUT:
        output = torch.empty(data.logical_numel, dtype=torch.bfloat16, device=device)
        return output, output
    output = torch.empty(data.size, dtype=torch.uint8, device=device)
    return output, torch.empty_like(output)


def _launch_pointwise_compressed_dense(data: CompressedTensor, other: torch.Tensor,
                                       operation: PointwiseOp, policy: int, *,
                                       alpha: torch.Tensor | None = None,
                                       beta: torch.Tensor | None = None,
                                       alpha_is_one: bool = False):
    """One fused launch: decode ``data``, apply ``operation`` with ``other``."""
    scaled = operation is SCALAR_MUL_ADD
    other = other.contiguous().view(-1)
    _, _, rare_length = get_distribution_tables(data.distribution, data.data.device)
    block_symbols, lanes, steps, fixed_words = data.codec_geometry
    output, auxiliary = _allocate_outputs(data, policy)
    if data.logical_numel:
        dispatch.pointwise_dense(
            data.data, data.sign_mantissa, other, output, auxiliary, shifted_decode_table(data),
            data.size, data.center, alpha if scaled else None, beta if scaled else None,
            rare_length=rare_length, logical_numel=data.logical_numel,
            block_symbols=block_symbols, lanes=lanes, steps=steps, fixed_words=fixed_words,
            output_policy=policy, op=operation.code,
            alpha_is_one=(not scaled) or alpha_is_one, beta_is_one=(not scaled) or beta is None,
            overflow=overlay_of(data))
    return output, auxiliary


def _launch_scalar_mul_add_compressed_compressed(data: CompressedTensor,
                                                 other: CompressedTensor,
                                                 alpha: torch.Tensor, policy: int):
    """One fused launch of ``alpha * data + other`` (both compressed)."""
    _, _, rare_a = get_distribution_tables(data.distribution, data.data.device)
    _, _, rare_b = get_distribution_tables(other.distribution, other.data.device)
    if rare_a != rare_b:
        raise ValueError("two-compressed path requires matching RARE_LENGTH")
    block_symbols, lanes, steps, fixed_words = data.codec_geometry
    output, auxiliary = _allocate_outputs(data, policy)
    if data.logical_numel:
        dispatch.dual_mapped(
            data.data, data.sign_mantissa, shifted_decode_table(data), data.center,
            overlay_of(data),
            other.data, other.sign_mantissa, shifted_decode_table(other), other.center,
            overlay_of(other),
            output, auxiliary, alpha, data.size, rare_length=rare_a,
            logical_numel=data.logical_numel, block_symbols=block_symbols, lanes=lanes,
            steps=steps, fixed_words=fixed_words, output_policy=policy)
    return output, auxiliary


def pointwise_scale_add_compressed(data: CompressedTensor, other: CompressedTensor,
                                   alpha: torch.Tensor, *, dense_output: bool = True,
                                   buffer: TensorBuffer | None = None,
                                   distribution: Distribution | None = None):
    """``alpha * compA + compB`` (``LCT/codec/pointwise.py:159-210``)."""
    same_layout = (data.layout == StorageLayout.COMPRESSED
                   and other.layout == StorageLayout.COMPRESSED)
    same_buffering = (data.fallback_descriptor is None) == (other.fallback_descriptor is None)
    assert same_buffering, (
        "pointwise_scale_add_compressed requires both inputs to be buffer-backed "
        "or both to be non-buffer-backed")
    if same_layout and data.codec_geometry == other.codec_geometry:
        result_distribution = distribution or data.distribution
        if not dense_output and geometry(result_distribution) != data.codec_geometry:
            raise ValueError("matrix compressed output must preserve the input stream geometry")
        policy = DENSE_OUTPUT if dense_output else COMPRESSED_OUTPUT
        values, auxiliary = _launch_scalar_mul_add_compressed_compressed(
            data, other, alpha, policy)
        if dense_output:
            return values.reshape(data.shape)
        return compress_components(auxiliary, values, data.size, result_distribution, buffer,
                                   data.shape, precomputed=True,
                                   logical_numel=data.logical_numel)
    if other.layout == StorageLayout.RAW:
        other_dense = other.data.reshape(other.shape)
    else:
        other_dense = decode_dense(other)
    return pointwise_compressed_dense(data, other_dense, SCALAR_MUL_ADD, alpha=alpha,
                                      dense_output=dense_output, buffer=buffer,
                                      distribution=distribution)


def pointwise_compressed_dense(data: CompressedTensor, other: torch.Tensor,
                               operation: PointwiseOp, *, alpha: torch.Tensor | None = None,
                               beta: torch.Tensor | None = None, alpha_is_one: bool = False,
                               dense_output: bool = True, buffer: TensorBuffer | None = None,
                               distribution: Distribution | None = None):
    """``alpha * compA + beta * B`` or ``compA (+|*) B``
    (``LCT/codec/pointwise.py:213-278``)."""
    if tuple(other.shape) != data.shape:
        raise ValueError(f"{operation.name} expects tensors with the same shape")
    result_distribution = distribution or data.distribution
    if operation is SCALAR_MUL_ADD and alpha is None:
        raise ValueError("scalar_mul_add requires an alpha argument")
    if (data.layout == StorageLayout.COMPRESSED and not dense_output
            and geometry(result_distribution) != data.codec_geometry):
        raise ValueError("matrix compressed output must preserve the input stream geometry")

    if data.layout == StorageLayout.RAW:
        # Raw storage holds the dense tensor itself: plain torch arithmetic
        # (pointwise.py:242-261).
        left = data.data.reshape(data.shape)
        if operation is SCALAR_MUL_ADD:
            if alpha_is_one:
                if beta is None:
                    result = (left.float() + other.float()).to(torch.bfloat16)
                else:
                    result = torch.addcmul(left.float(), other.float(), beta).to(torch.bfloat16)
            elif beta is None:
                result = operation.torch_fn(left, other, alpha)
            else:
                result = torch.addcmul(other.float() * beta, left.float(),
                                       alpha).to(torch.bfloat16)
        else:
            result = operation.torch_fn(left, other)
        if dense_output:
            return result
        return compress_dense(result, result_distribution, buffer)

    policy = DENSE_OUTPUT if dense_output else COMPRESSED_OUTPUT
    values, auxiliary = _launch_pointwise_compressed_dense(
        data, other, operation, policy, alpha=alpha, beta=beta, alpha_is_one=alpha_is_one)
    if dense_output:
        return values.reshape(data.shape)
    return compress_components(auxiliary, values, data.size, result_distribution, buffer,
                               data.shape, precomputed=True, logical_numel=data.logical_numel)


__all__ = [
    "ADD", "MULTIPLY", "SCALAR_MUL_ADD", "POINTWISE_OPS", "PointwiseOp",
    "DENSE_OUTPUT", "COMPRESSED_OUTPUT",
    "pointwise_compressed_dense", "pointwise_scale_add_compressed", "storage_of",
]
