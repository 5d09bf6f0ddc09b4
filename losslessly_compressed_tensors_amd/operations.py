"""Public API: lossless BF16 compression, decompression and fused updates.

Same functions, arguments and errors as ``LCT/operations.py:18-136``; the
compute runs in the gfx950 library ``liblct_hip.so``.
"""
from __future__ import annotations

import torch
from torch import Tensor

from .codec.decode import decode as decode_dense
from .codec.encode import encode as compress_dense
from .codec.encode import encode_batch
from .codec.pointwise import (
    ADD,
    MULTIPLY,
    SCALAR_MUL_ADD,
    fused_update_batch,
    pointwise_compressed_dense,
    pointwise_scale_add_compressed,
)
from .comp_format import Distribution, StorageLayout
from .comp_tensor import CompressedTensor
from .tensor_buffer import TensorBuffer


@torch.compiler.disable
def compress(data: Tensor, distribution: Distribution | None = None,
             buffer: TensorBuffer | None = None, allow_raw: bool = False) -> CompressedTensor:
    """Losslessly encode the exponent byte of a GPU bfloat16 tensor."""
    if distribution is None:
        distribution = Distribution()
    return compress_dense(data.detach(), distribution, buffer, allow_raw=allow_raw)


def compress_batch(tensors, distribution=None, buffer: TensorBuffer | None = None) -> list:
    """:func:`compress` of several GPU bfloat16 tensors into ``buffer``, one
    fused compress launch and one compaction launch per 16 tensors (the
    reference compresses one tensor per call).  ``distribution``: one for all,
    or one per tensor.  The records equal those of :func:`compress` except
    where in the buffer's arena each overflow region lies."""
    tensors = [t.detach() for t in tensors]
    if distribution is None or isinstance(distribution, Distribution):
        distributions = [distribution or Distribution()] * len(tensors)
    else:
        distributions = [Distribution() if d is None else d for d in distribution]
        if len(distributions) != len(tensors):
            raise ValueError("one distribution per tensor")
    return encode_batch(tensors, distributions, buffer)


@torch.compiler.disable
def decompress(data: CompressedTensor) -> Tensor:
    """Decode a tensor produced by :func:`compress`."""
    if data.layout == StorageLayout.COMPRESSED:
        return decode_dense(data)
    return data.data.reshape(data.shape)


def A_compBT(A: Tensor, B_comp: CompressedTensor) -> Tensor:
    """``A @ B_comp.T``."""
    if A.ndim != 2 or A.shape[1] != B_comp.shape[1]:
        raise ValueError("activation and weight inner dimensions must match")
    return A.contiguous() @ decompress(B_comp).T


def A_compB(A: Tensor, B_comp: CompressedTensor) -> Tensor:
    """``A @ B_comp``."""
    if A.ndim != 2 or A.shape[1] != B_comp.shape[0]:
        raise ValueError("activation and weight inner dimensions must match")
    return A.contiguous() @ decompress(B_comp)


def compA_add_B(A_comp: CompressedTensor, B: Tensor, *, dense_output: bool = True,
                buffer: TensorBuffer | None = None, distribution=None):
    """``A + B`` with ``A`` compressed."""
    return pointwise_compressed_dense(A_comp, B, ADD, dense_output=dense_output,
                                      buffer=buffer, distribution=distribution)


def compA_mul_B(A_comp: CompressedTensor, B: Tensor, *, dense_output: bool = True,
                buffer: TensorBuffer | None = None, distribution=None):
    """``A * B`` elementwise with ``A`` compressed."""
    return pointwise_compressed_dense(A_comp, B, MULTIPLY, dense_output=dense_output,
                                      buffer=buffer, distribution=distribution)


def _alpha_operand(a, device) -> Tensor:
    """The scalar operand as the kernels read it: the first element of a
    device tensor, as FP32 (a tensor of another float dtype is cast on the
    device's stream, without a host sync)."""
    if not isinstance(a, torch.Tensor):
        raise TypeError("alpha must be a torch.Tensor")
    if a.device != device:
        raise ValueError("alpha must be on the compressed tensor's device")
    if a.numel() == 0:
        raise ValueError("alpha must hold at least one element")
    return a if a.dtype == torch.float32 else a.reshape(-1)[:1].to(torch.float32)


def a_compA_add_B(A_comp: CompressedTensor, a: Tensor, B: Tensor, *, alpha_is_one: bool = False,
                  dense_output: bool = True, buffer: TensorBuffer | None = None,
                  distribution=None):
    """``a * A_comp + B`` in one fused pass (FP32 fma, BF16 rounding).

    ``alpha_is_one=True`` treats ``a`` as 1 without reading it.
    """
    if not isinstance(a, torch.Tensor):
        raise TypeError("alpha must be a torch.Tensor")
    if not alpha_is_one:
        a = _alpha_operand(a, A_comp.data.device)
    return pointwise_compressed_dense(A_comp, B, SCALAR_MUL_ADD, alpha=a,
                                      alpha_is_one=alpha_is_one, dense_output=dense_output,
                                      buffer=buffer, distribution=distribution)


def a_compA_add_b_B(A_comp: CompressedTensor, a: Tensor, B: Tensor, b: Tensor, *,
                    alpha_is_one: bool = False, dense_output: bool = True,
                    buffer: TensorBuffer | None = None, distribution=None):
    """``a * A_comp + b * B``: ``B*b`` in FP32, then fma(A, a, B*b).

    ``alpha_is_one=True`` uses fma(B, b, A) instead.  ``a`` and ``b`` are
    float32 one-element tensors on the compressed tensor's device.
    """
    for name, scalar in (("alpha", a), ("beta", b)):
        if not isinstance(scalar, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if (scalar.numel() != 1 or scalar.dtype != torch.float32
                or scalar.device != A_comp.data.device):
            raise ValueError(f"{name} must be a float32 scalar on the compressed tensor's device")
    return pointwise_compressed_dense(A_comp, B, SCALAR_MUL_ADD, alpha=a, beta=b,
                                      alpha_is_one=alpha_is_one, dense_output=dense_output,
                                      buffer=buffer, distribution=distribution)


def a_compA_add_b_B_batch(A_comps, a: Tensor, Bs, b: Tensor | None = None, *,
                          alpha_is_one: bool = False, buffer: TensorBuffer,
                          distributions=None) -> list:
    """``a * A + b * B`` (``a * A + B`` when ``b`` is None) with compressed
    output into ``buffer`` for each pair: the ``dense_output=False`` form of
    :func:`a_compA_add_B` / :func:`a_compA_add_b_B`, one sampler, encoder and
    compaction launch per 8 tensors (the reference updates one tensor per
    call).  ``distributions``: the results' (default: each A's).  The records
    equal those of the one-tensor calls except where in the buffer's arena
    each overflow region lies."""
    A_comps, Bs = list(A_comps), list(Bs)
    if len(A_comps) != len(Bs):
        raise ValueError("one B per compressed A")
    if not A_comps:
        return []
    device = A_comps[0].data.device
    if not isinstance(a, torch.Tensor):
        raise TypeError("alpha must be a torch.Tensor")
    if b is None:
        if not alpha_is_one:
            a = _alpha_operand(a, device)
    else:
        for name, scalar in (("alpha", a), ("beta", b)):
            if not isinstance(scalar, torch.Tensor):
                raise TypeError(f"{name} must be a torch.Tensor")
            if scalar.numel() != 1 or scalar.dtype != torch.float32 or scalar.device != device:
                raise ValueError(
                    f"{name} must be a float32 scalar on the compressed tensors' device")
    if distributions is None:
        distributions = [A.distribution for A in A_comps]
    distributions = list(distributions)
    if len(distributions) != len(A_comps):
        raise ValueError("one distribution per compressed A")
    return fused_update_batch(list(zip(A_comps, Bs, distributions)), SCALAR_MUL_ADD, buffer,
                              alpha=a, beta=b, alpha_is_one=alpha_is_one)


def a_compA_add_compB(A_comp: CompressedTensor, a: Tensor, B_comp: CompressedTensor, *,
                      dense_output: bool = True, buffer: TensorBuffer | None = None,
                      distribution=None):
    """``a * A_comp + B_comp`` with both operands compressed (one fused pass)."""
    a = _alpha_operand(a, A_comp.data.device)
    return pointwise_scale_add_compressed(A_comp, B_comp, a, dense_output=dense_output,
                                          buffer=buffer, distribution=distribution)
