"""Pointwise operations on compressed tensors.

Host logic of ``LCT/codec/pointwise.py:28-304``:

* ``pointwise_compressed_dense``: ``compA + B``, ``compA * B`` or
  ``alpha * compA + beta * B`` with one compressed and one dense operand;
* ``pointwise_scale_add_compressed``: ``alpha * compA + compB`` with both
  compressed (one fused launch when geometries and buffering modes agree,
  else decode B and use the dense path).

Dense output is BF16.  Compressed output equals ``compress(result)`` with a
freshly sampled center.  With a dense operand it is produced in a single pass
over the compressed operand (decode, operate, re-encode; see
``_fused_compressed_output``), and so with two compressed operands
(``_fused_dual_compressed_output``).
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
from .encode import CENTER_SAMPLE_SIZE, finish_encode, finish_fused
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


def _bookkept(blocks: int) -> bool:
    """Whether a fused update's encoder launch does its own overflow
    bookkeeping (``_encode_with_bookkeeping``)."""
    return 0 < blocks <= dispatch.MAX_CODEC_BLOCKS


def _encode_with_bookkeeping(launch_encoder, exponents, side, encoded, extra_starts, summaries,
                             size, distribution, buffer, shape, *, center, shifted_decode,
                             logical_numel, sample_values, samples=None) -> CompressedTensor:
    """Run a fused update's encoder launch, ``launch_encoder(record)``, with
    the overflow bookkeeping in the same launch when the block count allows
    (a ``dispatch.bookkeeping`` record: prefix scan and, for a shared buffer,
    the deferred frees and the reservation), then the compaction; otherwise
    the encoder alone followed by ``finish_encode``'s bookkeeping launches.
    Either way the stored tensor is the same (``LCT/codec/encode.py:77-186``).
    ``samples``: the record's in-launch sampling operands (only with the
    bookkeeping in the launch)."""
    device = encoded.device
    blocks = size // geometry(distribution)[0]
    if not _bookkept(blocks):
        if samples is not None:
            raise ValueError("in-launch center sampling needs the in-launch bookkeeping")
        launch_encoder(None)
        return finish_encode(exponents, side, encoded, extra_starts, summaries, size,
                             distribution, buffer, shape, precomputed=True, center=center,
                             shifted_decode=shifted_decode, logical_numel=logical_numel,
                             sample_values=sample_values)
    counts = torch.empty(4, dtype=torch.int32, device=device)
    blocks_out = torch.empty(3 * blocks, dtype=torch.int32, device=device)
    descriptor = None
    frees = ()
    if buffer is not None:
        descriptor = torch.empty(4, dtype=torch.int32, device=device)
        frees = buffer._take_frees()
    try:
        launch_encoder(dispatch.bookkeeping(device, blocks, counts, blocks_out, buffer,
                                            descriptor, frees, samples=samples))
    except BaseException:
        # Nothing was launched: the deferred frees wait for the next call.
        if buffer is not None:
            buffer._restore_frees(frees)
        raise
    return finish_fused(exponents, side, encoded, extra_starts, size, distribution, buffer,
                        shape, precomputed=True, center=center, shifted_decode=shifted_decode,
                        logical_numel=logical_numel, sample_values=sample_values,
                        counts=counts, blocks_out=blocks_out, descriptor=descriptor)


def _fused_compressed_output(data: CompressedTensor, other: torch.Tensor,
                             operation: PointwiseOp, result_distribution: Distribution,
                             buffer: TensorBuffer | None, *, alpha: torch.Tensor | None,
                             beta: torch.Tensor | None, alpha_is_one: bool) -> CompressedTensor:
    """``operation(compA, B)`` re-encoded in one pass over A's payload, A's side
    bytes and B.

    The reference writes the result's side and exponent bytes, then encodes
    them (``LCT/codec/pointwise.py:262-278`` -> ``LCT/codec/encode.py:22-186``).
    Here ``lct_pointwise_sample`` computes the result at the center's sample
    positions (from A's recorded sample values when A has them, else by
    decoding the sampled streams' prefixes), ``lct_pointwise_encode`` derives
    the center and encodes the result as it is computed, and only the exponent
    bytes of overflow rows reach HBM (for the compaction's tails).  The stored
    tensor is identical.
    """
    device = data.data.device
    scaled = operation is SCALAR_MUL_ADD
    alpha_is_one = (not scaled) or alpha_is_one
    beta_is_one = (not scaled) or beta is None
    other = other.contiguous().view(-1)
    block_symbols, lanes, steps, fixed_words = data.codec_geometry
    blocks = data.size // block_symbols
    streams = blocks * lanes
    n = data.logical_numel
    _, _, rare_length = get_distribution_tables(data.distribution, device)
    base_encode, base_decode, _ = get_distribution_tables(result_distribution, device)
    sample_size = min(n, CENTER_SAMPLE_SIZE)
    launch = dict(rare_length=rare_length, logical_numel=n, block_symbols=block_symbols,
                  lanes=lanes, steps=steps, fixed_words=fixed_words, op=operation.code,
                  alpha_is_one=alpha_is_one, beta_is_one=beta_is_one, sample_size=sample_size,
                  overflow=overlay_of(data))
    alpha_arg = None if alpha_is_one else alpha
    beta_arg = None if beta_is_one else beta
    decode_table = shifted_decode_table(data)
    partials = torch.empty(2 * -(-sample_size // 64), dtype=torch.int32, device=device)
    # A's recorded values at the sample positions spare the sampler a walk
    # through A's streams; the result's are recorded for the next update.  (The
    # sampler stays a launch of its own: inside the encoder launch, B's 4096
    # scattered reads delayed every block's center by more than it costs.)
    a_samples = data.sample_values
    if a_samples is not None and a_samples.numel() != sample_size:
        a_samples = None
    result_samples = torch.empty(sample_size, dtype=torch.int16, device=device)
    dispatch.pointwise_sample(data.data, data.sign_mantissa, decode_table, data.center, other,
                              alpha_arg, beta_arg, partials, data.size, a_samples=a_samples,
                              result_samples=result_samples, **launch)
    center = torch.empty(1, dtype=torch.int32, device=device)
    shifted_decode = torch.empty(1024, dtype=torch.int32, device=device)
    side = torch.empty(data.size, dtype=torch.uint8, device=device)
    encoded = torch.empty(streams * fixed_words + 4, dtype=torch.int32, device=device)
    extra_starts = torch.empty(streams, dtype=torch.uint8, device=device)
    summaries = torch.empty(dispatch.summaries_length(blocks), dtype=torch.int32,
                            device=device)
    # Only the rows of overflowing streams are written (and read back by the
    # compaction); the rest stays unwritten.
    exponents = torch.empty(n, dtype=torch.uint8, device=device)

    def launch_encoder(record):
        dispatch.pointwise_encode(data.data, data.sign_mantissa, decode_table, data.center,
                                  other, alpha_arg, beta_arg, partials, base_encode,
                                  base_decode, center, shifted_decode, side, encoded,
                                  extra_starts, summaries, exponents, data.size, record=record,
                                  **launch)

    return _encode_with_bookkeeping(launch_encoder, exponents, side, encoded, extra_starts,
                                    summaries, data.size, result_distribution, buffer,
                                    data.shape, center=center, shifted_decode=shifted_decode,
                                    logical_numel=n, sample_values=result_samples)


def _fused_dual_compressed_output(data: CompressedTensor, other: CompressedTensor,
                                  alpha: torch.Tensor, result_distribution: Distribution,
                                  buffer: TensorBuffer | None) -> CompressedTensor:
    """``alpha * compA + compB`` re-encoded in one pass over both operands'
    payloads and side bytes.

    The reference runs the dual kernel with compressed output and encodes its
    side and exponent bytes (``LCT/codec/pointwise.py:191-202`` ->
    ``LCT/codec/encode.py:22-186``).  Here ``lct_dual_sample`` computes the
    result at the center's sample positions (from an operand's recorded
    sample values when it has them, else by decoding the sampled streams'
    prefixes) and ``lct_dual_encode`` decodes both operands, applies
    ``fma(a, alpha, b)`` and encodes the result as it is computed; with both
    operands' recorded values and the bookkeeping in the encoder launch, that
    launch also samples.  The stored tensor is identical.
    """
    device = data.data.device
    _, _, rare_a = get_distribution_tables(data.distribution, device)
    _, _, rare_b = get_distribution_tables(other.distribution, device)
    if rare_a != rare_b:
        raise ValueError("two-compressed path requires matching RARE_LENGTH")
    base_encode, base_decode, _ = get_distribution_tables(result_distribution, device)
    block_symbols, lanes, steps, fixed_words = data.codec_geometry
    blocks = data.size // block_symbols
    streams = blocks * lanes
    n = data.logical_numel
    sample_size = min(n, CENTER_SAMPLE_SIZE)
    launch = dict(rare_length=rare_a, logical_numel=n, block_symbols=block_symbols, lanes=lanes,
                  steps=steps, fixed_words=fixed_words, sample_size=sample_size)
    a_table, b_table = shifted_decode_table(data), shifted_decode_table(other)
    a_storage, b_storage = overlay_of(data), overlay_of(other)

    def recorded(tensor: CompressedTensor):
        values = tensor.sample_values
        return values if values is not None and values.numel() == sample_size else None

    result_samples = torch.empty(sample_size, dtype=torch.int16, device=device)
    a_samples, b_samples = recorded(data), recorded(other)
    # With both operands' recorded values and the bookkeeping in the encoder
    # launch, that launch samples the center itself.
    in_launch = a_samples is not None and b_samples is not None and _bookkept(blocks)
    partials = None
    if not in_launch:
        partials = torch.empty(2 * -(-sample_size // 64), dtype=torch.int32, device=device)
        dispatch.dual_sample(data.data, data.sign_mantissa, a_table, data.center, a_storage,
                             other.data, other.sign_mantissa, b_table, other.center, b_storage,
                             alpha, partials, data.size, a_samples=a_samples,
                             b_samples=b_samples, result_samples=result_samples, **launch)
    center = torch.empty(1, dtype=torch.int32, device=device)
    shifted_decode = torch.empty(1024, dtype=torch.int32, device=device)
    side = torch.empty(data.size, dtype=torch.uint8, device=device)
    encoded = torch.empty(streams * fixed_words + 4, dtype=torch.int32, device=device)
    extra_starts = torch.empty(streams, dtype=torch.uint8, device=device)
    summaries = torch.empty(dispatch.summaries_length(blocks), dtype=torch.int32,
                            device=device)
    # Only the rows of overflowing streams are written (and read back by the
    # compaction); the rest stays unwritten.
    exponents = torch.empty(n, dtype=torch.uint8, device=device)

    def launch_encoder(record):
        dispatch.dual_encode(data.data, data.sign_mantissa, a_table, data.center, a_storage,
                             other.data, other.sign_mantissa, b_table, other.center, b_storage,
                             alpha, partials, base_encode, base_decode, center, shifted_decode,
                             side, encoded, extra_starts, summaries, exponents, data.size,
                             record=record, **launch)

    return _encode_with_bookkeeping(launch_encoder, exponents, side, encoded, extra_starts,
                                    summaries, data.size, result_distribution, buffer,
                                    data.shape, center=center, shifted_decode=shifted_decode,
                                    logical_numel=n, sample_values=result_samples,
                                    samples=(a_samples, b_samples, result_samples) if in_launch
                                    else None)


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
        dispatch.dual(
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
        # Both operands' streams are walked with A's size (the reference reads B
        # out of bounds otherwise).
        if data.shape != other.shape:
            raise ValueError(f"{SCALAR_MUL_ADD.name} expects tensors with the same shape")
        result_distribution = distribution or data.distribution
        if not dense_output and geometry(result_distribution) != data.codec_geometry:
            raise ValueError("matrix compressed output must preserve the input stream geometry")
        if not dense_output and data.logical_numel > 0:
            if buffer is not None and buffer.capacity_bytes % 4:
                raise ValueError("TensorBuffer capacity must be divisible by 4")
            return _fused_dual_compressed_output(data, other, alpha, result_distribution,
                                                 buffer)
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


def fused_update_batch(items, operation: PointwiseOp, buffer: TensorBuffer, *,
                       alpha: torch.Tensor | None = None, beta: torch.Tensor | None = None,
                       alpha_is_one: bool = False) -> list[CompressedTensor]:
    """``operation(compA, B)`` with compressed output into ``buffer`` for each
    ``(A, B, result_distribution)`` of ``items``: the single-pass update of
    ``pointwise_compressed_dense(..., dense_output=False)``, with one sampler,
    one encoder and one compaction launch (``lct_pointwise_update_batch``)
    per ``hip.MAX_UPDATE_BATCH`` tensors of one step count.  Each record equals
    that call's, except where in the arena its overflow region lies.  Pairs
    the batched launch does not take (RAW or empty A, a result geometry other
    than A's) go through ``pointwise_compressed_dense`` one by one."""
    if buffer is None:
        raise ValueError("fused_update_batch stores into a TensorBuffer")
    if buffer.capacity_bytes % 4:
        raise ValueError("TensorBuffer capacity must be divisible by 4")
    if operation is SCALAR_MUL_ADD and alpha is None:
        raise ValueError("scalar_mul_add requires an alpha argument")
    scaled = operation is SCALAR_MUL_ADD
    alpha_is_one = (not scaled) or alpha_is_one
    beta_is_one = (not scaled) or beta is None
    alpha_arg = None if alpha_is_one else alpha
    beta_arg = None if beta_is_one else beta
    device = buffer.device
    results: list[CompressedTensor | None] = [None] * len(items)
    pending: dict[int, list] = {}
    for index, (data, other, distribution) in enumerate(items):
        result_distribution = distribution or data.distribution
        if tuple(other.shape) != data.shape:
            raise ValueError(f"{operation.name} expects tensors with the same shape")
        if (data.layout != StorageLayout.COMPRESSED or data.logical_numel == 0
                or geometry(result_distribution) != data.codec_geometry):
            results[index] = pointwise_compressed_dense(
                data, other, operation, alpha=alpha, beta=beta, alpha_is_one=alpha_is_one,
                dense_output=False, buffer=buffer, distribution=result_distribution)
            continue
        _require_bf16(other, operation)
        dispatch.require_device(data.data, other)
        other = other.contiguous().view(-1)
        block_symbols, lanes, steps, fixed_words = data.codec_geometry
        blocks = data.size // block_symbols
        streams = blocks * lanes
        n = data.logical_numel
        _, _, rare_length = get_distribution_tables(data.distribution, device)
        base_encode, base_decode, _ = get_distribution_tables(result_distribution, device)
        sample_size = min(n, CENTER_SAMPLE_SIZE)
        a_samples = data.sample_values
        if a_samples is not None and a_samples.numel() != sample_size:
            a_samples = None
        payload_bytes = 4 * (streams * fixed_words + 4)
        packed = torch.empty(data.size + payload_bytes, dtype=torch.uint8, device=device)
        record = torch.empty(1033 + 3 * blocks, dtype=torch.int32, device=device)
        result_samples = torch.empty(sample_size, dtype=torch.int16, device=device)
        # Only the rows of overflowing streams are written (and read back by
        # the compaction); the rest stays unwritten.
        exponents = torch.empty(n, dtype=torch.uint8, device=device)
        overflow = overlay_of(data)
        p_side, p_record = packed.data_ptr(), record.data_ptr()
        job = hip.UpdateJob()
        job.encoded, job.side = data.data.data_ptr(), data.sign_mantissa.data_ptr()
        job.shifted_decode = shifted_decode_table(data).data_ptr()
        job.center = data.center.data_ptr()
        job.has_overflow = int(overflow is not None)
        if overflow is not None:
            job.overflow = overflow.as_overflow()
        job.a_samples = None if a_samples is None else a_samples.data_ptr()
        job.other = other.data_ptr()
        job.base_encode, job.base_decode = base_encode.data_ptr(), base_decode.data_ptr()
        job.center_out, job.shifted_decode_out = p_record + 4 * 1032, p_record
        job.side_out, job.encoded_out = p_side, p_side + data.size
        job.result_samples = result_samples.data_ptr()
        job.exponents = exponents.data_ptr()
        job.counts, job.descriptor = p_record + 4 * 1024, p_record + 4 * 1028
        job.blocks = p_record + 4 * 1033
        job.size, job.logical_numel, job.sample_size = data.size, n, sample_size
        job.geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
        job.rare_length = rare_length
        pending.setdefault(steps, []).append(
            (index, job, (data, other, exponents), packed, record, result_samples,
             result_distribution, blocks, payload_bytes))
    stream = torch._C._cuda_getCurrentRawStream(device.index)
    for members in pending.values():
        for start in range(0, len(members), hip.MAX_UPDATE_BATCH):
            part = members[start:start + hip.MAX_UPDATE_BATCH]
            frees = buffer._take_frees()
            try:
                dispatch.pointwise_update_batch_pointers(
                    [m[1] for m in part], operation.code, alpha_is_one, beta_is_one, alpha_arg,
                    beta_arg, buffer, frees, device, stream)
            except BaseException:
                buffer._restore_frees(frees)
                raise
            for (index, _, (data, _, _), packed, record, result_samples, result_distribution,
                 blocks, payload_bytes) in part:
                side, payload = packed.split_with_sizes((data.size, payload_bytes))
                shifted_decode, counts, descriptor, center, blocks_out = record.split_with_sizes(
                    (1024, 4, 4, 1, 3 * blocks))
                count_view, used_view = counts.split_with_sizes((1, 1, 2))[:2]
                results[index] = CompressedTensor(
                    payload.view(torch.int32), data.size, side,
                    fallback_blocks=blocks_out,
                    fallback_buffer=buffer.data,
                    fallback_descriptor=descriptor,
                    buffer=buffer,
                    fallback_count=count_view,
                    fallback_used=used_view,
                    distribution=result_distribution, center=center,
                    decode_table=shifted_decode, shape=data.shape,
                    layout=StorageLayout.COMPRESSED,
                    stream_geometry=geometry(result_distribution),
                    sample_values=result_samples,
                )
    return results


def _require_bf16(other: torch.Tensor, operation: PointwiseOp) -> None:
    """The kernels read the dense operand as BF16.  The reference's kernel
    loads it with its own dtype (``LCT/kernels/generic/pointwise.py:154``);
    here any other dtype raises rather than being read with the wrong
    element size."""
    if other.dtype != torch.bfloat16:
        raise TypeError(f"{operation.name}: the dense operand must be bfloat16, "
                        f"got {other.dtype}")


def pointwise_compressed_dense(data: CompressedTensor, other: torch.Tensor,
                               operation: PointwiseOp, *, alpha: torch.Tensor | None = None,
                               beta: torch.Tensor | None = None, alpha_is_one: bool = False,
                               dense_output: bool = True, buffer: TensorBuffer | None = None,
                               distribution: Distribution | None = None):
    """``alpha * compA + beta * B`` or ``compA (+|*) B``
    (``LCT/codec/pointwise.py:213-278``)."""
    if tuple(other.shape) != data.shape:
        raise ValueError(f"{operation.name} expects tensors with the same shape")
    if data.layout == StorageLayout.COMPRESSED:
        _require_bf16(other, operation)
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

    if not dense_output and data.logical_numel > 0:
        if buffer is not None and buffer.capacity_bytes % 4:
            raise ValueError("TensorBuffer capacity must be divisible by 4")
        return _fused_compressed_output(data, other, operation, result_distribution, buffer,
                                        alpha=alpha, beta=beta, alpha_is_one=alpha_is_one)
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
    "fused_update_batch",
]
