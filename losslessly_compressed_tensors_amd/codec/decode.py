"""Decompression: one decoder launch with the overflow overlay fused.

Host sequencing of ``LCT/codec/decode.py:16-92``.  The reference keeps a
separate scatter pass for backends without a fused overlay; the gfx950
decoder always overlays overflow tails in the same pass, so decompression is
exactly one launch and never syncs.
"""
from __future__ import annotations

import torch

from ..comp_tensor import CompressedTensor
from ..compression.huffman_tables import get_distribution_tables
from ..kernels import dispatch
from ..kernels.dispatch import FallbackStorage


def _buffered(data: CompressedTensor) -> bool:
    return data.fallback_descriptor is not None


def storage_of(data: CompressedTensor) -> FallbackStorage:
    """Overflow storage view of a compressed tensor (``decode.py:38-60``)."""
    if _buffered(data):
        arena = data.fallback_buffer
        return FallbackStorage(tail=arena, count=data.fallback_count, lanes=arena,
                               starts=arena, blocks=data.fallback_blocks,
                               descriptor=data.fallback_descriptor,
                               allocation=data.fallback_descriptor)
    return FallbackStorage(tail=data.fallback_buffer, count=data.fallback_count,
                           lanes=data.fallback_lanes, starts=data.fallback_starts,
                           blocks=data.fallback_blocks, allocation=data.fallback_lanes,
                           base=data.fallback_base)


def has_fallback(data: CompressedTensor) -> bool:
    """True when the tensor may carry overflow streams (``decode.py:63-69``)."""
    if data.layout != data.layout.COMPRESSED:
        return False
    if _buffered(data):
        return True
    return data.fallback_lanes is not None and data.fallback_lanes.numel() > 0


def overlay_of(data: CompressedTensor) -> FallbackStorage | None:
    return storage_of(data) if has_fallback(data) else None


def shifted_decode_table(data: CompressedTensor) -> torch.Tensor:
    """The tensor's shifted decode table, rebuilt from its center if absent."""
    if data.decode_table is not None:
        return data.decode_table
    _, decode_table, _ = get_distribution_tables(data.distribution, data.data.device)
    return dispatch.shift_decoding_table(decode_table, data.center)


def decode(data: CompressedTensor) -> torch.Tensor:
    """Decode the fixed payload and overlay overflow tails; returns BF16."""
    logical_numel = data.logical_numel
    output = torch.empty(logical_numel, dtype=torch.int16, device=data.data.device)
    if logical_numel:
        _, _, rare_length = get_distribution_tables(data.distribution, data.data.device)
        block_symbols, lanes, steps, fixed_words = data.codec_geometry
        dispatch.decode_kernel(
            data.data, data.sign_mantissa, output, shifted_decode_table(data), data.center,
            data.size, logical_numel=logical_numel, block_symbols=block_symbols, lanes=lanes,
            steps=steps, fixed_words=fixed_words, rare_length=rare_length,
            overflow=overlay_of(data))
    return output.view(torch.bfloat16).reshape(data.shape)


def decode_batch(tensors: list[CompressedTensor]) -> list[torch.Tensor]:
    """Decode several compressed tensors with as few launches as possible: one
    ``lct_decode_batch`` launch per ``MAX_DECODE_BATCH`` non-empty tensors.
    Each result equals ``decode`` of its tensor.  For tensors of a few codec
    blocks each (a layer's weights), whose decodes are bound by one block's
    latency, one launch replaces one per tensor."""
    from ..kernels import hip

    outputs = []
    jobs = []
    for data in tensors:
        if data.layout != data.layout.COMPRESSED:
            outputs.append(data.data.reshape(data.shape))
            continue
        output = torch.empty(data.logical_numel, dtype=torch.int16, device=data.data.device)
        outputs.append(output.view(torch.bfloat16).reshape(data.shape))
        if not data.logical_numel:
            continue
        _, _, rare_length = get_distribution_tables(data.distribution, data.data.device)
        jobs.append((data.data, data.sign_mantissa, output, shifted_decode_table(data),
                     data.center, data.size, data.logical_numel, data.codec_geometry,
                     rare_length, overlay_of(data)))
    for start in range(0, len(jobs), hip.MAX_DECODE_BATCH):
        dispatch.decode_batch(jobs[start:start + hip.MAX_DECODE_BATCH])
    return outputs
