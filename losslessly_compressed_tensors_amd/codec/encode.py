"""Compression pipeline: center + tables, encoder, scans/allocation, compaction.

Host sequencing of ``LCT/codec/encode.py:22-218`` on the gfx950 library:

1. ``lct_sample_center`` samples the center's positions over many
   workgroups (the sampling half of the reference's table kernel);
2. ``lct_encode_sampled`` derives the center and the center-shifted tables
   in every workgroup, then splits fields and writes the fixed payload,
   per-stream overflow starts and per-block overflow summaries (with a given
   center: ``lct_shift_tables`` then ``lct_encode``);
3. ``lct_prefix_allocate`` scans the summaries and, for a shared
   ``TensorBuffer``, reserves the overflow region on the device;
4. private storage only: one device->host sync reads the overflow totals so
   exact-size lane/start/tail arrays can be allocated (as the reference does);
5. ``lct_compact_extra`` writes the per-block overflow list and tails.

The tensors allocated (and hence ``memory_size()``) match the reference's.
"""
from __future__ import annotations

import torch

from ..comp_format import Distribution, StorageLayout
from ..comp_tensor import CompressedTensor
from ..compression.huffman_tables import get_distribution_tables
from ..kernels import dispatch
from ..kernels.dispatch import MAX_CODEC_BLOCKS, FallbackStorage
from ..tensor_buffer import TensorBuffer
from .geometry import geometry

CENTER_SAMPLE_SIZE = 4096


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def encode_components(
    source_values: torch.Tensor,
    sign_mantissa: torch.Tensor,
    size: int,
    distribution: Distribution,
    buffer: TensorBuffer | None,
    shape: tuple[int, ...],
    *,
    precomputed: bool,
    center: torch.Tensor | None = None,
    logical_numel: int,
) -> CompressedTensor:
    """Encode BF16 bits (or precomputed exponent bytes + side bytes).

    Args mirror ``LCT/codec/encode.py:22-47``: ``source_values`` is int16 BF16
    bits, or uint8 raw exponent bytes in logical order when ``precomputed``
    (``sign_mantissa`` then already holds the side bytes); ``size`` is the
    padded storage element count; ``center`` an optional device int32[1].
    """
    if buffer is not None and buffer.capacity_bytes % 4:
        raise ValueError("TensorBuffer capacity must be divisible by 4")
    device = source_values.device
    stream_geometry = geometry(distribution)
    block_symbols, lanes, steps, fixed_words = stream_geometry
    blocks = _cdiv(size, block_symbols)
    streams = blocks * lanes
    if blocks > MAX_CODEC_BLOCKS:
        raise ValueError(
            f"tensor too large: {blocks} codec blocks; the storage format's int32 offsets "
            f"allow {MAX_CODEC_BLOCKS} ({MAX_CODEC_BLOCKS * block_symbols} elements here)")
    encode_table, decode_table, _ = get_distribution_tables(distribution, device)
    shifted_decode = torch.empty_like(decode_table)
    encoded = torch.empty(streams * fixed_words + 4, dtype=torch.int32, device=device)
    extra_starts = torch.empty(streams, dtype=torch.uint8, device=device)
    # Per-block overflow counts/bytes, their scans and the list of blocks
    # that overflow (int32[5*blocks + 1], see lct_prefix_allocate), then the
    # ready word of lct_allocate_compact.
    summaries = torch.empty(dispatch.summaries_length(blocks), dtype=torch.int32,
                            device=device)
    launch = dict(precomputed=precomputed, logical_numel=logical_numel,
                  block_symbols=block_symbols, lanes=lanes, steps=steps, fixed_words=fixed_words)
    sample_values = None
    if center is None and logical_numel > 0:
        # The center's samples are taken by many workgroups; the encoder
        # reduces their partial sums and shifts the tables itself.  A BF16
        # source's sampled values are kept for later fused updates.
        center = torch.empty(1, dtype=torch.int32, device=device)
        sample_size = min(logical_numel, CENTER_SAMPLE_SIZE)
        partials = torch.empty(2 * _cdiv(sample_size, 64), dtype=torch.int32, device=device)
        if not precomputed:
            sample_values = torch.empty(sample_size, dtype=torch.int16, device=device)
        dispatch.sample_center(source_values, logical_numel, sample_size, precomputed, partials,
                               sample_values)
        dispatch.encode_sampled(source_values, sign_mantissa, encoded, partials, sample_size,
                                encode_table, decode_table, center, shifted_decode, extra_starts,
                                summaries, size, **launch)
    else:
        if center is None:
            center = torch.zeros(1, dtype=torch.int32, device=device)   # empty: tables.py:47
        shifted_encode = torch.empty(256, dtype=torch.int32, device=device)
        dispatch.shift_encoding_table(encode_table, center, shifted_encode, decode_table,
                                      shifted_decode)
        if blocks > 0:
            dispatch.encode_kernel(source_values, sign_mantissa, encoded, shifted_encode,
                                   extra_starts, summaries, size, streams, write_summary=True,
                                   **launch)
    return finish_encode(source_values, sign_mantissa, encoded, extra_starts, summaries, size,
                         distribution, buffer, shape, precomputed=precomputed, center=center,
                         shifted_decode=shifted_decode, logical_numel=logical_numel,
                         sample_values=sample_values)


def finish_encode(
    tail_source: torch.Tensor,
    sign_mantissa: torch.Tensor,
    encoded: torch.Tensor,
    extra_starts: torch.Tensor,
    summaries: torch.Tensor,
    size: int,
    distribution: Distribution,
    buffer: TensorBuffer | None,
    shape: tuple[int, ...],
    *,
    precomputed: bool,
    center: torch.Tensor,
    shifted_decode: torch.Tensor,
    logical_numel: int,
    sample_values: torch.Tensor | None = None,
) -> CompressedTensor:
    """Overflow bookkeeping after an encoder pass and the CompressedTensor
    (``LCT/codec/encode.py:77-186``): block scans and, for a shared buffer, the
    arena reservation; for private storage one device->host sync that sizes
    the exact lane/start/tail arrays; then the compaction, which reads the
    tails' exponents from ``tail_source`` (BF16 bits, or exponent bytes in
    logical order when ``precomputed``).  For a shared buffer the scans, the
    reservation (after the buffer's deferred frees) and the compaction are one
    launch; ``summaries`` then holds ``dispatch.summaries_length(blocks)``
    entries."""
    device = encoded.device
    stream_geometry = geometry(distribution)
    block_symbols, lanes, steps, _ = stream_geometry
    blocks = _cdiv(size, block_symbols)
    counts = torch.empty(4, dtype=torch.int32, device=device)
    blocks_out = torch.empty(3 * blocks, dtype=torch.int32, device=device)
    buffered = buffer is not None
    descriptor = torch.empty(4, dtype=torch.int32, device=device) if buffered else counts
    if blocks > 0 and buffered:
        frees = buffer._take_frees()
        try:
            dispatch.allocate_compact(
                tail_source, summaries, counts, descriptor, buffer, blocks_out, extra_starts,
                frees, blocks, size, logical_numel=logical_numel, block_symbols=block_symbols,
                lanes=lanes, steps=steps, precomputed=precomputed)
        except BaseException:
            # Nothing was launched: the deferred frees wait for the next call.
            buffer._restore_frees(frees)
            raise
    elif blocks > 0:
        dispatch.prefix_allocate(summaries, counts, descriptor, buffer, blocks_out, blocks,
                                 False, 256)
    else:
        counts.zero_()
        if buffered:
            # An empty request still yields a descriptor (status 2).
            buffer_descriptor = buffer.allocate(counts[1:2])
            descriptor = buffer_descriptor.descriptor

    final_count, final_total = counts[:1], counts[1:2]
    needs_compaction = False
    if buffered:
        arena = buffer.data
        storage = FallbackStorage(tail=arena, count=final_count, lanes=arena, starts=arena,
                                  blocks=blocks_out, descriptor=descriptor,
                                  allocation=descriptor)
    else:
        count, tail_bytes = (int(v) for v in counts[:2].tolist())
        needs_compaction = blocks > 0 and count > 0
        storage = FallbackStorage(
            tail=torch.empty(tail_bytes, dtype=torch.uint8, device=device),
            count=final_count,
            lanes=torch.empty(count, dtype=torch.uint8, device=device),
            starts=torch.empty(count, dtype=torch.uint8, device=device),
            blocks=blocks_out, allocation=counts[2:3], base=0)
    if needs_compaction:
        dispatch.compact_extra(
            tail_source, storage, blocks, size, precomputed=precomputed, buffered=buffered,
            logical_numel=logical_numel, block_symbols=block_symbols, lanes=lanes,
            steps=steps, extra_starts=extra_starts, summaries=summaries)
    return CompressedTensor(
        encoded, size, sign_mantissa,
        fallback_starts=None if buffered else storage.starts,
        fallback_lanes=None if buffered else storage.lanes,
        fallback_blocks=storage.blocks,
        fallback_buffer=storage.tail,
        fallback_descriptor=descriptor if buffered else None,
        buffer=buffer,
        fallback_count=final_count,
        fallback_used=final_total,
        distribution=distribution, center=center, decode_table=shifted_decode,
        shape=shape, layout=StorageLayout.COMPRESSED, stream_geometry=stream_geometry,
        sample_values=sample_values,
    )


def encode(data: torch.Tensor, distribution: Distribution, buffer: TensorBuffer | None = None,
           *, allow_raw: bool = False) -> CompressedTensor:
    """Compress a BF16 tensor through the flattened 1-D block layout
    (``LCT/codec/encode.py:189-218``)."""
    shape = tuple(data.shape)
    source = data.contiguous().view(-1)
    logical_numel = source.numel()
    block_symbols, lanes, _, fixed_words = geometry(distribution)
    blocks = _cdiv(logical_numel, block_symbols)
    storage_numel = blocks * block_symbols
    streams = blocks * lanes
    minimum_bytes = storage_numel + (streams * fixed_words + 4) * 4
    if allow_raw and minimum_bytes > logical_numel * data.element_size():
        return CompressedTensor(source, logical_numel, buffer=buffer,
                                distribution=distribution, shape=shape,
                                layout=StorageLayout.RAW)
    if source.element_size() != 2:
        raise TypeError(f"LCT compresses 16-bit (bfloat16) tensors, got {source.dtype}")
    if source.data_ptr() % 16:
        # The encoder reads its input with 16-byte vector loads.
        source = source.clone()
    sign_mantissa = torch.empty(storage_numel, dtype=torch.uint8, device=source.device)
    return encode_components(source.view(torch.int16), sign_mantissa, storage_numel,
                             distribution, buffer, shape, precomputed=False,
                             logical_numel=logical_numel)
