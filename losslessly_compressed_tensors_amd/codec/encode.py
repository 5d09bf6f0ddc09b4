"""Compression pipeline: center + tables, encoder, scans/allocation, compaction.

Host sequencing of ``LCT/codec/encode.py:22-218`` on the gfx950 library.  A
compress (the center sampled from the input) is two launches:

1. ``lct_encode_fused``, one workgroup per codec block: the first 64 first
   publish the center's partial sums; every workgroup reduces them to the
   center, shifts the tables, splits fields, writes its block's fixed payload
   and per-stream overflow starts and publishes its block's overflow summary;
   workgroup 0, after its block, scans the summaries into the block metadata
   and the overflow-block list and, for a shared ``TensorBuffer``, applies the
   buffer's deferred frees and reserves the overflow region;
2. private storage only: one device->host sync reads the overflow totals so
   exact-size lane/start/tail arrays can be allocated (as the reference does);
3. ``lct_compact_extra`` (one workgroup per block, from the block metadata)
   writes the per-block overflow entries and tails (``finish_fused``, shared
   with the fused pointwise updates).

With a given center (``lct_shift_tables`` then ``lct_encode``), the
bookkeeping runs as its own launches after the encoder (``finish_encode``).
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
        # One launch samples the center (its partial sums over many
        # workgroups, which every encoding workgroup reduces to the center),
        # encodes, and scans the blocks' overflow (for a shared buffer also
        # reserving the overflow region); the compaction follows.  A BF16
        # source's sampled values are kept for later fused updates.
        center = torch.empty(1, dtype=torch.int32, device=device)
        sample_size = min(logical_numel, CENTER_SAMPLE_SIZE)
        if not precomputed:
            sample_values = torch.empty(sample_size, dtype=torch.int16, device=device)
        return _encode_fused(source_values, sign_mantissa, encoded, extra_starts, summaries, size,
                             distribution, buffer, shape, encode_table, decode_table, center,
                             shifted_decode, sample_size, sample_values, launch)
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


def _encode_fused(source_values, sign_mantissa, encoded, extra_starts, summaries, size,
                  distribution, buffer, shape, encode_table, decode_table, center,
                  shifted_decode, sample_size, sample_values, launch) -> CompressedTensor:
    """``lct_encode_fused`` then ``lct_compact_extra``: the buffered form takes
    the buffer's deferred frees into the launch and needs no host sync; the
    private form reads the overflow totals once (as the reference does) to
    allocate exact-size lane/start/tail arrays."""
    device = encoded.device
    block_symbols = geometry(distribution)[0]
    blocks = _cdiv(size, block_symbols)
    counts = torch.empty(4, dtype=torch.int32, device=device)
    blocks_out = torch.empty(3 * blocks, dtype=torch.int32, device=device)
    descriptor = None
    fused = dict(size=size, **launch)
    if buffer is not None:
        descriptor = torch.empty(4, dtype=torch.int32, device=device)
        frees = buffer._take_frees()
        try:
            dispatch.encode_fused(source_values, sign_mantissa, encoded, sample_size,
                                  encode_table, decode_table, center, shifted_decode,
                                  sample_values, extra_starts, summaries, blocks_out, counts,
                                  buffer=buffer, descriptor=descriptor, frees=frees, **fused)
        except BaseException:
            # Nothing was launched: the deferred frees wait for the next call.
            buffer._restore_frees(frees)
            raise
    else:
        dispatch.encode_fused(source_values, sign_mantissa, encoded, sample_size, encode_table,
                              decode_table, center, shifted_decode, sample_values, extra_starts,
                              summaries, blocks_out, counts, **fused)
    return finish_fused(source_values, sign_mantissa, encoded, extra_starts, size, distribution,
                        buffer, shape, precomputed=launch["precomputed"], center=center,
                        shifted_decode=shifted_decode, logical_numel=launch["logical_numel"],
                        sample_values=sample_values, counts=counts, blocks_out=blocks_out,
                        descriptor=descriptor)


def finish_fused(tail_source, sign_mantissa, encoded, extra_starts, size, distribution, buffer,
                 shape, *, precomputed, center, shifted_decode, logical_numel, sample_values,
                 counts, blocks_out, descriptor) -> CompressedTensor:
    """After an encoder launch that made its own overflow bookkeeping
    (``lct_encode_fused``, ``lct_pointwise_encode_fused``,
    ``lct_dual_encode_fused``; ``LCT/codec/encode.py:77-186``): the compaction
    (``lct_compact_extra`` over the block metadata that launch wrote) and the
    CompressedTensor.  ``tail_source`` holds the tails' exponents (BF16 bits,
    or exponent bytes in logical order when ``precomputed``).  With a buffer
    nothing syncs; private storage reads the totals once to size exact
    lane/start/tail arrays and raises if a device-side wait gave up."""
    device = encoded.device
    stream_geometry = geometry(distribution)
    block_symbols, lanes, steps, _ = stream_geometry
    blocks = _cdiv(size, block_symbols)
    compaction = dict(precomputed=precomputed, logical_numel=logical_numel,
                      block_symbols=block_symbols, lanes=lanes, steps=steps,
                      extra_starts=extra_starts, summaries=None)
    if buffer is not None:
        arena = buffer.data
        storage = FallbackStorage(tail=arena, count=counts[:1], lanes=arena, starts=arena,
                                  blocks=blocks_out, descriptor=descriptor,
                                  allocation=descriptor)
        dispatch.compact_extra(tail_source, storage, blocks, size, buffered=True, **compaction)
    else:
        count, tail_bytes, _, incomplete = (int(v) for v in counts.tolist())
        if incomplete:
            raise RuntimeError(
                "compress: a device-side wait of the encoder gave up (a block's summary or "
                "the center's samples did not arrive); the tensor was not stored")
        storage = FallbackStorage(
            tail=torch.empty(tail_bytes, dtype=torch.uint8, device=device),
            count=counts[:1],
            lanes=torch.empty(count, dtype=torch.uint8, device=device),
            starts=torch.empty(count, dtype=torch.uint8, device=device),
            blocks=blocks_out, allocation=counts[2:3], base=0)
        if count > 0:
            dispatch.compact_extra(tail_source, storage, blocks, size, buffered=False,
                                   **compaction)
    buffered = buffer is not None
    return CompressedTensor(
        encoded, size, sign_mantissa,
        fallback_starts=None if buffered else storage.starts,
        fallback_lanes=None if buffered else storage.lanes,
        fallback_blocks=storage.blocks,
        fallback_buffer=storage.tail,
        fallback_descriptor=storage.descriptor,
        buffer=buffer,
        fallback_count=counts[:1],
        fallback_used=counts[1:2],
        distribution=distribution, center=center, decode_table=shifted_decode,
        shape=shape, layout=StorageLayout.COMPRESSED, stream_geometry=stream_geometry,
        sample_values=sample_values,
    )


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
