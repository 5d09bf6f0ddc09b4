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
2. private storage only: the host waits for the overflow totals so exact-size
   lane/start/tail arrays can be allocated (the reference reads them with a
   sync); the launch's bookkeeping also posts them to two words of pinned host
   memory, which the host polls, so it can allocate and enqueue the
   compaction as soon as the totals exist;
3. ``lct_compact_extra`` (one workgroup per block, from the block metadata)
   writes the per-block overflow entries and tails (``_compress_bf16``;
   ``finish_fused`` for the fused pointwise updates).

With a given center (``lct_shift_tables`` then ``lct_encode``), the
bookkeeping runs as its own launches after the encoder (``finish_encode``).
The tensors allocated (and hence ``memory_size()``) match the reference's.
"""
from __future__ import annotations

import torch

from ..comp_format import Distribution, StorageLayout
from ..comp_tensor import CompressedTensor
from ..compression.huffman_tables import get_distribution_tables
from ..kernels import dispatch, hip
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
    encoded: torch.Tensor | None = None,
) -> CompressedTensor:
    """Encode BF16 bits (or precomputed exponent bytes + side bytes).

    Args mirror ``LCT/codec/encode.py:22-47``: ``source_values`` is int16 BF16
    bits, or uint8 raw exponent bytes in logical order when ``precomputed``
    (``sign_mantissa`` then already holds the side bytes); ``size`` is the
    padded storage element count; ``center`` an optional device int32[1];
    ``encoded`` an optional preallocated payload (int32[streams * W + 4],
    16-byte aligned).
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
    if encoded is None:
        encoded = torch.empty(streams * fixed_words + 4, dtype=torch.int32, device=device)
    launch = dict(precomputed=precomputed, logical_numel=logical_numel,
                  block_symbols=block_symbols, lanes=lanes, steps=steps, fixed_words=fixed_words)
    sample_values = None
    if center is None and logical_numel > 0:
        # One launch samples the center (its partial sums over many
        # workgroups, which every encoding workgroup reduces to the center),
        # encodes, and scans the blocks' overflow (for a shared buffer also
        # reserving the overflow region); the compaction follows.  A BF16
        # source's sampled values are kept for later fused updates.
        sample_size = min(logical_numel, CENTER_SAMPLE_SIZE)
        if not precomputed:
            sample_values = torch.empty(sample_size, dtype=torch.int16, device=device)
        return _encode_fused(source_values, sign_mantissa, encoded, size, distribution, buffer,
                             shape, encode_table, decode_table, sample_size, sample_values,
                             launch)
    shifted_decode = torch.empty_like(decode_table)
    extra_starts = torch.empty(streams, dtype=torch.uint8, device=device)
    # Per-block overflow counts/bytes, their scans and the list of blocks
    # that overflow (int32[5*blocks + 1], see lct_prefix_allocate), then the
    # ready word of lct_allocate_compact.
    summaries = torch.empty(dispatch.summaries_length(blocks), dtype=torch.int32,
                            device=device)
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


def record_arrays(device, blocks: int, buffered: bool):
    """The stored record's small int32 arrays as views of one allocation:
    ``(shifted_decode[1024], counts[4], fallback_count[1], fallback_used[1],
    descriptor[4] or None, center[1], blocks_out[3 * blocks])``, where the
    count and used views are counts[0] and counts[1].  ``memory_size()``
    counts each distinct allocation once by its size, so one allocation of the
    summed size counts what the separate arrays would."""
    if buffered:
        record = torch.empty(1024 + 4 + 4 + 1 + 3 * blocks, dtype=torch.int32, device=device)
        shifted, counts, descriptor, center, blocks_out = record.split_with_sizes(
            (1024, 4, 4, 1, 3 * blocks))
    else:
        record = torch.empty(1024 + 4 + 1 + 3 * blocks, dtype=torch.int32, device=device)
        shifted, counts, center, blocks_out = record.split_with_sizes((1024, 4, 1, 3 * blocks))
        descriptor = None
    count, used = counts.split_with_sizes((1, 1, 2))[:2]
    return shifted, counts, count, used, descriptor, center, blocks_out


def _encode_fused(source_values, sign_mantissa, encoded, size, distribution, buffer, shape,
                  encode_table, decode_table, sample_size, sample_values,
                  launch) -> CompressedTensor:
    """``lct_encode_fused`` then ``lct_compact_extra``: the buffered form takes
    the buffer's deferred frees into the launch and needs no host sync; the
    private form waits for the overflow totals once (the reference reads them
    with a sync) to allocate exact-size lane/start/tail arrays.  The extra
    starts and block summaries are working arrays no stored tensor keeps: they
    come from the thread's per-stream workspace."""
    dispatch.require_device(source_values, sign_mantissa, encoded)
    device = encoded.device
    block_symbols = launch["block_symbols"]
    blocks = _cdiv(size, block_symbols)
    buffered = buffer is not None
    shifted_decode, counts, count, used, descriptor, center, blocks_out = record_arrays(
        device, blocks, buffered)
    extra_starts, summaries = dispatch.compress_workspace(device, blocks,
                                                          blocks * launch["lanes"])
    fused = dict(size=size, **launch)
    totals = None
    if buffered:
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
        mailbox = dispatch.host_totals()
        epoch = dispatch.encode_fused(source_values, sign_mantissa, encoded, sample_size,
                                      encode_table, decode_table, center, shifted_decode,
                                      sample_values, extra_starts, summaries, blocks_out, counts,
                                      host_totals=mailbox, **fused)
        totals = mailbox.wait(epoch, counts, device)
    return finish_fused(source_values, sign_mantissa, encoded, extra_starts, size, distribution,
                        buffer, shape, precomputed=launch["precomputed"], center=center,
                        shifted_decode=shifted_decode, logical_numel=launch["logical_numel"],
                        sample_values=sample_values, counts=counts, blocks_out=blocks_out,
                        descriptor=descriptor, totals=totals, count_views=(count, used))


def finish_fused(tail_source, sign_mantissa, encoded, extra_starts, size, distribution, buffer,
                 shape, *, precomputed, center, shifted_decode, logical_numel, sample_values,
                 counts, blocks_out, descriptor, totals=None,
                 count_views=None) -> CompressedTensor:
    """After an encoder launch that made its own overflow bookkeeping
    (``lct_encode_fused``, ``lct_pointwise_encode_fused``,
    ``lct_dual_encode_fused``; ``LCT/codec/encode.py:77-186``): the compaction
    (``lct_compact_extra`` over the block metadata that launch wrote) and the
    CompressedTensor.  ``tail_source`` holds the tails' exponents (BF16 bits,
    or exponent bytes in logical order when ``precomputed``).  With a buffer
    nothing syncs; private storage reads the totals once (``totals`` =
    (entries, tail bytes, incomplete) when the caller has them already) to size
    exact lane/start/tail arrays, which share one allocation, and raises if a
    device-side wait gave up.  ``count_views``: the record's fallback_count
    and fallback_used views (counts[0:1], counts[1:2]) when the caller has
    them."""
    device = encoded.device
    count_view, used_view = count_views if count_views is not None else (counts[:1],
                                                                          counts[1:2])
    stream_geometry = geometry(distribution)
    block_symbols, lanes, steps, _ = stream_geometry
    blocks = _cdiv(size, block_symbols)
    compaction = dict(precomputed=precomputed, logical_numel=logical_numel,
                      block_symbols=block_symbols, lanes=lanes, steps=steps,
                      extra_starts=extra_starts, summaries=None)
    if buffer is not None:
        arena = buffer.data
        storage = FallbackStorage(tail=arena, count=count_view, lanes=arena, starts=arena,
                                  blocks=blocks_out, descriptor=descriptor,
                                  allocation=descriptor)
        dispatch.compact_extra(tail_source, storage, blocks, size, buffered=True, **compaction)
    else:
        if totals is None:
            count, tail_bytes, _, incomplete = (int(v) for v in counts.tolist())
        else:
            count, tail_bytes, incomplete = totals
        if incomplete:
            raise RuntimeError(
                "compress: a device-side wait of the encoder gave up (a block's summary or "
                "the center's samples did not arrive); the tensor was not stored")
        # lanes | starts | tails in one allocation of their summed size.
        lanes_out, starts_out, tail_out = torch.empty(
            2 * count + tail_bytes, dtype=torch.uint8, device=device).split_with_sizes(
                (count, count, tail_bytes))
        storage = FallbackStorage(tail=tail_out, count=count_view, lanes=lanes_out,
                                  starts=starts_out, blocks=blocks_out, base=0)
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
        fallback_count=count_view,
        fallback_used=used_view,
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
    if logical_numel > 0:
        return _compress_bf16(source, shape, distribution, buffer, logical_numel, storage_numel)
    sign_mantissa = torch.empty(storage_numel, dtype=torch.uint8, device=source.device)
    return encode_components(source.view(torch.int16), sign_mantissa, storage_numel,
                             distribution, buffer, shape, precomputed=False,
                             logical_numel=logical_numel)


def _compress_bf16(source: torch.Tensor, shape, distribution: Distribution,
                   buffer: TensorBuffer | None, logical_numel: int,
                   storage_numel: int) -> CompressedTensor:
    """The public compress of a non-empty BF16 tensor: ``lct_encode_fused``
    (center, encoder and overflow bookkeeping), then ``lct_compact_extra``,
    into the record's arrays of ``encode_components``.

    The stored arrays come from three allocations: side bytes with the payload
    words after them, the small int32 arrays (``record_arrays``), and the
    recorded sample values; ``memory_size()`` counts each allocation once by
    its size, so the total is that of separate arrays.  The launch takes raw
    addresses; the record's views are made while it runs, so that a private
    compress, which waits for the overflow totals (the reference reads them
    with a sync), has only the overflow arrays' allocation and the
    compaction's launch between the totals' arrival and its return."""
    if source.device.type != "cuda":
        raise ValueError(f"LCT kernels require GPU tensors, got {source.device}")
    if buffer is not None and buffer.capacity_bytes % 4:
        raise ValueError("TensorBuffer capacity must be divisible by 4")
    stream_geometry = geometry(distribution)
    block_symbols, lanes, steps, fixed_words = stream_geometry
    blocks = storage_numel // block_symbols
    if blocks > MAX_CODEC_BLOCKS:
        raise ValueError(
            f"tensor too large: {blocks} codec blocks; the storage format's int32 offsets "
            f"allow {MAX_CODEC_BLOCKS} ({MAX_CODEC_BLOCKS * block_symbols} elements here)")
    device = source.device
    streams = blocks * lanes
    buffered = buffer is not None
    payload_bytes = 4 * (streams * fixed_words + 4)
    # storage_numel is a multiple of the block size, so the payload words
    # start 16-byte aligned.
    packed = torch.empty(storage_numel + payload_bytes, dtype=torch.uint8, device=device)
    head = 1028 + (4 if buffered else 0)
    record = torch.empty(head + 1 + 3 * blocks, dtype=torch.int32, device=device)
    sample_size = min(logical_numel, CENTER_SAMPLE_SIZE)
    sample_values = torch.empty(sample_size, dtype=torch.int16, device=device)
    encode_table, decode_table, _ = get_distribution_tables(distribution, device)
    extra_starts, summaries = dispatch.compress_workspace(device, blocks, streams)
    stream = torch._C._cuda_getCurrentRawStream(device.index)
    p_source, p_side, p_record = source.data_ptr(), packed.data_ptr(), record.data_ptr()
    p_counts, p_extra = p_record + 4 * 1024, extra_starts.data_ptr()
    p_descriptor = p_record + 4 * 1028 if buffered else None
    p_blocks = p_record + 4 * (head + 1)
    g = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    launch = (p_source, p_side, p_side + storage_numel, sample_size, encode_table.data_ptr(),
              decode_table.data_ptr(), p_record + 4 * head, p_record, sample_values.data_ptr(),
              p_extra, summaries.data_ptr(), p_blocks, p_counts, storage_numel, logical_numel, g,
              device, stream)
    mailbox = None
    if buffered:
        frees = buffer._take_frees()
        try:
            dispatch.encode_fused_pointers(*launch, descriptor=p_descriptor, buffer=buffer,
                                           frees=frees)
        except BaseException:
            # Nothing was launched: the deferred frees wait for the next call.
            buffer._restore_frees(frees)
            raise
        arena = buffer.data.data_ptr()
        dispatch.compact_extra_pointers(p_source, arena, arena, arena, p_descriptor, p_counts,
                                        p_blocks, p_extra, storage_numel, logical_numel, g, True,
                                        stream)
    else:
        mailbox = dispatch.host_totals()
        epoch = dispatch.encode_fused_pointers(*launch, host_totals=mailbox)
    # The record's views, while the launch runs.
    side, payload = packed.split_with_sizes((storage_numel, payload_bytes))
    encoded = payload.view(torch.int32)
    if buffered:
        shifted_decode, counts, descriptor, center, blocks_out = record.split_with_sizes(
            (1024, 4, 4, 1, 3 * blocks))
    else:
        shifted_decode, counts, center, blocks_out = record.split_with_sizes(
            (1024, 4, 1, 3 * blocks))
        descriptor = None
    count_view, used_view = counts.split_with_sizes((1, 1, 2))[:2]
    if buffered:
        arena = buffer.data
        lanes_out = starts_out = None
        tail_out = arena
    else:
        count, tail_bytes, incomplete = mailbox.wait(epoch, counts, device)
        if incomplete:
            raise RuntimeError(
                "compress: a device-side wait of the encoder gave up (a block's summary or "
                "the center's samples did not arrive); the tensor was not stored")
        # lanes | starts | tails in one allocation of their summed size.
        overflow = torch.empty(2 * count + tail_bytes, dtype=torch.uint8, device=device)
        if count > 0:
            base = overflow.data_ptr()
            dispatch.compact_extra_pointers(p_source, base, base + count, base + 2 * count, None,
                                            p_counts, p_blocks, p_extra, storage_numel,
                                            logical_numel, g, False, stream)
        lanes_out, starts_out, tail_out = overflow.split_with_sizes(
            (count, count, tail_bytes))
    return CompressedTensor(
        encoded, storage_numel, side,
        fallback_starts=starts_out,
        fallback_lanes=lanes_out,
        fallback_blocks=blocks_out,
        fallback_buffer=tail_out,
        fallback_descriptor=descriptor,
        buffer=buffer,
        fallback_count=count_view,
        fallback_used=used_view,
        distribution=distribution, center=center, decode_table=shifted_decode,
        shape=shape, layout=StorageLayout.COMPRESSED, stream_geometry=stream_geometry,
        sample_values=sample_values,
    )


def encode_batch(tensors, distributions, buffer: TensorBuffer) -> list[CompressedTensor]:
    """``encode`` of several BF16 tensors into ``buffer``: one fused compress
    launch and one compaction launch (``lct_compress_batch``) per
    ``hip.MAX_COMPRESS_BATCH`` tensors of one step count.  Each record equals
    the one ``encode`` makes, except where in the arena its overflow region
    lies.  The buffer's deferred frees are applied before the first
    reservation.  Empty tensors take ``encode``."""
    if buffer is None:
        raise ValueError("encode_batch stores into a TensorBuffer")
    if buffer.capacity_bytes % 4:
        raise ValueError("TensorBuffer capacity must be divisible by 4")
    results: list[CompressedTensor | None] = [None] * len(tensors)
    # (index, job, record pieces) per launchable tensor, grouped by step count.
    pending: dict[int, list] = {}
    for index, (data, distribution) in enumerate(zip(tensors, distributions)):
        shape = tuple(data.shape)
        source = data.contiguous().view(-1)
        if source.element_size() != 2:
            raise TypeError(f"LCT compresses 16-bit (bfloat16) tensors, got {source.dtype}")
        if source.device.type != "cuda":
            raise ValueError(f"LCT kernels require GPU tensors, got {source.device}")
        if source.device != buffer.device:
            raise ValueError("tensors must be on the buffer's device")
        logical_numel = source.numel()
        if logical_numel == 0:
            results[index] = encode(data, distribution, buffer)
            continue
        if source.data_ptr() % 16:
            source = source.clone()
        stream_geometry = geometry(distribution)
        block_symbols, lanes, steps, fixed_words = stream_geometry
        blocks = _cdiv(logical_numel, block_symbols)
        if blocks > MAX_CODEC_BLOCKS:
            raise ValueError(f"tensor too large: {blocks} codec blocks (at most "
                             f"{MAX_CODEC_BLOCKS})")
        storage_numel = blocks * block_symbols
        payload_bytes = 4 * (blocks * lanes * fixed_words + 4)
        device = source.device
        packed = torch.empty(storage_numel + payload_bytes, dtype=torch.uint8, device=device)
        record = torch.empty(1033 + 3 * blocks, dtype=torch.int32, device=device)
        sample_size = min(logical_numel, CENTER_SAMPLE_SIZE)
        sample_values = torch.empty(sample_size, dtype=torch.int16, device=device)
        encode_table, decode_table, _ = get_distribution_tables(distribution, device)
        p_side, p_record = packed.data_ptr(), record.data_ptr()
        job = hip.CompressJob(
            source.data_ptr(), p_side, p_side + storage_numel, encode_table.data_ptr(),
            decode_table.data_ptr(), p_record + 4 * 1032, p_record, sample_values.data_ptr(),
            p_record + 4 * 1033, p_record + 4 * 1024, p_record + 4 * 1028, sample_size,
            storage_numel, logical_numel, hip.Geometry(*stream_geometry))
        pending.setdefault(steps, []).append(
            (index, job, source, packed, record, sample_values, shape, distribution,
             stream_geometry, storage_numel, payload_bytes, blocks))
    device = buffer.device
    stream = torch._C._cuda_getCurrentRawStream(device.index)
    for members in pending.values():
        for start in range(0, len(members), hip.MAX_COMPRESS_BATCH):
            part = members[start:start + hip.MAX_COMPRESS_BATCH]
            frees = buffer._take_frees()
            try:
                dispatch.compress_batch_pointers([m[1] for m in part], buffer, frees, device,
                                                 stream)
            except BaseException:
                buffer._restore_frees(frees)
                raise
            for (index, _, source, packed, record, sample_values, shape, distribution,
                 stream_geometry, storage_numel, payload_bytes, blocks) in part:
                side, payload = packed.split_with_sizes((storage_numel, payload_bytes))
                shifted_decode, counts, descriptor, center, blocks_out = record.split_with_sizes(
                    (1024, 4, 4, 1, 3 * blocks))
                count_view, used_view = counts.split_with_sizes((1, 1, 2))[:2]
                results[index] = CompressedTensor(
                    payload.view(torch.int32), storage_numel, side,
                    fallback_blocks=blocks_out,
                    fallback_buffer=buffer.data,
                    fallback_descriptor=descriptor,
                    buffer=buffer,
                    fallback_count=count_view,
                    fallback_used=used_view,
                    distribution=distribution, center=center, decode_table=shifted_decode,
                    shape=shape, layout=StorageLayout.COMPRESSED,
                    stream_geometry=stream_geometry, sample_values=sample_values,
                )
    return results
