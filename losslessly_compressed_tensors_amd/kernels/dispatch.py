"""Launch wrappers: one function per codec kernel launch.

Mirrors the reference's operator boundary ``LCT/kernels/dispatch.py``: each
function takes caller-allocated torch tensors, enqueues exactly one HIP
kernel on the current stream through ``liblct_hip.so`` and returns nothing
(except ``shift_decoding_table``, which returns its new table as the
reference's does).  There is no backend selection: the gfx950 library is the
only engine.
"""
from __future__ import annotations

import itertools
import os
import threading
from dataclasses import dataclass

import torch

from . import hip

# Largest codec block count of one tensor.  The reference switches to an
# atomic compaction path above 8192 blocks (LCT/kernels/autotune.py:54,
# LCT/codec/encode.py:80); here one deterministic path serves every size up to
# the storage format's int32 offsets: fewer than 2^31 storage elements.
MAX_CODEC_BLOCKS = 65535


def _ptr(tensor: torch.Tensor | None):
    return None if tensor is None else tensor.data_ptr()


def _stream(tensor: torch.Tensor) -> int:
    """The raw handle of the current stream of ``tensor``'s device."""
    return torch._C._cuda_getCurrentRawStream(tensor.get_device())


def _byref(storage: FallbackStorage | None):
    """The storage as a C-ABI overflow argument, or None when it holds no
    entries: absent, or private with exact-size arrays of length 0."""
    if storage is None or (not storage.buffered and storage.lanes.numel() == 0):
        return None
    return hip.ctypes.byref(storage.as_overflow())


def require_device(*tensors: torch.Tensor) -> None:
    """Raise ``ValueError`` for any host tensor among ``tensors`` (None skipped)."""
    for tensor in tensors:
        if tensor is not None and tensor.device.type != "cuda":
            raise ValueError(f"LCT kernels require GPU tensors, got {tensor.device}")


_require_device = require_device


@dataclass
class FallbackStorage:
    """Overflow lanes/starts/tails of one tensor (``LCT/kernels/backends.py:36-50``).

    Buffered storage has ``descriptor`` set and all three arrays pointing at
    the TensorBuffer arena; private storage has exact-size arrays.
    """

    tail: torch.Tensor
    count: torch.Tensor
    lanes: torch.Tensor
    starts: torch.Tensor
    blocks: torch.Tensor
    descriptor: torch.Tensor | None = None
    allocation: torch.Tensor | None = None
    base: int = 0

    @property
    def buffered(self) -> bool:
        return self.descriptor is not None

    def as_overflow(self) -> hip.Overflow:
        return hip.Overflow(
            _ptr(self.lanes), _ptr(self.starts), _ptr(self.tail), _ptr(self.blocks),
            _ptr(self.count), _ptr(self.descriptor), int(self.base))


# ---------------------------------------------------------------------------
# Tables (dispatch.py:16-62)
# ---------------------------------------------------------------------------


def shift_encoding_table(encode_table, center, shifted_encode, decode_table,
                         shifted_decode=None) -> None:
    """Encode/decode tables for a given device center (``dispatch.py:16-30``)."""
    _require_device(encode_table, center)
    if shifted_decode is None:
        shifted_decode = torch.empty_like(decode_table)
    hip.call("lct_shift_tables", _ptr(encode_table), _ptr(center), _ptr(shifted_encode),
             _ptr(decode_table), _ptr(shifted_decode), _stream(encode_table))


def estimate_and_shift_encoding_table(source, center, size, encode_table, shifted_encode,
                                      decode_table, shifted_decode, sample_size,
                                      precomputed) -> None:
    """Sample the center from ``source`` and shift both tables (``dispatch.py:33-48``)."""
    _require_device(source, center)
    if shifted_decode is None:
        shifted_decode = torch.empty_like(decode_table)
    hip.call("lct_estimate_and_shift_tables", _ptr(source), int(bool(precomputed)), int(size),
             int(sample_size), _ptr(encode_table), _ptr(decode_table), _ptr(center),
             _ptr(shifted_encode), _ptr(shifted_decode), _stream(source))


def sample_center(source, logical_numel, sample_size, precomputed, partials,
                  sample_values=None) -> None:
    """Center samples spread over 64-sample workgroups: per-group exponent
    sums and counts into ``partials`` (the sampling half of ``dispatch.py:33-48``);
    the sampled BF16 values into ``sample_values`` when given."""
    _require_device(source, partials)
    hip.call("lct_sample_center", _ptr(source), int(bool(precomputed)), int(logical_numel),
             int(sample_size), _ptr(partials), _ptr(sample_values), _stream(source))


def shift_decoding_table(decode_table, center) -> torch.Tensor:
    """Return a center-shifted copy of ``decode_table`` (``dispatch.py:51-62``)."""
    _require_device(decode_table, center)
    shifted = torch.empty(1024, dtype=torch.int32, device=decode_table.device)
    hip.call("lct_shift_decoding_table", _ptr(decode_table), _ptr(center), _ptr(shifted),
             _stream(decode_table))
    return shifted


# ---------------------------------------------------------------------------
# Encoder, scans, compaction (dispatch.py:70-130, 294-316)
# ---------------------------------------------------------------------------


def encode_kernel(source, side, encoded, encode_table, extra_starts, summaries, size, streams,
                  *, precomputed, logical_numel, block_symbols, lanes, steps, fixed_words,
                  write_summary) -> None:
    """Field split + fixed-payload encoder (``dispatch.py:294-316``)."""
    _require_device(source, side, encoded)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    hip.call("lct_encode", _ptr(source), _ptr(side), _ptr(encoded), _ptr(encode_table),
             _ptr(extra_starts), _ptr(summaries) if write_summary else None, int(size),
             int(logical_numel), geometry, int(bool(precomputed)), int(bool(write_summary)),
             _stream(source))


def encode_sampled(source, side, encoded, partials, sample_size, encode_table, decode_table,
                   center, shifted_decode, extra_starts, summaries, size, *, precomputed,
                   logical_numel, block_symbols, lanes, steps, fixed_words) -> None:
    """The encoder with the table step folded in: the center and both shifted
    tables come from ``sample_center``'s partials (``dispatch.py:33-48`` then
    ``:294-316``)."""
    _require_device(source, side, encoded, partials)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    hip.call("lct_encode_sampled", _ptr(source), _ptr(side), _ptr(encoded), _ptr(partials),
             int(sample_size), _ptr(encode_table), _ptr(decode_table), _ptr(center),
             _ptr(shifted_decode), _ptr(extra_starts), _ptr(summaries), int(size),
             int(logical_numel), geometry, int(bool(precomputed)), 1, _stream(source))


def prefix_allocate(summaries, counts, descriptor, buffer, blocks_out, blocks, buffered,
                    max_free_regions) -> None:
    """Block scans, block metadata, overflow-block list and optional arena
    reservation (``dispatch.py:70-85`` plus the metadata half of
    ``compact_extra``).  ``summaries`` is int32[5*blocks + 1]."""
    _require_device(summaries, counts)
    meta = buffer.storage if buffer is not None else None
    if buffered:
        buffer._flush_frees()
    hip.call("lct_prefix_allocate", _ptr(summaries), _ptr(counts),
             _ptr(descriptor) if buffered else None, _ptr(meta) if buffered else None,
             _ptr(blocks_out), int(blocks), int(bool(buffered)), int(max_free_regions),
             _stream(summaries))


MAX_PENDING_FREES = hip.MAX_PENDING_FREES

# Values stored to the ready word of lct_allocate_compact: unique within the
# process (a counter) and, in the high half, a per-process random salt, so no
# earlier call's value (nor, in practice, stale memory) equals a new one.
_EPOCHS = itertools.count((int.from_bytes(os.urandom(4), "little") | 1) << 32)

# int32 entries of a summaries tensor for lct_allocate_compact: the 5*nb + 1
# of lct_prefix_allocate, then an 8-byte aligned uint64 ready word.


def summaries_length(blocks: int) -> int:
    return 5 * blocks + 5


def _ready_pointer(summaries: torch.Tensor, blocks: int) -> int:
    return (summaries.data_ptr() + 4 * (5 * blocks + 1) + 7) & ~7


def allocate_compact(source, summaries, counts, descriptor, buffer, blocks_out, extra_starts,
                     frees, n_blocks, size, *, logical_numel, block_symbols, lanes, steps,
                     precomputed) -> None:
    """Buffered overflow bookkeeping in one launch: the deferred ``frees``
    (device descriptors, at most ``hip.MAX_PENDING_FREES``), then what
    ``prefix_allocate`` and ``compact_extra`` do for a shared buffer
    (``dispatch.py:70-85, 113-130``).  ``summaries`` holds
    ``summaries_length(n_blocks)`` entries."""
    _require_device(source, summaries, counts)
    pending = hip.PendingFrees()
    pending.count = len(frees)
    for i, freed in enumerate(frees):
        pending.descriptor[i] = freed.data_ptr()
    geometry = hip.Geometry(block_symbols, lanes, steps, 2)
    hip.call("lct_allocate_compact", _ptr(source), _ptr(summaries), _ptr(counts),
             _ptr(descriptor), _ptr(buffer.storage), int(buffer.max_free_regions),
             _ptr(buffer.data), _ptr(blocks_out), _ptr(extra_starts), hip.ctypes.byref(pending),
             _ready_pointer(summaries, n_blocks), next(_EPOCHS), int(size), int(logical_numel),
             geometry, int(bool(precomputed)), _stream(source))


# lct_encode_fused's control arrays: one per (device, stream), zeroed when
# created and never cleared again (each call's words carry its epoch), grown
# when a tensor has more codec blocks than the array holds words for.
CONTROL_PARTIALS = 64
_control_arrays: dict = {}
_control_lock = threading.Lock()

# Epochs of lct_encode_fused: unique within the process (a 32-bit counter from
# a random start, 0 skipped), so no word an earlier call left in a control
# array matches a later call's epoch before 2^32 calls.
_FUSED_EPOCHS = itertools.count(int.from_bytes(os.urandom(4), "little"))


def _next_fused_epoch() -> int:
    while True:
        epoch = next(_FUSED_EPOCHS) & 0xFFFFFFFF
        if epoch != 0:
            return epoch


def control_array(device: torch.device, n_blocks: int) -> torch.Tensor:
    """The current stream's control array on ``device`` with room for
    ``n_blocks`` codec blocks (int64 words, reinterpreted as uint64 by the
    kernel).  A new or larger array is zeroed on the current stream, so the
    launch that follows on that stream sees it zeroed."""
    stream = torch._C._cuda_getCurrentRawStream(device.index)
    key = (device.index, stream)
    need = CONTROL_PARTIALS + n_blocks
    with _control_lock:
        array = _control_arrays.get(key)
        if array is None or array.numel() < need:
            size = max(need, CONTROL_PARTIALS + 4096)
            if array is not None:
                size = max(size, 2 * array.numel())
            array = torch.zeros(size, dtype=torch.int64, device=device)
            _control_arrays[key] = array
        return array


def bookkeeping(device, n_blocks, counts, blocks_out, buffer=None, descriptor=None, frees=(),
                samples=None):
    """The ``lct_bookkeeping`` record of a fused update encoder launch on the
    current stream of ``device``: its control array and a fresh epoch, the
    totals and block metadata outputs and, for a shared ``buffer``, the
    reservation's descriptor and the deferred ``frees``.  ``samples``:
    ``(a_samples, b_samples, result_samples)`` for a launch that samples the
    result's center itself (no sampler launch before it), or None."""
    control = control_array(device, n_blocks)
    record = hip.Bookkeeping()
    record.control = _ptr(control)
    record.control_words = int(control.numel())
    record.epoch = _next_fused_epoch()
    record.counts = _ptr(counts)
    record.blocks = _ptr(blocks_out)
    if buffer is not None:
        record.descriptor = _ptr(descriptor)
        record.buffer_meta = _ptr(buffer.storage)
        record.max_free_regions = int(buffer.max_free_regions)
        record.frees.count = len(frees)
        for i, freed in enumerate(frees):
            record.frees.descriptor[i] = freed.data_ptr()
    if samples is not None:
        record.a_samples, record.b_samples, record.result_samples = (_ptr(t) for t in samples)
    return record


def encode_fused(source, side, encoded, sample_size, encode_table, decode_table, center,
                 shifted_decode, sample_values, extra_starts, summaries, blocks_out, counts,
                 size, *, precomputed, logical_numel, block_symbols, lanes, steps, fixed_words,
                 buffer=None, descriptor=None, frees=(), host_totals=None) -> int:
    """Center sampling, encoder and overflow bookkeeping in one launch
    (``dispatch.py:33-48``, ``:294-316`` and ``:70-85`` as
    ``LCT/codec/encode.py:22-186`` sequences them): for a shared ``buffer``
    also the deferred ``frees`` and the arena reservation into
    ``descriptor``.  ``compact_extra`` then writes the entries and tails.
    ``host_totals`` (private storage only): a :class:`HostTotals` the launch
    also posts the overflow totals to.  Returns the launch's epoch."""
    _require_device(source, side, encoded, summaries, counts)
    n_blocks = size // block_symbols
    control = control_array(source.device, n_blocks)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    buffered = buffer is not None
    pending = None
    if buffered:
        pending = hip.PendingFrees()
        pending.count = len(frees)
        for i, freed in enumerate(frees):
            pending.descriptor[i] = freed.data_ptr()
    epoch = _next_fused_epoch()
    hip.call("lct_encode_fused", _ptr(source), _ptr(side), _ptr(encoded), int(sample_size),
             _ptr(encode_table), _ptr(decode_table), _ptr(center), _ptr(shifted_decode),
             _ptr(sample_values), _ptr(extra_starts), _ptr(summaries), _ptr(blocks_out),
             _ptr(counts), _ptr(control), int(control.numel()), epoch,
             _ptr(descriptor) if buffered else None, _ptr(buffer.storage) if buffered else None,
             int(buffer.max_free_regions) if buffered else 0,
             hip.ctypes.byref(pending) if buffered else None,
             host_totals.address if host_totals is not None else None, int(size),
             int(logical_numel), geometry, int(bool(precomputed)), _stream(source))
    return epoch


def encode_fused_pointers(source, side, encoded, sample_size, encode_table, decode_table,
                          center, shifted_decode, sample_values, extra_starts, summaries,
                          blocks_out, counts, size, logical_numel, geometry, device, stream, *,
                          descriptor=None, buffer=None, frees=(), host_totals=None) -> int:
    """``encode_fused`` with every array given as a device address (int) and
    the stream as its raw handle, for the public compress, which places
    several arrays in one allocation and checks its tensors itself.  Returns
    the launch's epoch."""
    control = control_array(device, size // geometry.block_symbols)
    pending = None
    if buffer is not None:
        pending = hip.PendingFrees()
        pending.count = len(frees)
        for i, freed in enumerate(frees):
            pending.descriptor[i] = freed.data_ptr()
    epoch = _next_fused_epoch()
    hip.call("lct_encode_fused", source, side, encoded, sample_size, encode_table, decode_table,
             center, shifted_decode, sample_values, extra_starts, summaries, blocks_out, counts,
             control.data_ptr(), control.numel(), epoch, descriptor,
             None if buffer is None else buffer.storage.data_ptr(),
             0 if buffer is None else buffer.max_free_regions,
             None if pending is None else hip.ctypes.byref(pending),
             None if host_totals is None else host_totals.address, size, logical_numel,
             geometry, 0, stream)
    return epoch


def compress_batch_pointers(jobs, buffer, frees, device, stream) -> None:
    """``lct_compress_batch``: the buffered compress of ``jobs`` (at most
    ``hip.MAX_COMPRESS_BATCH`` ``hip.CompressJob``s with device addresses,
    all of one step count) into ``buffer``, applying the deferred ``frees``
    first, on the raw stream handle ``stream`` of ``device``."""
    n_blocks = [job.size // job.geometry.block_symbols for job in jobs]
    total = sum(n_blocks)
    # One working array each, partitioned by the entry point in job order:
    # extra starts (256 per block), summaries (5 nb + 1 per job) and control
    # words (a gate word, then 64 + nb per job).
    extra_starts, summaries = compress_workspace(device, total + len(jobs), total * 256)
    control = control_array(device, total + (CONTROL_PARTIALS + 1) * len(jobs))
    pending = hip.PendingFrees()
    pending.count = len(frees)
    for i, freed in enumerate(frees):
        pending.descriptor[i] = freed.data_ptr()
    array = (hip.CompressJob * len(jobs))(*jobs)
    hip.call("lct_compress_batch", array, len(jobs), extra_starts.data_ptr(),
             extra_starts.numel(), summaries.data_ptr(), summaries.numel(), control.data_ptr(),
             control.numel(), _next_fused_epoch(), buffer.storage.data_ptr(),
             buffer.max_free_regions, buffer.data.data_ptr(), hip.ctypes.byref(pending), stream)


def pointwise_update_batch_pointers(jobs, op, alpha_is_one, beta_is_one, alpha, beta, buffer,
                                    frees, device, stream) -> None:
    """``lct_pointwise_update_batch``: the fused compressed-output updates of
    ``jobs`` (at most ``hip.MAX_UPDATE_BATCH`` ``hip.UpdateJob``s with device
    addresses, one step count) into ``buffer``, applying the deferred
    ``frees`` first, on the raw stream handle ``stream`` of ``device``.
    ``alpha``/``beta``: float32 device scalars or None."""
    n_blocks = [job.size // job.geometry.block_symbols for job in jobs]
    total = sum(n_blocks)
    groups = sum(-(-job.sample_size // 64) for job in jobs)
    extra_starts, summaries = compress_workspace(device, total + len(jobs), total * 256)
    control = control_array(device, total + (CONTROL_PARTIALS + 1) * len(jobs))
    partials = torch.empty(2 * groups, dtype=torch.int32, device=device)
    pending = hip.PendingFrees()
    pending.count = len(frees)
    for i, freed in enumerate(frees):
        pending.descriptor[i] = freed.data_ptr()
    array = (hip.UpdateJob * len(jobs))(*jobs)
    hip.call("lct_pointwise_update_batch", array, len(jobs), int(op), int(alpha_is_one),
             int(beta_is_one), None if alpha is None else alpha.data_ptr(),
             None if beta is None else beta.data_ptr(), partials.data_ptr(), partials.numel(),
             extra_starts.data_ptr(), extra_starts.numel(), summaries.data_ptr(),
             summaries.numel(), control.data_ptr(), control.numel(), _next_fused_epoch(),
             buffer.storage.data_ptr(), buffer.max_free_regions, buffer.data.data_ptr(),
             hip.ctypes.byref(pending), stream)


def compact_extra_pointers(source, lanes, starts, tail, descriptor, count, blocks, extra_starts,
                           size, logical_numel, geometry, buffered, stream) -> None:
    """``compact_extra`` over every block whose metadata ``encode_fused`` wrote
    (no summaries, tail base 0), with device addresses (ints) and a raw
    stream handle; BF16 tail source."""
    hip.call("lct_compact_extra", source, lanes, starts, tail, descriptor, count, blocks, 0,
             extra_starts, None, size, logical_numel, geometry, 0, int(buffered), stream)


class HostTotals:
    """Two uint64 words of pinned host memory that ``lct_encode_fused`` posts a
    private compress's overflow totals to (``epoch << 32 | entries |
    incomplete << 31`` and ``epoch << 32 | tail bytes``).  The reference reads
    the totals with a blocking device->host copy after the launch
    (``LCT/codec/encode.py:137-171``); polling these words instead lets the
    host size the exact overflow arrays and enqueue the compaction as soon as
    the launch's bookkeeping has the totals, before the launch ends."""

    def __init__(self):
        self.words = torch.zeros(2, dtype=torch.int64, pin_memory=True)
        self.address = self.words.data_ptr()
        self._view = self.words.numpy().view("uint64")

    def wait(self, epoch: int, counts: torch.Tensor, device) -> tuple[int, int, int]:
        """(entries, tail bytes, incomplete) of the launch with ``epoch``, made
        on the current stream of ``device``.  Polls the words; once that
        stream has no work left and they still do not carry the epoch, reads
        ``counts`` from the device instead."""
        view = self._view
        spins = 0
        stream = None
        while True:
            w0 = int(view[0])
            w1 = int(view[1])
            if w0 >> 32 == epoch and w1 >> 32 == epoch:
                return w0 & 0x7FFFFFFF, w1 & 0xFFFFFFFF, (w0 >> 31) & 1
            spins += 1
            if spins % 64 != 0:
                continue
            if stream is None:
                stream = torch.cuda.current_stream(device)
            if stream.query():
                w0 = int(view[0])
                w1 = int(view[1])
                if w0 >> 32 == epoch and w1 >> 32 == epoch:
                    return w0 & 0x7FFFFFFF, w1 & 0xFFFFFFFF, (w0 >> 31) & 1
                count, tail_bytes, _, incomplete = (int(v) for v in counts.tolist())
                return count, tail_bytes, incomplete


class _ThreadState(threading.local):
    def __init__(self):
        self.workspaces = {}
        self.host_totals = None


_thread_state = _ThreadState()


def host_totals() -> HostTotals:
    """This thread's :class:`HostTotals` (a compress waits on it before it
    returns, so one per thread serves every stream)."""
    state = _thread_state
    if state.host_totals is None:
        state.host_totals = HostTotals()
    return state.host_totals


def compress_workspace(device: torch.device, n_blocks: int, n_streams: int):
    """``(extra_starts uint8[n_streams], summaries int32[summaries_length(n_blocks)])``
    for a compress on the current stream of ``device``: working arrays that no
    stored tensor keeps, held per thread and stream and grown on demand.  The
    next compress of the same thread on the same stream reuses them; stream
    order puts its writes after every read of this one."""
    stream = torch._C._cuda_getCurrentRawStream(device.index)
    key = (device.index, stream)
    cached = _thread_state.workspaces.get(key)
    if cached is not None and cached[0] == (n_blocks, n_streams):
        return cached[2]
    need_extra, need_summaries = n_streams, summaries_length(n_blocks)
    arrays = None if cached is None else cached[1]
    if arrays is None or arrays[0].numel() < need_extra or arrays[1].numel() < need_summaries:
        arrays = (torch.empty(max(need_extra, 0 if arrays is None else arrays[0].numel()),
                              dtype=torch.uint8, device=device),
                  torch.empty(max(need_summaries, 0 if arrays is None else arrays[1].numel()),
                              dtype=torch.int32, device=device))
    views = (arrays[0][:need_extra], arrays[1][:need_summaries])
    _thread_state.workspaces[key] = ((n_blocks, n_streams), arrays, views)
    return views


def count_bad_streams(extra_starts, count, total, streams, steps) -> None:
    """Atomic-path totals (``dispatch.py:88-95``): adds the overflowing
    streams and their tail bytes to ``count[0]`` and ``total[0]`` (zeroed by
    the caller)."""
    _require_device(extra_starts, count, total)
    hip.call("lct_count_bad_streams", _ptr(extra_starts), _ptr(count), _ptr(total),
             int(streams), int(steps), _stream(extra_starts))


def compact_bad_streams(extra_starts, storage: FallbackStorage, final_counts, bad_count,
                        fallback_total, n_streams, steps, n_blocks, buffered, lanes) -> None:
    """Atomic-path entries and block metadata (``dispatch.py:98-110``): each
    block reserves its slice with atomics on ``bad_count``/``fallback_total``
    (zeroed by the caller); ``compact_extra(..., summaries=None)`` then writes
    the tails."""
    _require_device(extra_starts, storage.blocks, bad_count, fallback_total)
    if lanes != 256:
        raise ValueError("LCT streams have 256 lanes per block")
    hip.call("lct_compact_bad_streams", _ptr(extra_starts), _ptr(storage.lanes),
             _ptr(storage.starts), _ptr(storage.descriptor), _ptr(storage.blocks),
             _ptr(final_counts), _ptr(bad_count), _ptr(fallback_total), int(n_streams),
             int(steps), int(n_blocks), int(bool(buffered)), _stream(extra_starts))


def compact_extra(source, storage: FallbackStorage, n_blocks, n_elements, *, precomputed,
                  buffered, logical_numel, block_symbols, lanes, steps, extra_starts,
                  summaries) -> None:
    """Overflow entries and tails (``dispatch.py:113-130``): of the blocks
    ``prefix_allocate`` listed, or, with ``summaries=None``, of every block
    whose metadata ``compact_bad_streams`` or ``encode_fused`` wrote (one
    workgroup per block)."""
    _require_device(source, extra_starts)
    geometry = hip.Geometry(block_symbols, lanes, steps, 2)
    hip.call("lct_compact_extra", _ptr(source), _ptr(storage.lanes), _ptr(storage.starts),
             _ptr(storage.tail), _ptr(storage.descriptor), _ptr(storage.count),
             _ptr(storage.blocks), int(storage.base), _ptr(extra_starts), _ptr(summaries),
             int(n_elements), int(logical_numel), geometry, int(bool(precomputed)),
             int(bool(buffered)), _stream(source))


# ---------------------------------------------------------------------------
# Decoder and fused pointwise (dispatch.py:168-286, 319-361)
# ---------------------------------------------------------------------------


def decode_kernel(encoded, side, output, shifted_decode, center, size, *, logical_numel,
                  block_symbols, lanes, steps, fixed_words, rare_length,
                  overflow: FallbackStorage | None = None) -> None:
    """Decoder with the overflow overlay fused when ``overflow`` is given."""
    _require_device(encoded, side, output)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    ov = overflow.as_overflow() if overflow is not None else None
    hip.call("lct_decode", _ptr(encoded), _ptr(side), _ptr(output), _ptr(shifted_decode),
             _ptr(center), int(size), int(logical_numel), geometry, int(rare_length),
             ov if ov is None else hip.ctypes.byref(ov), _stream(encoded))


def decode_batch(jobs) -> None:
    """Several decodes in one launch (``lct_decode_batch``).  ``jobs``: at most
    ``hip.MAX_DECODE_BATCH`` tuples ``(encoded, side, output, shifted_decode,
    center, size, logical_numel, (B, L, S, W), rare_length, overflow)`` with
    ``decode_kernel``'s meanings, all on the current stream's device."""
    array = (hip.DecodeJob * len(jobs))()
    for job, (encoded, side, output, shifted_decode, center, size, logical_numel, geometry,
              rare_length, overflow) in zip(array, jobs):
        _require_device(encoded, side, output)
        job.encoded, job.side, job.output = _ptr(encoded), _ptr(side), _ptr(output)
        job.shifted_decode, job.center = _ptr(shifted_decode), _ptr(center)
        job.size, job.logical_numel = int(size), int(logical_numel)
        job.geometry = hip.Geometry(*(int(v) for v in geometry))
        job.rare_length = int(rare_length)
        job.has_overflow = int(overflow is not None)
        if overflow is not None:
            job.overflow = overflow.as_overflow()
    hip.call("lct_decode_batch", array, len(jobs), _stream(jobs[0][0]))


def scatter_fallback(storage: FallbackStorage, sign_mantissa, output, n_elements,
                     logical_numel, block_symbols, lanes, steps) -> None:
    """Overflow rows of a decode made without the overlay
    (``dispatch.py:146-165``)."""
    _require_device(sign_mantissa, output)
    overflow = _byref(storage)
    if overflow is None:
        return
    geometry = hip.Geometry(block_symbols, lanes, steps, 2)
    hip.call("lct_scatter_fallback", overflow, _ptr(sign_mantissa), _ptr(output),
             int(n_elements), int(logical_numel), geometry, _stream(sign_mantissa))


def pointwise_fallback(storage: FallbackStorage, sign_mantissa, other, output, auxiliary,
                       n_elements, alpha, beta, *, logical_numel, block_symbols, lanes, steps,
                       output_policy, op, alpha_is_one, beta_is_one) -> None:
    """Overflow rows of a pointwise result computed without the overlay
    (``dispatch.py:190-212``); the operation's flags are the reference's
    ``operation_meta`` (OP, ALPHA_IS_ONE, BETA_IS_ONE) as plain arguments."""
    _require_device(sign_mantissa, other, output)
    overflow = _byref(storage)
    if overflow is None:
        return
    geometry = hip.Geometry(block_symbols, lanes, steps, 2)
    hip.call("lct_pointwise_fallback", overflow, _ptr(sign_mantissa), _ptr(other),
             _ptr(output), _ptr(auxiliary), _ptr(alpha), _ptr(beta), int(n_elements),
             int(logical_numel), geometry, int(op), int(bool(alpha_is_one)),
             int(bool(beta_is_one)), int(output_policy), _stream(sign_mantissa))


def pointwise_dense(encoded, sign_mantissa, other, output, auxiliary, shifted_decode, size,
                    center, alpha, beta, *, rare_length, logical_numel, block_symbols, lanes,
                    steps, fixed_words, output_policy, op, alpha_is_one, beta_is_one,
                    overflow: FallbackStorage | None = None) -> None:
    """Decode + op against a dense operand, overflow rows overlaid in the same pass."""
    _require_device(encoded, sign_mantissa, other, output)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    ov = overflow.as_overflow() if overflow is not None else None
    hip.call("lct_pointwise_dense", _ptr(encoded), _ptr(sign_mantissa), _ptr(other),
             _ptr(output), _ptr(auxiliary), _ptr(shifted_decode), _ptr(center), _ptr(alpha),
             _ptr(beta), int(size), int(logical_numel), geometry, int(rare_length), int(op),
             int(bool(alpha_is_one)), int(bool(beta_is_one)), int(output_policy),
             ov if ov is None else hip.ctypes.byref(ov), _stream(encoded))


def dual(a_encoded, a_sign_mantissa, a_shifted_decode, a_center, a_storage,
         b_encoded, b_sign_mantissa, b_shifted_decode, b_center, b_storage,
         output, auxiliary, alpha, size, *, rare_length, logical_numel,
         block_symbols, lanes, steps, fixed_words, output_policy) -> None:
    """Fused ``alpha * A + B`` over two compressed operands: the reference's
    ``dual_maps_init`` + ``dual_tables_and_maps`` + ``dual_mapped``
    (``dispatch.py:215-286``) in one launch."""
    _require_device(a_encoded, b_encoded, output, alpha)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    a_ov = a_storage.as_overflow() if a_storage is not None else None
    b_ov = b_storage.as_overflow() if b_storage is not None else None
    hip.call("lct_dual", _ptr(a_encoded), _ptr(a_sign_mantissa), _ptr(a_shifted_decode),
             _ptr(a_center), a_ov if a_ov is None else hip.ctypes.byref(a_ov), _ptr(b_encoded),
             _ptr(b_sign_mantissa), _ptr(b_shifted_decode), _ptr(b_center),
             b_ov if b_ov is None else hip.ctypes.byref(b_ov), _ptr(alpha), _ptr(output),
             _ptr(auxiliary), int(size), int(logical_numel), geometry, int(rare_length),
             int(output_policy), _stream(a_encoded))


def dual_maps_init(a_stream_starts, a_stream_offsets, b_stream_starts, b_stream_offsets,
                   a_count, b_count, n_streams, steps) -> None:
    """Both operands' per-stream maps to "no overflow" (``dispatch.py:215-225``;
    the counts are not needed to initialise them)."""
    _require_device(a_stream_starts, b_stream_starts)
    hip.call("lct_dual_maps_init", _ptr(a_stream_starts), _ptr(a_stream_offsets),
             _ptr(b_stream_starts), _ptr(b_stream_offsets), int(n_streams), int(steps),
             _stream(a_stream_starts))


def dual_tables_and_maps(a_decode_table, a_center, a_shifted, b_decode_table, b_center,
                         b_shifted, a_storage, b_storage, a_stream_starts, a_stream_offsets,
                         b_stream_starts, b_stream_offsets, blocks, *, lanes, steps,
                         buffered) -> None:
    """Shift both decode tables and expand both compact overflow lists into
    the per-stream maps (``dispatch.py:228-252``)."""
    _require_device(a_decode_table, b_decode_table, a_stream_starts, b_stream_starts)
    if lanes != 256:
        raise ValueError("LCT streams have 256 lanes per block")
    hip.call("lct_dual_tables_and_maps", _ptr(a_decode_table), _ptr(a_center), _ptr(a_shifted),
             _ptr(b_decode_table), _ptr(b_center), _ptr(b_shifted), _byref(a_storage),
             _byref(b_storage), _ptr(a_stream_starts), _ptr(a_stream_offsets),
             _ptr(b_stream_starts), _ptr(b_stream_offsets), int(blocks), int(steps),
             _stream(a_decode_table))


def dual_mapped(a_encoded, a_sign_mantissa, a_shifted, a_center, a_stream_starts,
                a_stream_offsets, a_storage, b_encoded, b_sign_mantissa, b_shifted, b_center,
                b_stream_starts, b_stream_offsets, b_storage, output, auxiliary, alpha,
                n_elements, n_streams, blocks, *, rare_length, logical_numel, buffered,
                block_symbols, lanes, steps, fixed_words, output_policy) -> None:
    """``alpha * A + B`` with each operand's overlay read from its per-stream
    maps (``dispatch.py:255-286``)."""
    _require_device(a_encoded, b_encoded, output, alpha)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    hip.call("lct_dual_mapped", _ptr(a_encoded), _ptr(a_sign_mantissa), _ptr(a_shifted),
             _ptr(a_center), _ptr(a_stream_starts), _ptr(a_stream_offsets), _byref(a_storage),
             _ptr(b_encoded), _ptr(b_sign_mantissa), _ptr(b_shifted), _ptr(b_center),
             _ptr(b_stream_starts), _ptr(b_stream_offsets), _byref(b_storage), _ptr(alpha),
             _ptr(output), _ptr(auxiliary), int(n_elements), int(logical_numel), geometry,
             int(rare_length), int(output_policy), _stream(a_encoded))


def pointwise_sample(encoded, sign_mantissa, shifted_decode, center, other, alpha, beta,
                     partials, size, *, rare_length, logical_numel, block_symbols, lanes, steps,
                     fixed_words, op, alpha_is_one, beta_is_one, sample_size,
                     overflow: FallbackStorage | None = None, a_samples=None,
                     result_samples=None) -> None:
    """The operation's result at the center sample positions only: exponent
    sum and count per group of 64 samples into ``partials``
    (int32[2*ceil(sample_size/64)]).  ``a_samples``: A's recorded values at
    those positions (then A's streams are not read); ``result_samples``
    receives the result's."""
    _require_device(encoded, sign_mantissa, other, partials)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    ov = overflow.as_overflow() if overflow is not None else None
    hip.call("lct_pointwise_sample", _ptr(encoded), _ptr(sign_mantissa), _ptr(shifted_decode),
             _ptr(center), ov if ov is None else hip.ctypes.byref(ov), _ptr(a_samples),
             _ptr(other), _ptr(alpha), _ptr(beta), int(size), int(logical_numel), geometry,
             int(rare_length), int(op), int(bool(alpha_is_one)), int(bool(beta_is_one)),
             int(sample_size), _ptr(partials), _ptr(result_samples), _stream(encoded))


def pointwise_encode(encoded, sign_mantissa, shifted_decode, center, other, alpha, beta,
                     partials, base_encode, base_decode, center_out, shifted_decode_out,
                     side_out, encoded_out, extra_starts, summaries, exponents, size, *,
                     rare_length, logical_numel, block_symbols, lanes, steps, fixed_words, op,
                     alpha_is_one, beta_is_one, sample_size,
                     overflow: FallbackStorage | None = None, record=None) -> None:
    """Decode + op + re-encode in one pass: the single-pass form of the
    compressed-output ``pointwise_dense`` launch followed by the encoder
    launch of ``encode_components(precomputed=True)``; with a ``record``
    (``bookkeeping()``) also the prefix scan and reservation of
    ``encode_components`` in the same launch (``lct_pointwise_encode_fused``)."""
    _require_device(encoded, sign_mantissa, other, partials, encoded_out)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    ov = overflow.as_overflow() if overflow is not None else None
    args = [_ptr(encoded), _ptr(sign_mantissa), _ptr(shifted_decode), _ptr(center),
            ov if ov is None else hip.ctypes.byref(ov), _ptr(other), _ptr(alpha), _ptr(beta),
            _ptr(partials), int(sample_size), _ptr(base_encode), _ptr(base_decode),
            _ptr(center_out), _ptr(shifted_decode_out), _ptr(side_out), _ptr(encoded_out),
            _ptr(extra_starts), _ptr(summaries), _ptr(exponents), int(size), int(logical_numel),
            geometry, int(rare_length), int(op), int(bool(alpha_is_one)),
            int(bool(beta_is_one))]
    if record is None:
        hip.call("lct_pointwise_encode", *args, _stream(encoded))
    else:
        hip.call("lct_pointwise_encode_fused", *args, hip.ctypes.byref(record),
                 _stream(encoded))


def dual_sample(a_encoded, a_sign_mantissa, a_shifted_decode, a_center, a_storage, b_encoded,
                b_sign_mantissa, b_shifted_decode, b_center, b_storage, alpha, partials, size, *,
                rare_length, logical_numel, block_symbols, lanes, steps, fixed_words,
                sample_size, a_samples=None, b_samples=None, result_samples=None) -> None:
    """``fma(a, alpha, b)`` at the center sample positions only, for two
    compressed operands: exponent sum and count per group of 64 samples into
    ``partials``.  ``a_samples``/``b_samples``: an operand's recorded values at
    those positions (then its streams are not read); ``result_samples``
    receives the result's."""
    _require_device(a_encoded, b_encoded, alpha, partials)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    hip.call("lct_dual_sample", _ptr(a_encoded), _ptr(a_sign_mantissa), _ptr(a_shifted_decode),
             _ptr(a_center), _byref(a_storage), _ptr(a_samples), _ptr(b_encoded),
             _ptr(b_sign_mantissa), _ptr(b_shifted_decode), _ptr(b_center), _byref(b_storage),
             _ptr(b_samples), _ptr(alpha), int(size), int(logical_numel), geometry,
             int(rare_length), int(sample_size), _ptr(partials), _ptr(result_samples),
             _stream(a_encoded))


def dual_encode(a_encoded, a_sign_mantissa, a_shifted_decode, a_center, a_storage, b_encoded,
                b_sign_mantissa, b_shifted_decode, b_center, b_storage, alpha, partials,
                base_encode, base_decode, center_out, shifted_decode_out, side_out,
                encoded_out, extra_starts, summaries, exponents, size, *, rare_length,
                logical_numel, block_symbols, lanes, steps, fixed_words, sample_size,
                record=None) -> None:
    """Decode A and B, ``fma(a, alpha, b)`` and re-encode in one pass: the
    single-pass form of the compressed-output ``dual_mapped`` launch followed
    by the encoder launch of ``encode_components(precomputed=True)``; with a
    ``record`` also the prefix scan and reservation (``lct_dual_encode_fused``)."""
    _require_device(a_encoded, b_encoded, alpha, partials, encoded_out)
    geometry = hip.Geometry(block_symbols, lanes, steps, fixed_words)
    args = [_ptr(a_encoded), _ptr(a_sign_mantissa), _ptr(a_shifted_decode), _ptr(a_center),
            _byref(a_storage), _ptr(b_encoded), _ptr(b_sign_mantissa), _ptr(b_shifted_decode),
            _ptr(b_center), _byref(b_storage), _ptr(alpha), _ptr(partials), int(sample_size),
            _ptr(base_encode), _ptr(base_decode), _ptr(center_out), _ptr(shifted_decode_out),
            _ptr(side_out), _ptr(encoded_out), _ptr(extra_starts), _ptr(summaries),
            _ptr(exponents), int(size), int(logical_numel), geometry, int(rare_length)]
    if record is None:
        hip.call("lct_dual_encode", *args, _stream(a_encoded))
    else:
        hip.call("lct_dual_encode_fused", *args, hip.ctypes.byref(record), _stream(a_encoded))


# ---------------------------------------------------------------------------
# TensorBuffer allocator (LCT/tensor_buffer.py:93-136, tensor_buffer_ops.py)
# ---------------------------------------------------------------------------


def buffer_reset(storage, max_free_regions, capacity_bytes) -> None:
    hip.call("lct_buffer_reset", _ptr(storage), int(max_free_regions), int(capacity_bytes),
             _stream(storage))


def buffer_allocate(storage, max_free_regions, requested, item_count, item_bytes,
                    descriptor) -> None:
    hip.call("lct_buffer_allocate", _ptr(storage), int(max_free_regions), _ptr(requested),
             _ptr(item_count), int(item_bytes), _ptr(descriptor), _stream(storage))


def buffer_free(storage, max_free_regions, descriptor, status, *, stream=None) -> None:
    """``stream``: a raw stream handle; the current stream when None."""
    hip.call("lct_buffer_free", _ptr(storage), int(max_free_regions), _ptr(descriptor),
             _ptr(status), _stream(storage) if stream is None else stream)


MAX_FREE_BATCH = hip.MAX_FREE_BATCH


def buffer_free_batch(storage, max_free_regions, descriptors, status=None, *,
                      stream=None) -> None:
    """Free up to ``MAX_FREE_BATCH`` descriptors in order in one launch;
    ``status``: int32[len(descriptors)] or None.  ``stream`` as for
    ``buffer_free``."""
    if not 1 <= len(descriptors) <= MAX_FREE_BATCH:
        raise ValueError(f"1 to {MAX_FREE_BATCH} descriptors per batch, got {len(descriptors)}")
    # The kernel reads 4 ints of each descriptor and writes one status each.
    if any(d.dtype != torch.int32 or d.numel() < 4 for d in descriptors):
        raise ValueError("descriptors are int32[4] tensors")
    if status is not None and (status.dtype != torch.int32 or status.numel() < len(descriptors)):
        raise ValueError(f"status must be int32[{len(descriptors)}] or None")
    _require_device(storage, *descriptors, status)
    array = (hip.ctypes.c_void_p * len(descriptors))(*(d.data_ptr() for d in descriptors))
    hip.call("lct_buffer_free_batch", _ptr(storage), int(max_free_regions), array,
             len(descriptors), _ptr(status), _stream(storage) if stream is None else stream)
