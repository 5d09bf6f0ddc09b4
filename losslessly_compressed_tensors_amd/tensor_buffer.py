"""GPU-resident first-fit allocator for overflow tails (``TensorBuffer``).

Same interface and semantics as ``LCT/tensor_buffer.py:13-201``: one device
byte array holds ``free_starts[R] | free_sizes[R] | free_count | lock |
generation`` (padded to 16 bytes) followed by the payload arena; allocation
and free run on the device (``lct_buffer_allocate`` / ``lct_buffer_free``)
and return ``[offset, size, status, generation]`` descriptors without a host
sync.  ``reset()`` bumps the generation so older descriptors become stale.

A compressed tensor whose overflow reservation fails (no fit, lock not taken,
or an incomplete compaction) also sets a bit of a failure word kept in the
metadata's padding; ``verify_buffer``, ``TensorBuffer.check`` and the
tensor's own ``memory_size()`` raise ``BufferReservationError`` at their
synchronisation.  The reference never reports this case
(``LCT/kernels/tensor_buffer.py:84-89``).

``CompressedTensor.free()`` (which reports no status) defers its free to the
buffer's next reservation on the same stream: the compressed-output paths
reserve and compact in one launch (``lct_allocate_compact``) that first
applies the deferred frees, in order and under the same lock, so the arena
holds exactly what an immediate free would have left.  Every other operation
on the buffer (``allocate``, ``free``, ``reset``, the free-list snapshot
helpers) and a change of stream first launch the deferred frees as they are.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernels import dispatch

_ALIGNMENT = 16

# Descriptor statuses (LCT/kernels/tensor_buffer.py:37-192; 7 is this
# build's: a reservation whose compaction did not complete).
STATUS_OK, STATUS_NO_FIT, STATUS_EMPTY, STATUS_FREE_LIST_FULL = 0, 1, 2, 3
STATUS_INVALID, STATUS_FREED, STATUS_LOCK, STATUS_INCOMPLETE = 4, 5, 6, 7

# Bits of the buffer's failure word (int32 after the generation): a compressed
# tensor's overflow reservation found no fit, could not take the arena lock, or
# its compaction did not complete.  Kept until reset().
FAIL_NO_FIT, FAIL_LOCK, FAIL_INCOMPLETE = 1, 2, 4
_FAILURE_TEXT = {
    FAIL_NO_FIT: "no free region was large enough",
    FAIL_LOCK: "the arena lock could not be taken",
    FAIL_INCOMPLETE: "the overflow bookkeeping or compaction did not complete",
}
_STATUS_FAILURE = {STATUS_NO_FIT: FAIL_NO_FIT, STATUS_LOCK: FAIL_LOCK,
                   STATUS_INCOMPLETE: FAIL_INCOMPLETE}


class BufferReservationError(RuntimeError):
    """A compressed tensor's overflow data could not be stored in its
    ``TensorBuffer``; the tensor does not decode to its input.  The reference
    leaves such a tensor unflagged (``LCT/kernels/tensor_buffer.py:84-89``)."""


def _describe(bits: int) -> str:
    return "; ".join(text for bit, text in _FAILURE_TEXT.items() if bits & bit)


def check_reservation(status: int, count: int) -> None:
    """Raise ``BufferReservationError`` for a codec reservation with ``count``
    overflow entries whose descriptor status says the entries were not
    stored, and for every incomplete one (status 7: its bookkeeping or
    compaction did not finish, so even ``count`` may be short)."""
    if status == STATUS_INCOMPLETE or (count > 0 and status in _STATUS_FAILURE):
        raise BufferReservationError(
            f"compressed tensor's overflow reservation failed (status {status}: "
            f"{_describe(_STATUS_FAILURE[status])}); its {count} overflow streams were not "
            "stored and it does not decode to its input. Size the TensorBuffer for all "
            "live compressed tensors.")


@dataclass(frozen=True)
class Allocation:
    """A device ``[offset, aligned_size, status, generation]`` descriptor."""

    descriptor: torch.Tensor
    owner: object

    @property
    def offset(self) -> torch.Tensor:
        return self.descriptor[0]

    @property
    def size(self) -> torch.Tensor:
        return self.descriptor[1]

    @property
    def status(self) -> torch.Tensor:
        return self.descriptor[2]

    @property
    def generation(self) -> torch.Tensor:
        return self.descriptor[3]


def _free_now(storage: torch.Tensor, descriptor: torch.Tensor,
              max_free_regions: int, stream: int | None = None) -> torch.Tensor:
    status = torch.empty(1, dtype=torch.int32, device=storage.device)
    dispatch.buffer_free(storage, max_free_regions, descriptor, status, stream=stream)
    return status


def _free_many(storage: torch.Tensor, descriptors: list[torch.Tensor], max_free_regions: int,
               stream: int | None = None) -> None:
    """Free ``descriptors`` in order, ``dispatch.MAX_FREE_BATCH`` per launch
    (``lct_buffer_free_batch``: one hold of the lock each); statuses are not
    kept, as for the frees that ride on a reservation."""
    step = dispatch.MAX_FREE_BATCH
    for i in range(0, len(descriptors), step):
        dispatch.buffer_free_batch(storage, max_free_regions, descriptors[i:i + step], None,
                                   stream=stream)


@torch.library.custom_op("lct::tensor_buffer_free", mutates_args=("storage", "descriptor"))
def tensor_buffer_free(storage: torch.Tensor, descriptor: torch.Tensor,
                       max_free_regions: int) -> torch.Tensor:
    """Opaque free for ``torch.compile`` (``LCT/kernels/tensor_buffer_ops.py:5-15``)."""
    return _free_now(storage, descriptor, max_free_regions)


@tensor_buffer_free.register_fake
def _tensor_buffer_free_fake(storage, descriptor, max_free_regions):
    return torch.empty(1, dtype=torch.int32, device=storage.device)


class TensorBuffer:
    """Device-resident first-fit allocator returning device-side descriptors."""

    def __init__(self, capacity_bytes: int, *, max_free_regions: int = 256,
                 device: torch.device | str | None = None) -> None:
        if capacity_bytes > torch.iinfo(torch.int32).max:
            raise ValueError("capacity_bytes must fit in int32")
        if max_free_regions <= 0 or max_free_regions & (max_free_regions - 1):
            raise ValueError("max_free_regions must be a positive power of two")
        if max_free_regions > 4096:
            raise ValueError("max_free_regions above 4096 is not supported")
        self.capacity_bytes = int(capacity_bytes)
        self.max_free_regions = int(max_free_regions)
        self._metadata_bytes = self._align(8 * self.max_free_regions + 12)
        self._storage = torch.zeros(self._metadata_bytes + self.capacity_bytes,
                                    dtype=torch.uint8, device=torch.device(device or "cuda"))
        self.device = self._storage.device
        regions = self.max_free_regions
        meta = self._storage.narrow(0, 0, 8 * regions + 16).view(torch.int32)
        self._free_starts = meta.narrow(0, 0, regions)
        self._free_sizes = meta.narrow(0, regions, regions)
        self._free_count = meta.narrow(0, 2 * regions, 1)
        self._lock = meta.narrow(0, 2 * regions + 1, 1)
        self._generation = meta.narrow(0, 2 * regions + 2, 1)
        # In the metadata's alignment padding (8R + 12 rounded up to 16).
        self._failures = meta.narrow(0, 2 * regions + 3, 1)
        self._data = self._storage.narrow(0, self._metadata_bytes, self.capacity_bytes)
        # Descriptors whose free waits for the next reservation, and the raw
        # handle of the stream they were freed on.
        self._pending_frees: list[torch.Tensor] = []
        self._pending_stream = 0
        self.reset()

    @staticmethod
    def _align(nbytes: int) -> int:
        return (nbytes + _ALIGNMENT - 1) // _ALIGNMENT * _ALIGNMENT

    @property
    def data(self) -> torch.Tensor:
        """The payload arena (descriptor offsets index into it)."""
        return self._data

    @property
    def storage(self) -> torch.Tensor:
        """Metadata followed by the arena; the allocator kernels take its base."""
        return self._storage

    def _current_stream(self) -> int:
        return torch._C._cuda_getCurrentRawStream(self._storage.get_device())

    def _defer_free(self, descriptor: torch.Tensor) -> None:
        """Free ``descriptor`` at the next reservation on the current stream
        (up to ``dispatch.MAX_FREE_BATCH`` frees wait; a full list is launched
        first, in one launch)."""
        stream = self._current_stream()
        if self._pending_frees and (stream != self._pending_stream
                                    or len(self._pending_frees) == dispatch.MAX_FREE_BATCH):
            self._flush_frees()
        self._pending_frees.append(descriptor)
        self._pending_stream = stream

    def _restore_frees(self, frees: list[torch.Tensor]) -> None:
        """Put back frees taken for a reservation that was not launched."""
        self._pending_frees = [*frees, *self._pending_frees]

    def _take_frees(self) -> list[torch.Tensor]:
        """The deferred frees for a reservation on the current stream: the
        last ``dispatch.MAX_PENDING_FREES`` (a reservation applies that many);
        earlier ones are launched first, in one launch, and those deferred on
        another stream are launched there instead."""
        if not self._pending_frees:
            return []
        if self._pending_stream != self._current_stream():
            self._flush_frees()
            return []
        keep = dispatch.MAX_PENDING_FREES
        if len(self._pending_frees) > keep:
            # Dropped from the list once launched: a launch that raises (at
            # most MAX_FREE_BATCH wait, so it is one launch) leaves them
            # deferred.
            _free_many(self._storage, self._pending_frees[:-keep], self.max_free_regions,
                       stream=self._pending_stream)
            del self._pending_frees[:-keep]
        frees, self._pending_frees = self._pending_frees, []
        return frees

    def _flush_frees(self) -> None:
        """Launch the deferred frees, in order, on the stream they were made
        on; when that is not the current stream, the current stream then
        waits for them, so work enqueued on it from here on (after any
        ``wait_stream`` the caller made since the frees) follows them, as it
        would have followed an immediate free.  That stream must still exist."""
        if not self._pending_frees:
            return
        _free_many(self._storage, self._pending_frees, self.max_free_regions,
                   stream=self._pending_stream)
        self._pending_frees = []   # only once launched, as in _take_frees
        if self._pending_stream != self._current_stream():
            done = torch.cuda.Event()
            done.record(torch.cuda.ExternalStream(self._pending_stream, device=self.device))
            torch.cuda.current_stream(self.device).wait_event(done)

    def allocate(self, nbytes: torch.Tensor) -> Allocation:
        """Reserve ``nbytes`` (a one-element device int32 tensor) without a sync."""
        self._flush_frees()
        descriptor = torch.empty(4, dtype=torch.int32, device=self.device)
        dispatch.buffer_allocate(self._storage, self.max_free_regions, nbytes, None, 0,
                                 descriptor)
        return Allocation(descriptor, self)

    def allocate_with_items(self, payload_bytes: torch.Tensor, item_count: torch.Tensor,
                            item_bytes: int) -> Allocation:
        """Reserve ``payload_bytes + item_count * item_bytes`` asynchronously."""
        if item_bytes <= 0:
            raise ValueError("item_bytes must be positive")
        self._flush_frees()
        descriptor = torch.empty(4, dtype=torch.int32, device=self.device)
        dispatch.buffer_allocate(self._storage, self.max_free_regions, payload_bytes,
                                 item_count, int(item_bytes), descriptor)
        return Allocation(descriptor, self)

    def free(self, allocation: Allocation) -> torch.Tensor:
        """Return an allocation; the device status comes back asynchronously."""
        if allocation.owner is not self:
            raise ValueError("allocation belongs to a different allocator")
        if allocation.descriptor.device != self.device:
            raise ValueError("allocation must be on the allocator device")
        if torch.compiler.is_compiling():
            return tensor_buffer_free(self._storage, allocation.descriptor,
                                      self.max_free_regions)
        # Eager callers skip the operator dispatch (same kernel, same stream).
        self._flush_frees()
        return _free_now(self._storage, allocation.descriptor, self.max_free_regions)

    def reset(self) -> None:
        """Reset asynchronously; previously returned descriptors become stale
        and the failure word is cleared."""
        self._flush_frees()
        dispatch.buffer_reset(self._storage, self.max_free_regions, self.capacity_bytes)

    def failures(self) -> int:
        """Synchronize and return the failure word: ``FAIL_*`` bits of the
        compressed tensors whose overflow reservation failed since the last
        reset (0 if none)."""
        self._flush_frees()
        return int(self._failures.item())

    def check(self) -> None:
        """Synchronize and raise ``BufferReservationError`` if a compressed
        tensor's overflow reservation failed since the last reset."""
        bits = self.failures()
        if bits:
            raise BufferReservationError(
                f"a compressed tensor's overflow reservation in this TensorBuffer failed "
                f"({_describe(bits)}); that tensor does not decode to its input. Size the "
                "buffer for all live compressed tensors, then reset() it.")


def _free_regions_snapshot(buffer: TensorBuffer) -> list[tuple[int, int]]:
    """Synchronize and copy the free list as ``[(start, size), ...]``."""
    buffer._flush_frees()
    regions = buffer.max_free_regions
    meta = buffer._storage.narrow(0, 0, buffer._metadata_bytes).view(torch.int32).cpu()
    count = int(meta[2 * regions].item())
    if not 0 <= count <= regions:
        raise RuntimeError(f"corrupt free-list count: {count}")
    return [(int(meta[i].item()), int(meta[regions + i].item())) for i in range(count)]


def verify_buffer(buffer: TensorBuffer) -> None:
    """Synchronize and check the free-list invariants (``tensor_buffer.py:158-170``),
    and that no compressed tensor's overflow reservation failed since the last
    reset (``BufferReservationError``)."""
    buffer.check()
    previous_end = 0
    free_bytes = 0
    for start, size in _free_regions_snapshot(buffer):
        if size <= 0 or start < previous_end or start + size > buffer.capacity_bytes:
            raise RuntimeError(f"invalid free region: [{start}, {start + size})")
        if start == previous_end and previous_end != 0:
            raise RuntimeError("adjacent free regions were not coalesced")
        previous_end = start + size
        free_bytes += size
    if free_bytes > buffer.capacity_bytes:
        raise RuntimeError("free regions exceed payload capacity")


def visualize_buffer(buffer: TensorBuffer, width: int = 80) -> str:
    """Synchronize and return an ASCII map of arena usage."""
    if buffer is None:
        return ""
    if width < 8:
        raise ValueError("width must be at least 8")
    free_regions = _free_regions_snapshot(buffer)
    capacity = buffer.capacity_bytes
    free_bytes = sum(size for _, size in free_regions)
    used_bytes = capacity - free_bytes
    cells = ["#"] * width
    for start, size in free_regions:
        left = start * width // capacity
        right = ((start + size) * width + capacity - 1) // capacity
        for cell in range(left, min(width, max(left + 1, right))):
            cells[cell] = "."
    ranges = [f"[{start}, {start + size})" for start, size in free_regions]
    if len(ranges) > 8:
        ranges = [*ranges[:4], "...", *ranges[-4:]]
    return "\n".join((
        f"payload: {used_bytes}/{capacity} B used ({used_bytes / capacity:.1%}); "
        f"{len(free_regions)} free region(s)",
        f"0 [{''.join(cells)}] {capacity}",
        "# used  . free",
        f"free: {', '.join(ranges) or 'none'}",
    ))
