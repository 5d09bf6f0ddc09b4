"""``CompressedTensor``: the storage record of one compressed BF16 tensor.

Field names, defaults and methods follow ``LCT/comp_tensor.py:12-96`` so code
written against the reference reads the same attributes.  ``memory_size()``
is the compressed-size metric: bytes of every distinct device allocation the
record holds (payload, side bytes, overflow metadata, counts, center and the
4 KiB shifted decode table), excluding a shared arena, plus the arena bytes
this tensor reserved.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, fields
from typing import TYPE_CHECKING, Optional, Tuple, Union

import torch

from .comp_format import Distribution, DistType, NoiseLevel, StorageLayout

if TYPE_CHECKING:
    from .tensor_buffer import TensorBuffer


@dataclass(frozen=True)
class CompressedTensor:
    data: torch.Tensor  # fixed exponent payload (or the raw tensor for RAW layout)
    size: int  # storage element count, including padding
    sign_mantissa: Optional[torch.Tensor] = None  # sign + 7 mantissa bits per element
    offsets: Optional[torch.Tensor] = None  # legacy slot, unused
    fallback_starts: Optional[torch.Tensor] = None  # first overflow step per entry (private)
    fallback_offsets: Optional[torch.Tensor] = None  # legacy slot, unused
    fallback_buffer: Optional[torch.Tensor] = None  # tail bytes (private) or the arena
    fallback_descriptor: Optional[torch.Tensor] = None  # arena allocation descriptor
    buffer: Optional["TensorBuffer"] = None
    fallback_base: int = 0
    fallback_count: Optional[torch.Tensor] = None  # total overflow entries
    fallback_used: Optional[torch.Tensor] = None  # total tail bytes
    distribution: Distribution = field(default_factory=Distribution)
    center: Union[torch.Tensor, int] = 0
    shape: Tuple[int, ...] = ()
    layout: StorageLayout = StorageLayout.RAW
    stream_geometry: Optional[Tuple[int, int, int, int]] = None
    fallback_lanes: Optional[torch.Tensor] = None  # overflow lane per entry (private)
    fallback_blocks: Optional[torch.Tensor] = None  # int32[3*nb] count/first/byte_base
    decode_table: Optional[torch.Tensor] = None  # center-shifted decode table
    # The tensor's BF16 values at the center's sample positions (uint16[min(n,
    # 4096)]), recorded when the tensor is made so that a fused update can
    # sample its result without decoding streams.  An acceleration record, not
    # part of the reference's storage record: memory_size() does not count it.
    sample_values: Optional[torch.Tensor] = None

    @property
    def codec_geometry(self) -> tuple[int, int, int, int]:
        """Stored ``(B, L, S, W)`` (``comp_tensor.py:40-55``)."""
        if self.layout == StorageLayout.COMPRESSED and self.fallback_blocks is None:
            raise ValueError(
                "legacy compressed layout: decode with the original codec and recompress")
        if self.stream_geometry is not None:
            return self.stream_geometry
        from .codec.geometry import geometry

        if (self.distribution.family == DistType.GAUSSIAN
                and self.distribution.noise_level == NoiseLevel.CLEAN):
            return 65536, 256, 256, 24
        return geometry(self.distribution)

    def _reserved_bytes(self) -> int:
        """Arena bytes of this tensor's reservation (syncs).  Raises
        ``BufferReservationError`` when the tensor has overflow entries whose
        reservation failed (no fit, lock not taken, or a compaction that did
        not complete): its overflow tails were never stored, so it cannot be
        decoded."""
        from .tensor_buffer import check_reservation

        size, status, count = (int(v) for v in torch.cat(
            (self.fallback_descriptor[1:3], self.fallback_count[:1])).tolist())
        check_reservation(status, count)
        return size

    def memory_size(self) -> int:
        """Device bytes owned by this tensor (syncs when buffer-backed)."""
        allocations: dict[tuple[torch.device, int], int] = {}
        for f in fields(self):
            value = getattr(self, f.name)
            if not isinstance(value, torch.Tensor):
                continue
            if f.name == "fallback_buffer" and self.fallback_descriptor is not None:
                continue
            if f.name == "sample_values":
                continue
            storage = value.untyped_storage()
            allocations[(value.device, storage.data_ptr())] = storage.nbytes()
        total = sum(allocations.values())
        if self.fallback_descriptor is not None:
            total += self._reserved_bytes()
        return total

    def memory_buffer_size(self) -> int:
        """Arena bytes reserved by this tensor (syncs)."""
        if self.fallback_descriptor is None:
            return 0
        return self._reserved_bytes()

    def free(self) -> None:
        """Release this tensor's arena reservation, if buffer-backed
        (``LCT/comp_tensor.py:80-86``).  Eagerly the free rides on the
        buffer's next reservation on this stream (the arena then holds what an
        immediate free would have left); under ``torch.compile`` it is the
        ``lct::tensor_buffer_free`` operator."""
        if self.fallback_descriptor is None or self.buffer is None:
            return
        from .tensor_buffer import Allocation

        if torch.compiler.is_compiling():
            self.buffer.free(Allocation(self.fallback_descriptor, self.buffer))
        else:
            self.buffer._defer_free(self.fallback_descriptor)

    @property
    def logical_numel(self) -> int:
        return math.prod(self.shape)

    @property
    def storage_numel(self) -> int:
        return self.size
