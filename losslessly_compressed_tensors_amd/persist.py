"""A versioned file format for ``CompressedTensor``.

The reference keeps no compressed form on disk: its checkpoints decode
compressed weights and momentum to dense tensors before ``torch.save``
(``examples/nanogpt/train_gpt_lct.py:280-286, 305-312``).  This module stores
the compressed record itself, so a checkpoint stays at the compressed size and
reloads without re-encoding.

Format ``lct-v1`` is a safetensors container (named tensors plus string
metadata, readable without executing anything from the file):

* metadata ``format`` = ``"lct-v1"``, ``layout`` (``"compressed"`` or ``"raw"``),
  ``shape`` (JSON list), ``family``, ``param``, ``mean``, ``zero_prob`` (JSON,
  may be null), ``noise_level``; for the compressed layout also ``size``
  (storage elements), ``geometry`` (JSON ``[B, L, S, W]``), ``center``,
  ``overflow_count`` and ``overflow_bytes``;
* compressed layout tensors: ``payload`` int32[nb*256*W + 4], ``side``
  uint8[size], ``blocks`` int32[3*nb] (count, first entry, tail byte base per
  codec block), ``lanes`` and ``starts`` uint8[overflow_count], ``tails``
  uint8[overflow_bytes], and, when the record has them, ``decode_table``
  int32[1024] and ``sample_values`` (int16 view of the BF16 values at the
  center's sample positions);
* raw layout: ``data``, the tensor itself.

These are the reference's own storage fields (``LCT/comp_tensor.py:12-96``,
the compact overflow list of ``LCT/kernels/generic/compaction.py:3-16``), so a
record whose fields were produced by the reference's encoder loads and decodes
the same way.  A buffer-backed tensor is written in the private layout (its
entries and tails copied out of the arena); loading into a ``TensorBuffer``
reserves a region and copies them back in.
"""
from __future__ import annotations

import json
import math
from pathlib import Path
from typing import BinaryIO, Union

import numpy as np
import torch

from .codec.geometry import geometry as layout_geometry
from .comp_format import Distribution, DistType, NoiseLevel, StorageLayout
from .comp_tensor import CompressedTensor
from .compression.huffman_tables import distribution_codebook
from .tensor_buffer import TensorBuffer, check_reservation

FORMAT = "lct-v1"

PathLike = Union[str, Path]


def _distribution_metadata(d: Distribution) -> dict[str, str]:
    return {
        "family": d.family.value,
        "param": repr(float(d.param)),
        "mean": repr(float(d.mean)),
        "zero_prob": json.dumps(d.zero_prob),
        "noise_level": d.noise_level.name,
    }


def _distribution_from(meta: dict[str, str]) -> Distribution:
    return Distribution(DistType(meta["family"]), param=float(meta["param"]),
                        mean=float(meta["mean"]), noise_level=NoiseLevel[meta["noise_level"]],
                        zero_prob=json.loads(meta["zero_prob"]))


def _overflow_arrays(ct: CompressedTensor):
    """(lanes, starts, tails) of the record as exact-size host arrays."""
    count = int(ct.fallback_count.item()) if ct.fallback_count is not None else 0
    nbytes = int(ct.fallback_used.item()) if ct.fallback_used is not None else 0
    empty = torch.empty(0, dtype=torch.uint8)
    if count == 0:
        return empty, empty, empty.clone(), 0, nbytes
    if ct.fallback_descriptor is not None:
        descriptor = ct.fallback_descriptor.cpu()
        check_reservation(int(descriptor[2]), count)
        if int(descriptor[2]) != 0:
            raise ValueError("buffer-backed tensor has no overflow storage "
                             f"(allocation status {int(descriptor[2])})")
        offset = int(descriptor[0])
        region = ct.fallback_buffer[offset:offset + 2 * count + nbytes].cpu()
        return region[:count], region[count:2 * count], region[2 * count:], count, nbytes
    tails = ct.fallback_buffer[ct.fallback_base:ct.fallback_base + nbytes]
    return ct.fallback_lanes.cpu(), ct.fallback_starts.cpu(), tails.cpu(), count, nbytes


def state_of(ct: CompressedTensor) -> tuple[dict[str, torch.Tensor], dict[str, str]]:
    """The record as (host tensors, string metadata) in format ``lct-v1``.
    Synchronises with the device."""
    meta = {"format": FORMAT, "shape": json.dumps(list(ct.shape))}
    meta.update(_distribution_metadata(ct.distribution))
    if ct.layout == StorageLayout.RAW:
        meta["layout"] = "raw"
        return {"data": ct.data.detach().cpu().contiguous()}, meta
    lanes, starts, tails, count, nbytes = _overflow_arrays(ct)
    center = ct.center.item() if isinstance(ct.center, torch.Tensor) else ct.center
    meta.update({
        "layout": "compressed",
        "size": str(int(ct.size)),
        "geometry": json.dumps(list(ct.codec_geometry)),
        "center": str(int(center)),
        "overflow_count": str(count),
        "overflow_bytes": str(nbytes),
    })
    tensors = {
        "payload": ct.data.detach().cpu().contiguous(),
        "side": ct.sign_mantissa.detach().cpu().contiguous(),
        "blocks": ct.fallback_blocks.detach().cpu().contiguous(),
        "lanes": lanes.contiguous(),
        "starts": starts.contiguous(),
        "tails": tails.contiguous(),
    }
    if ct.decode_table is not None:
        tensors["decode_table"] = ct.decode_table.detach().cpu().contiguous()
    if ct.sample_values is not None:
        tensors["sample_values"] = ct.sample_values.detach().cpu().contiguous().view(torch.int16)
    return tensors, meta


def _shifted_decode(base: np.ndarray, center: int) -> np.ndarray:
    """The center-shifted decode table (``LCT/kernels/common/tables.py:102-118``):
    ``len | exponent << 8`` per entry, 0 for continuation entries."""
    base = base.astype(np.int64)
    length = base & 255
    symbol = (base >> 8) & 255
    zero_delta = (-127 - center) & 255
    delta = symbol - (symbol <= zero_delta)
    delta = np.where(delta >= 128, delta - 256, delta)
    exponent = np.where(symbol == 0, -127, delta + center)
    entry = np.where(length == 0, 0, (length | (exponent << 8)) & 0xFFFFFFFF)
    return entry.astype(np.uint32).view(np.int32)


def _validate(tensors: dict[str, torch.Tensor], meta: dict[str, str],
              distribution: Distribution, shape: tuple[int, ...]):
    """Check every field the device kernels index with before anything is
    uploaded: geometry, sizes, the per-block overflow metadata against the
    entries it describes, the center and the tables.  Returns (size, (B, L,
    S, W), count, nbytes); raises ``ValueError`` on any mismatch.  A record
    that passes cannot make a kernel read or write outside its arrays."""
    def fail(what: str):
        raise ValueError(f"corrupt {FORMAT} record: {what}")

    def tensor(name: str, dtype: torch.dtype) -> np.ndarray:
        value = tensors.get(name)
        if value is None:
            fail(f"missing field {name!r}")
        if value.dtype != dtype or value.dim() != 1:
            fail(f"field {name!r} is not a 1-D {dtype} tensor")
        return value.numpy()

    try:
        size = int(meta["size"])
        stored = tuple(int(v) for v in json.loads(meta["geometry"]))
        count = int(meta["overflow_count"])
        nbytes = int(meta["overflow_bytes"])
        center = int(meta["center"])
    except (KeyError, TypeError, ValueError) as error:
        fail(f"metadata {error}")
    if len(stored) != 4 or stored != tuple(layout_geometry(distribution)):
        fail(f"geometry {list(stored)} is not the layout of {distribution}")
    B, L, S, W = stored
    n = math.prod(shape)
    if any(d < 0 for d in shape) or size <= 0 or size % B or not size - B < n <= size:
        fail(f"{size} storage elements do not hold shape {list(shape)} in blocks of {B}")
    if not -128 <= center <= 127:
        fail(f"center {center} outside [-128, 127]")
    nb = size // B
    payload = tensor("payload", torch.int32)
    side = tensor("side", torch.uint8)
    blocks = tensor("blocks", torch.int32)
    lanes = tensor("lanes", torch.uint8)
    starts = tensor("starts", torch.uint8)
    tails = tensor("tails", torch.uint8)
    if payload.size != nb * L * W + 4 or side.size != size or blocks.size != 3 * nb:
        fail("payload, side or block metadata size does not match the geometry")
    if lanes.size != count or starts.size != count or tails.size != nbytes:
        fail("overflow entry or tail sizes do not match the counts")
    per_count = blocks[:nb].astype(np.int64)
    if np.any(per_count < 0) or np.any(per_count > L) or int(per_count.sum()) != count:
        fail("per-block overflow counts")
    first = np.concatenate(([0], np.cumsum(per_count)[:-1])) if nb else per_count
    if not np.array_equal(blocks[nb:2 * nb], first):
        fail("per-block first entries are not the scan of the counts")
    starts64 = starts.astype(np.int64)
    if np.any(starts64 >= S) or np.any(starts64 & 1):
        fail("an overflow start step is odd or past the block")
    entry_block = np.repeat(np.arange(nb), per_count)
    per_bytes = np.bincount(entry_block, weights=S - starts64, minlength=nb).astype(np.int64)
    if int(per_bytes.sum()) != nbytes:
        fail("tail bytes do not match the overflow starts")
    base = np.concatenate(([0], np.cumsum(per_bytes)[:-1])) if nb else per_bytes
    if not np.array_equal(blocks[2 * nb:], base):
        fail("per-block tail bases are not the scan of the tail bytes")
    if count > 1:
        same_block = entry_block[1:] == entry_block[:-1]
        if np.any(same_block & (lanes[1:].astype(np.int64) <= lanes[:-1])):
            fail("overflow lanes do not ascend within a block")
    table = tensors.get("decode_table")
    if table is not None:
        expect = _shifted_decode(distribution_codebook(distribution).decode, center)
        if table.dtype != torch.int32 or not np.array_equal(table.numpy(), expect):
            fail("decode table is not the distribution's table shifted by the center")
    samples = tensors.get("sample_values")
    if samples is not None and (samples.dtype != torch.int16
                                or samples.numel() != min(n, 4096)):
        fail("sample values are not one int16 per center sample")
    return size, stored, count, nbytes


def from_state(tensors: dict[str, torch.Tensor], meta: dict[str, str],
               device: Union[str, torch.device] = "cuda",
               buffer: TensorBuffer | None = None) -> CompressedTensor:
    """Rebuild a record from ``state_of``'s output on ``device``, private or,
    with ``buffer``, with its overflow entries and tails in a reserved arena
    region.  Raises ``ValueError`` for another format, missing or inconsistent
    fields, or an arena without room."""
    if meta.get("format") != FORMAT:
        raise ValueError(f"not an {FORMAT} record (format={meta.get('format')!r})")
    device = torch.device(device)
    try:
        shape = tuple(int(d) for d in json.loads(meta["shape"]))
        distribution = _distribution_from(meta)
    except (KeyError, TypeError, ValueError) as error:
        raise ValueError(f"corrupt {FORMAT} record: metadata {error}") from None
    if meta["layout"] == "raw":
        data = tensors["data"].to(device)
        return CompressedTensor(data, data.numel(), distribution=distribution, shape=shape,
                                layout=StorageLayout.RAW)
    if meta["layout"] != "compressed":
        raise ValueError(f"unknown layout {meta['layout']!r}")
    tensors = {name: value.cpu() for name, value in tensors.items()}
    size, (B, L, S, W), count, nbytes = _validate(tensors, meta, distribution, shape)
    payload, side, blocks = tensors["payload"], tensors["side"], tensors["blocks"]
    # One 4-entry counts array, as the encoder's host sequence allocates it
    # (memory_size() counts its 16 bytes).
    counts = torch.tensor([count, nbytes, 0, 0], dtype=torch.int32, device=device)
    decode_table = tensors.get("decode_table")
    sample_values = tensors.get("sample_values")
    common = dict(
        distribution=distribution,
        center=torch.tensor([int(meta["center"])], dtype=torch.int32, device=device),
        shape=shape, layout=StorageLayout.COMPRESSED, stream_geometry=(B, L, S, W),
        fallback_blocks=blocks.to(device), fallback_count=counts[:1], fallback_used=counts[1:2],
        decode_table=None if decode_table is None else decode_table.to(device),
        sample_values=None if sample_values is None else sample_values.to(device),
    )
    payload, side = payload.to(device), side.to(device)
    if buffer is None:
        return CompressedTensor(payload, size, side,
                                fallback_starts=tensors["starts"].to(device),
                                fallback_lanes=tensors["lanes"].to(device),
                                fallback_buffer=tensors["tails"].to(device), **common)
    if buffer.data.device != payload.device:
        raise ValueError("the buffer must be on the load device")
    allocation = buffer.allocate_with_items(counts[1:2], counts[:1], 2)
    descriptor = allocation.descriptor
    status = descriptor.cpu()
    if int(status[2]) not in (0, 2):
        raise ValueError(f"TensorBuffer reservation failed (status {int(status[2])})")
    if count:
        offset = int(status[0])
        region = torch.cat([tensors["lanes"], tensors["starts"], tensors["tails"]])
        buffer.data[offset:offset + region.numel()].copy_(region.to(device))
    return CompressedTensor(payload, size, side, fallback_buffer=buffer.data,
                            fallback_descriptor=descriptor, buffer=buffer, **common)


def save_compressed(ct: CompressedTensor, path: Union[PathLike, BinaryIO]) -> None:
    """Write ``ct`` to ``path`` (a file name or a binary file object)."""
    from safetensors.torch import save

    tensors, meta = state_of(ct)
    blob = save(tensors, metadata=meta)
    if hasattr(path, "write"):
        path.write(blob)
    else:
        Path(path).write_bytes(blob)


def load_compressed(path: Union[PathLike, BinaryIO], device: Union[str, torch.device] = "cuda",
                    buffer: TensorBuffer | None = None) -> CompressedTensor:
    """Read a record written by ``save_compressed``."""
    from safetensors.torch import load

    blob = path.read() if hasattr(path, "read") else Path(path).read_bytes()
    tensors = load(blob)
    # The string metadata sits in the container's JSON header: an 8-byte
    # little-endian length, then the header with its "__metadata__" entry.
    header_len = int.from_bytes(blob[:8], "little")
    meta = json.loads(blob[8:8 + header_len]).get("__metadata__", {})
    return from_state(tensors, meta, device=device, buffer=buffer)
