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
from pathlib import Path
from typing import BinaryIO, Union

import torch

from .comp_format import Distribution, DistType, NoiseLevel, StorageLayout
from .comp_tensor import CompressedTensor
from .tensor_buffer import TensorBuffer

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
    shape = tuple(json.loads(meta["shape"]))
    distribution = _distribution_from(meta)
    if meta["layout"] == "raw":
        data = tensors["data"].to(device)
        return CompressedTensor(data, data.numel(), distribution=distribution, shape=shape,
                                layout=StorageLayout.RAW)
    if meta["layout"] != "compressed":
        raise ValueError(f"unknown layout {meta['layout']!r}")
    size = int(meta["size"])
    B, L, S, W = (int(v) for v in json.loads(meta["geometry"]))
    nb = size // B
    count = int(meta["overflow_count"])
    nbytes = int(meta["overflow_bytes"])
    payload, side, blocks = tensors["payload"], tensors["side"], tensors["blocks"]
    if (size % B or payload.dtype != torch.int32 or payload.numel() != nb * L * W + 4
            or side.dtype != torch.uint8 or side.numel() != size
            or blocks.dtype != torch.int32 or blocks.numel() != 3 * nb
            or tensors["lanes"].numel() != count or tensors["starts"].numel() != count
            or tensors["tails"].numel() != nbytes):
        raise ValueError("lct-v1 record fields do not match its geometry and counts")
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
