"""The lct-v1 file format on the CPU: a record assembled from the oracle's
reference-format fields (payload, side bytes, compact overflow list) survives
save and load field for field, and the format rejects foreign or
inconsistent files."""
import io
import json

import numpy as np
import pytest
import torch

import oracle
from losslessly_compressed_tensors_amd.comp_format import (
    DistType,
    Distribution,
    NoiseLevel,
    StorageLayout,
)
from losslessly_compressed_tensors_amd.comp_tensor import CompressedTensor
from losslessly_compressed_tensors_amd.compression.huffman_tables import distribution_codebook
from losslessly_compressed_tensors_amd.persist import (
    FORMAT,
    from_state,
    load_compressed,
    save_compressed,
    state_of,
)


def _oracle_record(bits: np.ndarray, dist: Distribution, shape):
    book = distribution_codebook(dist)
    geometry = oracle.geometry_of(dist.family.value, dist.noise_level.name)
    o = oracle.compress(bits, geometry, book.encode, book.decode, book.rare_length)
    counts = torch.tensor([int(o.counts[0]), int(o.counts[1]), 0, 0], dtype=torch.int32)
    ct = CompressedTensor(
        torch.from_numpy(o.encoded.copy()), o.size, torch.from_numpy(o.side.copy()),
        fallback_starts=torch.from_numpy(o.starts.copy()),
        fallback_lanes=torch.from_numpy(o.lanes.copy()),
        fallback_buffer=torch.from_numpy(o.tail.copy()), fallback_count=counts[:1],
        fallback_used=counts[1:2], distribution=dist,
        center=torch.tensor([o.center], dtype=torch.int32), shape=tuple(shape),
        layout=StorageLayout.COMPRESSED, stream_geometry=tuple(geometry),
        fallback_blocks=torch.from_numpy(o.blocks.copy()),
        decode_table=torch.from_numpy(o.shifted_decode.copy()))
    return ct, o


def _patterns(n, seed):
    rng = np.random.default_rng(seed)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    return np.resize(bits, n)


CASES = [
    ("patterns-sparse", Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE),
     (256, 256), 1),
    ("patterns-ragged", Distribution(DistType.GAUSSIAN, zero_prob=0.02), (3, 33333), 2),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_record_survives_save_and_load(case):
    name, dist, shape, seed = case
    bits = _patterns(int(np.prod(shape)), seed)
    ct, o = _oracle_record(bits.view(np.int16), dist, shape)
    assert o.counts[0] > 0, "the case must carry overflow entries"
    blob = io.BytesIO()
    save_compressed(ct, blob)
    blob.seek(0)
    back = load_compressed(blob, device="cpu")
    assert back.shape == ct.shape and back.size == ct.size
    assert back.distribution == dist and back.codec_geometry == ct.codec_geometry
    for field in ("data", "sign_mantissa", "fallback_blocks", "fallback_lanes",
                  "fallback_starts", "fallback_buffer", "decode_table", "center",
                  "fallback_count", "fallback_used"):
        assert torch.equal(getattr(back, field), getattr(ct, field)), field
    assert back.memory_size() == ct.memory_size() == o.memory_size()
    # What the oracle decodes from the reloaded fields is the input.
    tensors, meta = state_of(back)
    assert meta["format"] == FORMAT and json.loads(meta["geometry"]) == list(o.geometry)
    o.encoded = tensors["payload"].numpy()
    o.side = tensors["side"].numpy()
    assert np.array_equal(oracle.decompress(o), bits)


def test_raw_layout_round_trip():
    data = torch.arange(77, dtype=torch.int16).view(torch.bfloat16)
    ct = CompressedTensor(data, data.numel(), distribution=Distribution(DistType.GAMMA),
                          shape=(7, 11), layout=StorageLayout.RAW)
    blob = io.BytesIO()
    save_compressed(ct, blob)
    blob.seek(0)
    back = load_compressed(blob, device="cpu")
    assert back.layout == StorageLayout.RAW and back.shape == (7, 11)
    assert torch.equal(back.data.view(torch.int16), data.view(torch.int16))


def test_foreign_and_inconsistent_records_are_rejected():
    bits = _patterns(65536, 3)
    ct, _ = _oracle_record(bits.view(np.int16), Distribution(DistType.GAUSSIAN), (65536,))
    tensors, meta = state_of(ct)
    with pytest.raises(ValueError, match="not an lct-v1"):
        from_state(tensors, dict(meta, format="lct-v0"), device="cpu")
    short = dict(tensors, side=tensors["side"][:-1])
    with pytest.raises(ValueError, match="do not match"):
        from_state(short, meta, device="cpu")
