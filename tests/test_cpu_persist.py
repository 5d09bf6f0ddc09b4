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
    with pytest.raises(ValueError, match="does not match"):
        from_state(short, meta, device="cpu")


def _corruptions():
    """(name, edit of (tensors, meta)) pairs: each breaks one field a kernel
    indexes with, in a way a plausible bit flip or a foreign file would."""
    def blocks_edit(fn):
        def edit(t, m):
            b = t["blocks"].clone()
            fn(b, b.numel() // 3)
            t["blocks"] = b
        return edit

    def bump(name, index, delta):
        def edit(t, m):
            v = t[name].clone()
            v[index] = (int(v[index]) + delta) % 256 if v.dtype == torch.uint8 else v[index] + delta
            t[name] = v
        return edit

    def set_meta(key, value):
        def edit(t, m):
            m[key] = value
        return edit

    def first_overflow_block(b, nb):
        return int(torch.nonzero(b[:nb])[0])

    return [
        ("count above 256", blocks_edit(lambda b, nb: b.__setitem__(0, 300))),
        ("negative count", blocks_edit(lambda b, nb: b.__setitem__(nb - 1, -1))),
        ("count moved between blocks", blocks_edit(
            lambda b, nb: (b.__setitem__(first_overflow_block(b, nb), b[first_overflow_block(b, nb)] - 1),
                           b.__setitem__(nb - 1, b[nb - 1] + 1)))),
        ("first entry off by one", blocks_edit(lambda b, nb: b.__setitem__(nb + nb - 1, b[2 * nb - 1] + 1))),
        ("tail base off by one", blocks_edit(lambda b, nb: b.__setitem__(3 * nb - 1, b[3 * nb - 1] + 1))),
        ("start past the block", bump("starts", 0, 200)),
        ("odd start", bump("starts", 0, 1)),
        ("lanes out of order", lambda t, m: t.__setitem__("lanes", t["lanes"].flip(0))),
        ("fewer tail bytes", lambda t, m: t.__setitem__("tails", t["tails"][:-1])),
        ("overflow count", set_meta("overflow_count", "1")),
        ("overflow bytes", lambda t, m: (m.__setitem__("overflow_bytes", str(int(m["overflow_bytes"]) + 1)),
                                          t.__setitem__("tails", torch.cat((t["tails"], t["tails"][:1]))))),
        ("zero block size", set_meta("geometry", "[0, 256, 0, 12]")),
        ("foreign geometry", set_meta("geometry", "[65536, 256, 256, 24]")),
        ("too many words", set_meta("geometry", "[32768, 256, 128, 13]")),
        ("size not whole blocks", set_meta("size", "65537")),
        ("shape larger than storage", set_meta("shape", "[65536, 2]")),
        ("shape not a list of ints", set_meta("shape", '["a"]')),
        ("center out of range", set_meta("center", "300")),
        ("decode table for another center", set_meta("center", "1")),
        ("decode table entry", bump("decode_table", 5, 1)),
        ("payload words", lambda t, m: t.__setitem__("payload", t["payload"][:-1])),
        ("payload dtype", lambda t, m: t.__setitem__("payload", t["payload"].to(torch.int64))),
        ("sample values", lambda t, m: t.__setitem__("sample_values", torch.zeros(5, dtype=torch.int16))),
        ("missing blocks", lambda t, m: t.pop("blocks")),
        ("missing metadata", lambda t, m: m.pop("size")),
        ("unknown family", set_meta("family", "cauchy")),
    ]


@pytest.mark.parametrize("name,edit", _corruptions(), ids=[c[0] for c in _corruptions()])
def test_corrupt_record_is_rejected_before_upload(name, edit):
    """Every field the decoder indexes with is checked on the CPU, so a
    corrupt or crafted file raises ValueError instead of reaching a kernel
    (the uploads would fail loudly here anyway: device "meta" holds no data)."""
    bits = _patterns(65536 * 3, 4)
    ct, o = _oracle_record(bits.view(np.int16), Distribution(DistType.GAUSSIAN), (65536 * 3,))
    assert o.counts[0] > 1
    tensors, meta = state_of(ct)
    tensors["sample_values"] = torch.zeros(4096, dtype=torch.int16)
    tensors, meta = dict(tensors), dict(meta)
    from_state(dict(tensors), dict(meta), device="cpu")   # the intact record loads
    edit(tensors, meta)
    with pytest.raises(ValueError):
        from_state(tensors, meta, device="meta")
