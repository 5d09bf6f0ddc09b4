"""Helpers for GPU parity tests: seeded CPU inputs and oracle comparisons."""
from __future__ import annotations

import numpy as np
import torch

import oracle
from losslessly_compressed_tensors_amd.compression.huffman_tables import distribution_codebook


def require_gpu():
    import pytest
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def bits_of(x: torch.Tensor) -> np.ndarray:
    return x.detach().cpu().contiguous().view(torch.int16).numpy().reshape(-1).view(np.uint16)


def oracle_compress(x: torch.Tensor, dist, buffer=None, **kw):
    """Oracle compress of a (CPU or GPU) BF16 tensor with ``dist``'s codebook."""
    book = distribution_codebook(dist)
    geometry = oracle.geometry_of(dist.family.value, dist.noise_level.name)
    return oracle.compress(bits_of(x), geometry, book.encode, book.decode, book.rare_length,
                           buffer=buffer, **kw)


def oracle_from_components(side: np.ndarray, exponents: np.ndarray, dist, buffer=None):
    """Oracle compress of precomputed components: side bytes (storage order,
    uint8[size]) and exponent bytes (logical order, uint8[n]), as the fused
    pointwise kernels hand them to the encoder."""
    book = distribution_codebook(dist)
    geometry = oracle.geometry_of(dist.family.value, dist.noise_level.name)
    return oracle.compress(np.ascontiguousarray(exponents, dtype=np.uint8), geometry,
                           book.encode, book.decode, book.rare_length, precomputed=True,
                           side=side, buffer=buffer)


def assert_matches_oracle(ct, o: "oracle.Compressed"):
    """Every written field of a GPU CompressedTensor equals the oracle's."""
    B, L, S, W = ct.codec_geometry
    ns = (ct.size // B) * L
    assert int(ct.center.item()) == o.center
    assert np.array_equal(ct.decode_table.cpu().numpy(), o.shifted_decode)
    enc = ct.data.cpu().numpy()
    assert np.array_equal(enc[: ns * W], o.encoded[: ns * W]), "payload words differ"
    assert np.array_equal(ct.sign_mantissa.cpu().numpy(), o.side), "side bytes differ"
    assert int(ct.fallback_count.item()) == int(o.counts[0])
    assert int(ct.fallback_used.item()) == int(o.counts[1])
    assert np.array_equal(ct.fallback_blocks.cpu().numpy(), o.blocks)
    if o.buffered:
        desc = ct.fallback_descriptor.cpu().numpy()
        assert np.array_equal(desc, o.descriptor)
        if desc[2] == 0:
            lo, hi = int(desc[0]), int(desc[0]) + int(o.counts[1]) + 2 * int(o.counts[0])
            arena = ct.buffer.data.cpu().numpy()
            assert np.array_equal(arena[lo:hi], o.tail[lo:hi]), "arena overflow region differs"
    else:
        assert np.array_equal(ct.fallback_lanes.cpu().numpy(), o.lanes)
        assert np.array_equal(ct.fallback_starts.cpu().numpy(), o.starts)
        assert np.array_equal(ct.fallback_buffer.cpu().numpy(), o.tail)
    assert ct.memory_size() == o.memory_size()
