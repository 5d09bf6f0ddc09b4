"""Why the fused update kernels decode one symbol per table lookup (CPU).

A pair table indexed by the next 8 bits would let a wave skip the second,
dependent lookup of a step pair only when every one of its 64 lanes has both
codes within those 8 bits and neither escapes.  From the codebooks and data of
the C4 momentum and of a trained-scale weight, per lane most pairs fit, but the
64-lane conjunction holds for under a tenth of the wave steps, so such a table
would remove the second lookup from almost none of them.  The lengths come
from the oracle's center estimate and shifted encode table.
"""
import numpy as np
import pytest
import torch

import oracle
from losslessly_compressed_tensors_amd.codec.geometry import geometry
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.compression.huffman_tables import distribution_codebook


def _fit_rates(x: torch.Tensor, dist, bits: int, blocks: int = 16):
    book = distribution_codebook(dist)
    B, L, S, W = geometry(dist)
    values = x.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)
    center = oracle.estimate_center(values.view(np.int16))
    encode = oracle.shift_tables(book.encode, book.decode, center)[0]
    lengths = (np.asarray(encode, dtype=np.int64) >> 20) & 0xFFF
    rows = np.arange(blocks * S)[:, None]
    lanes = np.arange(L)[None, :]
    logical = rows * L + (lanes ^ (rows & 254))
    length = lengths[((values[logical] >> 7) & 255).astype(np.int64)]
    l0, l1 = length[0::2], length[1::2]
    fits = (l0 <= 8) & (l1 <= 8) & (l0 + l1 <= bits)
    lane_rate = float(fits.mean())
    wave_rate = float(fits.reshape(fits.shape[0], L // 64, 64).all(axis=2).mean())
    return lane_rate, wave_rate


@pytest.mark.parametrize("name, dist, std", [
    ("C4 momentum", Distribution(DistType.EMPIRICAL), 1e-3),
    ("weight", Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN), 0.02),
])
def test_eight_bit_pairs_rarely_fit_a_whole_wave(name, dist, std):
    x = (torch.randn(16 * 65536, generator=torch.Generator().manual_seed(4)) * std).to(torch.bfloat16)
    lane_rate, wave_rate = _fit_rates(x, dist, 8)
    assert lane_rate > 0.9, (name, lane_rate)          # most single pairs fit ...
    assert wave_rate < 0.1, (name, wave_rate)          # ... but rarely all 64 lanes at once
    _, wave_rate_12 = _fit_rates(x, dist, 12)
    assert wave_rate_12 > 0.7, (name, wave_rate_12)    # a 12-bit table would serve most steps
