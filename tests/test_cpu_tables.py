"""Codebook parity with the reference (CPU).

The product's probability model and table builder
(``compression/probabilities.py``, ``compression/huffman_tables.py``) against
the golden fixtures written from the reference's own builder
(``tests/golden/make_tables.py``; LCT/compression/probabilities.py:43-158,
LCT/compression/huffman_tables.py:18-279).  Probabilities must match to the
last bit and the tables exactly.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_cases
from losslessly_compressed_tensors_amd.comp_format import Distribution, DistType, NoiseLevel
from losslessly_compressed_tensors_amd.compression import huffman_tables as ht
from losslessly_compressed_tensors_amd.compression.probabilities import symbol_probabilities

CASES = golden_cases()


def _case_id(case):
    return f"{case['family']}-{case['param']}-{case['mean']}-{case['zero_prob']}"


@pytest.mark.parametrize("case", CASES, ids=[_case_id(c) for c in CASES])
def test_probabilities_and_tables_match_reference(case):
    density = ht._density(DistType(case["family"]), case["param"], case["mean"])
    probabilities = symbol_probabilities(density, case["zero_prob"])
    expected = np.array([float.fromhex(h) for h in case["probabilities_hex"]])
    assert np.array_equal(probabilities, expected), "probability model differs"
    book = ht.build_codebook(expected)
    assert book.encode.tolist() == case["encode"]
    assert book.decode.tolist() == case["decode"]
    assert book.rare_length == case["rare_length"]


def test_distribution_codebook_uses_rounded_parameters():
    # Distribution snaps param/mean to quarters (comp_format.py:59-67), so a
    # std of 0.98 selects the (1.0, 0.0, 0.0) Gaussian codebook.
    case = next(c for c in CASES if (c["family"], c["param"], c["mean"], c["zero_prob"])
                == ("gaussian", 1.0, 0.0, 0.0))
    book = ht.distribution_codebook(Distribution(DistType.GAUSSIAN, 0.98, 0.05,
                                                 noise_level=NoiseLevel.MEDIUM))
    assert book.encode.tolist() == case["encode"]
    assert book.rare_length == case["rare_length"]


@pytest.mark.parametrize("case", CASES[:3], ids=[_case_id(c) for c in CASES[:3]])
def test_codebook_is_prefix_free_and_decodable(case):
    """Every symbol's code decodes back to that symbol through the 10-bit
    first-level table (escaped symbols: ESC, then the 8-bit index)."""
    encode = np.array(case["encode"], dtype=np.int64)
    decode = np.array(case["decode"], dtype=np.int64)
    rare = case["rare_length"]
    for symbol in range(256):
        code, length = int(encode[symbol] & 0xFFFFF), int(encode[symbol] >> 20)
        assert 1 <= length <= 16
        entry = int(decode[code & 1023])
        if entry & 255:
            assert entry & 255 == length and entry >> 8 == symbol
        else:
            assert length == rare + 8
            assert (code >> rare) & 255 == symbol
    # Kraft equality over the direct codes and the ESC code.
    direct = [int(e >> 20) for e in encode if int(e >> 20) <= 8 and int(e >> 20) != rare + 8]
    kraft = sum(2.0 ** -length for length in direct) + 2.0 ** -rare
    assert kraft == pytest.approx(1.0)
