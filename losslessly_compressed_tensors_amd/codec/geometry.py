"""Stream geometry of the compressed format per distribution.

``geometry(dist) -> (block_symbols B, lanes L, steps S, fixed_words W)``,
identical to ``LCT/codec/geometry.py:13-39``: a block is L=256 parallel
Huffman streams of S symbols each; each stream owns W fixed 32-bit payload
words and spills what does not fit into overflow storage.

=============================  =====  ===  ===  ==
layout                             B    L    S   W
=============================  =====  ===  ===  ==
GAUSSIAN + CLEAN               32768  256  128  12  (3 bits/symbol)
other families + CLEAN         65536  256  256  25  (800 bits/stream)
SPARSE                         65536  256  256  20  (2.5 bits/symbol)
MEDIUM                         32768  256  128  19
HIGH                           32768  256  128  22
=============================  =====  ===  ===  ==
"""
from __future__ import annotations

from ..comp_format import Distribution, DistType, NoiseLevel

LANES = 256
BLOCK_SYMBOLS = 65536
LANE_BITS = 800
GAUSSIAN_BLOCK_SYMBOLS = 32768
GAUSSIAN_LANE_BITS = 3 * (GAUSSIAN_BLOCK_SYMBOLS // LANES)


def geometry(distribution: Distribution) -> tuple[int, int, int, int]:
    """Return ``(block_symbols, lanes, steps, fixed_words)`` for new storage."""
    level = distribution.noise_level
    if level == NoiseLevel.CLEAN:
        if distribution.family == DistType.GAUSSIAN:
            block, bits = GAUSSIAN_BLOCK_SYMBOLS, GAUSSIAN_LANE_BITS
        else:
            block, bits = BLOCK_SYMBOLS, LANE_BITS
    elif level == NoiseLevel.SPARSE:
        block, bits = BLOCK_SYMBOLS, 5 * (BLOCK_SYMBOLS // LANES) // 2
    elif level == NoiseLevel.MEDIUM:
        block, bits = BLOCK_SYMBOLS // 2, LANE_BITS - 6 * 32
    elif level == NoiseLevel.HIGH:
        block, bits = BLOCK_SYMBOLS // 2, LANE_BITS - 3 * 32
    else:
        raise ValueError(f"Unknown noise level: {level}")
    return block, LANES, block // LANES, bits // 32
