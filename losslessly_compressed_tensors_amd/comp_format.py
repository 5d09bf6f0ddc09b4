"""Codec format selectors: distribution family, noise level, storage layout.

Same names, values and validation as ``LCT/comp_format.py:6-74``, so code
written against the reference constructs identical selectors.  ``param`` and
``mean`` are snapped to multiples of 0.25 with Python's ``round`` (ties to
even) and ``param`` is at least 0.25; ``zero_prob`` is rounded to two
decimals (``comp_format.py:65-67``).  Rounding keeps the codebook cache small.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from enum import Enum, auto


class NoiseLevel(Enum):
    """Stream geometry selector (``comp_format.py:6-10``)."""

    CLEAN = auto()   # fixed-stream Huffman layout
    MEDIUM = auto()  # larger fixed payload per stream
    HIGH = auto()    # smaller blocks, more payload per stream
    SPARSE = auto()  # 2.5 fixed bits per exponent plus overflow storage


class DistType(Enum):
    """Codebook family (``comp_format.py:13-17``)."""

    EMPIRICAL = "empirical"
    GAUSSIAN = "gaussian"
    LAPLACE = "laplace"
    GAMMA = "gamma"


class StorageLayout(Enum):
    """Whether a tensor is stored raw or Huffman-coded (``comp_format.py:20-23``)."""

    RAW = auto()
    COMPRESSED = auto()


def _snap_quarter(value: float) -> float:
    return float(round(value / 0.25) * 0.25)


@dataclass
class Distribution:
    """Codebook selector (``comp_format.py:26-74``).

    ``param`` is the value scale (Gaussian std, Laplace/empirical scale),
    ``mean`` the location, ``zero_prob`` an extra point mass at exact zero
    (``None`` means none), ``noise_level`` the stream geometry.
    """

    family: DistType = DistType.EMPIRICAL
    param: float = 1.0
    mean: float = 0.0
    noise_level: NoiseLevel = NoiseLevel.CLEAN
    zero_prob: float | None = 0.0

    def __post_init__(self):
        if not isinstance(self.family, DistType):
            raise TypeError("family must be a DistType member")
        if not isinstance(self.noise_level, NoiseLevel):
            raise TypeError("noise_level must be a NoiseLevel member")
        param = float(self.param)
        mean = float(self.mean)
        zero_prob = 0.0 if self.zero_prob is None else float(self.zero_prob)
        if not math.isfinite(param) or param <= 0.0:
            raise ValueError("distribution parameter must be finite and positive")
        if not math.isfinite(mean):
            raise ValueError("distribution mean must be finite")
        if not math.isfinite(zero_prob) or not 0.0 <= zero_prob <= 1.0:
            raise ValueError("zero_prob must be finite and between 0 and 1")
        self.param = float(max(0.25, _snap_quarter(param)))
        self.mean = _snap_quarter(mean)
        self.zero_prob = round(max(0.0, min(1.0, zero_prob)), 2)

    def __str__(self) -> str:
        label = "std" if self.family == DistType.GAUSSIAN else "scale"
        return (f"{self.family.value}/{label}={self.param}/mean={self.mean}/"
                f"{self.noise_level.name.lower()}")
