"""Probability of each centred BF16 exponent symbol under a value distribution.

Host-side model behind the codebook, restated from
``LCT/compression/probabilities.py:307-437``.  The codebook must come out
bit-identical to the reference's, and its code lengths are decided by
comparisons of sums of these probabilities, so every density below evaluates
the same floating-point expression, in the same operation order, as the
reference's density, and every bin is integrated with the same SciPy QUADPACK
call and tolerances (``probabilities.py:322-326``).  Only the arithmetic order
is shared; the structure is this module's own.
"""
from __future__ import annotations

import math
from typing import Callable

import numpy as np
from scipy.integrate import quad

Density = Callable[[float], float]

# BF16 has 8 exponent bits: raw byte 0 is zero/subnormal, 255 is inf/NaN.
_EXPONENT_LOW = -127
_EXPONENT_HIGH = 128


def _folded(base: Density, mean: float) -> Density:
    """Density of |X| for X symmetric about ``mean`` (``probabilities.py:307-319``)."""
    mean = float(mean)

    def density(value: float) -> float:
        return 0.5 * (base(abs(value - mean)) + base(abs(value + mean)))

    return density


def gaussian_density(std: float = 1.0, mean: float = 0.0) -> Density:
    """|N(mean, std^2)| density (``probabilities.py:395-406``)."""
    sigma = float(std)
    scale = 2.0 / (sigma * math.sqrt(2.0 * math.pi))

    def base(value: float) -> float:
        return scale * math.exp(-0.5 * (value / sigma) ** 2)

    return _folded(base, mean)


def laplace_density(scale: float = 1.0, mean: float = 0.0) -> Density:
    """|Laplace(mean, scale)| density (``probabilities.py:409-417``)."""
    s = float(scale)

    def base(value: float) -> float:
        return math.exp(-value / s) / s

    return _folded(base, mean)


def empirical_density(scale: float = 1.0, mean: float = 0.0) -> Density:
    """Exponential body with a power-law tail (``probabilities.py:420-437``).

    The body holds 95 % of the mass; past ``-scale*ln(0.05)`` the survival
    decays as ``x^-1.8`` (tail exponent 2.8).
    """
    s = float(scale)
    tail_mass = 0.05
    tail_power = 2.8
    knee = -s * math.log(tail_mass)
    tail_scale = tail_mass * (tail_power - 1.0) / knee

    def base(value: float) -> float:
        if value <= knee:
            return math.exp(-value / s) / s
        return tail_scale * (knee / value) ** tail_power

    return _folded(base, mean)


def gamma_density(shape: float = 0.82, scale: float = 2.43) -> Density:
    """Gamma(shape, scale) magnitude density (``probabilities.py:375-392``).

    The defaults are the reference's fixed fit to ReLU-like activations; the
    GAMMA family ignores ``param`` and ``mean`` (``huffman_tables.py:267-269``).
    """
    shape = float(shape)
    scale = float(scale)
    log_norm = shape * math.log(scale) + math.lgamma(shape)

    def density(value: float) -> float:
        value = abs(value)
        return math.exp((shape - 1.0) * math.log(value) - value / scale - log_norm)

    return density


def _bin_mass(density: Density, exponent: int) -> float:
    """Mass of the magnitude bin whose BF16 exponent is ``exponent``."""
    low = 0.0 if exponent == _EXPONENT_LOW else math.ldexp(1.0, exponent)
    high = math.inf if exponent == _EXPONENT_HIGH else math.ldexp(1.0, exponent + 1)
    if low == high:
        return 0.0
    return quad(density, low, high, epsabs=1e-12, epsrel=1e-10, limit=200)[0]


def round_half_away(value: float) -> int:
    """Round to the nearest integer, halves away from zero."""
    if value >= 0.0:
        return math.floor(value + 0.5)
    return -math.floor(-value + 0.5)


def symbol_probabilities(density: Density, zero_prob: float = 0.0) -> np.ndarray:
    """Return float64[256] probabilities indexed by codebook *table index*.

    Mirrors ``_exponent_probabilities`` (``probabilities.py:329-372``):

    * exponent ``e`` (unbiased, -127..128) gets the mass of ``[2^e, 2^(e+1))``
      (``e=-127`` covers ``[0, 2^-126)``, ``e=128`` covers ``[2^128, inf)``);
    * the masses are normalised and their mean exponent, rounded half away
      from zero, is the distribution's own centre ``c``;
    * symbol ``delta = (e - c) & 255``; an exact-zero point mass ``zero_prob``
      is blended in at ``zd = (-127 - c) & 255``;
    * table index 0 is the zero symbol, deltas below ``zd`` move up by one.
    """
    exponents = np.arange(_EXPONENT_LOW, _EXPONENT_HIGH + 1)
    by_byte = np.zeros(256, dtype=np.float64)
    for e in exponents:
        by_byte[e & 255] = _bin_mass(density, int(e))
    by_byte /= by_byte.sum()

    mean_exponent = float(np.dot(exponents, by_byte[exponents & 255]))
    centre = round_half_away(mean_exponent)

    by_delta = np.zeros(256, dtype=np.float64)
    by_delta[(exponents - centre) & 255] = by_byte[exponents & 255]
    zero_delta = (-127 - centre) & 255
    if zero_prob:
        if not 0.0 <= zero_prob <= 1.0:
            raise ValueError("zero_prob must be between 0 and 1")
        by_delta = (1.0 - zero_prob) * by_delta
        by_delta[zero_delta] += zero_prob

    table = np.zeros(256, dtype=np.float64)
    deltas = np.arange(256)
    index = np.where(deltas == zero_delta, 0,
                     np.where(deltas < zero_delta, deltas + 1, deltas))
    # Each index receives exactly one delta, so a scatter equals the sum.
    table[index] = by_delta
    return table
