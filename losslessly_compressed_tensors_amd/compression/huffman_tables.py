"""Length-limited Huffman codebook with an optimal escape cutoff.

Host-side, built once per distribution and cached.  Restates
``LCT/compression/huffman_tables.py:18-279``:

* code lengths come from package-merge with an 8-bit length limit
  (``huffman_tables.py:18-95``), run over ``np.longdouble`` weights;
* the escape cutoff ``k`` (the ``k`` least likely table indices share one ESC
  code followed by an 8-bit literal) minimises the expected code length,
  first minimum wins (``huffman_tables.py:98-165``);
* codes are canonical in (length, symbol) order with ESC as the last symbol
  (``huffman_tables.py:168-185``) and stored bit-reversed, so the encoder can
  emit them LSB-first (``huffman_tables.py:196-242``).

The tie rules decide the lengths, so they are kept exactly: stable ascending
sort, an item placed before a package of equal weight, strict ``<`` when
comparing cut-off costs, and every sum formed in ``np.longdouble`` with the
same pairing.  The package-merge here is vectorised (``searchsorted`` merge,
counting backward pass) rather than the reference's list-walking loops; the
golden fixtures in ``tests/golden/tables.json`` pin that the results agree.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass
from functools import lru_cache

import numpy as np

from ..comp_format import DistType, Distribution
from .probabilities import (
    empirical_density,
    gamma_density,
    gaussian_density,
    laplace_density,
    symbol_probabilities,
)

# The decode table is indexed by the next FIRST_BITS bits of a stream.
FIRST_BITS = 10
FIRST_MASK = (1 << FIRST_BITS) - 1
# Length limit for direct codes and the ESC code (``huffman_tables.py:98,106``).
MAX_CODE_LENGTH = 8
# An escaped symbol is ESC followed by its 8-bit table index.
LITERAL_BITS = 8
# Encode-table packing: reversed code in the low 20 bits, length above.
ENCODE_LENGTH_SHIFT = 20


def package_merge_lengths(weights, limit: int) -> np.ndarray:
    """Optimal code lengths (each <= ``limit``) for non-negative ``weights``.

    Package-merge: level 0 is the sorted item list; each next level merges the
    items with the pairwise sums ("packages") of the level below.  The
    ``2n-2`` cheapest entries of the top level are selected and the selection
    is propagated down: every selected package selects its two children, and
    every selected item adds one bit to that symbol's length.
    """
    w = np.asarray(weights, dtype=np.longdouble)
    n = w.size
    if n == 0:
        return np.empty(0, dtype=np.int16)
    if np.any(w < 0) or not np.any(w > 0):
        raise ValueError("weights must be nonnegative and not all zero")
    if n > (1 << limit):
        raise ValueError("Too many symbols for requested maximum length")
    if n <= 2:
        return np.ones(n, dtype=np.int16)

    order = np.argsort(w, kind="stable")
    items = w[order]
    item_rank = np.arange(n)

    # package_flags[j] marks which entries of level j+1 are packages.
    package_flags = []
    level = items
    for _ in range(limit - 1):
        even = level.size & ~1
        packages = level[0:even:2] + level[1:even:2]
        # Stable merge, an item first on a tie with a package.
        item_pos = item_rank + np.searchsorted(packages, items, side="left")
        package_pos = np.arange(packages.size) + np.searchsorted(items, packages, side="right")
        merged = np.empty(n + packages.size, dtype=np.longdouble)
        merged[item_pos] = items
        merged[package_pos] = packages
        is_package = np.zeros(merged.size, dtype=bool)
        is_package[package_pos] = True
        package_flags.append(is_package)
        level = merged

    # Items appear in each level in ascending order, so the selected items of a
    # level are always the first ``selected - packages`` symbols.
    depth = np.zeros(n, dtype=np.int16)
    selected = 2 * n - 2
    for is_package in reversed(package_flags):
        prefix = is_package[:selected]
        chosen_packages = int(np.count_nonzero(prefix))
        depth[: prefix.size - chosen_packages] += 1
        selected = 2 * chosen_packages
    depth[:selected] += 1

    lengths = np.empty(n, dtype=np.int16)
    lengths[order] = depth
    return lengths


@dataclass(frozen=True)
class EscapeCode:
    """Chosen direct symbols, their lengths, and the ESC code length."""

    direct: np.ndarray        # table indices coded directly, most likely first
    escaped: np.ndarray       # table indices sent as ESC + literal
    direct_lengths: np.ndarray
    esc_length: int
    expected_bits: float


def choose_escape_cutoff(probabilities, limit: int = MAX_CODE_LENGTH) -> EscapeCode:
    """Pick the escape cutoff with the smallest expected code length.

    Cost of cutoff ``k`` (``huffman_tables.py:118-143``): the ``256-k`` most
    likely symbols plus one ESC symbol carrying the remaining tail mass are
    Huffman-coded; escaped symbols pay 8 literal bits on top of ESC.
    """
    p = np.asarray(probabilities, dtype=np.longdouble)
    p /= p.sum()
    n = p.size
    by_likelihood = np.argsort(-p, kind="stable")
    ranked = p[by_likelihood]
    tail_mass = np.zeros(n + 1, dtype=np.longdouble)
    tail_mass[1:] = np.cumsum(ranked[::-1], dtype=np.longdouble)

    best_lengths = package_merge_lengths(ranked, limit)
    best_cost = float(np.dot(ranked, best_lengths.astype(np.longdouble)))
    best_k = 0
    for k in range(1, n):
        kept = n - k
        weights = np.empty(kept + 1, dtype=np.longdouble)
        weights[:kept] = ranked[:kept]
        weights[kept] = tail_mass[k]
        lengths = package_merge_lengths(weights, limit)
        cost = float(np.dot(weights, lengths.astype(np.longdouble))
                     + LITERAL_BITS * tail_mass[k])
        if cost < best_cost:
            best_cost, best_k, best_lengths = cost, k, lengths.copy()

    if best_k == 0:
        return EscapeCode(by_likelihood, np.empty(0, dtype=np.int64),
                          best_lengths, 0, best_cost)
    kept = n - best_k
    return EscapeCode(by_likelihood[:kept], by_likelihood[kept:],
                      best_lengths[:kept], int(best_lengths[-1]), best_cost)


def canonical_codes(lengths) -> list[int]:
    """Canonical MSB-first codes, assigned in (length, symbol) order.

    Zero-length entries get no code (they only occur for an unused ESC).
    """
    lengths = [int(v) for v in lengths]
    longest = max(lengths, default=0)
    per_length = [0] * (longest + 1)
    for length in lengths:
        if length:
            per_length[length] += 1
    first = [0] * (longest + 1)
    code = 0
    for length in range(1, longest + 1):
        code = (code + per_length[length - 1]) << 1
        first[length] = code
    codes = [0] * len(lengths)
    for symbol in sorted(range(len(lengths)), key=lambda s: (lengths[s], s)):
        if lengths[symbol]:
            codes[symbol] = first[lengths[symbol]]
            first[lengths[symbol]] += 1
    return codes


def reverse_bits(value: int, width: int) -> int:
    """Reverse the low ``width`` bits of ``value``."""
    out = 0
    for _ in range(width):
        out = (out << 1) | (value & 1)
        value >>= 1
    return out


@dataclass(frozen=True)
class Codebook:
    """Encode/decode tables of one distribution, in table-index space.

    ``encode[i] = reversed(code) | length << 20``; ``decode[x]`` for a 10-bit
    stream prefix ``x`` is ``length | index << 8``, or 0 when the prefix
    starts with ESC and the escaped code is longer than 10 bits.
    """

    encode: np.ndarray   # int32[256]
    decode: np.ndarray   # int32[1024]
    rare_length: int     # ESC code length
    probabilities: np.ndarray

    def as_tuple(self):
        return self.encode, self.decode, self.rare_length


def build_codebook(probabilities) -> Codebook:
    """Tables for one probability vector (``huffman_tables.py:196-242``)."""
    choice = choose_escape_cutoff(probabilities)
    esc_symbol = len(choice.direct_lengths)
    all_lengths = list(choice.direct_lengths) + [choice.esc_length]
    codes = canonical_codes(all_lengths)

    code_of = {}
    for position, index in enumerate(choice.direct):
        code_of[int(index)] = (codes[position], int(all_lengths[position]))
    esc_code = codes[esc_symbol]
    for index in choice.escaped:
        literal = reverse_bits(int(index) & 255, LITERAL_BITS)
        code_of[int(index)] = ((esc_code << LITERAL_BITS) | literal,
                               choice.esc_length + LITERAL_BITS)

    encode = np.zeros(256, dtype=np.int32)
    decode = np.zeros(1 << FIRST_BITS, dtype=np.int32)
    for index in range(256):
        code, length = code_of[index]
        stream_order = reverse_bits(code, length)
        encode[index] = stream_order | (length << ENCODE_LENGTH_SHIFT)
        if length <= FIRST_BITS:
            entry = length | (index << 8)
            for suffix in range(1 << (FIRST_BITS - length)):
                decode[stream_order | (suffix << length)] = entry
        else:
            decode[stream_order & FIRST_MASK] = 0
    return Codebook(encode, decode, choice.esc_length,
                    np.asarray(probabilities, dtype=np.float64))


def _density(family: DistType, param: float, mean: float):
    if family == DistType.EMPIRICAL:
        return empirical_density(param, mean)
    if family == DistType.GAUSSIAN:
        return gaussian_density(param, mean)
    if family == DistType.LAPLACE:
        return laplace_density(param, mean)
    if family == DistType.GAMMA:
        return gamma_density()
    raise ValueError(f"unknown distribution family: {family!r}")


@lru_cache(maxsize=None)
def _codebook(family: DistType, param: float, mean: float, zero_prob: float) -> Codebook:
    probabilities = symbol_probabilities(_density(family, param, mean), zero_prob)
    return build_codebook(probabilities)


def distribution_codebook(dist: Distribution) -> Codebook:
    """Host tables for ``dist``; noise level does not change the codebook."""
    if not isinstance(dist, Distribution):
        raise TypeError("distribution must be a Distribution instance")
    return _codebook(dist.family, dist.param, dist.mean, dist.zero_prob)


_device_lock = threading.Lock()
_device_tables: dict = {}


def get_distribution_tables(dist: Distribution, device=None):
    """Return ``(encode int32[256], decode int32[1024], rare_length)``.

    Same contract as ``huffman_tables.py:245-279``: the two tables are device
    tensors (uploaded once per distribution and device), ``rare_length`` is
    the ESC code length.
    """
    import torch

    book = distribution_codebook(dist)
    device = torch.device(device if device is not None else "cuda")
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    key = (dist.family, dist.param, dist.mean, dist.zero_prob, str(device))
    with _device_lock:
        cached = _device_tables.get(key)
        if cached is None:
            cached = (
                torch.from_numpy(book.encode.copy()).to(device),
                torch.from_numpy(book.decode.copy()).to(device),
            )
            _device_tables[key] = cached
    return cached[0], cached[1], book.rare_length
