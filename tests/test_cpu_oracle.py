"""Pinning the C oracle (CPU).

The oracle (``oracle/lct_oracle.c``) restates the reference's kernels; these
tests fix it by checks that do not retype its code: exhaustive round trips,
an independent bit-string writer built from the storage format
(LCT/kernels/generic/encode.py:10-169, layout.py:15-18), brute-force
overflow recounts, the memory_size closed form (LCT/comp_tensor.py:57-72),
the center sampler's closed form (LCT/kernels/common/tables.py:9-49),
exact-rational FP32-FMA / BF16-RTNE arithmetic
(LCT/kernels/generic/pointwise.py:352-363) and a Python model of the
first-fit allocator (LCT/kernels/tensor_buffer.py:37-179).
"""
from __future__ import annotations

import math
import random
from fractions import Fraction

import numpy as np
import pytest
import torch

from conftest import golden_tables

GEOMETRIES = {
    "gaussian-clean": (32768, 256, 128, 12),
    "other-clean": (65536, 256, 256, 25),
    "sparse": (65536, 256, 256, 20),
    "medium": (32768, 256, 128, 19),
    "high": (32768, 256, 128, 22),
}
TABLES = [("gaussian", 1.0, 0.0, 0.0), ("laplace", 1.0, 0.0, 0.5), ("empirical", 1.0, 0.0, 0.0)]


def _bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().reshape(-1).view(np.uint16)


def _compress(oracle, bits, geometry, table=("gaussian", 1.0, 0.0, 0.0), **kw):
    enc, dec, rare = golden_tables(*table)
    return oracle.compress(bits, geometry, enc, dec, rare, **kw)


# ---- round trips -----------------------------------------------------------


@pytest.mark.parametrize("geometry", list(GEOMETRIES), ids=list(GEOMETRIES))
@pytest.mark.parametrize("table", TABLES, ids=[t[0] for t in TABLES])
def test_every_bf16_pattern_round_trips(oracle_lib, geometry, table):
    """All 65536 BF16 bit patterns (NaN payloads, infinities, subnormals,
    signed zeros), shuffled so every stream mixes them and many overflow."""
    rng = np.random.default_rng(7)
    bits = rng.permutation(np.arange(65536, dtype=np.uint32)).astype(np.uint16)
    c = _compress(oracle_lib, bits, GEOMETRIES[geometry], table)
    assert np.array_equal(oracle_lib.decompress(c), bits)


@pytest.mark.parametrize("n", [1, 2, 255, 256, 257, 32767, 32769, 100003])
def test_ragged_sizes_round_trip(oracle_lib, n):
    gen = torch.Generator().manual_seed(n)
    bits = _bf16_bits(torch.randn(n, generator=gen))
    c = _compress(oracle_lib, bits, GEOMETRIES["gaussian-clean"])
    assert np.array_equal(oracle_lib.decompress(c), bits)


# ---- payload words, overflow and tails against a naive bit writer ----------


def _logical_index(block, step, lane, steps):
    row = block * steps + step
    return row * 256 + (lane ^ (row & 254))


def _naive_streams(bits, shifted_encode, geometry):
    """Per stream: (W payload words, first overflowing step or None, tail
    bytes), built as a bit string from the format description."""
    B, L, S, W = geometry
    n = bits.size
    nb = -(-n // B)
    exponents = (bits.astype(np.int64) >> 7) & 0xFF
    out = {}
    for block in range(nb):
        for lane in range(L):
            stream_bits, used, start = 0, 0, None
            for step in range(0, S, 2):
                pair_code, pair_len = 0, 0
                for k in (0, 1):
                    index = _logical_index(block, step + k, lane, S)
                    if index < n:
                        entry = int(shifted_encode[exponents[index]])
                        code, length = entry & 0xFFFFF, entry >> 20
                        pair_code |= code << pair_len
                        pair_len += length
                if used + pair_len > 32 * W:
                    start = step
                    break
                stream_bits |= pair_code << used
                used += pair_len
            words = [(stream_bits >> (32 * w)) & 0xFFFFFFFF for w in range(W)]
            tail = []
            if start is not None:
                for step in range(start, S):
                    index = _logical_index(block, step, lane, S)
                    e = int(exponents[index]) if index < n else 0
                    tail.append((e - 127) & 0xFF)
            out[(block, lane)] = (words, start, tail)
    return out


@pytest.mark.parametrize("geometry", ["gaussian-clean", "sparse"])
def test_payload_and_overflow_match_naive_writer(oracle_lib, geometry):
    """Half the streams carry Gaussian data, half uniformly random bits (many
    escapes), so both clean streams and overflowing streams are covered."""
    B, L, S, W = GEOMETRIES[geometry]
    n = B + B // 2 + 77    # two blocks, the second partial
    gen = torch.Generator().manual_seed(3)
    bits = _bf16_bits(torch.randn(n, generator=gen))
    rng = np.random.default_rng(4)
    noisy = rng.random(n) < 0.5
    bits[noisy] = rng.integers(0, 65536, noisy.sum(), dtype=np.uint32).astype(np.uint16)
    c = _compress(oracle_lib, bits, (B, L, S, W))
    naive = _naive_streams(bits, c.shifted_encode, (B, L, S, W))
    nb, ns = c.n_blocks, c.n_blocks * L
    payload = c.encoded[: ns * W].reshape(W, ns).view(np.uint32)
    overflowing = 0
    tails = bytearray()
    lanes, starts = [], []
    for block in range(nb):
        for lane in range(L):
            words, start, tail = naive[(block, lane)]
            stream = block * L + lane
            assert payload[:, stream].tolist() == words, (block, lane)
            assert c.extra_starts[stream] == (255 if start is None else start)
            if start is not None:
                overflowing += 1
                lanes.append(lane)
                starts.append(start)
                tails += bytes(tail)
    assert overflowing > 0
    assert int(c.counts[0]) == overflowing
    assert int(c.counts[1]) == len(tails)
    assert c.lanes.tolist() == lanes and c.starts.tolist() == starts
    assert bytes(c.tail) == bytes(tails)


def test_overflow_blocks_metadata(oracle_lib):
    """fallback_blocks = {count, first entry, first tail byte} per block."""
    B, L, S, W = GEOMETRIES["gaussian-clean"]
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 65536, 3 * B, dtype=np.uint32).astype(np.uint16)
    c = _compress(oracle_lib, bits, (B, L, S, W))
    nb = c.n_blocks
    counts = c.blocks[:nb]
    firsts = c.blocks[nb:2 * nb]
    bases = c.blocks[2 * nb:]
    assert counts.sum() == c.counts[0]
    assert firsts.tolist() == np.concatenate([[0], np.cumsum(counts)[:-1]]).tolist()
    per_stream_bytes = np.where(c.extra_starts == 255, 0, S - c.extra_starts.astype(np.int64))
    block_bytes = per_stream_bytes.reshape(nb, L).sum(axis=1)
    assert bases.tolist() == np.concatenate([[0], np.cumsum(block_bytes)[:-1]]).tolist()


# ---- memory_size closed form ------------------------------------------------


def test_memory_size_closed_form_c1(oracle_lib):
    """C1: randn(1024, 1024) seed 0; 32 blocks of (32768, 256, 128, 12).
    Fixed part 393232 + 1048576 + 384 + 16 + 4 + 4096 = 1446308 bytes; each
    overflowing stream adds 2 bytes plus its tail bytes."""
    gen = torch.Generator().manual_seed(0)
    bits = _bf16_bits(torch.randn(1024, 1024, generator=gen))
    c = _compress(oracle_lib, bits, GEOMETRIES["gaussian-clean"])
    count, tails = int(c.counts[0]), int(c.counts[1])
    assert c.memory_size() == 1446308 + 2 * count + tails
    assert np.array_equal(oracle_lib.decompress(c), bits)


# ---- center sampler -----------------------------------------------------------


def _positions_closed_form(n: int) -> list[int]:
    """tables.py:24-31 restated: sample i of M = min(n, 4096) at a hashed
    offset inside region [i*n/M, (i+1)*n/M)."""
    m = min(n, 4096)
    out = []
    for i in range(m):
        start = i * n // m
        end = (i + 1) * n // m
        offset = ((i * 0x9E3779B9) & 0xFFFFFFFF) * (end - start) >> 32
        out.append(start + offset)
    return out


def _center_closed_form(exponents: np.ndarray) -> int:
    """tables.py:15-49 restated: M = min(n, 4096) hashed positions, keep
    exponents >= -120, mean rounded half away from zero, clamped."""
    total, count = 0, 0
    for position in _positions_closed_form(exponents.size):
        e = int(exponents[position])
        if e >= -120:
            total += e
            count += 1
    if count == 0:
        return 0
    mean = Fraction(total, count)
    rounded = math.floor(mean + Fraction(1, 2)) if mean >= 0 else -math.floor(-mean + Fraction(1, 2))
    return max(-128, min(127, rounded))


@pytest.mark.parametrize("n", [1, 5, 4095, 4096, 4097, 10007, 123457])
def test_center_matches_closed_form(oracle_lib, n):
    rng = np.random.default_rng(n)
    scale = np.exp2(rng.integers(-30, 30, n)).astype(np.float32)
    values = torch.from_numpy(rng.standard_normal(n).astype(np.float32) * scale)
    bits = _bf16_bits(values)
    exponents = ((bits.astype(np.int64) >> 7) & 0xFF) - 127
    assert oracle_lib.estimate_center(bits.view(np.int16)) == _center_closed_form(exponents)
    raw = ((bits.astype(np.int64) >> 7) & 0xFF).astype(np.uint8)
    assert oracle_lib.estimate_center(raw, precomputed=True) == _center_closed_form(exponents)


@pytest.mark.parametrize("n", [1, 7, 4095, 4096, 4097, 65536 * 3 + 5, 45088768])
def test_sample_positions_match_closed_form(oracle_lib, n):
    """The positions the fused pointwise sampler is checked against: one per
    region, strictly increasing, inside the tensor."""
    positions = oracle_lib.sample_positions(n)
    assert positions.tolist() == _positions_closed_form(n)
    m = positions.size
    regions = np.arange(m, dtype=np.int64)
    assert np.all(positions >= regions * n // m)
    assert np.all(positions < (regions + 1) * n // m)


def test_center_special_cases(oracle_lib):
    zeros = np.zeros(1000, dtype=np.int16)            # all exponents -127: none kept
    assert oracle_lib.estimate_center(zeros) == 0
    halves = _bf16_bits(torch.full((64,), 1.5))        # exponent 0
    assert oracle_lib.estimate_center(halves.view(np.int16)) == 0
    big = _bf16_bits(torch.full((64,), 2.0 ** 100))
    assert oracle_lib.estimate_center(big.view(np.int16)) == 100
    # mean exactly -0.5 rounds away from zero to -1
    mixed = _bf16_bits(torch.tensor([1.0, 0.5] * 2048))
    assert oracle_lib.estimate_center(mixed.view(np.int16)) == -1


# ---- shifted tables -----------------------------------------------------------


@pytest.mark.parametrize("center", [-128, -3, 0, 1, 17, 127])
def test_shifted_tables_map_raw_exponents(oracle_lib, center):
    """Raw exponent byte -> table index: 0 for e == 0, else delta + (delta <
    zd) with delta = (e - 127 - c) & 255, zd = (-127 - c) & 255; decoding the
    code found for a byte gives that byte's unbiased exponent back."""
    enc, dec, rare = golden_tables("laplace", 1.0, 0.0, 0.0)
    shifted_encode, shifted_decode = oracle_lib.shift_tables(enc, dec, center)
    zd = (-127 - center) & 255
    for e in range(256):
        if e == 0:
            index = 0
        else:
            delta = (e - 127 - center) & 255
            index = delta + (1 if delta < zd else 0)
        assert shifted_encode[e] == enc[index]
        code, length = int(shifted_encode[e]) & 0xFFFFF, int(shifted_encode[e]) >> 20
        entry = int(shifted_decode[code & 1023])
        if length <= 8 and entry & 255:
            assert entry & 255 == length
            assert ((entry >> 8) + 127) & 255 == e
        else:
            assert length == rare + 8


# ---- swizzle ------------------------------------------------------------------


def test_side_bytes_follow_the_swizzle(oracle_lib):
    """Side byte at storage (block k, step t, lane l) is that of logical
    element (k*S + t)*256 + (l ^ ((k*S + t) & 254)); the map is a bijection."""
    B, L, S, W = GEOMETRIES["gaussian-clean"]
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 65536, 2 * B, dtype=np.uint32).astype(np.uint16)
    c = _compress(oracle_lib, bits, (B, L, S, W))
    rows = np.arange(2 * S)[:, None]
    lanes = np.arange(L)[None, :]
    logical = (rows * 256 + (lanes ^ (rows & 254))).reshape(-1)
    assert np.array_equal(np.sort(logical), np.arange(2 * B))
    expected = ((bits & 0x7F) | ((bits >> 8) & 0x80)).astype(np.uint8)[logical]
    assert np.array_equal(c.side, expected)


# ---- pointwise arithmetic -------------------------------------------------------


def _bf16_value(bits: int) -> Fraction | None:
    sign = -1 if bits & 0x8000 else 1
    e = (bits >> 7) & 0xFF
    m = bits & 0x7F
    if e == 0xFF:
        return None
    if e == 0:
        return sign * Fraction(m, 1 << 7) * Fraction(1, 1 << 126)
    return sign * (1 + Fraction(m, 128)) * (Fraction(2) ** (e - 127))


def _round_to(value: Fraction, mant_bits: int, min_exp: int, max_exp: int):
    """Round an exact rational to a binary float with ``mant_bits`` stored
    mantissa bits, ties to even; returns a Fraction or +-inf."""
    if value == 0:
        return Fraction(0)
    sign = -1 if value < 0 else 1
    a = abs(value)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, min_exp)
    ulp = Fraction(2) ** (e - mant_bits)
    q, r = divmod(a, ulp)
    q = int(q)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    result = q * ulp
    if result >= Fraction(2) ** (max_exp + 1):
        return sign * math.inf
    return sign * result


def _to_f32(v):
    return _round_to(v, 23, -126, 127)


def _to_bf16_bits(v) -> int:
    if v == math.inf or v == -math.inf:
        return 0x7F80 if v > 0 else 0xFF80
    r = _round_to(v, 7, -126, 127)
    if r == math.inf or r == -math.inf:
        return 0x7F80 if r > 0 else 0xFF80
    return int(torch.tensor(float(r), dtype=torch.float64).to(torch.bfloat16)
               .view(torch.int16).item()) & 0xFFFF


def _finite_bf16(rng, count):
    out = []
    while len(out) < count:
        b = int(rng.integers(0, 65536))
        if ((b >> 7) & 0xFF) not in (0xFF,) and ((b >> 7) & 0xFF) > 90 and ((b >> 7) & 0xFF) < 170:
            out.append(b)
    return out


def test_f32_to_bf16_is_round_to_nearest_even(oracle_lib):
    rng = np.random.default_rng(1)
    values = np.concatenate([
        rng.standard_normal(4000).astype(np.float32),
        # exact ties: bf16 value + half an ulp, both parities
        (np.arange(1, 2000, dtype=np.float32) * np.float32(1.0 / 128) + np.float32(1 / 256.0)),
        np.array([0.0, -0.0, 1e-40, -1e-40, 3.4e38, -3.4e38, np.inf, -np.inf], np.float32),
    ])
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle_lib.f32_to_bf16(float(v)) for v in values], dtype=np.uint16)
    assert np.array_equal(got, expected)
    assert (oracle_lib.f32_to_bf16(float("nan")) & 0x7F80) == 0x7F80


def _cancellation_pairs(alpha: float, limit: int):
    """BF16 pairs (a, b) with b close to -a*alpha, where rounding a*alpha to
    FP32 before the add changes the BF16 result: exactly the cases that tell
    a fused multiply-add from a multiply then an add."""
    a = np.arange(0x3F80, 0x4000, dtype=np.uint32)                   # [1, 2)
    a_val = (a << 16).view(np.float32).astype(np.float64)
    product = a_val * np.float64(np.float32(alpha))                    # exact in f64
    near = torch.from_numpy(product).to(torch.bfloat16).view(torch.int16).numpy().astype(np.int64)
    pairs = []
    for delta in (-2, -1, 0, 1, 2):
        b = ((near + delta) & 0xFFFF) ^ 0x8000                         # -(product +- ulps)
        b_val = ((b.astype(np.uint32) << 16).view(np.float32)).astype(np.float64)
        fused = (product + b_val).astype(np.float32)                   # exact sum, one rounding
        unfused = (product.astype(np.float32) + b_val.astype(np.float32)).astype(np.float32)
        fb = torch.from_numpy(fused).to(torch.bfloat16).view(torch.int16).numpy()
        ub = torch.from_numpy(unfused).to(torch.bfloat16).view(torch.int16).numpy()
        for i in np.nonzero(fb != ub)[0][:limit]:
            pairs.append((int(a[i]), int(b[i])))
    return pairs


def test_scalar_mul_add_is_one_fma_then_rtne(oracle_lib):
    """SCALAR_MUL_ADD with alpha != 1, beta == 1 is bf16(fl32(a*alpha + b))
    with a single rounding to FP32 (fused), unlike mul-then-add."""
    rng = np.random.default_rng(2)
    alphas = [0.95, -0.5, 1.0 / 3.0, 0.999, 7.25]
    for a_bits, b_bits in zip(_finite_bf16(rng, 400), _finite_bf16(rng, 400)):
        alpha = float(np.float32(alphas[a_bits % len(alphas)]))
        exact = _bf16_value(a_bits) * Fraction(alpha) + _bf16_value(b_bits)
        got = oracle_lib.apply(oracle_lib.OP_SCALAR_MUL_ADD, a_bits, b_bits, alpha=alpha)
        assert got == _to_bf16_bits(_to_f32(exact)), (hex(a_bits), hex(b_bits), alpha)
    checked = 0
    for alpha in (float(np.float32(v)) for v in (0.95, 1.0 / 3.0, 0.999)):
        pairs = _cancellation_pairs(alpha, 40)
        checked += len(pairs)
        _check_fused(oracle_lib, alpha, pairs)
    assert checked >= 10


def _check_fused(oracle_lib, alpha, pairs):
    for a_bits, b_bits in pairs:
        a, b = _bf16_value(a_bits), _bf16_value(b_bits)
        fused = _to_bf16_bits(_to_f32(a * Fraction(alpha) + b))
        unfused = _to_bf16_bits(_to_f32(_to_f32(a * Fraction(alpha)) + b))
        assert fused != unfused
        assert oracle_lib.apply(oracle_lib.OP_SCALAR_MUL_ADD, a_bits, b_bits,
                                alpha=alpha) == fused, (hex(a_bits), hex(b_bits))


@pytest.mark.parametrize("op", ["add", "multiply"])
def test_add_and_multiply_are_correctly_rounded(oracle_lib, op):
    rng = np.random.default_rng(3)
    code = oracle_lib.OP_ADD if op == "add" else oracle_lib.OP_MULTIPLY
    for a_bits, b_bits in zip(_finite_bf16(rng, 800), _finite_bf16(rng, 800)):
        a, b = _bf16_value(a_bits), _bf16_value(b_bits)
        exact = a + b if op == "add" else a * b
        assert oracle_lib.apply(code, a_bits, b_bits) == _to_bf16_bits(exact)


def test_scalar_mul_add_flag_forms(oracle_lib):
    """alpha_is_one / beta_is_one select fma(a, alpha, b), fma(a, alpha,
    fl(b*beta)), fma(b, beta, a) and a + b (pointwise.py:352-363)."""
    rng = np.random.default_rng(9)
    alpha, beta = float(np.float32(0.7)), float(np.float32(-1.3))
    for a_bits, b_bits in zip(_finite_bf16(rng, 300), _finite_bf16(rng, 300)):
        a, b = _bf16_value(a_bits), _bf16_value(b_bits)
        fa, fb = Fraction(alpha), Fraction(beta)
        cases = [
            (False, False, _to_f32(a * fa + _to_f32(b * fb))),
            (True, False, _to_f32(b * fb + a)),
            (True, True, _to_f32(a + b)),
        ]
        for alpha_is_one, beta_is_one, value in cases:
            got = oracle_lib.apply(oracle_lib.OP_SCALAR_MUL_ADD, a_bits, b_bits, alpha=alpha,
                                   beta=beta, alpha_is_one=alpha_is_one, beta_is_one=beta_is_one)
            assert got == _to_bf16_bits(value), (alpha_is_one, beta_is_one)


# ---- allocator ------------------------------------------------------------------


class _FreeListModel:
    """First-fit free list with coalescing and a region cap, statuses as the
    reference's allocator kernels report them."""

    def __init__(self, capacity, regions, generation):
        self.regions, self.free, self.generation = regions, [(0, capacity)], generation

    def allocate(self, request):
        size = (request + 15) // 16 * 16
        if request <= 0:
            return (-1, 0, 2, self.generation)
        for i, (start, length) in enumerate(self.free):
            if length >= size:
                if length == size:
                    self.free.pop(i)
                else:
                    self.free[i] = (start + size, length - size)
                return (start, size, 0, self.generation)
        return (-1, 0, 1, self.generation)

    def release(self, descriptor):
        offset, size, status, generation = descriptor
        if status != 0 or generation != self.generation or offset < 0 or size <= 0:
            return 4
        i = sum(1 for s, _ in self.free if s < offset)
        merge_prev = i > 0 and sum(self.free[i - 1]) == offset
        merge_next = i < len(self.free) and offset + size == self.free[i][0]
        if merge_prev and merge_next:
            prev, nxt = self.free[i - 1], self.free[i]
            self.free[i - 1:i + 1] = [(prev[0], prev[1] + size + nxt[1])]
        elif merge_prev:
            self.free[i - 1] = (self.free[i - 1][0], self.free[i - 1][1] + size)
        elif merge_next:
            self.free[i] = (offset, self.free[i][1] + size)
        elif len(self.free) < self.regions:
            self.free.insert(i, (offset, size))
        else:
            return 3
        return 0


@pytest.mark.parametrize("seed", range(4))
def test_allocator_matches_free_list_model(oracle_lib, seed):
    rng = random.Random(seed)
    capacity, regions = 1 << 16, 8
    buffer = oracle_lib.Buffer(capacity, regions)
    # reset increments the generation (kernels/tensor_buffer.py:34)
    assert int(buffer.meta[2 * regions + 2]) == 1
    model = _FreeListModel(capacity, regions, 1)
    live = []
    for _ in range(400):
        if live and rng.random() < 0.45:
            descriptor = live.pop(rng.randrange(len(live)))
            before = tuple(int(v) for v in descriptor)
            status = buffer.free(descriptor)
            assert status == model.release(before)
            if status == 0:
                assert int(descriptor[2]) == 5      # marked freed
                assert buffer.free(descriptor) == 4  # double free rejected
        else:
            request = rng.choice([0, 1, 15, 16, 17, 100, 1000, 4096, 9000])
            descriptor = buffer.allocate(request)
            assert tuple(int(v) for v in descriptor) == model.allocate(request)
            if descriptor[2] == 0:
                live.append(descriptor)
        assert buffer.free_regions() == model.free
        starts = [s for s, _ in model.free]
        assert starts == sorted(starts)
        assert all(a[0] + a[1] < b[0] for a, b in zip(model.free, model.free[1:]))
    for descriptor in live:
        before = tuple(int(v) for v in descriptor)
        assert buffer.free(descriptor) == model.release(before)


def test_reset_invalidates_older_descriptors(oracle_lib):
    buffer = oracle_lib.Buffer(4096, 4)
    old = buffer.allocate(100)
    assert int(old[2]) == 0 and int(old[3]) == 1
    buffer.reset()
    assert buffer.free_regions() == [(0, 4096)]
    assert buffer.free(old) == 4
    fresh = buffer.allocate(100)
    assert int(fresh[3]) == 2 and buffer.free(fresh) == 0
    assert buffer.free_regions() == [(0, 4096)]
