"""Pinning the oracle's fused pointwise functions by composition (CPU).

``lcto_pointwise`` decodes a block and applies the operation in one pass, and
``lcto_dual`` decodes two operands and computes its FMA inline
(``oracle/lct_oracle.c``; reference ``LCT/kernels/generic/pointwise.py:14-363``
and ``LCT/kernels/generic/pointwise_scalar_dual.py:17-346``).  Each is checked
here against an independent composition of oracle functions that are pinned on
their own: the whole-tensor decoder (exhaustive round trips) followed by the
elementwise arithmetic ``lcto_apply`` (exact rational FMA/RTNE checks).  The
compressed-output policy (side bytes in storage order, exponent bytes in
logical order) must re-encode and decode to the dense result.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_tables

OPS = {"add": 0, "multiply": 1, "scalar_mul_add": 2}
# (alpha, beta, alpha_is_one, beta_is_one): the four forms of
# LCT/kernels/generic/pointwise.py:352-363.
FORMS = {
    "a*x+y": (0.95, 1.0, False, True),
    "a*x+b*y": (-0.5, 3.0, False, False),
    "x+b*y": (1.0, -0.01, True, False),
    "x+y": (1.0, 1.0, True, True),
}
# Geometry and codebook pairs: GAUSSIAN CLEAN, a 256-step layout with the
# Laplace half-zero codebook, MEDIUM.
LAYOUTS = {
    "gaussian-clean": ((32768, 256, 128, 12), ("gaussian", 1.0, 0.0, 0.0)),
    "sparse": ((65536, 256, 256, 20), ("laplace", 1.0, 0.0, 0.5)),
    "medium": ((32768, 256, 128, 19), ("empirical", 1.0, 0.0, 0.0)),
}
SIZES = [1, 777, 2 * 32768 + 5, 3 * 65536 - 1]


def _operand(n, seed, kind):
    """BF16 bits: N(0, 1) values, or every bit pattern shuffled (escapes,
    overflowing streams, NaN payloads, infinities, subnormals)."""
    rng = np.random.default_rng(seed)
    if kind == "patterns":
        return np.resize(rng.permutation(np.arange(65536, dtype=np.uint32)).astype(np.uint16), n)
    values = rng.standard_normal(n).astype(np.float32)
    bits = values.view(np.uint32)
    rounded = bits + 0x7FFF + ((bits >> 16) & 1)
    return (rounded >> 16).astype(np.uint16)


def _compress(oracle, bits, layout):
    geometry, table = LAYOUTS[layout]
    enc, dec, rare = golden_tables(*table)
    return oracle.compress(bits, geometry, enc, dec, rare), (geometry, enc, dec, rare)


def _reencode(oracle, side, exponents, codec):
    geometry, enc, dec, rare = codec
    return oracle.decompress(oracle.compress(exponents, geometry, enc, dec, rare,
                                             precomputed=True, side=side))


@pytest.mark.parametrize("layout", list(LAYOUTS))
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("kind", ["normal", "patterns"])
def test_pointwise_equals_decode_then_apply(oracle_lib, layout, n, kind):
    a_bits = _operand(n, n + 1, kind)
    b_bits = _operand(n, n + 2, "normal" if kind == "patterns" else "patterns")
    c, codec = _compress(oracle_lib, a_bits, layout)
    decoded = oracle_lib.decompress(c)
    assert np.array_equal(decoded, a_bits)
    for op_name, op in OPS.items():
        forms = FORMS.items() if op == 2 else [("-", (1.0, 1.0, False, True))]
        for form, (alpha, beta, alpha_one, beta_one) in forms:
            kw = dict(alpha=alpha, beta=beta, alpha_is_one=alpha_one, beta_is_one=beta_one)
            fused = oracle_lib.pointwise(c, b_bits, op, **kw)
            expect = oracle_lib.apply_array(op, decoded, b_bits, alpha, beta, alpha_one,
                                            beta_one)
            assert np.array_equal(fused, expect), (op_name, form)
            side, exponents = oracle_lib.pointwise(c, b_bits, op, policy=1, **kw)
            assert np.array_equal(_reencode(oracle_lib, side, exponents, codec), expect), \
                (op_name, form, "components")


@pytest.mark.parametrize("layout", list(LAYOUTS))
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("alpha", [-0.01, 0.95, 1.0, -3.5])
def test_dual_equals_fma_of_two_decodes(oracle_lib, layout, n, alpha):
    a_bits = _operand(n, 3 * n + 1, "patterns")
    b_bits = _operand(n, 3 * n + 2, "normal")
    a, codec = _compress(oracle_lib, a_bits, layout)
    b, _ = _compress(oracle_lib, b_bits, layout)
    expect = oracle_lib.apply_array(2, oracle_lib.decompress(a), oracle_lib.decompress(b),
                                    alpha, 1.0, False, True)
    assert np.array_equal(oracle_lib.dual(a, b, alpha), expect)
    side, exponents = oracle_lib.dual(a, b, alpha, policy=1)
    assert np.array_equal(_reencode(oracle_lib, side, exponents, codec), expect)


def test_composition_catches_a_planted_operand_swap(oracle_lib):
    """The check has teeth: the FMA with its operands swapped (b*alpha + a, a
    plausible mistake) differs from the dual's result."""
    n = 4096
    a, _ = _compress(oracle_lib, _operand(n, 5, "normal"), "gaussian-clean")
    b, _ = _compress(oracle_lib, _operand(n, 6, "normal"), "gaussian-clean")
    swapped = oracle_lib.apply_array(2, oracle_lib.decompress(b), oracle_lib.decompress(a),
                                     0.95, 1.0, False, True)
    assert not np.array_equal(oracle_lib.dual(a, b, 0.95), swapped)
