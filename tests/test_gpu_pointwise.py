"""GPU parity of the fused pointwise paths against the CPU oracle.

One compressed operand with a dense one (LCT/codec/pointwise.py:213-278,
LCT/kernels/generic/pointwise.py:14-363), two compressed operands
(LCT/codec/pointwise.py:89-210, pointwise_scalar_dual.py) and the LCTTensor
in-place updates (LCT/LCTensor.py:70-99).  Dense results must equal the
oracle's bits; compressed results must equal, field by field, the oracle's
re-encode of the oracle's output components (new center included).
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import (
    assert_matches_oracle,
    bits_of,
    oracle_compress,
    oracle_from_components,
    require_gpu,
)
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
from losslessly_compressed_tensors_amd.operations import (
    a_compA_add_B,
    a_compA_add_b_B,
    a_compA_add_compB,
    compA_add_B,
    compA_mul_B,
    compress,
    decompress,
)
from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer, verify_buffer

pytestmark = pytest.mark.gpu

ALPHA = float(np.float32(0.95))
BETA = float(np.float32(-1.25))


def _gaussian(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def _patterns(seed):
    """All 65536 BF16 patterns, shuffled: escapes, overflow, NaN and inf."""
    rng = np.random.default_rng(seed)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


CASES = [
    ("gaussian", Distribution(DistType.GAUSSIAN), lambda: _gaussian((1024, 1024), 0),
     lambda: _gaussian((1024, 1024), 1, 0.5)),
    ("patterns-sparse", Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE),
     lambda: _patterns(2), lambda: _gaussian((65536,), 3)),
    ("ragged-medium", Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM),
     lambda: _gaussian((3, 33333), 4),
     lambda: torch.cat([_patterns(5), _patterns(6)])[:99999].reshape(3, 33333)),
]

# (name, op code, operation call, alpha, beta, alpha_is_one, beta_is_one)
OPS = [
    ("add", oracle.OP_ADD, lambda A, B, **kw: compA_add_B(A, B, **kw), 1.0, 1.0, False, True),
    ("mul", oracle.OP_MULTIPLY, lambda A, B, **kw: compA_mul_B(A, B, **kw), 1.0, 1.0, False,
     True),
    ("axpy", oracle.OP_SCALAR_MUL_ADD,
     lambda A, B, **kw: a_compA_add_B(A, _scalar(ALPHA), B, **kw), ALPHA, 1.0, False, True),
    ("axpy-alpha-one", oracle.OP_SCALAR_MUL_ADD,
     lambda A, B, **kw: a_compA_add_B(A, _scalar(ALPHA), B, alpha_is_one=True, **kw),
     ALPHA, 1.0, True, True),
    ("axpby", oracle.OP_SCALAR_MUL_ADD,
     lambda A, B, **kw: a_compA_add_b_B(A, _scalar(ALPHA), B, _scalar(BETA), **kw),
     ALPHA, BETA, False, False),
    ("axpby-alpha-one", oracle.OP_SCALAR_MUL_ADD,
     lambda A, B, **kw: a_compA_add_b_B(A, _scalar(ALPHA), B, _scalar(BETA),
                                        alpha_is_one=True, **kw),
     ALPHA, BETA, True, False),
]


def _scalar(value):
    return torch.tensor([value], dtype=torch.float32, device="cuda")


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("op", OPS, ids=[o[0] for o in OPS])
def test_pointwise_dense_output(case, op):
    require_gpu()
    name, dist, make_a, make_b = case
    op_name, code, call, alpha, beta, alpha_is_one, beta_is_one = op
    print(f"case pointwise dense {name} {op_name}", flush=True)
    a, b = make_a(), make_b()
    ct = compress(a.cuda(), dist)
    result = call(ct, b.cuda(), dense_output=True)
    o = oracle_compress(a, dist)
    expected = oracle.pointwise(o, bits_of(b), code, alpha, beta, alpha_is_one, beta_is_one)
    assert result.shape == a.shape and result.dtype == torch.bfloat16
    assert np.array_equal(bits_of(result), expected)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("op", [OPS[0], OPS[2], OPS[4]], ids=["add", "axpy", "axpby"])
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_pointwise_compressed_output(case, op, buffered):
    require_gpu()
    name, dist, make_a, make_b = case
    op_name, code, call, alpha, beta, alpha_is_one, beta_is_one = op
    print(f"case pointwise compressed {name} {op_name} buffered={buffered}", flush=True)
    a, b = make_a(), make_b()
    buffer = TensorBuffer(8 << 20, max_free_regions=64, device="cuda") if buffered else None
    host = oracle.Buffer(8 << 20, 64) if buffered else None
    ct = compress(a.cuda(), dist, buffer=buffer)
    o = oracle_compress(a, dist, buffer=host)
    result = call(ct, b.cuda(), dense_output=False, buffer=buffer)
    side, exponents = oracle.pointwise(o, bits_of(b), code, alpha, beta, alpha_is_one,
                                       beta_is_one, policy=1)
    expected = oracle_from_components(side, exponents, dist, buffer=host)
    assert_matches_oracle(result, expected)
    dense = oracle.pointwise(o, bits_of(b), code, alpha, beta, alpha_is_one, beta_is_one)
    assert np.array_equal(bits_of(decompress(result)), dense)
    if buffered:
        result.free()
        ct.free()
        verify_buffer(buffer)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("dense_output", [True, False], ids=["dense", "compressed"])
def test_dual_compressed_operands(case, dense_output):
    require_gpu()
    name, dist, make_a, make_b = case
    print(f"case dual {name} dense={dense_output}", flush=True)
    a, b = make_a(), make_b().reshape(make_a().shape)
    ca, cb = compress(a.cuda(), dist), compress(b.cuda(), dist)
    oa, ob = oracle_compress(a, dist), oracle_compress(b, dist)
    result = a_compA_add_compB(ca, _scalar(ALPHA), cb, dense_output=dense_output)
    dense = oracle.dual(oa, ob, ALPHA)
    if dense_output:
        assert np.array_equal(bits_of(result), dense)
    else:
        side, exponents = oracle.dual(oa, ob, ALPHA, policy=1)
        assert_matches_oracle(result, oracle_from_components(side, exponents, dist))
        assert np.array_equal(bits_of(decompress(result)), dense)


def test_dual_matches_dense_path_through_a_decode():
    """alpha*A + B with both compressed equals alpha*A + decompress(B)."""
    require_gpu()
    dist = Distribution(DistType.GAUSSIAN)
    a, b = _gaussian((777, 1001), 8), _gaussian((777, 1001), 9, 3.0)
    ca, cb = compress(a.cuda(), dist), compress(b.cuda(), dist)
    fused = a_compA_add_compB(ca, _scalar(ALPHA), cb)
    unfused = a_compA_add_B(ca, _scalar(ALPHA), decompress(cb))
    assert torch.equal(fused.view(torch.int16), unfused.view(torch.int16))


def test_lcttensor_updates_track_the_oracle():
    """mul_add_, add_ and add_comp_ on one LCTTensor, checked after each step
    against the oracle's pointwise + re-encode (buffer-backed, then freed)."""
    require_gpu()
    dist = Distribution(DistType.EMPIRICAL)
    shape = (512, 1100)
    buffer = TensorBuffer(16 << 20, max_free_regions=64, device="cuda")
    host = oracle.Buffer(16 << 20, 64)
    m0 = _gaussian(shape, 4, 1e-3)
    tensor = LCTTensor(m0.cuda(), buffer, dist)
    state = oracle_compress(m0, dist, buffer=host)
    assert_matches_oracle(tensor.x, state)
    for step in range(6):
        g = _gaussian(shape, 100 + step, 1e-2)
        print(f"case lcttensor step {step}", flush=True)
        update, update_state = None, None
        if step % 3 == 0:
            tensor.mul_add_(_scalar(ALPHA), g.cuda())
            side, exponents = oracle.pointwise(state, bits_of(g), oracle.OP_SCALAR_MUL_ADD,
                                               ALPHA, policy=1)
        elif step % 3 == 1:
            tensor.add_(g.cuda())
            side, exponents = oracle.pointwise(state, bits_of(g), oracle.OP_ADD, policy=1)
        else:
            update = LCTTensor(g.cuda(), buffer, dist)
            update_state = oracle_compress(g, dist, buffer=host)
            tensor.add_comp_(update, _scalar(ALPHA))
            side, exponents = oracle.dual(update_state, state, ALPHA, policy=1)
        # Same arena order as the GPU: the new state is reserved, then the
        # previous one released, then the temporary update.
        previous = state
        state = oracle_from_components(side, exponents, dist, buffer=host)
        host.free(previous.descriptor)
        if update is not None:
            update.free()
            host.free(update_state.descriptor)
        assert_matches_oracle(tensor.x, state)
    dense = tensor.decompress_free()
    assert np.array_equal(bits_of(dense), oracle.decompress(state))
    verify_buffer(buffer)
    host.free(state.descriptor)
    assert host.free_regions() == [(0, 16 << 20)]
