"""GPU tests of the public API's thinner corners against the CPU oracle.

* ``A_compBT`` / ``A_compB`` (LCT/operations.py:39-50): the compressed
  operand is decoded on the device and multiplied densely; the result equals
  the same dense product of the oracle's decode, and the shape checks raise.
* ``LCTTensor.__torch_dispatch__`` (LCT/LCTensor.py:30-47): ``t``,
  ``permute`` (which returns the transpose whatever the permutation, as the
  reference's does) and ``mm`` with an ``LCTTensor`` on either side.
* RAW storage (LCT/codec/encode.py:205-211): a tensor too small to gain from
  the codec, compressed with ``allow_raw=True``, keeps its dense values, and
  the pointwise ops take torch's arithmetic on them
  (LCT/codec/pointwise.py:242-261); a RAW ``B_comp`` in ``a_compA_add_compB``
  is read densely by the fused kernel (LCT/codec/pointwise.py:203-210).
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
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, StorageLayout
from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
from losslessly_compressed_tensors_amd.operations import (
    A_compB,
    A_compBT,
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
GAUSS = Distribution(DistType.GAUSSIAN)
EMPIRICAL = Distribution(DistType.EMPIRICAL)


def _gaussian(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def _scalar(value):
    return torch.tensor([value], dtype=torch.float32, device="cuda")


def _oracle_dense(x, dist):
    """The oracle's decode of the oracle's compress of ``x``, as a device BF16
    tensor of ``x``'s shape."""
    o = oracle_compress(x, dist)
    dense = oracle.decompress(o)
    return torch.from_numpy(dense.view(np.int16).copy()).view(torch.bfloat16) \
        .reshape(x.shape).cuda()


# ---- A_compBT / A_compB


@pytest.mark.parametrize("dist", [GAUSS, EMPIRICAL], ids=["gaussian", "empirical"])
def test_A_compBT_and_A_compB(dist):
    require_gpu()
    print(f"case A_compBT/A_compB {dist.family.value}", flush=True)
    a = _gaussian((192, 768), 1).cuda()
    w = _gaussian((1024, 768), 2, 0.02)
    v = _gaussian((768, 640), 3, 0.02)
    w_comp, v_comp = compress(w.cuda(), dist), compress(v.cuda(), dist)
    w_dense, v_dense = _oracle_dense(w, dist), _oracle_dense(v, dist)
    assert torch.equal(w_dense.cpu().view(torch.int16), w.view(torch.int16))
    got_bt = A_compBT(a, w_comp)
    got_b = A_compB(a, v_comp)
    # The same dense products of the oracle's decodes, bit for bit (same
    # operand layouts, so the same GEMM).
    assert torch.equal(got_bt, a @ w_dense.T)
    assert torch.equal(got_b, a @ v_dense)
    # And close to an FP32 product on the host.
    ref_bt = a.float().cpu() @ w.float().T
    ref_b = a.float().cpu() @ v.float()
    assert torch.allclose(got_bt.float().cpu(), ref_bt, rtol=2e-2, atol=2e-2)
    assert torch.allclose(got_b.float().cpu(), ref_b, rtol=2e-2, atol=2e-2)
    # A non-contiguous activation is made contiguous first.
    a_t = _gaussian((768, 192), 4).cuda().T
    assert torch.equal(A_compBT(a_t, w_comp), a_t.contiguous() @ w_dense.T)
    with pytest.raises(ValueError):
        A_compBT(a[:, :700], w_comp)
    with pytest.raises(ValueError):
        A_compB(a[:, :700], v_comp)
    with pytest.raises(ValueError):
        A_compB(a.reshape(2, 96, 768), v_comp)


# ---- LCTTensor dispatch


def test_lcttensor_t_permute_and_mm():
    require_gpu()
    print("case LCTTensor t/permute/mm", flush=True)
    w = _gaussian((384, 256), 5, 0.02)
    buffer = TensorBuffer(4 << 20, device="cuda")
    t = LCTTensor(w.cuda(), buffer, GAUSS)
    dense = _oracle_dense(w, GAUSS)
    assert isinstance(t, LCTTensor) and t.shape == (384, 256)
    assert torch.equal(t.t(), dense.T)
    assert torch.equal(t.permute(1, 0), dense.T)
    # The reference maps every permute to the transpose, the identity
    # permutation included.
    assert torch.equal(t.permute(0, 1), dense.T)
    x = _gaussian((64, 384), 6).cuda()
    y = _gaussian((256, 96), 7).cuda()
    assert torch.equal(torch.mm(x, t), x @ dense)
    assert torch.equal(torch.mm(t, y), dense @ y)
    with pytest.raises(NotImplementedError):
        torch.add(t, t)
    assert t.nbytes == t.x.memory_size() < t.dense_nbytes
    assert t.layout == "LCT compressed"
    assert torch.equal(t.decompress_free(), dense)
    verify_buffer(buffer)


# ---- RAW storage


def _raw(x, dist):
    ct = compress(x.cuda(), dist, allow_raw=True)
    assert ct.layout == StorageLayout.RAW
    return ct


def _torch_unfused(left, right, alpha):
    """``(left * alpha + right)`` with one FP32 rounding per operation, then
    BF16 (the reference's RAW scalar_mul_add, evaluated on the host)."""
    return (left.float() * alpha + right.float()).to(torch.bfloat16)


def _either(got, fused_bits, unfused):
    """Every element equals the fused (one rounding) or the unfused (two
    roundings) evaluation; torch's ``addcmul`` may contract its multiply-add."""
    g = bits_of(got)
    u = bits_of(unfused)
    ok = (g == fused_bits) | (g == u)
    assert ok.all(), f"{int((~ok).sum())} elements match neither evaluation"


# (name, public call on (A, B), expected(A bits, B bits) -> either a bit array
# (exact) or a (fused, unfused) pair)
def _ops():
    alpha, beta = _scalar(ALPHA), _scalar(BETA)

    def add(a, b):
        return oracle.apply_array(oracle.OP_ADD, bits_of(a), bits_of(b))

    def mul(a, b):
        return oracle.apply_array(oracle.OP_MULTIPLY, bits_of(a), bits_of(b))

    def axpy(a, b):
        return bits_of(_torch_unfused(a, b, ALPHA))

    def axpy_one(a, b):
        return oracle.apply_array(oracle.OP_ADD, bits_of(a), bits_of(b))

    def axpby(a, b):
        fused = oracle.apply_array(oracle.OP_SCALAR_MUL_ADD, bits_of(a), bits_of(b), ALPHA,
                                   BETA, False, False)
        unfused = (b.float() * BETA + a.float() * ALPHA).to(torch.bfloat16)
        return fused, unfused

    def axpby_one(a, b):
        fused = oracle.apply_array(oracle.OP_SCALAR_MUL_ADD, bits_of(a), bits_of(b), ALPHA,
                                   BETA, True, False)
        unfused = (a.float() + b.float() * BETA).to(torch.bfloat16)
        return fused, unfused

    return [
        ("add", lambda A, B, **kw: compA_add_B(A, B, **kw), add),
        ("mul", lambda A, B, **kw: compA_mul_B(A, B, **kw), mul),
        ("axpy", lambda A, B, **kw: a_compA_add_B(A, alpha, B, **kw), axpy),
        ("axpy-alpha-one", lambda A, B, **kw: a_compA_add_B(A, alpha, B, alpha_is_one=True,
                                                            **kw), axpy_one),
        ("axpby", lambda A, B, **kw: a_compA_add_b_B(A, alpha, B, beta, **kw), axpby),
        ("axpby-alpha-one", lambda A, B, **kw: a_compA_add_b_B(A, alpha, B, beta,
                                                               alpha_is_one=True, **kw),
         axpby_one),
    ]


OP_NAMES = ["add", "mul", "axpy", "axpy-alpha-one", "axpby", "axpby-alpha-one"]


@pytest.mark.parametrize("op_index", range(len(OP_NAMES)), ids=OP_NAMES)
@pytest.mark.parametrize("dist", [GAUSS, EMPIRICAL], ids=["gaussian", "empirical"])
def test_raw_A_pointwise(op_index, dist):
    require_gpu()
    name, call, expect = _ops()[op_index]
    print(f"case raw-A {name} {dist.family.value}", flush=True)
    a = _gaussian((97, 131), 10)
    b = _gaussian((97, 131), 11, 0.5)
    ct = _raw(a, dist)
    dense = call(ct, b.cuda())
    expected = expect(a, b)
    if isinstance(expected, tuple):
        _either(dense, *expected)
    else:
        assert np.array_equal(bits_of(dense), expected)
    # Compressed output: the dense result compressed with the result
    # distribution, every stored field as the oracle's.
    buffer = TensorBuffer(4 << 20, device="cuda")
    host = oracle.Buffer(4 << 20, 256)
    result = call(ct, b.cuda(), dense_output=False, buffer=buffer)
    assert result.layout == StorageLayout.COMPRESSED
    assert_matches_oracle(result, oracle_compress(dense.cpu(), dist, buffer=host))
    assert torch.equal(decompress(result), dense)
    result.free()
    verify_buffer(buffer)


@pytest.mark.parametrize("dense_output", [True, False], ids=["dense", "compressed"])
def test_raw_B_comp_in_the_two_operand_update(dense_output):
    """``a * compA + B_comp`` with a RAW ``B_comp``: the fused one-operand
    kernel reads B's dense values (one FP32 fma, one BF16 rounding)."""
    require_gpu()
    print(f"case raw-B dual dense={dense_output}", flush=True)
    a = _gaussian((97, 131), 12)
    b = _gaussian((97, 131), 13, 0.5)
    ca, cb = compress(a.cuda(), GAUSS), _raw(b, GAUSS)
    oa = oracle_compress(a, GAUSS)
    result = a_compA_add_compB(ca, _scalar(ALPHA), cb, dense_output=dense_output)
    if dense_output:
        expected = oracle.pointwise(oa, bits_of(b), oracle.OP_SCALAR_MUL_ADD, ALPHA)
        assert np.array_equal(bits_of(result), expected)
    else:
        side, exponents = oracle.pointwise(oa, bits_of(b), oracle.OP_SCALAR_MUL_ADD, ALPHA,
                                           policy=1)
        assert_matches_oracle(result, oracle_from_components(side, exponents, GAUSS))


def test_raw_A_in_the_two_operand_update():
    """``a * A_raw + compB``: B is decoded and torch's unfused arithmetic runs
    on A's dense values, as in the reference."""
    require_gpu()
    print("case raw-A dual", flush=True)
    a = _gaussian((97, 131), 14)
    b = _gaussian((97, 131), 15, 0.5)
    ca, cb = _raw(a, GAUSS), compress(b.cuda(), GAUSS)
    result = a_compA_add_compB(ca, _scalar(ALPHA), cb)
    assert np.array_equal(bits_of(result), bits_of(_torch_unfused(a, b, ALPHA)))


def test_raw_round_trip_and_size():
    """RAW storage decodes to its input and reports its dense size; a tensor
    large enough to gain from the codec is compressed even with allow_raw."""
    require_gpu()
    a = _gaussian((97, 131), 16)
    ct = _raw(a, GAUSS)
    assert torch.equal(decompress(ct).cpu().view(torch.int16), a.view(torch.int16))
    assert ct.memory_size() == a.numel() * 2
    big = _gaussian((256, 256), 17)
    assert compress(big.cuda(), GAUSS, allow_raw=True).layout == StorageLayout.COMPRESSED
