"""Heavy overflow with several workgroups resident on every CU.

A 50304 x 768 tensor (590 codec blocks at LAPLACE CLEAN, more than two per CU)
that is 99 % exact zeros: under ``zero_prob=0.01`` the zero symbol takes 7
bits, so nearly every stream overflows at step 114 and each block's tails
(about 36 KiB) are read from HBM by the step loops.  This is the shape of a
zero-initialised projection weight compressed with the trainer's weight
codebook.  Every kernel that stores 16 bytes per lane is run here, each
result compared with the oracle bit for bit, the decoder three times.
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
from losslessly_compressed_tensors_amd.codec.decode import overlay_of, shifted_decode_table
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.compression.huffman_tables import get_distribution_tables
from losslessly_compressed_tensors_amd.kernels import dispatch
from losslessly_compressed_tensors_amd.operations import (
    a_compA_add_b_B,
    a_compA_add_compB,
    compress,
    decompress,
)
from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer, verify_buffer

pytestmark = pytest.mark.gpu

SHAPE = (50304, 768)
DIST = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN, zero_prob=0.01)
ALPHA = float(np.float32(0.95))
BETA = float(np.float32(-1.25))


def _sprinkled(seed, fraction=0.01):
    """Exact zeros with a seeded `fraction` of N(0, 1) entries."""
    g = torch.Generator().manual_seed(seed)
    n = SHAPE[0] * SHAPE[1]
    x = torch.zeros(n)
    idx = torch.randperm(n, generator=g)[: int(n * fraction)]
    x[idx] = torch.randn(idx.numel(), generator=g)
    return x.reshape(SHAPE).to(torch.bfloat16)


def _scalar(value):
    return torch.tensor([value], dtype=torch.float32, device="cuda")


@pytest.fixture(scope="module")
def operands():
    a, b = _sprinkled(0), _sprinkled(1)
    o = oracle_compress(a, DIST)
    B, L, S, W = o.geometry
    nb = a.numel() // B + 1
    assert nb >= 512, "needs more blocks than two per CU"
    assert int(o.counts[0]) > 0.9 * nb * L, "nearly every stream overflows"
    assert int(o.counts[1]) // nb > 1024, "tails per block exceed the LDS copy"
    return a, b, o


@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_decode_every_slot(operands, buffered):
    require_gpu()
    a, _, _ = operands
    print(f"case occupancy decode buffered={buffered}", flush=True)
    buffer = TensorBuffer(64 << 20, device="cuda") if buffered else None
    host = oracle.Buffer(64 << 20) if buffered else None
    ct = compress(a.cuda(), DIST, buffer=buffer)
    assert_matches_oracle(ct, oracle_compress(a, DIST, buffer=host))
    B, L, S, W = ct.codec_geometry
    _, _, rare = get_distribution_tables(DIST, "cuda")
    expected = bits_of(a)
    for fill in (0x5555, 0x1234, 0x7FFF):
        out = torch.full((ct.logical_numel,), fill, dtype=torch.int16, device="cuda")
        dispatch.decode_kernel(ct.data, ct.sign_mantissa, out, shifted_decode_table(ct),
                               ct.center, ct.size, logical_numel=ct.logical_numel,
                               block_symbols=B, lanes=L, steps=S, fixed_words=W,
                               rare_length=rare, overflow=overlay_of(ct))
        assert np.array_equal(bits_of(out), expected), f"decode differs (fill {fill:#x})"
    assert np.array_equal(bits_of(decompress(ct)), expected)
    if buffered:
        ct.free()
        verify_buffer(buffer)


@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_fused_update_every_slot(operands, buffered):
    """Single-pass compressed output (pointwise_encode_kernel) and the dense
    output of the same operation."""
    require_gpu()
    a, b, o = operands
    print(f"case occupancy fused buffered={buffered}", flush=True)
    buffer = TensorBuffer(64 << 20, device="cuda") if buffered else None
    host = oracle.Buffer(64 << 20) if buffered else None
    ct = compress(a.cuda(), DIST, buffer=buffer)
    if buffered:
        o = oracle_compress(a, DIST, buffer=host)
    result = a_compA_add_b_B(ct, _scalar(ALPHA), b.cuda(), _scalar(BETA), dense_output=False,
                             buffer=buffer)
    side, exponents = oracle.pointwise(o, bits_of(b), oracle.OP_SCALAR_MUL_ADD, ALPHA, BETA,
                                       False, False, policy=1)
    assert_matches_oracle(result, oracle_from_components(side, exponents, DIST, buffer=host))
    dense = oracle.pointwise(o, bits_of(b), oracle.OP_SCALAR_MUL_ADD, ALPHA, BETA, False, False)
    assert np.array_equal(bits_of(decompress(result)), dense)
    got = a_compA_add_b_B(ct, _scalar(ALPHA), b.cuda(), _scalar(BETA))
    assert np.array_equal(bits_of(got), dense)
    if buffered:
        result.free()
        ct.free()
        verify_buffer(buffer)


def test_two_pass_components_every_slot(operands):
    """lct_pointwise_dense with COMPRESSED_OUTPUT (16-byte side-byte stores)."""
    require_gpu()
    a, b, o = operands
    print("case occupancy two-pass components", flush=True)
    ct = compress(a.cuda(), DIST)
    B, L, S, W = ct.codec_geometry
    _, _, rare = get_distribution_tables(DIST, "cuda")
    side = torch.empty(ct.size, dtype=torch.uint8, device="cuda")
    exponents = torch.empty(ct.logical_numel, dtype=torch.uint8, device="cuda")
    dispatch.pointwise_dense(ct.data, ct.sign_mantissa, b.cuda().reshape(-1), side, exponents,
                             shifted_decode_table(ct), ct.size, ct.center, _scalar(ALPHA),
                             _scalar(BETA), output_policy=1, rare_length=rare,
                             logical_numel=ct.logical_numel, block_symbols=B, lanes=L, steps=S,
                             fixed_words=W, op=oracle.OP_SCALAR_MUL_ADD, alpha_is_one=False,
                             beta_is_one=False, overflow=overlay_of(ct))
    expect_side, expect_exponents = oracle.pointwise(o, bits_of(b), oracle.OP_SCALAR_MUL_ADD,
                                                     ALPHA, BETA, False, False, policy=1)
    assert np.array_equal(side.cpu().numpy(), expect_side)
    assert np.array_equal(exponents.cpu().numpy(), expect_exponents)


@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_dual_every_slot(operands, buffered):
    """Both operands overflow almost everywhere (dual_encode_kernel)."""
    require_gpu()
    a, b, _ = operands
    print(f"case occupancy dual buffered={buffered}", flush=True)
    buffer = TensorBuffer(128 << 20, device="cuda") if buffered else None
    host = oracle.Buffer(128 << 20) if buffered else None
    ca, cb = compress(a.cuda(), DIST, buffer=buffer), compress(b.cuda(), DIST, buffer=buffer)
    oa, ob = oracle_compress(a, DIST, buffer=host), oracle_compress(b, DIST, buffer=host)
    result = a_compA_add_compB(ca, _scalar(ALPHA), cb, dense_output=False, buffer=buffer)
    side, exponents = oracle.dual(oa, ob, ALPHA, policy=1)
    assert_matches_oracle(result, oracle_from_components(side, exponents, DIST, buffer=host))
    assert np.array_equal(bits_of(decompress(result)), oracle.dual(oa, ob, ALPHA))
    if buffered:
        for t in (result, cb, ca):
            t.free()
        verify_buffer(buffer)
