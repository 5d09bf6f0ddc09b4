"""The benchmark configurations as GPU parity tests.

Inputs are drawn on the CPU with torch.Generator seeds and cast to BF16 on
the CPU, then copied to the GPU; every compressed field is compared with the
CPU oracle, and decompression must restore the input bits.
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
from losslessly_compressed_tensors_amd.operations import compress, decompress
from losslessly_compressed_tensors_amd.tensor_buffer import (
    TensorBuffer,
    _free_regions_snapshot,
    verify_buffer,
)

pytestmark = pytest.mark.gpu


def _randn(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_headline_tensor_matches_oracle(buffered):
    """The benchmark's own input: randn(16384, 8192) with CPU seed 0 in BF16
    (256 MiB), GAUSSIAN CLEAN.  Every field equals the oracle's, the ratio is
    the bench's 1.45409 and decompression restores the input."""
    require_gpu()
    print(f"case headline tensor buffered={buffered}", flush=True)
    x = _randn((16384, 8192), 0).to(torch.bfloat16)
    dist = Distribution(DistType.GAUSSIAN)
    capacity = 64 << 20
    buffer = TensorBuffer(capacity, device="cuda") if buffered else None
    ct = compress(x.cuda(), dist, buffer=buffer)
    o = oracle_compress(x, dist, buffer=oracle.Buffer(capacity, 256) if buffered else None)
    assert int(o.counts[0]) == 771, "771 streams of the headline tensor overflow"
    assert_matches_oracle(ct, o)
    if not buffered:
        assert round(2 * x.numel() / ct.memory_size(), 5) == 1.45409
    assert np.array_equal(bits_of(decompress(ct)), bits_of(x))


def test_c2_weight_medium():
    """8192x8192 from N(0, 0.02^2), seed 1; GAUSSIAN, MEDIUM layout."""
    require_gpu()
    print("case C2", flush=True)
    x = _randn((8192, 8192), 1, 0.02).to(torch.bfloat16)
    dist = Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM)
    ct = compress(x.cuda(), dist)
    assert_matches_oracle(ct, oracle_compress(x, dist))
    assert np.array_equal(bits_of(decompress(ct)), bits_of(x))


def test_c3_sparse_activation_with_outliers():
    """relu(N(0,1)) of 8x2048x4096 (seed 2), 0.1% of entries (randperm seed 3)
    scaled by 1e4; LAPLACE(1, zero_prob=0.5) SPARSE in a 64 MiB TensorBuffer;
    compress, decompress, free, and the arena's free list is whole again."""
    require_gpu()
    print("case C3", flush=True)
    z = torch.relu(_randn((8, 2048, 4096), 2))
    n = z.numel()
    idx = torch.randperm(n, generator=torch.Generator().manual_seed(3))[: n // 1000]
    z.view(-1)[idx] *= 1e4
    x = z.to(torch.bfloat16)
    assert 0.45 < (x == 0).float().mean().item() < 0.55
    dist = Distribution(DistType.LAPLACE, 1.0, zero_prob=0.5, noise_level=NoiseLevel.SPARSE)
    capacity = 64 << 20
    buffer = TensorBuffer(capacity, device="cuda")
    host = oracle.Buffer(capacity, 256)
    ct = compress(x.cuda(), dist, buffer=buffer)
    o = oracle_compress(x, dist, buffer=host)
    assert int(o.counts[0]) > 0, "the outliers must overflow some streams"
    assert_matches_oracle(ct, o)
    assert np.array_equal(bits_of(decompress(ct)), bits_of(x))
    ct.free()
    verify_buffer(buffer)
    assert _free_regions_snapshot(buffer) == [(0, capacity)]


@pytest.mark.timeout(900)
def test_c4_momentum_50_steps():
    """m0 ~ N(0, 1e-3^2) of 4096x11008 (seed 4), EMPIRICAL CLEAN; 50 steps of
    m = 0.95*m + g_t with g_t ~ N(0, 1e-2^2) (seed 100+t) through
    LCTTensor.mul_add_, every compressed field checked after every step."""
    require_gpu()
    dist = Distribution(DistType.EMPIRICAL)
    shape = (4096, 11008)
    alpha = torch.tensor([0.95], dtype=torch.float32, device="cuda")
    alpha_f32 = float(np.float32(0.95))
    m0 = _randn(shape, 4, 1e-3).to(torch.bfloat16)
    momentum = LCTTensor(m0.cuda(), None, dist)
    state = oracle_compress(m0, dist)
    assert_matches_oracle(momentum.x, state)
    for step in range(50):
        print(f"case C4 step {step}", flush=True)
        g = _randn(shape, 100 + step, 1e-2).to(torch.bfloat16)
        momentum.mul_add_(alpha, g.cuda())
        side, exponents = oracle.pointwise(state, bits_of(g), oracle.OP_SCALAR_MUL_ADD,
                                           alpha_f32, policy=1)
        state = oracle_from_components(side, exponents, dist)
        assert_matches_oracle(momentum.x, state)
    assert np.array_equal(bits_of(momentum.decompress()), oracle.decompress(state))


@pytest.mark.timeout(600)
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_more_blocks_than_one_scan_chunk(buffered):
    """9000 Gaussian-CLEAN blocks (295 M elements): the block scan runs in
    chunks of 8192 with carried totals; random bits in every 97th block put
    overflow entries on both sides of the chunk boundary."""
    require_gpu()
    print(f"case large buffered={buffered}", flush=True)
    B = 32768
    nb = 9000
    x = _randn((nb * B,), 11).to(torch.bfloat16)
    rng = np.random.default_rng(12)
    bits = x.view(torch.int16).numpy()
    for block in range(0, nb, 97):
        lo = block * B + int(rng.integers(0, B - 4096))
        bits[lo:lo + 4096] = rng.integers(-32768, 32768, 4096, dtype=np.int16)
    dist = Distribution(DistType.GAUSSIAN)
    buffer = TensorBuffer(256 << 20, device="cuda") if buffered else None
    host = oracle.Buffer(256 << 20, 256) if buffered else None
    ct = compress(x.cuda(), dist, buffer=buffer)
    o = oracle_compress(x, dist, buffer=host)
    listed = np.nonzero(o.blocks[:nb])[0]
    assert listed.min() < 8192 < listed.max()
    assert_matches_oracle(ct, o)
    assert np.array_equal(bits_of(decompress(ct)), bits_of(x))
    if buffered:
        ct.free()
        verify_buffer(buffer)
