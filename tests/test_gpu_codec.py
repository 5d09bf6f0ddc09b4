"""GPU parity: compress/decompress through the C-ABI against the CPU oracle.

Every written field of the GPU CompressedTensor (center, shifted decode table,
payload words, side bytes, overflow list, tails, block metadata, descriptor,
memory_size) must equal the oracle's bit for bit, and decompression must
restore the input bits exactly.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_matches_oracle, bits_of, oracle_compress, require_gpu

pytestmark = pytest.mark.gpu

from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.operations import compress, decompress
from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer, verify_buffer


def _gaussian(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def _laplace(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    u = torch.rand(*shape, generator=g) - 0.5
    return (-scale * torch.sign(u) * torch.log1p(-2.0 * u.abs())).to(torch.bfloat16)


LAYOUTS = [
    (DistType.GAUSSIAN, NoiseLevel.CLEAN),
    (DistType.GAUSSIAN, NoiseLevel.MEDIUM),
    (DistType.LAPLACE, NoiseLevel.HIGH),
    (DistType.LAPLACE, NoiseLevel.SPARSE),
    (DistType.EMPIRICAL, NoiseLevel.CLEAN),
]


@pytest.mark.parametrize("family,noise", LAYOUTS)
@pytest.mark.parametrize("shape", [(1024, 1024), (3, 50001), (7,)])
def test_private_roundtrip_matches_oracle(family, noise, shape):
    require_gpu()
    print(f"case private {family.name} {noise.name} {shape}", flush=True)
    dist = Distribution(family, noise_level=noise)
    x = _gaussian(shape, 0) if family == DistType.GAUSSIAN else _laplace(shape, 1)
    ct = compress(x.cuda(), dist)
    o = oracle_compress(x, dist)
    assert_matches_oracle(ct, o)
    y = decompress(ct)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == tuple(shape)
    assert np.array_equal(bits_of(y), bits_of(x))


@pytest.mark.parametrize("family,noise", LAYOUTS)
def test_all_bf16_patterns_roundtrip(family, noise):
    """All 65536 bit patterns (NaNs, infs, subnormals): heavy escapes and overflow."""
    require_gpu()
    print(f"case patterns {family.name} {noise.name}", flush=True)
    rng = np.random.default_rng(7)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    dist = Distribution(family, noise_level=noise)
    ct = compress(x.cuda(), dist)
    o = oracle_compress(x, dist)
    assert o.counts[0] > 0
    assert_matches_oracle(ct, o)
    assert np.array_equal(bits_of(decompress(ct)), bits)


@pytest.mark.parametrize("family,noise", LAYOUTS)
def test_buffered_roundtrip_matches_oracle(family, noise):
    require_gpu()
    import oracle
    print(f"case buffered {family.name} {noise.name}", flush=True)
    dist = Distribution(family, noise_level=noise)
    capacity = 1 << 20
    buffer = TensorBuffer(capacity, max_free_regions=64, device="cuda")
    host = oracle.Buffer(capacity, 64)
    tensors = []
    for seed in range(3):
        rng = np.random.default_rng(seed)
        bits = rng.integers(0, 65536, size=40000 + 977 * seed, dtype=np.uint16)
        x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
        ct = compress(x.cuda(), dist, buffer=buffer)
        o = oracle_compress(x, dist, buffer=host)
        assert_matches_oracle(ct, o)
        assert np.array_equal(bits_of(decompress(ct)), bits)
        tensors.append((ct, o))
    # Free the middle one, then the rest; the free list must coalesce back.
    for index in (1, 0, 2):
        ct, o = tensors[index]
        ct.free()
        host.free(o.descriptor)
    verify_buffer(buffer)
    meta = buffer.storage[: 4 * (2 * 64 + 3)].view(torch.int32).cpu().numpy()
    assert np.array_equal(meta[:2 * 64 + 1], host.meta[:2 * 64 + 1])
    assert host.free_regions() == [(0, capacity)]


def test_c1_ratio_and_size():
    """Config 1: randn(1024,1024) seed 0, GAUSSIAN CLEAN, private."""
    require_gpu()
    x = _gaussian((1024, 1024), 0)
    ct = compress(x.cuda(), Distribution(DistType.GAUSSIAN))
    o = oracle_compress(x, Distribution(DistType.GAUSSIAN))
    assert ct.memory_size() == o.memory_size()
    assert np.array_equal(bits_of(decompress(ct)), bits_of(x))
    assert x.numel() * 2 / ct.memory_size() > 1.42


def test_unaligned_view_roundtrip():
    """A view starting 2 bytes into its storage still compresses bit-exactly."""
    require_gpu()
    base = _gaussian((300001,), 5).cuda()
    x = base[1:]
    assert x.data_ptr() % 16 != 0
    dist = Distribution(DistType.GAUSSIAN)
    ct = compress(x, dist)
    o = oracle_compress(x.cpu(), dist)
    assert_matches_oracle(ct, o)
    assert np.array_equal(bits_of(decompress(ct)), bits_of(x))


def test_large_block_count_metadata():
    """7000 codec blocks (458 MB): the prefix scan's large-LDS configuration."""
    require_gpu()
    g = torch.Generator(device="cuda").manual_seed(11)
    n = 7000 * 32768 - 12345
    x = torch.randn(n, device="cuda", generator=g).to(torch.bfloat16)
    dist = Distribution(DistType.GAUSSIAN)
    ct = compress(x, dist)
    o = oracle_compress(x.cpu(), dist)
    assert np.array_equal(ct.fallback_blocks.cpu().numpy(), o.blocks)
    assert ct.memory_size() == o.memory_size()
    assert np.array_equal(ct.fallback_lanes.cpu().numpy(), o.lanes)
    assert np.array_equal(ct.fallback_buffer.cpu().numpy(), o.tail)
    assert torch.equal(decompress(ct).view(torch.int16), x.view(torch.int16))


@pytest.mark.parametrize("mode", ["wide", "compact"])
@pytest.mark.parametrize("family,noise", LAYOUTS)
def test_both_decoders_restore_every_case(family, noise, mode):
    """lct_decode has two kernels (a 16-byte-tile one and a compact one that
    keeps 8 workgroups per CU at larger W); each, forced, restores every bit
    pattern (escapes, overflow in LDS and in HBM), a ragged last block and a
    buffered tensor, on every layout."""
    require_gpu()
    from losslessly_compressed_tensors_amd.kernels import hip
    print(f"case decoder {mode} {family.name} {noise.name}", flush=True)
    dist = Distribution(family, noise_level=noise)
    rng = np.random.default_rng(17)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    inputs = [
        torch.from_numpy(np.resize(bits, 5 * 65536 + 777).view(np.int16).copy())
        .view(torch.bfloat16),
        _gaussian((3, 50001), 2) if family == DistType.GAUSSIAN else _laplace((3, 50001), 3),
    ]
    buffer = TensorBuffer(16 << 20, device="cuda")
    hip.call("lct_set_decoder", 2 if mode == "compact" else 1)
    try:
        for x in inputs:
            for buf in (None, buffer):
                ct = compress(x.cuda(), dist, buffer=buf)
                assert np.array_equal(bits_of(decompress(ct)), bits_of(x))
                ct.free()
    finally:
        hip.call("lct_set_decoder", 0)
    verify_buffer(buffer)


def test_decode_batch_equals_single_decodes():
    """decode_batch (lct_decode_batch: up to 16 tensors per launch) restores
    every tensor bit for bit: 20 tensors (two launches) of every layout, private
    and buffered, with escapes and overflow, ragged and single-block sizes."""
    require_gpu()
    from losslessly_compressed_tensors_amd.codec.decode import decode_batch
    print("case decode batch", flush=True)
    rng = np.random.default_rng(23)
    buffer = TensorBuffer(16 << 20, device="cuda")
    inputs, tensors = [], []
    for i in range(20):
        family, noise = LAYOUTS[i % len(LAYOUTS)]
        n = int(rng.integers(1, 4 * 65536))
        if i % 3 == 0:
            bits = rng.integers(0, 65536, size=n, dtype=np.uint16)
            x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
        else:
            x = _gaussian((n,), 100 + i, 0.02)
        inputs.append(x)
        tensors.append(compress(x.cuda(), Distribution(family, noise_level=noise),
                                buffer=buffer if i % 2 else None))
    outputs = decode_batch(tensors)
    for x, ct, y in zip(inputs, tensors, outputs):
        assert y.shape == x.shape and y.dtype == torch.bfloat16
        assert np.array_equal(bits_of(y), bits_of(x))
        assert torch.equal(y.view(torch.int16), decompress(ct).view(torch.int16))
    for ct in tensors:
        ct.free()
    verify_buffer(buffer)
