"""GPU parity of the reference-shaped launches that the public API does not
sequence: the atomic overflow path (``dispatch.py:88-110`` with
``compact_extra(BUILD_META=False)``), the decode scatter (``dispatch.py:146-165``)
and the pointwise fallback (``dispatch.py:190-212``).

The public path fuses these into other kernels (block scan, decode overlay,
pointwise overlay).  Here each is launched in the reference's own sequence
and checked against the oracle:

* the atomic path's totals equal the oracle's; every block's entries and
  tails, wherever its atomically reserved slice lies, equal the oracle's
  slice of that block; the slices tile the entry list and the tail bytes;
  and a tensor assembled from them decodes to the input bits, private and
  buffered;
* a decode without the overlay is wrong at the overflow positions and the
  scatter makes it equal to the input;
* a pointwise launch without the overlay followed by the fallback equals the
  oracle's dense result and compressed-output components.
"""
import dataclasses

import numpy as np
import pytest
import torch

import oracle
from gpu_util import bits_of, oracle_compress, require_gpu
from losslessly_compressed_tensors_amd.codec.decode import shifted_decode_table, storage_of
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.compression.huffman_tables import get_distribution_tables
from losslessly_compressed_tensors_amd.kernels import dispatch
from losslessly_compressed_tensors_amd.kernels.dispatch import FallbackStorage
from losslessly_compressed_tensors_amd.operations import compress, decompress
from losslessly_compressed_tensors_amd.tensor_buffer import Allocation, TensorBuffer, verify_buffer

pytestmark = pytest.mark.gpu

ALPHA = float(np.float32(0.95))
BETA = float(np.float32(-1.25))


def _patterns(seed, n=65536):
    rng = np.random.default_rng(seed)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    bits = np.resize(bits, n)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def _gaussian(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


# (name, distribution, input): every case overflows some streams.
CASES = [
    ("patterns-sparse", Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE),
     lambda: _patterns(1)),
    ("patterns-ragged", Distribution(DistType.GAUSSIAN),
     lambda: _patterns(2, 5 * 32768 + 777)),
    ("patterns-many-blocks", Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM),
     lambda: _patterns(3, 700 * 32768)),
]


def _scalar(value):
    return torch.tensor([value], dtype=torch.float32, device="cuda")


def _atomic_storage(x, dist, o, buffer):
    """Run the reference's atomic overflow sequence (codec/encode.py:95-170,
    nb > 8192) on the oracle's extra starts; returns the storage and counts."""
    B, L, S, W = o.geometry
    nb = o.size // B
    ns = nb * L
    extra = torch.from_numpy(o.extra_starts.copy()).cuda()
    counts = torch.zeros(4, dtype=torch.int32, device="cuda")
    dispatch.count_bad_streams(extra, counts[0:1], counts[1:2], ns, S)
    blocks = torch.empty(3 * nb, dtype=torch.int32, device="cuda")
    if buffer is not None:
        allocation = buffer.allocate_with_items(counts[1:2], counts[0:1], 2)
        arena = buffer.data
        storage = FallbackStorage(tail=arena, count=counts[0:1], lanes=arena, starts=arena,
                                  blocks=blocks, descriptor=allocation.descriptor,
                                  allocation=allocation.descriptor)
        final_counts = counts[0:1]
    else:
        count, total = (int(v) for v in counts[:2].tolist())
        storage = FallbackStorage(
            tail=torch.empty(total, dtype=torch.uint8, device="cuda"), count=counts[2:3],
            lanes=torch.empty(count, dtype=torch.uint8, device="cuda"),
            starts=torch.empty(count, dtype=torch.uint8, device="cuda"), blocks=blocks,
            allocation=counts[2:3])
        final_counts = counts[2:3]
    dispatch.compact_bad_streams(extra, storage, final_counts, counts[2:3], counts[3:4], ns, S,
                                 nb, buffer is not None, L)
    storage.count = counts[0:1] if buffer is not None else counts[2:3]
    source = x.cuda().reshape(-1).view(torch.int16)
    dispatch.compact_extra(source, storage, nb, o.size, precomputed=False,
                           buffered=buffer is not None, logical_numel=o.n, block_symbols=B,
                           lanes=L, steps=S, extra_starts=extra, summaries=None)
    return storage, counts


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_atomic_overflow_path(case, buffered):
    require_gpu()
    name, dist, make = case
    print(f"case atomic path {name} buffered={buffered}", flush=True)
    x = make()
    o = oracle_compress(x, dist)
    assert o.counts[0] > 0
    need = int(o.counts[1]) + 2 * int(o.counts[0])
    capacity = max(8 << 20, (2 * need + 4095) // 4096 * 4096)
    buffer = TensorBuffer(capacity, max_free_regions=64, device="cuda") if buffered else None
    storage, counts = _atomic_storage(x, dist, o, buffer)
    c = counts.cpu().numpy()
    assert c[0] == o.counts[0] and c[1] == o.counts[1], "totals"
    assert c[2] == o.counts[0] and c[3] == o.counts[1], "atomic bump counters"

    B, L, S, W = o.geometry
    nb = o.size // B
    got_blocks = storage.blocks.cpu().numpy()
    assert np.array_equal(got_blocks[:nb], o.blocks[:nb]), "per-block counts"
    if buffered:
        desc = storage.descriptor.cpu().numpy()
        assert desc[2] == 0
        arena = buffer.data.cpu().numpy()
        total = int(o.counts[0])
        lanes = arena[desc[0]:desc[0] + total]
        starts = arena[desc[0] + total:desc[0] + 2 * total]
        tail = arena[desc[0] + 2 * total:desc[0] + 2 * total + int(o.counts[1])]
    else:
        lanes = storage.lanes.cpu().numpy()
        starts = storage.starts.cpu().numpy()
        tail = storage.tail.cpu().numpy()
    entry_slices, byte_slices = [], []
    for b in np.nonzero(o.blocks[:nb])[0]:
        count = int(o.blocks[b])
        first, base = int(got_blocks[nb + b]), int(got_blocks[2 * nb + b])
        o_first, o_base = int(o.blocks[nb + b]), int(o.blocks[2 * nb + b])
        nbytes = int(np.sum(S - o.starts[o_first:o_first + count].astype(np.int64)))
        assert np.array_equal(lanes[first:first + count], o.lanes[o_first:o_first + count])
        assert np.array_equal(starts[first:first + count], o.starts[o_first:o_first + count])
        assert np.array_equal(tail[base:base + nbytes], o.tail[o_base:o_base + nbytes])
        entry_slices.append((first, count))
        byte_slices.append((base, nbytes))
    for slices, total in ((entry_slices, int(o.counts[0])), (byte_slices, int(o.counts[1]))):
        covered = 0
        for start, length in sorted(slices):
            assert start == covered, "slices must tile the list without gaps or overlap"
            covered += length
        assert covered == total

    ct = compress(x.cuda(), dist)
    if buffered:
        assembled = dataclasses.replace(
            ct, fallback_buffer=buffer.data, fallback_descriptor=storage.descriptor,
            buffer=buffer, fallback_count=counts[0:1], fallback_used=counts[1:2],
            fallback_blocks=storage.blocks, fallback_lanes=None, fallback_starts=None)
    else:
        assembled = dataclasses.replace(
            ct, fallback_buffer=storage.tail, fallback_lanes=storage.lanes,
            fallback_starts=storage.starts, fallback_blocks=storage.blocks,
            fallback_count=counts[2:3], fallback_used=counts[3:4])
    assert np.array_equal(bits_of(decompress(assembled)), bits_of(x))
    if not buffered:
        # The atomic path's exact-size arrays are the oracle's sizes, so a
        # record holding them has the oracle's memory_size (ct's small arrays
        # share one allocation, so the two records' fields are not mixed).
        assert (storage.lanes.numel(), storage.starts.numel(), storage.tail.numel()) == \
            (o.lanes.size, o.starts.size, o.tail.size)
        assert ct.memory_size() == o.memory_size()
    if buffered:
        buffer.free(Allocation(storage.descriptor, buffer))
        verify_buffer(buffer)


@pytest.mark.parametrize("case", CASES[:2], ids=[c[0] for c in CASES[:2]])
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_scatter_fallback_restores_a_plain_decode(case, buffered):
    require_gpu()
    name, dist, make = case
    print(f"case scatter {name} buffered={buffered}", flush=True)
    x = make()
    buffer = TensorBuffer(8 << 20, max_free_regions=64, device="cuda") if buffered else None
    ct = compress(x.cuda(), dist, buffer=buffer)
    B, L, S, W = ct.codec_geometry
    n = ct.logical_numel
    _, _, rare = get_distribution_tables(dist, "cuda")
    out = torch.empty(n, dtype=torch.int16, device="cuda")
    dispatch.decode_kernel(ct.data, ct.sign_mantissa, out, shifted_decode_table(ct), ct.center,
                           ct.size, logical_numel=n, block_symbols=B, lanes=L, steps=S,
                           fixed_words=W, rare_length=rare, overflow=None)
    expected = bits_of(x)
    assert not np.array_equal(bits_of(out), expected), "overflow rows need the scatter"
    dispatch.scatter_fallback(storage_of(ct), ct.sign_mantissa, out, ct.size, n, B, L, S)
    assert np.array_equal(bits_of(out), expected)
    if buffered:
        ct.free()
        verify_buffer(buffer)


# (name, op code, alpha, beta, alpha_is_one, beta_is_one)
OPS = [
    ("add", oracle.OP_ADD, 1.0, 1.0, False, True),
    ("mul", oracle.OP_MULTIPLY, 1.0, 1.0, False, True),
    ("axpby", oracle.OP_SCALAR_MUL_ADD, ALPHA, BETA, False, False),
    ("bxpa", oracle.OP_SCALAR_MUL_ADD, ALPHA, BETA, True, False),
]


@pytest.mark.parametrize("case", CASES[:2], ids=[c[0] for c in CASES[:2]])
@pytest.mark.parametrize("op", OPS, ids=[o[0] for o in OPS])
@pytest.mark.parametrize("policy", [0, 1], ids=["dense", "components"])
def test_pointwise_fallback_completes_a_plain_pointwise(case, op, policy):
    require_gpu()
    name, dist, make = case
    op_name, code, alpha, beta, alpha_is_one, beta_is_one = op
    print(f"case pointwise fallback {name} {op_name} policy={policy}", flush=True)
    x = make()
    other = _gaussian((x.numel(),), 9)
    ct = compress(x.cuda(), dist)
    B, L, S, W = ct.codec_geometry
    n = ct.logical_numel
    _, _, rare = get_distribution_tables(dist, "cuda")
    scaled = code == oracle.OP_SCALAR_MUL_ADD
    flags = dict(op=code, alpha_is_one=(not scaled) or alpha_is_one,
                 beta_is_one=(not scaled) or beta_is_one)
    a_arg = None if flags["alpha_is_one"] else _scalar(alpha)
    b_arg = None if flags["beta_is_one"] else _scalar(beta)
    b = other.cuda()
    if policy == 0:
        output = torch.empty(n, dtype=torch.int16, device="cuda")
        auxiliary = output
    else:
        output = torch.empty(ct.size, dtype=torch.uint8, device="cuda")
        auxiliary = torch.empty(ct.size, dtype=torch.uint8, device="cuda")
    dispatch.pointwise_dense(ct.data, ct.sign_mantissa, b, output, auxiliary,
                             shifted_decode_table(ct), ct.size, ct.center, a_arg, b_arg,
                             rare_length=rare, logical_numel=n, block_symbols=B, lanes=L,
                             steps=S, fixed_words=W, output_policy=policy, overflow=None, **flags)
    dispatch.pointwise_fallback(storage_of(ct), ct.sign_mantissa, b, output, auxiliary, ct.size,
                                a_arg, b_arg, logical_numel=n, block_symbols=B, lanes=L,
                                steps=S, output_policy=policy, **flags)
    o = oracle_compress(x, dist)
    expected = oracle.pointwise(o, bits_of(other), code, alpha, beta, alpha_is_one, beta_is_one,
                                policy=policy)
    if policy == 0:
        assert np.array_equal(bits_of(output), expected)
    else:
        side, exponents = expected
        assert np.array_equal(output.cpu().numpy(), side)
        assert np.array_equal(auxiliary.cpu().numpy()[:n], exponents[:n])


# Two compressed operands of one geometry; the patterns overflow in both.
DUAL_CASES = [
    ("patterns-both", Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE),
     lambda: _patterns(11), lambda: _patterns(12)),
    ("gaussian-a-patterns-b-ragged", Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM),
     lambda: _gaussian((3 * 32768 + 555,), 13), lambda: _patterns(14, 3 * 32768 + 555)),
]


@pytest.mark.parametrize("case", DUAL_CASES, ids=[c[0] for c in DUAL_CASES])
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
@pytest.mark.parametrize("policy", [0, 1], ids=["dense", "components"])
def test_dual_three_launch_sequence(case, buffered, policy):
    """dual_maps_init -> dual_tables_and_maps -> dual_mapped, as
    LCT/codec/pointwise.py:88-156 sequences them, equals the oracle's dual."""
    require_gpu()
    name, dist, make_a, make_b = case
    print(f"case dual three-launch {name} buffered={buffered} policy={policy}", flush=True)
    a, b = make_a(), make_b()
    buffer = TensorBuffer(16 << 20, max_free_regions=64, device="cuda") if buffered else None
    ca, cb = compress(a.cuda(), dist, buffer=buffer), compress(b.cuda(), dist, buffer=buffer)
    B, L, S, W = ca.codec_geometry
    nb = ca.size // B
    ns = nb * L
    n = ca.logical_numel
    _, decode_table, rare = get_distribution_tables(dist, "cuda")
    maps = [torch.full((ns,), -5, dtype=torch.int32, device="cuda") for _ in range(4)]
    shifted = [torch.empty(1024, dtype=torch.int32, device="cuda") for _ in range(2)]
    dispatch.dual_maps_init(maps[0], maps[1], maps[2], maps[3], ca.fallback_count,
                            cb.fallback_count, ns, S)
    dispatch.dual_tables_and_maps(decode_table, ca.center, shifted[0], decode_table, cb.center,
                                  shifted[1], storage_of(ca), storage_of(cb), maps[0], maps[1],
                                  maps[2], maps[3], nb, lanes=L, steps=S, buffered=buffered)
    if policy == 0:
        output = torch.empty(n, dtype=torch.int16, device="cuda")
        auxiliary = output
    else:
        output = torch.empty(ca.size, dtype=torch.uint8, device="cuda")
        auxiliary = torch.empty(ca.size, dtype=torch.uint8, device="cuda")
    dispatch.dual_mapped(ca.data, ca.sign_mantissa, shifted[0], ca.center, maps[0], maps[1],
                         storage_of(ca), cb.data, cb.sign_mantissa, shifted[1], cb.center,
                         maps[2], maps[3], storage_of(cb), output, auxiliary, _scalar(ALPHA),
                         ca.size, ns, nb, rare_length=rare, logical_numel=n, buffered=buffered,
                         block_symbols=B, lanes=L, steps=S, fixed_words=W, output_policy=policy)
    assert torch.equal(shifted[0], ca.decode_table) and torch.equal(shifted[1], cb.decode_table)
    oa, ob = oracle_compress(a, dist), oracle_compress(b, dist)
    assert oa.counts[0] > 0 or ob.counts[0] > 0
    # Maps: every overflowing stream's start and tail offset, S / 0 elsewhere.
    for m_start, m_offset, o in ((maps[0], maps[1], oa), (maps[2], maps[3], ob)):
        start = np.full(ns, S, dtype=np.int64)
        offset = np.zeros(ns, dtype=np.int64)
        for blk in np.nonzero(o.blocks[:nb])[0]:
            first, base = int(o.blocks[nb + blk]), int(o.blocks[2 * nb + blk])
            local = 0
            for e in range(int(o.blocks[blk])):
                stream = blk * L + int(o.lanes[first + e])
                start[stream] = int(o.starts[first + e])
                offset[stream] = base + local
                local += S - int(o.starts[first + e])
        assert np.array_equal(m_start.cpu().numpy(), start)
        assert np.array_equal(m_offset.cpu().numpy(), offset)
    expected = oracle.dual(oa, ob, ALPHA, policy=policy)
    if policy == 0:
        assert np.array_equal(bits_of(output), expected)
    else:
        side, exponents = expected
        assert np.array_equal(output.cpu().numpy(), side)
        assert np.array_equal(auxiliary.cpu().numpy()[:n], exponents[:n])
    if buffered:
        cb.free()
        ca.free()
        verify_buffer(buffer)
