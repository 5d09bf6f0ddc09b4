"""GPU parity of the one-launch buffered bookkeeping and of deferred frees.

``lct_allocate_compact`` replaces, for a shared TensorBuffer, the sequence
free(s) -> prefix scan + reservation -> compaction
(``LCT/tensor_buffer.py:121-128``, ``LCT/kernels/dispatch.py:70-85, 113-130``).
Checked here:

* on the same encoder output and the same fragmented buffer, the one launch
  with pending frees leaves the counts, descriptor, block metadata, overflow
  list, freed descriptors, free list and the whole arena byte-identical to
  ``lct_buffer_free`` + ``lct_prefix_allocate`` + ``lct_compact_extra``
  (overflowing inputs, a reservation that does not fit, a double free);
* ``CompressedTensor.free()`` (deferred to the next reservation) gives the
  same descriptors, free list and decoded tensors as immediate frees over a
  random compress/free sequence, including more frees in a row than one launch
  takes, a stream change and an explicit ``TensorBuffer.allocate``.
"""
import numpy as np
import pytest
import torch

from gpu_util import require_gpu
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.compression.huffman_tables import get_distribution_tables
from losslessly_compressed_tensors_amd.codec.geometry import geometry
from losslessly_compressed_tensors_amd.kernels import dispatch
from losslessly_compressed_tensors_amd.kernels.dispatch import FallbackStorage
from losslessly_compressed_tensors_amd.operations import compress, decompress
from losslessly_compressed_tensors_amd.tensor_buffer import (
    FAIL_NO_FIT, Allocation, BufferReservationError, TensorBuffer, _free_regions_snapshot,
    verify_buffer,
)

pytestmark = pytest.mark.gpu

SPARSE = Distribution(DistType.LAPLACE, 1.0, zero_prob=0.5, noise_level=NoiseLevel.SPARSE)
GAUSS = Distribution(DistType.GAUSSIAN)
MEDIUM = Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM)


def _patterns(seed, n):
    """Every BF16 bit pattern, shuffled and repeated: escapes and overflow in
    every layout."""
    rng = np.random.default_rng(seed)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    return torch.from_numpy(np.resize(bits, n).view(np.int16).copy()).view(torch.bfloat16)


def _sparse_activation(seed, shape=(2, 1024, 4096)):
    """relu(N(0,1)) with 0.1% of the entries scaled by 1e4 (config C3's recipe)."""
    z = torch.relu(torch.randn(*shape, generator=torch.Generator().manual_seed(seed)))
    n = z.numel()
    idx = torch.randperm(n, generator=torch.Generator().manual_seed(seed + 1))[: n // 1000]
    z.view(-1)[idx] *= 1e4
    return z.to(torch.bfloat16)


def _gaussian(n, seed):
    return torch.randn(n, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


def _encode(x, dist):
    """The sampled encoder's outputs for ``x`` (as compress produces them)."""
    src = x.cuda().reshape(-1).view(torch.int16)
    n = src.numel()
    B, L, S, W = geometry(dist)
    nb = -(-n // B)
    size = nb * B
    enc_table, dec_table, _ = get_distribution_tables(dist, src.device)
    sample = min(n, 4096)
    partials = torch.empty(2 * (-(-sample // 64)), dtype=torch.int32, device="cuda")
    dispatch.sample_center(src, n, sample, False, partials)
    side = torch.empty(size, dtype=torch.uint8, device="cuda")
    encoded = torch.empty(nb * L * W + 4, dtype=torch.int32, device="cuda")
    center = torch.empty(1, dtype=torch.int32, device="cuda")
    shifted = torch.empty(1024, dtype=torch.int32, device="cuda")
    extra = torch.empty(nb * L, dtype=torch.uint8, device="cuda")
    summaries = torch.empty(dispatch.summaries_length(nb), dtype=torch.int32, device="cuda")
    dispatch.encode_sampled(src, side, encoded, partials, sample, enc_table, dec_table, center,
                            shifted, extra, summaries, size, precomputed=False, logical_numel=n,
                            block_symbols=B, lanes=L, steps=S, fixed_words=W)
    return src, extra, summaries, (B, L, S, W), nb, size, n


def _fragmented(capacity):
    """A buffer with five reservations, the 2nd and 4th freed (three free
    regions); returns it and the five allocations."""
    buffer = TensorBuffer(capacity, device="cuda")
    allocations = [buffer.allocate(torch.tensor([nbytes], dtype=torch.int32, device="cuda"))
                   for nbytes in (4096, 12345, 777, 50000, 1024)]
    buffer.free(allocations[1])
    buffer.free(allocations[3])
    return buffer, allocations


CASES = [
    ("patterns-sparse", SPARSE, lambda: _patterns(11, 3 * 65536 + 999), 8 << 20),
    ("patterns-medium-many-blocks", MEDIUM, lambda: _patterns(12, 300 * 32768), 32 << 20),
    ("c3-like", SPARSE, lambda: _sparse_activation(13), 16 << 20),
    ("gaussian-ragged", GAUSS, lambda: _gaussian(40 * 32768 + 5, 14), 1 << 20),
    ("no-fit", SPARSE, lambda: _patterns(15, 65536), 24 << 10),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("frees", ["one", "double-free", "same-twice", "none"])
def test_one_launch_equals_free_scan_compact(case, frees):
    require_gpu()
    name, dist, make, capacity = case
    print(f"case allocate_compact {name} frees={frees}", flush=True)
    x = make()
    src, extra, summaries, (B, L, S, W), nb, size, n = _encode(x, dist)
    buf_a, alloc_a = _fragmented(capacity)
    buf_b, alloc_b = _fragmented(capacity)
    pending = {"one": [2], "double-free": [2, 1], "same-twice": [2, 2], "none": []}[frees]

    # Reference-shaped sequence: immediate frees, scan + reservation, compaction.
    statuses = [buf_a.free(alloc_a[i]) for i in pending]
    sum_a = summaries.clone()
    counts_a = torch.empty(4, dtype=torch.int32, device="cuda")
    desc_a = torch.empty(4, dtype=torch.int32, device="cuda")
    blocks_a = torch.empty(3 * nb, dtype=torch.int32, device="cuda")
    dispatch.prefix_allocate(sum_a, counts_a, desc_a, buf_a, blocks_a, nb, True,
                             buf_a.max_free_regions)
    arena_a = buf_a.data
    storage = FallbackStorage(tail=arena_a, count=counts_a[:1], lanes=arena_a, starts=arena_a,
                              blocks=blocks_a, descriptor=desc_a, allocation=desc_a)
    dispatch.compact_extra(src, storage, nb, size, precomputed=False, buffered=True,
                           logical_numel=n, block_symbols=B, lanes=L, steps=S,
                           extra_starts=extra, summaries=sum_a)

    # One launch with the frees pending.
    sum_b = summaries.clone()
    counts_b = torch.empty(4, dtype=torch.int32, device="cuda")
    desc_b = torch.empty(4, dtype=torch.int32, device="cuda")
    blocks_b = torch.empty(3 * nb, dtype=torch.int32, device="cuda")
    dispatch.allocate_compact(src, sum_b, counts_b, desc_b, buf_b, blocks_b, extra,
                              [alloc_b[i].descriptor for i in pending], nb, size,
                              logical_numel=n, block_symbols=B, lanes=L, steps=S,
                              precomputed=False)
    torch.cuda.synchronize()

    if frees in ("double-free", "same-twice"):
        assert [int(s.item()) for s in statuses] == [0, 4]
    assert torch.equal(counts_a, counts_b)
    assert torch.equal(desc_a, desc_b)
    assert torch.equal(blocks_a, blocks_b)
    # The overflow-block list and its length (the one launch leaves the scans
    # [2nb, 4nb) to the block metadata, compared above).
    assert torch.equal(sum_a[4 * nb: 5 * nb + 1], sum_b[4 * nb: 5 * nb + 1])
    for a, b in zip(alloc_a, alloc_b):
        assert torch.equal(a.descriptor, b.descriptor)
    assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    assert torch.equal(buf_a.data, buf_b.data), "arena bytes differ"
    status = int(desc_b[2].item())
    if name == "no-fit":
        assert status == 1
        # Both paths record the failed codec reservation in the buffer.
        assert buf_a.failures() == buf_b.failures() == FAIL_NO_FIT
        with pytest.raises(BufferReservationError):
            verify_buffer(buf_b)
    else:
        assert status == 0 and int(counts_b[0].item()) > 0
        verify_buffer(buf_b)


def _inputs():
    return [
        (_patterns(21, 2 * 65536 + 333), SPARSE),
        (_sparse_activation(22, (1, 512, 4096)), SPARSE),
        (_gaussian(7 * 32768 + 11, 23), GAUSS),
        (_patterns(24, 5 * 32768), MEDIUM),
    ]


def _assert_same_allocation(ct_a, ct_b):
    assert torch.equal(ct_a.fallback_descriptor, ct_b.fallback_descriptor)
    assert torch.equal(ct_a.fallback_blocks, ct_b.fallback_blocks)
    assert torch.equal(ct_a.fallback_count, ct_b.fallback_count)


def test_deferred_frees_equal_immediate_frees():
    require_gpu()
    print("case deferred frees, random sequence", flush=True)
    inputs = [(x.cuda(), d) for x, d in _inputs()]
    rng = np.random.default_rng(5)
    buf_a = TensorBuffer(6 << 20, device="cuda")   # immediate frees
    buf_b = TensorBuffer(6 << 20, device="cuda")   # CompressedTensor.free(): deferred
    live = []
    for step in range(60):
        if live and (rng.random() < 0.45 or len(live) > 7):
            ct_a, ct_b, _ = live.pop(int(rng.integers(len(live))))
            buf_a.free(Allocation(ct_a.fallback_descriptor, buf_a))
            ct_b.free()
        else:
            i = int(rng.integers(len(inputs)))
            x, dist = inputs[i]
            ct_a = compress(x, dist, buffer=buf_a)
            ct_b = compress(x, dist, buffer=buf_b)
            _assert_same_allocation(ct_a, ct_b)
            live.append((ct_a, ct_b, i))
        if step % 15 == 14:
            assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    # Six frees in a row (more than one launch takes), then one reservation.
    for _ in range(6):
        x, dist = inputs[int(rng.integers(len(inputs)))]
        live.append((compress(x, dist, buffer=buf_a), compress(x, dist, buffer=buf_b), None))
    for ct_a, ct_b, _ in live[-6:]:
        buf_a.free(Allocation(ct_a.fallback_descriptor, buf_a))
        ct_b.free()
    del live[-6:]
    x, dist = inputs[0]
    ct_a, ct_b = compress(x, dist, buffer=buf_a), compress(x, dist, buffer=buf_b)
    _assert_same_allocation(ct_a, ct_b)
    live.append((ct_a, ct_b, 0))
    torch.cuda.synchronize()
    assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    verify_buffer(buf_b)
    for ct_a, ct_b, i in live:
        if i is None:
            continue
        x, _ = inputs[i]
        assert torch.equal(decompress(ct_b).view(torch.int16).reshape(-1),
                           x.view(torch.int16).reshape(-1))


def test_deferred_free_then_explicit_allocate_and_stream_change():
    require_gpu()
    print("case deferred frees, allocate and stream change", flush=True)
    x, dist = _patterns(31, 65536), SPARSE
    x = x.cuda()
    buf_a = TensorBuffer(1 << 20, device="cuda")
    buf_b = TensorBuffer(1 << 20, device="cuda")
    cts = [(compress(x, dist, buffer=buf_a), compress(x, dist, buffer=buf_b)) for _ in range(3)]
    # A deferred free, then TensorBuffer.allocate: the free is applied first.
    buf_a.free(Allocation(cts[0][0].fallback_descriptor, buf_a))
    cts[0][1].free()
    request = torch.tensor([1000], dtype=torch.int32, device="cuda")
    assert torch.equal(buf_a.allocate(request).descriptor, buf_b.allocate(request).descriptor)
    assert torch.equal(cts[0][0].fallback_descriptor, cts[0][1].fallback_descriptor)
    # A deferred free on the default stream, a reservation on another stream
    # ordered after it.
    buf_a.free(Allocation(cts[1][0].fallback_descriptor, buf_a))
    cts[1][1].free()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ct_a = compress(x, dist, buffer=buf_a)
        ct_b = compress(x, dist, buffer=buf_b)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _assert_same_allocation(ct_a, ct_b)
    assert int(cts[1][1].fallback_descriptor[2].item()) == 5   # freed
    assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    assert torch.equal(decompress(ct_b).view(torch.int16), x.view(torch.int16))
    # reset() applies a pending free before the generation changes.
    cts[2][1].free()
    buf_b.reset()
    torch.cuda.synchronize()
    assert int(cts[2][1].fallback_descriptor[2].item()) == 5
    assert _free_regions_snapshot(buf_b) == [(0, 1 << 20)]


def test_one_launch_free_list_full():
    """A deferred free that needs a new region when the list is full (status 3
    in the reference) changes nothing, as an immediate free would."""
    require_gpu()
    print("case allocate_compact free list full", flush=True)
    x = _patterns(41, 65536)
    src, extra, summaries, (B, L, S, W), nb, size, n = _encode(x, SPARSE)
    buffers = []
    for _ in range(2):
        buffer = TensorBuffer(1 << 20, max_free_regions=4, device="cuda")
        allocations = [buffer.allocate(torch.tensor([4096], dtype=torch.int32, device="cuda"))
                       for _ in range(8)]
        for i in (0, 2, 4):
            buffer.free(allocations[i])   # three holes + the tail: the list is full
        buffers.append((buffer, allocations))
    (buf_a, alloc_a), (buf_b, alloc_b) = buffers
    status = buf_a.free(alloc_a[6])
    sum_a, sum_b = summaries.clone(), summaries.clone()
    outs = [tuple(torch.empty(k, dtype=torch.int32, device="cuda") for k in (4, 4, 3 * nb))
            for _ in range(2)]
    dispatch.prefix_allocate(sum_a, outs[0][0], outs[0][1], buf_a, outs[0][2], nb, True,
                             buf_a.max_free_regions)
    arena_a = buf_a.data
    storage = FallbackStorage(tail=arena_a, count=outs[0][0][:1], lanes=arena_a, starts=arena_a,
                              blocks=outs[0][2], descriptor=outs[0][1], allocation=outs[0][1])
    dispatch.compact_extra(src, storage, nb, size, precomputed=False, buffered=True,
                           logical_numel=n, block_symbols=B, lanes=L, steps=S,
                           extra_starts=extra, summaries=sum_a)
    dispatch.allocate_compact(src, sum_b, outs[1][0], outs[1][1], buf_b, outs[1][2], extra,
                              [alloc_b[6].descriptor], nb, size, logical_numel=n,
                              block_symbols=B, lanes=L, steps=S, precomputed=False)
    torch.cuda.synchronize()
    assert int(status.item()) == 3
    assert int(alloc_b[6].descriptor[2].item()) == 0   # not freed
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
    assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    assert torch.equal(buf_a.data, buf_b.data)


def test_two_streams_share_one_buffer():
    """Compress + free on two streams at once into one TensorBuffer: the
    versioned lock serialises the reservations (a snapshot taken while the
    other stream holds or changes the list is read again), so the free list
    stays valid, every tensor decodes to its input and all space comes back."""
    require_gpu()
    print("case two streams, one buffer", flush=True)
    inputs = [(x.cuda(), d) for x, d in _inputs()]
    buffer = TensorBuffer(16 << 20, max_free_regions=64, device="cuda")
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    kept = [[], []]
    for round_ in range(12):
        for k, s in enumerate(streams):
            with torch.cuda.stream(s):
                x, dist = inputs[(round_ + k) % len(inputs)]
                ct = compress(x, dist, buffer=buffer)
                if round_ % 3 == 2:
                    ct.free()
                else:
                    kept[k].append((ct, x))
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    verify_buffer(buffer)
    for k in range(2):
        for ct, x in kept[k]:
            assert int(ct.fallback_descriptor[2].item()) == 0
            assert torch.equal(decompress(ct).view(torch.int16).reshape(-1),
                               x.view(torch.int16).reshape(-1))
    for k in range(2):
        for ct, _ in kept[k]:
            ct.free()
    torch.cuda.synchronize()
    assert _free_regions_snapshot(buffer) == [(0, 16 << 20)]


def test_deferred_frees_with_the_largest_free_list():
    """4096 free regions: the LDS copy of the list is 32 KiB and every thread
    holds 16 entries in the shifts; many small holes are freed and refilled."""
    require_gpu()
    print("case 4096-region buffer", flush=True)
    x, dist = _patterns(51, 65536), SPARSE
    x = x.cuda()
    bufs = [TensorBuffer(4 << 20, max_free_regions=4096, device="cuda") for _ in range(2)]
    cts = [[compress(x, dist, buffer=b) for _ in range(40)] for b in bufs]
    for i in range(0, 40, 2):   # every other tensor: twenty holes
        bufs[0].free(Allocation(cts[0][i].fallback_descriptor, bufs[0]))
        cts[1][i].free()
    again = [[compress(x, dist, buffer=b) for _ in range(10)] for b in bufs]
    for a, b in zip(again[0], again[1]):
        _assert_same_allocation(a, b)
    torch.cuda.synchronize()
    assert _free_regions_snapshot(bufs[0]) == _free_regions_snapshot(bufs[1])
    assert len(_free_regions_snapshot(bufs[1])) > 5
    verify_buffer(bufs[1])
    assert torch.equal(decompress(again[1][-1]).view(torch.int16), x.view(torch.int16))


def test_freeing_one_tensor_twice_changes_nothing_the_second_time():
    """CompressedTensor.free() twice: both frees ride on one reservation; the
    second is rejected as the immediate second free is (status 4)."""
    require_gpu()
    print("case double CompressedTensor.free()", flush=True)
    x, dist = _patterns(61, 65536), SPARSE
    x = x.cuda()
    buf_a = TensorBuffer(1 << 20, device="cuda")
    buf_b = TensorBuffer(1 << 20, device="cuda")
    cts = [(compress(x, dist, buffer=buf_a), compress(x, dist, buffer=buf_b)) for _ in range(3)]
    first = buf_a.free(Allocation(cts[1][0].fallback_descriptor, buf_a))
    second = buf_a.free(Allocation(cts[1][0].fallback_descriptor, buf_a))
    cts[1][1].free()
    cts[1][1].free()
    ct_a, ct_b = compress(x, dist, buffer=buf_a), compress(x, dist, buffer=buf_b)
    torch.cuda.synchronize()
    assert (int(first.item()), int(second.item())) == (0, 4)
    _assert_same_allocation(ct_a, ct_b)
    assert torch.equal(cts[1][0].fallback_descriptor, cts[1][1].fallback_descriptor)
    assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    verify_buffer(buf_b)


def test_free_batch_equals_single_frees():
    """``lct_buffer_free_batch`` against ``lct_buffer_free`` one descriptor at a
    time on twin buffers: the same statuses, descriptors and free list.  The
    order lists one descriptor twice (freed once, status 4 the second time)
    and overfills a four-region free list (status 3), then merges holes."""
    require_gpu()
    print("case lct_buffer_free_batch against single frees", flush=True)
    bufs = [TensorBuffer(1 << 20, max_free_regions=4, device="cuda") for _ in range(2)]
    request = torch.tensor([1000], dtype=torch.int32, device="cuda")
    allocs = [[b.allocate(request) for _ in range(12)] for b in bufs]
    order = [1, 3, 3, 5, 7, 9, 0, 11, 2, 10]
    single = [int(bufs[0].free(allocs[0][i]).item()) for i in order]
    status = torch.full((len(order),), -1, dtype=torch.int32, device="cuda")
    dispatch.buffer_free_batch(bufs[1].storage, 4, [allocs[1][i].descriptor for i in order],
                               status)
    torch.cuda.synchronize()
    assert status.tolist() == single
    assert 3 in single and 4 in single and 0 in single   # full list, double free, ok
    for a, b in zip(allocs[0], allocs[1]):
        assert torch.equal(a.descriptor, b.descriptor)
    assert _free_regions_snapshot(bufs[0]) == _free_regions_snapshot(bufs[1])


def test_many_deferred_frees_equal_immediate_frees():
    """40 CompressedTensor.free() calls before the next reservation (a full
    batch launched at the 33rd, the rest before and inside the reservation)
    against 40 immediate frees."""
    require_gpu()
    print("case 40 deferred frees", flush=True)
    x, dist = _patterns(71, 65536), SPARSE
    x = x.cuda()
    buf_a = TensorBuffer(8 << 20, max_free_regions=64, device="cuda")
    buf_b = TensorBuffer(8 << 20, max_free_regions=64, device="cuda")
    cts = [(compress(x, dist, buffer=buf_a), compress(x, dist, buffer=buf_b)) for _ in range(48)]
    for ct_a, ct_b in cts[:40]:
        buf_a.free(Allocation(ct_a.fallback_descriptor, buf_a))
        ct_b.free()
    assert len(buf_b._pending_frees) == 40 - dispatch.MAX_FREE_BATCH
    ct_a, ct_b = compress(x, dist, buffer=buf_a), compress(x, dist, buffer=buf_b)
    assert not buf_b._pending_frees
    torch.cuda.synchronize()
    _assert_same_allocation(ct_a, ct_b)
    for a, b in cts[:40]:
        assert torch.equal(a.fallback_descriptor, b.fallback_descriptor)
    assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    verify_buffer(buf_b)
    assert torch.equal(decompress(ct_b).view(torch.int16), x.view(torch.int16))


def test_free_batch_of_stale_descriptors_after_reset():
    """Descriptors made before a reset are stale (another generation): a batch
    of them gets status 4 for each and leaves the reset free list whole."""
    require_gpu()
    print("case lct_buffer_free_batch after reset", flush=True)
    buffer = TensorBuffer(1 << 20, max_free_regions=16, device="cuda")
    request = torch.tensor([2000], dtype=torch.int32, device="cuda")
    allocs = [buffer.allocate(request) for _ in range(5)]
    buffer.reset()
    status = torch.full((5,), -1, dtype=torch.int32, device="cuda")
    dispatch.buffer_free_batch(buffer.storage, 16, [a.descriptor for a in allocs], status)
    torch.cuda.synchronize()
    assert status.tolist() == [4] * 5
    assert _free_regions_snapshot(buffer) == [(0, 1 << 20)]
