"""Device-side failures of a compressed tensor's overflow reservation reach the
host at the synchronisations the path already makes.

The reference leaves a failed reservation unflagged: the allocator stores
offset -1 and nothing reads the status (``LCT/kernels/tensor_buffer.py:84-89``),
so the tensor silently decodes without its overflow tails.  Here the three ways
a codec reservation can fail are driven from the host, with every kernel
leaving through its own bounded wait:

* no free region fits (a buffer too small for the tails): status 1;
* the arena lock is held (an odd version written into the lock word from the
  host, the lock wait bounded by ``lct_set_wait_limits``): status 6;
* a compacting workgroup of the separate bookkeeping launch stops waiting
  for the reservation (its poll bound lowered to one poll): status 7, the
  region still held and freeable (the one-launch compress's own give-up path
  is tested with it, in test_gpu_fused_compress.py).

In each case ``CompressedTensor.memory_size()``, ``verify_buffer`` and
``TensorBuffer.check`` raise ``BufferReservationError``, the free list is left
as it was (or, for status 7, holds the reservation until it is freed), and
``reset()`` clears the failure word.
"""
import numpy as np
import pytest
import torch

from gpu_util import require_gpu
from losslessly_compressed_tensors_amd.codec.encode import encode_components
from losslessly_compressed_tensors_amd.codec.geometry import geometry
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.compression.huffman_tables import get_distribution_tables
from losslessly_compressed_tensors_amd.kernels import dispatch, hip
from losslessly_compressed_tensors_amd.operations import compress, decompress
from losslessly_compressed_tensors_amd.tensor_buffer import (
    FAIL_INCOMPLETE, FAIL_LOCK, FAIL_NO_FIT, STATUS_INCOMPLETE, STATUS_LOCK, STATUS_NO_FIT,
    BufferReservationError, TensorBuffer, _free_regions_snapshot, verify_buffer,
)

pytestmark = pytest.mark.gpu

SPARSE = Distribution(DistType.LAPLACE, 1.0, zero_prob=0.5, noise_level=NoiseLevel.SPARSE)
GAUSS = Distribution(DistType.GAUSSIAN)


def _overflowing(seed, n=3 * 65536 + 77):
    """Every BF16 bit pattern, shuffled: thousands of overflowing streams."""
    rng = np.random.default_rng(seed)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    return torch.from_numpy(np.resize(bits, n).view(np.int16).copy()).view(torch.bfloat16).cuda()


def _clean(seed=4, shape=(256, 512)):
    """N(0, 1) with CPU seed 4: no stream overflows under GAUSSIAN CLEAN (the
    oracle's encode of it has no overflow entries)."""
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(
        torch.bfloat16).cuda()


@pytest.fixture
def wait_limits():
    """Set the device waits' bounds for one test; the defaults come back after."""
    def set_limits(lock_polls, ready_polls):
        hip.call("lct_set_wait_limits", lock_polls, ready_polls)

    yield set_limits
    hip.call("lct_set_wait_limits", 0, 0)


def _descriptor(ct):
    return [int(v) for v in ct.fallback_descriptor.tolist()]


def test_reservation_that_does_not_fit_raises_at_memory_size():
    require_gpu()
    print("case failures no-fit", flush=True)
    buffer = TensorBuffer(1 << 10, device="cuda")
    before = _free_regions_snapshot(buffer)
    ct = compress(_overflowing(1), SPARSE, buffer=buffer)
    torch.cuda.synchronize()
    assert _descriptor(ct)[2] == STATUS_NO_FIT
    assert int(ct.fallback_count.item()) > 0
    with pytest.raises(BufferReservationError, match="status 1"):
        ct.memory_size()
    with pytest.raises(BufferReservationError):
        ct.memory_buffer_size()
    assert buffer.failures() == FAIL_NO_FIT
    with pytest.raises(BufferReservationError, match="no free region"):
        verify_buffer(buffer)
    assert _free_regions_snapshot(buffer) == before   # nothing was reserved
    buffer.reset()
    assert buffer.failures() == 0
    verify_buffer(buffer)


def test_a_successful_reservation_sets_no_failure():
    require_gpu()
    print("case failures none", flush=True)
    buffer = TensorBuffer(8 << 20, device="cuda")
    x = _overflowing(2)
    ct = compress(x, SPARSE, buffer=buffer)
    assert ct.memory_size() > 0
    assert torch.equal(decompress(ct).view(torch.int16), x.view(torch.int16))
    assert buffer.failures() == 0
    verify_buffer(buffer)


def test_held_lock_gives_status_6_and_raises(wait_limits):
    require_gpu()
    print("case failures lock held", flush=True)
    buffer = TensorBuffer(8 << 20, device="cuda")
    keep = buffer.allocate(torch.tensor([4096], dtype=torch.int32, device="cuda"))
    before = _free_regions_snapshot(buffer)
    version = int(buffer._lock.item())
    assert version % 2 == 0
    wait_limits(64, 0)   # the lock waits give up after 64 polls
    buffer._lock.fill_(version + 1)   # held by "someone else"
    try:
        plain = buffer.allocate(torch.tensor([256], dtype=torch.int32, device="cuda"))
        freed = buffer.free(keep)
        ct = compress(_overflowing(3), SPARSE, buffer=buffer)
        clean = compress(_clean(), GAUSS, buffer=buffer)
        torch.cuda.synchronize()
        assert int(plain.status.item()) == STATUS_LOCK
        assert int(freed.item()) == STATUS_LOCK
        assert _descriptor(ct)[2] == STATUS_LOCK
        assert int(buffer._lock.item()) == version + 1   # nobody touched the held lock
        # A plain allocate reports its status in its descriptor only; the
        # codec's reservation also records the failure.
        assert int(buffer._failures.item()) == FAIL_LOCK
        with pytest.raises(BufferReservationError, match="status 6"):
            ct.memory_size()
        # Without overflow entries nothing was lost: the tensor is usable.
        assert int(clean.fallback_count.item()) == 0 and _descriptor(clean)[2] == STATUS_LOCK
        clean.memory_size()
        assert torch.equal(decompress(clean).view(torch.int16), _clean().view(torch.int16))
    finally:
        buffer._lock.fill_(version + 2)
    assert _free_regions_snapshot(buffer) == before
    with pytest.raises(BufferReservationError, match="lock"):
        verify_buffer(buffer)
    buffer.reset()
    verify_buffer(buffer)


def test_prefix_allocate_records_a_lock_failure(wait_limits):
    """The reference-shaped lct_prefix_allocate (buffered) flags its failure
    the same way as the one-launch path."""
    require_gpu()
    print("case failures prefix_allocate lock", flush=True)
    buffer = TensorBuffer(8 << 20, device="cuda")
    dist = SPARSE
    src = _overflowing(5).reshape(-1).view(torch.int16)
    n = src.numel()
    B, L, S, W = geometry(dist)
    nb = -(-n // B)
    enc_table, dec_table, _ = get_distribution_tables(dist, src.device)
    partials = torch.empty(2 * 64, dtype=torch.int32, device="cuda")
    dispatch.sample_center(src, n, 4096, False, partials)
    summaries = torch.empty(dispatch.summaries_length(nb), dtype=torch.int32, device="cuda")
    dispatch.encode_sampled(src, torch.empty(nb * B, dtype=torch.uint8, device="cuda"),
                            torch.empty(nb * L * W + 4, dtype=torch.int32, device="cuda"),
                            partials, 4096, enc_table, dec_table,
                            torch.empty(1, dtype=torch.int32, device="cuda"),
                            torch.empty(1024, dtype=torch.int32, device="cuda"),
                            torch.empty(nb * L, dtype=torch.uint8, device="cuda"), summaries,
                            nb * B, precomputed=False, logical_numel=n, block_symbols=B,
                            lanes=L, steps=S, fixed_words=W)
    counts = torch.empty(4, dtype=torch.int32, device="cuda")
    descriptor = torch.empty(4, dtype=torch.int32, device="cuda")
    blocks = torch.empty(3 * nb, dtype=torch.int32, device="cuda")
    version = int(buffer._lock.item())
    wait_limits(64, 0)
    buffer._lock.fill_(version + 1)
    try:
        dispatch.prefix_allocate(summaries, counts, descriptor, buffer, blocks, nb, True,
                                 buffer.max_free_regions)
        torch.cuda.synchronize()
    finally:
        buffer._lock.fill_(version + 2)
    assert int(descriptor[2].item()) == STATUS_LOCK and int(counts[0].item()) > 0
    assert buffer.failures() == FAIL_LOCK


def _compress_given_center(x, dist, buffer, center):
    """A buffered compress through the separate launches that a given center
    takes (shifted tables, encoder, then the one-launch bookkeeping
    lct_allocate_compact), as the fused updates' re-encodes use them."""
    src = x.reshape(-1).view(torch.int16)
    n = src.numel()
    nb = -(-n // geometry(dist)[0])
    size = nb * geometry(dist)[0]
    side = torch.empty(size, dtype=torch.uint8, device="cuda")
    return encode_components(src, side, size, dist, buffer, tuple(x.shape), precomputed=False,
                             center=center, logical_numel=n)


def test_compaction_that_stops_waiting_marks_the_reservation_incomplete(wait_limits):
    require_gpu()
    print("case failures incomplete compaction", flush=True)
    buffer = TensorBuffer(8 << 20, device="cuda")
    before = _free_regions_snapshot(buffer)
    x = _overflowing(6, n=40 * 65536)
    center = compress(x, SPARSE).center
    wait_limits(0, 1)   # compacting workgroups poll the ready word once
    statuses = []
    for attempt in range(4):
        ct = _compress_given_center(x, SPARSE, buffer, center)
        status = _descriptor(ct)[2]
        statuses.append(status)
        print(f"attempt {attempt}: status {status}", flush=True)
        assert status in (0, STATUS_INCOMPLETE)
        if status == 0:
            # Every workgroup saw the reservation in its one poll.
            assert torch.equal(decompress(ct).view(torch.int16), x.view(torch.int16))
            ct.memory_size()
            ct.free()
            continue
        with pytest.raises(BufferReservationError, match="status 7"):
            ct.memory_size()
        assert buffer.failures() & FAIL_INCOMPLETE
        assert len(_free_regions_snapshot(buffer)) == 1 and _free_regions_snapshot(buffer) != before
        ct.free()   # the region is held like a status-0 one and comes back
        assert _free_regions_snapshot(buffer) == before
        break
    assert STATUS_INCOMPLETE in statuses, statuses
    with pytest.raises(BufferReservationError, match="did not complete"):
        buffer.check()
    buffer.reset()
    buffer.check()
