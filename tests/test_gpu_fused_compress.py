"""GPU parity of the one-launch compress (``lct_encode_fused``).

``lct_encode_fused`` replaces the launch sequence center sampling -> encoder ->
prefix scan (+ arena reservation after the buffer's deferred frees)
(``LCT/kernels/dispatch.py:33-48, 294-316, 70-85`` as
``LCT/codec/encode.py:22-186`` runs them).  Checked here, on the same input
and the same fragmented buffer, against that sequence built from the
reference-shaped entry points (``lct_sample_center``, ``lct_encode_sampled``,
``lct_buffer_free``, ``lct_prefix_allocate``), each followed by the same
``lct_compact_extra``:

* every output equal: side bytes, payload, center, shifted decode table,
  sampled values, extra starts, counts, descriptor, block metadata, the
  overflow-block list, the freed descriptors, the free list and the whole
  arena (overflowing inputs, more than one pass of the polled scan, a ragged
  tail block, a reservation that does not fit, double frees);
* private storage: the same counts, metadata and exact-size arrays;
* consecutive calls on one stream reuse the stream's control array (each call
  sees only its own epoch's words), including a smaller tensor after a larger;
* a bookkeeping wait that gives up (its poll bound lowered from the host)
  marks the tensor incomplete: status 7 and ``BufferReservationError`` at
  ``memory_size()`` with a buffer, ``RuntimeError`` from a private compress;
  the region is still freed.
"""
import numpy as np
import pytest
import torch

from gpu_util import require_gpu
from losslessly_compressed_tensors_amd.codec.geometry import geometry
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.compression.huffman_tables import get_distribution_tables
from losslessly_compressed_tensors_amd.kernels import dispatch, hip
from losslessly_compressed_tensors_amd.kernels.dispatch import FallbackStorage
from losslessly_compressed_tensors_amd.operations import compress, decompress
from losslessly_compressed_tensors_amd.tensor_buffer import (
    FAIL_INCOMPLETE, FAIL_NO_FIT, STATUS_INCOMPLETE, BufferReservationError, TensorBuffer,
    _free_regions_snapshot, verify_buffer,
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


def _outputs(n, dist, buffered):
    B, L, S, W = geometry(dist)
    nb = -(-n // B)
    dev = "cuda"
    return dict(
        side=torch.empty(nb * B, dtype=torch.uint8, device=dev),
        encoded=torch.empty(nb * L * W + 4, dtype=torch.int32, device=dev),
        center=torch.empty(1, dtype=torch.int32, device=dev),
        shifted=torch.empty(1024, dtype=torch.int32, device=dev),
        samples=torch.empty(min(n, 4096), dtype=torch.int16, device=dev),
        extra=torch.empty(nb * L, dtype=torch.uint8, device=dev),
        summaries=torch.empty(dispatch.summaries_length(nb), dtype=torch.int32, device=dev),
        counts=torch.empty(4, dtype=torch.int32, device=dev),
        blocks=torch.empty(3 * nb, dtype=torch.int32, device=dev),
        descriptor=torch.empty(4, dtype=torch.int32, device=dev) if buffered else None,
    )


def _compact(src, o, dist, n, buffer):
    """lct_compact_extra after either bookkeeping; returns the storage."""
    B, L, S, W = geometry(dist)
    nb = -(-n // B)
    if buffer is not None:
        arena = buffer.data
        storage = FallbackStorage(tail=arena, count=o["counts"][:1], lanes=arena, starts=arena,
                                  blocks=o["blocks"], descriptor=o["descriptor"],
                                  allocation=o["descriptor"])
    else:
        count, tail_bytes = (int(v) for v in o["counts"][:2].tolist())
        storage = FallbackStorage(
            tail=torch.empty(tail_bytes, dtype=torch.uint8, device="cuda"),
            count=o["counts"][:1], lanes=torch.empty(count, dtype=torch.uint8, device="cuda"),
            starts=torch.empty(count, dtype=torch.uint8, device="cuda"), blocks=o["blocks"],
            allocation=o["counts"][2:3])
        if count == 0:
            return storage
    dispatch.compact_extra(src, storage, nb, nb * B, precomputed=False,
                           buffered=buffer is not None, logical_numel=n, block_symbols=B,
                           lanes=L, steps=S, extra_starts=o["extra"], summaries=o["summaries"])
    return storage


def _sequence(x, dist, buffer=None, frees=()):
    """The reference-shaped launches: immediate frees, sampler, sampled encoder,
    prefix scan (+ reservation), compaction."""
    src = x.cuda().reshape(-1).view(torch.int16)
    n = src.numel()
    B, L, S, W = geometry(dist)
    nb = -(-n // B)
    o = _outputs(n, dist, buffer is not None)
    statuses = [buffer.free(a) for a in frees] if buffer is not None else []
    enc_table, dec_table, _ = get_distribution_tables(dist, src.device)
    sample = min(n, 4096)
    partials = torch.empty(2 * (-(-sample // 64)), dtype=torch.int32, device="cuda")
    dispatch.sample_center(src, n, sample, False, partials, o["samples"])
    dispatch.encode_sampled(src, o["side"], o["encoded"], partials, sample, enc_table, dec_table,
                            o["center"], o["shifted"], o["extra"], o["summaries"], nb * B,
                            precomputed=False, logical_numel=n, block_symbols=B, lanes=L,
                            steps=S, fixed_words=W)
    dispatch.prefix_allocate(o["summaries"], o["counts"], o["descriptor"], buffer, o["blocks"],
                             nb, buffer is not None,
                             buffer.max_free_regions if buffer is not None else 256)
    o["storage"] = _compact(src, o, dist, n, buffer)
    o["statuses"] = statuses
    return o


def _fused(x, dist, buffer=None, frees=()):
    """lct_encode_fused (the frees deferred into it) then the compaction."""
    src = x.cuda().reshape(-1).view(torch.int16)
    n = src.numel()
    B, L, S, W = geometry(dist)
    nb = -(-n // B)
    o = _outputs(n, dist, buffer is not None)
    enc_table, dec_table, _ = get_distribution_tables(dist, src.device)
    dispatch.encode_fused(src, o["side"], o["encoded"], min(n, 4096), enc_table, dec_table,
                          o["center"], o["shifted"], o["samples"], o["extra"], o["summaries"],
                          o["blocks"], o["counts"], nb * B, precomputed=False, logical_numel=n,
                          block_symbols=B, lanes=L, steps=S, fixed_words=W, buffer=buffer,
                          descriptor=o["descriptor"], frees=[a.descriptor for a in frees])
    o["storage"] = _compact(src, o, dist, n, buffer)
    return o


def _fragmented(capacity):
    """A buffer with five reservations, the 2nd and 4th freed (three free
    regions); returns it and the five allocations."""
    buffer = TensorBuffer(capacity, device="cuda")
    allocations = [buffer.allocate(torch.tensor([nbytes], dtype=torch.int32, device="cuda"))
                   for nbytes in (4096, 12345, 777, 50000, 1024)]
    buffer.free(allocations[1])
    buffer.free(allocations[3])
    return buffer, allocations


def _assert_same_codec_outputs(a, b, nb):
    for key in ("side", "center", "shifted", "samples", "extra", "counts", "blocks"):
        assert torch.equal(a[key], b[key]), key
    # The payload without its 4 words of read-ahead padding, which nobody writes.
    payload = a["encoded"].numel() - 4
    assert torch.equal(a["encoded"][:payload], b["encoded"][:payload]), "encoded"
    # The overflow-block list's length and entries (the fused launch writes no
    # other summary entries, and neither path writes past the list's length).
    listed = int(a["summaries"][5 * nb].item())
    assert int(b["summaries"][5 * nb].item()) == listed
    assert torch.equal(a["summaries"][4 * nb: 4 * nb + listed],
                       b["summaries"][4 * nb: 4 * nb + listed])


CASES = [
    ("patterns-sparse", SPARSE, lambda: _patterns(31, 3 * 65536 + 999), 8 << 20),
    ("patterns-medium-three-scan-passes", MEDIUM, lambda: _patterns(32, 2500 * 32768), 128 << 20),
    ("c3-like", SPARSE, lambda: _sparse_activation(33), 16 << 20),
    ("gaussian-ragged", GAUSS, lambda: _gaussian(40 * 32768 + 5, 34), 1 << 20),
    ("one-block", GAUSS, lambda: _gaussian(1000, 35), 1 << 20),
    ("no-fit", SPARSE, lambda: _patterns(36, 65536), 24 << 10),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("frees", ["none", "one", "double-free"])
def test_fused_equals_the_launch_sequence_buffered(case, frees):
    require_gpu()
    name, dist, make, capacity = case
    print(f"case fused buffered {name} frees={frees}", flush=True)
    x = make()
    n = x.numel()
    nb = -(-n // geometry(dist)[0])
    buf_a, alloc_a = _fragmented(capacity)
    buf_b, alloc_b = _fragmented(capacity)
    pending = {"none": [], "one": [2], "double-free": [2, 2]}[frees]
    a = _sequence(x, dist, buf_a, [alloc_a[i] for i in pending])
    b = _fused(x, dist, buf_b, [alloc_b[i] for i in pending])
    torch.cuda.synchronize()
    _assert_same_codec_outputs(a, b, nb)
    assert torch.equal(a["descriptor"], b["descriptor"])
    for p, q in zip(alloc_a, alloc_b):
        assert torch.equal(p.descriptor, q.descriptor)
    assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    assert torch.equal(buf_a.data, buf_b.data), "arena bytes differ"
    assert int(b["counts"][3].item()) == 0
    if name == "no-fit":
        assert int(b["descriptor"][2].item()) == 1
        assert buf_a.failures() == buf_b.failures() == FAIL_NO_FIT
    else:
        assert int(b["descriptor"][2].item()) in (0, 2)   # 2: nothing overflowed
        verify_buffer(buf_b)


@pytest.mark.parametrize("case", CASES[:5], ids=[c[0] for c in CASES[:5]])
def test_fused_equals_the_launch_sequence_private(case):
    require_gpu()
    name, dist, make, _ = case
    print(f"case fused private {name}", flush=True)
    x = make()
    n = x.numel()
    nb = -(-n // geometry(dist)[0])
    a = _sequence(x, dist)
    b = _fused(x, dist)
    torch.cuda.synchronize()
    _assert_same_codec_outputs(a, b, nb)
    for key in ("lanes", "starts", "tail"):
        assert torch.equal(getattr(a["storage"], key), getattr(b["storage"], key)), key


def test_consecutive_calls_share_the_streams_control_array():
    """Public compresses on one stream, larger then smaller then larger again,
    interleaved with another stream's: every call decodes bit for bit."""
    require_gpu()
    print("case fused consecutive calls", flush=True)
    inputs = [(_patterns(41, 300 * 32768), MEDIUM), (_gaussian(3 * 32768 + 17, 42), GAUSS),
              (_sparse_activation(43, (1, 512, 4096)), SPARSE), (_gaussian(5, 44), GAUSS)]
    inputs = [(x.cuda(), d) for x, d in inputs]
    buffer = TensorBuffer(64 << 20, device="cuda")
    other = torch.cuda.Stream()
    for round_ in range(3):
        for i, (x, dist) in enumerate(inputs):
            cts = [compress(x, dist), compress(x, dist, buffer=buffer)]
            with torch.cuda.stream(other):
                other.wait_stream(torch.cuda.current_stream())
                side = compress(x, dist)
            torch.cuda.current_stream().wait_stream(other)
            for ct in cts + [side]:
                assert torch.equal(decompress(ct).view(torch.int16), x.view(torch.int16)), \
                    (round_, i)
            cts[1].free()


def test_bookkeeping_that_stops_waiting_marks_the_tensor_incomplete():
    require_gpu()
    print("case fused incomplete", flush=True)
    # 3000 blocks: more than the device holds at once, so workgroup 0 finishes
    # its own block (and starts the bookkeeping) while later blocks have not
    # been dispatched yet.
    x = torch.randn(3000 * 32768, generator=torch.Generator(device="cuda").manual_seed(51),
                    device="cuda").to(torch.bfloat16)
    buffer = TensorBuffer(16 << 20, device="cuda")
    before = _free_regions_snapshot(buffer)
    # One poll round of the partial sums and of each block's summary: the
    # bookkeeping gives up long before the last blocks finish.
    hip.call("lct_set_wait_limits", 0, 1)
    try:
        ct = compress(x, GAUSS, buffer=buffer)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="gave up"):
            compress(x, GAUSS)
    finally:
        hip.call("lct_set_wait_limits", 0, 0)
    assert int(ct.fallback_descriptor[2].item()) == STATUS_INCOMPLETE
    with pytest.raises(BufferReservationError, match="status 7"):
        ct.memory_size()
    assert buffer.failures() & FAIL_INCOMPLETE
    ct.free()   # the reservation is held like a status-0 one and comes back
    buffer._flush_frees()
    assert _free_regions_snapshot(buffer) == before
    # With the default bounds again, both forms work.
    assert torch.equal(decompress(compress(x, GAUSS)).view(torch.int16), x.view(torch.int16))
    ok = compress(x, GAUSS, buffer=buffer)
    assert torch.equal(decompress(ok).view(torch.int16), x.view(torch.int16))
    with pytest.raises(BufferReservationError, match="did not complete"):
        buffer.check()
    buffer.reset()
    buffer.check()


def test_private_compress_host_totals():
    """A private compress's launch posts its overflow totals to the thread's
    pinned host words (tagged with the launch's epoch) and they equal the
    stored counts; a wait for an epoch that never posts falls back to reading
    the counts once the stream is idle."""
    require_gpu()
    print("case host totals", flush=True)
    x = _patterns(90, 7 * 65536 + 4321)
    ct = compress(x.cuda(), SPARSE)
    torch.cuda.synchronize()
    w0, w1 = (int(v) & 0xFFFFFFFFFFFFFFFF for v in dispatch.host_totals().words.tolist())
    assert w0 >> 32 == w1 >> 32 != 0, "both words carry the launch's epoch"
    count, used = int(ct.fallback_count.item()), int(ct.fallback_used.item())
    assert count > 0
    assert (w0 & 0x7FFFFFFF, (w0 >> 31) & 1, w1 & 0xFFFFFFFF) == (count, 0, used)
    counts = torch.tensor([count, used, 0, 0], dtype=torch.int32, device="cuda")
    stale = (w0 >> 32) ^ 0x5A5A5A5A
    assert dispatch.host_totals().wait(stale, counts, counts.device) == (count, used, 0)
    restored = decompress(ct)
    assert torch.equal(restored.cpu().view(torch.int16), x.view(torch.int16))
