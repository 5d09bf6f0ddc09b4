"""GPU parity of the batched buffered compress (``lct_compress_batch``).

The batched compress has no counterpart in the reference, which compresses
one tensor per call (``LCT/codec/encode.py:189-218``); each tensor of a batch
must store what that call stores.  Checked here:

* every tensor of a batch against the oracle's compress of the same tensor
  (center, shifted decode table, payload, side bytes, totals, block metadata,
  and the overflow region -- lanes | starts | tails -- at whatever arena
  offset the tensor's reservation got), with a bit-exact decode, over ragged
  tails, single-element and all-patterns tensors, and batches that mix step
  counts (one launch per count) or hold more than 16 tensors (several);
* against ``compress`` of the same tensor into another buffer: the same
  reservation size and ``memory_size()``;
* the buffer's deferred frees are applied before the batch's reservations:
  the freed descriptors read freed, the free list passes its invariants and
  a batch that only fits after the frees is stored.
"""
import numpy as np
import pytest
import torch

from gpu_util import bits_of, oracle_compress, require_gpu
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.operations import compress, compress_batch, decompress
from losslessly_compressed_tensors_amd.tensor_buffer import (
    STATUS_EMPTY, STATUS_FREED, STATUS_OK, TensorBuffer, verify_buffer,
)

pytestmark = pytest.mark.gpu

GAUSS = Distribution(DistType.GAUSSIAN)                        # 256 steps
LAPLACE = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN)
SPARSE = Distribution(DistType.LAPLACE, 1.0, zero_prob=0.5, noise_level=NoiseLevel.SPARSE)
MEDIUM = Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM)


def _gaussian(n, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * scale).to(torch.bfloat16)


def _patterns(n, seed):
    """Every BF16 bit pattern, shuffled and repeated: escapes and overflow."""
    rng = np.random.default_rng(seed)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    return torch.from_numpy(np.resize(bits, n).view(np.int16).copy()).view(torch.bfloat16)


def _relu_outliers(n, seed):
    z = torch.relu(torch.randn(n, generator=torch.Generator().manual_seed(seed)))
    z[torch.randperm(n, generator=torch.Generator().manual_seed(seed + 1))[: n // 1000]] *= 1e4
    return z.to(torch.bfloat16)


def _assert_record(ct, x, dist):
    """``ct`` (buffered) stores what the oracle's private compress of ``x`` does,
    its overflow region at its own descriptor's offset, and decodes to ``x``."""
    o = oracle_compress(x, dist)
    B, L, S, W = ct.codec_geometry
    ns = (ct.size // B) * L
    assert int(ct.center.item()) == o.center
    assert np.array_equal(ct.decode_table.cpu().numpy(), o.shifted_decode)
    assert np.array_equal(ct.data.cpu().numpy()[: ns * W], o.encoded[: ns * W]), "payload differs"
    assert np.array_equal(ct.sign_mantissa.cpu().numpy(), o.side), "side bytes differ"
    count, used = int(ct.fallback_count.item()), int(ct.fallback_used.item())
    assert (count, used) == (int(o.counts[0]), int(o.counts[1]))
    assert np.array_equal(ct.fallback_blocks.cpu().numpy(), o.blocks)
    desc = ct.fallback_descriptor.cpu().numpy()
    # A tensor without overflow asks for nothing: status "empty", as in compress.
    assert int(desc[2]) == (STATUS_OK if count else STATUS_EMPTY)
    region = ct.buffer.data.cpu().numpy()[int(desc[0]): int(desc[0]) + 2 * count + used]
    assert np.array_equal(region[:count], o.lanes), "overflow lanes differ"
    assert np.array_equal(region[count:2 * count], o.starts), "overflow starts differ"
    assert np.array_equal(region[2 * count:], o.tail), "overflow tails differ"
    assert np.array_equal(bits_of(decompress(ct)), bits_of(x)), "decode differs"


CASES = [
    ("gauss-ragged", lambda: _gaussian(5 * 65536 - 17, 1), GAUSS),
    ("laplace-one", lambda: _gaussian(1, 2), LAPLACE),
    ("patterns", lambda: _patterns(3 * 32768 + 5, 3), SPARSE),
    ("relu-outliers", lambda: _relu_outliers(9 * 32768, 4), SPARSE),
    ("gauss-wide", lambda: _gaussian(70 * 65536, 5, 30.0), MEDIUM),
    ("laplace-seven", lambda: _gaussian(7, 6), LAPLACE),
]


@pytest.fixture(autouse=True)
def _gpu():
    require_gpu()


def test_batch_matches_oracle_per_tensor():
    """One batch of tensors of both step counts, each as the oracle stores it."""
    buffer = TensorBuffer(256 << 20, device="cuda")
    xs = [make() for _, make, _ in CASES]
    dists = [dist for _, _, dist in CASES]
    records = compress_batch([x.cuda() for x in xs], dists, buffer=buffer)
    for (name, _, dist), ct, x in zip(CASES, records, xs):
        print(f"case {name}", flush=True)
        _assert_record(ct, x, dist)
    verify_buffer(buffer)


def test_batch_matches_single_compress():
    """Reservation sizes and memory_size() equal those of one compress each."""
    batch_buffer = TensorBuffer(256 << 20, device="cuda")
    single_buffer = TensorBuffer(256 << 20, device="cuda")
    xs = [make().cuda() for _, make, _ in CASES]
    dists = [dist for _, _, dist in CASES]
    records = compress_batch(xs, dists, buffer=batch_buffer)
    for x, dist, ct in zip(xs, dists, records):
        single = compress(x, distribution=dist, buffer=single_buffer)
        assert int(ct.fallback_descriptor[1].item()) == int(single.fallback_descriptor[1].item())
        assert ct.memory_size() == single.memory_size()
        assert np.array_equal(ct.sample_values.cpu().numpy(), single.sample_values.cpu().numpy())


def test_batches_of_more_than_sixteen():
    """37 tensors (three launches), freed and stored again into the same buffer."""
    buffer = TensorBuffer(64 << 20, device="cuda")
    xs = [_gaussian(32768 * (1 + i % 5) - 3 * i, 100 + i).cuda() for i in range(37)]
    for round_ in range(2):
        records = compress_batch(xs, LAPLACE, buffer=buffer)
        for x, ct in zip(xs, records):
            assert torch.equal(decompress(ct).view(torch.int16), x.view(torch.int16))
        for i in (0, 5, 17, 36):
            _assert_record(records[i], xs[i].cpu(), LAPLACE)
        for ct in records:
            ct.free()
        verify_buffer(buffer)


def test_deferred_frees_come_first():
    """A batch whose reservations fit only once the deferred frees are applied:
    the frees ride on the batch's launch (job 0 applies them before any
    reservation) and every tensor is stored."""
    x_big = _patterns(40 * 32768, 7).cuda()
    probe = compress(x_big, distribution=SPARSE, buffer=TensorBuffer(64 << 20, device="cuda"))
    need = int(probe.fallback_descriptor[1].item())
    # Room for two such reservations and a quarter: the second batch fits only
    # after the first batch's two tensors are freed.
    buffer = TensorBuffer(((2 * need + need // 4 + 15) // 16) * 16, device="cuda")
    first = compress_batch([x_big, x_big], SPARSE, buffer=buffer)
    assert need > 0
    assert [int(ct.fallback_descriptor[2].item()) for ct in first] == [STATUS_OK] * 2
    for ct in first:
        ct.free()                      # deferred to the next reservation
    assert len(buffer._pending_frees) == 2
    second = compress_batch([x_big, _patterns(40 * 32768, 8).cuda()], SPARSE, buffer=buffer)
    assert not buffer._pending_frees
    assert [int(ct.fallback_descriptor[2].item()) for ct in first] == [STATUS_FREED] * 2
    for ct, seed in zip(second, (7, 8)):
        _assert_record(ct, _patterns(40 * 32768, seed), SPARSE)
    verify_buffer(buffer)
