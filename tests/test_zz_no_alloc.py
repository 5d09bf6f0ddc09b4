"""lct_compress_buffered_noalloc against the compress sequence it replaces.

The entry point enqueues lct_sample_center -> lct_encode_sampled ->
lct_allocate_compact with their working arrays in the library's file-scope
device array, so it must leave exactly what that sequence leaves with
torch-allocated working arrays: every output array, the descriptor, the
TensorBuffer's free list and the whole arena.  Two calls in a row (the second
on a smaller input, with the first one's reservation as a pending free)
check that the array's leftover contents from the first call change nothing.
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import require_gpu
from losslessly_compressed_tensors_amd.codec.geometry import geometry
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.compression.huffman_tables import get_distribution_tables
from losslessly_compressed_tensors_amd.kernels import dispatch, hip
from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer, _free_regions_snapshot

pytestmark = pytest.mark.gpu

SPARSE = Distribution(DistType.LAPLACE, 1.0, zero_prob=0.5, noise_level=NoiseLevel.SPARSE)
GAUSS = Distribution(DistType.GAUSSIAN)


def _patterns(seed, n):
    rng = np.random.default_rng(seed)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    return torch.from_numpy(np.resize(bits, n).view(np.int16).copy()).cuda()


def _gaussian(seed, n):
    x = torch.randn(n, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    return x.view(torch.int16).cuda()


def _gaussian_device(seed, n):
    """Large inputs drawn on the device (the CPU draw of 2^28 values is slow)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(n, generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)


def _outputs(n, dist):
    B, L, S, W = geometry(dist)
    nb = -(-n // B)
    dev = "cuda"
    return dict(
        side=torch.full((nb * B,), 0xAB, dtype=torch.uint8, device=dev),
        encoded=torch.full((nb * L * W + 4,), -1, dtype=torch.int32, device=dev),
        center=torch.full((1,), 99, dtype=torch.int32, device=dev),
        shifted=torch.full((1024,), -1, dtype=torch.int32, device=dev),
        samples=torch.full((min(n, 4096),), -1, dtype=torch.int16, device=dev),
        blocks=torch.full((3 * nb,), -1, dtype=torch.int32, device=dev),
        counts=torch.full((4,), -1, dtype=torch.int32, device=dev),
        descriptor=torch.full((4,), -1, dtype=torch.int32, device=dev),
    ), (B, L, S, W), nb


def _sequence(src, dist, buffer, frees):
    """The existing entry points, working arrays from torch."""
    n = src.numel()
    out, (B, L, S, W), nb = _outputs(n, dist)
    enc, dec, _ = get_distribution_tables(dist, src.device)
    sample = min(n, 4096)
    partials = torch.empty(2 * (-(-sample // 64)), dtype=torch.int32, device="cuda")
    extra = torch.empty(nb * L, dtype=torch.uint8, device="cuda")
    summaries = torch.empty(dispatch.summaries_length(nb), dtype=torch.int32, device="cuda")
    dispatch.sample_center(src, n, sample, False, partials, out["samples"])
    dispatch.encode_sampled(src, out["side"], out["encoded"], partials, sample, enc, dec,
                            out["center"], out["shifted"], extra, summaries, nb * B,
                            precomputed=False, logical_numel=n, block_symbols=B, lanes=L,
                            steps=S, fixed_words=W)
    dispatch.allocate_compact(src, summaries, out["counts"], out["descriptor"], buffer,
                              out["blocks"], extra, frees, nb, nb * B, logical_numel=n,
                              block_symbols=B, lanes=L, steps=S, precomputed=False)
    return out, nb * L * W


def _no_alloc(src, dist, buffer, frees):
    """The new entry point, through the C-ABI."""
    n = src.numel()
    out, (B, L, S, W), nb = _outputs(n, dist)
    enc, dec, _ = get_distribution_tables(dist, src.device)
    pending = hip.PendingFrees()
    pending.count = len(frees)
    for i, d in enumerate(frees):
        pending.descriptor[i] = d.data_ptr()
    p = lambda t: t.data_ptr()
    hip.call("lct_compress_buffered_noalloc", p(src), n, nb * B, hip.Geometry(B, L, S, W),
             p(enc), p(dec), p(out["side"]), p(out["encoded"]), p(out["center"]),
             p(out["shifted"]), p(out["samples"]), p(out["blocks"]), p(out["counts"]),
             p(out["descriptor"]), p(buffer.storage), buffer.max_free_regions, p(buffer.data),
             ctypes.byref(pending), torch.cuda.current_stream().cuda_stream)
    return out, nb * L * W


def _same(a, b, written_words):
    for key in a:
        x, y = a[key], b[key]
        if key == "encoded":
            x, y = x[:written_words], y[:written_words]
        assert torch.equal(x, y), key


@pytest.mark.parametrize("dist,first,second", [
    (SPARSE, lambda: _patterns(1, 37 * 65536 + 999), lambda: _patterns(2, 5 * 65536 + 3)),
    (GAUSS, lambda: _gaussian(3, 300 * 32768 + 17), lambda: _gaussian(4, 3000)),
    # The size limit: 8192 blocks run in several rounds of workgroups, so
    # blocks that finish (and store their summaries) precede blocks that start
    # (and read the sampler's partial sums); the working regions must not meet.
    (GAUSS, lambda: _gaussian_device(5, 8192 * 32768), lambda: _gaussian_device(6, 5000 * 32768 - 9)),
], ids=["overflowing-sparse", "gaussian", "gaussian-8192-blocks"])
def test_no_alloc_compress_equals_the_sequence_twice(dist, first, second):
    require_gpu()
    print(f"case no-alloc compress {dist.family.value}", flush=True)
    buf_a = TensorBuffer(16 << 20, device="cuda")
    buf_b = TensorBuffer(16 << 20, device="cuda")
    x1, x2 = first(), second()
    assert x2.numel() < x1.numel()
    out_a, words = _sequence(x1, dist, buf_a, [])
    out_b, _ = _no_alloc(x1, dist, buf_b, [])
    torch.cuda.synchronize()
    _same(out_a, out_b, words)
    assert int(out_b["descriptor"][2].item()) == 0
    # The second call frees the first reservation on its way in.
    out2_a, words2 = _sequence(x2, dist, buf_a, [out_a["descriptor"]])
    out2_b, _ = _no_alloc(x2, dist, buf_b, [out_b["descriptor"]])
    torch.cuda.synchronize()
    _same(out2_a, out2_b, words2)
    assert torch.equal(out_a["descriptor"], out_b["descriptor"])   # both freed (status 5)
    assert int(out_b["descriptor"][2].item()) == 5
    assert _free_regions_snapshot(buf_a) == _free_regions_snapshot(buf_b)
    assert torch.equal(buf_a.storage, buf_b.storage), "metadata or arena bytes differ"
