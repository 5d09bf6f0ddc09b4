"""One tensor beyond the reference's 10^9-element decode cutoff.

The reference switches its decoder to on-demand payload loads above 10^9
logical elements (LCT/kernels/autotune.py:58, LCT/kernels/dispatch.py:346);
the stored format and the decoded values stay the same.  Here one code path
serves every size, so this test takes a Gaussian tensor of 36 000 codec blocks
(about 1.18 x 10^9 elements, 2.36 GB of BF16: byte offsets of the input and of
the decoded output pass 2^31) through the public compress, private and into a
shared TensorBuffer, and checks every stored field against the oracle and the
decode bit for bit.  Random bit patterns in a few scattered blocks and in the
last two (the last one ragged) make streams overflow early, in the middle and
at the very end, so overflow offsets are large too.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_matches_oracle, oracle_compress, require_gpu
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution
from losslessly_compressed_tensors_amd.operations import compress, decompress
from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer, verify_buffer

pytestmark = pytest.mark.gpu

N_BLOCKS = 36000
BLOCK_SYMBOLS = 32768      # GAUSSIAN CLEAN
RAGGED = 1234              # elements missing from the last block
GAUSS = Distribution(DistType.GAUSSIAN)


def _large_input(seed):
    n = N_BLOCKS * BLOCK_SYMBOLS - RAGGED
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(n, generator=g, device="cuda").to(torch.bfloat16)
    bits = x.view(torch.int16)
    rng = np.random.default_rng(seed)
    chosen = sorted(rng.choice(N_BLOCKS - 2, 10, replace=False).tolist())
    last_valid = BLOCK_SYMBOLS - RAGGED
    for k in chosen + [N_BLOCKS - 2, N_BLOCKS - 1]:
        lo = k * BLOCK_SYMBOLS + int(rng.integers(0, last_valid - 4096))
        bits[lo:lo + 4096] = torch.from_numpy(
            rng.integers(-32768, 32768, 4096, dtype=np.int16)).cuda()
    return x


@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_compress_beyond_one_billion_elements(buffered):
    require_gpu()
    print(f"case large compress {N_BLOCKS} blocks buffered={buffered}", flush=True)
    x = _large_input(70)
    assert x.numel() > 10**9 and 2 * x.numel() > 2**31
    buffer = TensorBuffer(64 << 20, max_free_regions=64, device="cuda") if buffered else None
    host = oracle.Buffer(64 << 20, 64) if buffered else None
    ct = compress(x, GAUSS, buffer=buffer)
    o = oracle_compress(x, GAUSS, buffer=host)
    assert o.n_blocks == N_BLOCKS
    counts = o.blocks[:N_BLOCKS]
    assert counts[-1] > 0 and counts[-2] > 0, "the last two blocks overflow"
    assert int(o.blocks[2 * N_BLOCKS + N_BLOCKS - 1]) > 0, "the last block's tails start late"
    print(f"  oracle: {int(o.counts[0])} overflowing streams, {int(o.counts[1])} tail bytes",
          flush=True)
    assert_matches_oracle(ct, o)
    restored = decompress(ct)
    assert torch.equal(restored.view(torch.int16), x.view(torch.int16)), "decode differs"
    del restored
    if buffered:
        ct.free()
        verify_buffer(buffer)
