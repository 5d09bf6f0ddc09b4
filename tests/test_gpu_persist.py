"""The lct-v1 file format on the GPU: compressed tensors (private and
buffer-backed, with overflow) survive save and load into private storage or a
TensorBuffer and decode bit for bit; a record assembled from the oracle's
reference-format fields decodes on the GPU; a loaded tensor takes a fused
update like any other."""
import io

import numpy as np
import pytest
import torch

import oracle
from gpu_util import assert_matches_oracle, bits_of, oracle_compress, oracle_from_components, require_gpu
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.operations import a_compA_add_B, compress, decompress
from losslessly_compressed_tensors_amd.persist import load_compressed, save_compressed
from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer, verify_buffer
from test_cpu_persist import _oracle_record, _patterns

pytestmark = pytest.mark.gpu

DIST = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE)


def _round_trip(ct, buffer=None):
    blob = io.BytesIO()
    save_compressed(ct, blob)
    blob.seek(0)
    return load_compressed(blob, device="cuda", buffer=buffer)


@pytest.mark.parametrize("source", ["private", "buffered"])
@pytest.mark.parametrize("target", ["private", "buffered"])
def test_compressed_tensor_round_trip(source, target):
    require_gpu()
    print(f"case persist {source} -> {target}", flush=True)
    bits = _patterns(5 * 65536 + 321, 7)
    x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    src_buffer = TensorBuffer(8 << 20, max_free_regions=64, device="cuda") \
        if source == "buffered" else None
    dst_buffer = TensorBuffer(8 << 20, max_free_regions=64, device="cuda") \
        if target == "buffered" else None
    ct = compress(x.cuda(), DIST, buffer=src_buffer)
    assert int(ct.fallback_count.item()) > 0
    back = _round_trip(ct, dst_buffer)
    assert np.array_equal(bits_of(decompress(back)), bits)
    assert torch.equal(back.data, ct.data) and torch.equal(back.sign_mantissa, ct.sign_mantissa)
    assert torch.equal(back.fallback_blocks, ct.fallback_blocks)
    if source == "private" and target == "private":
        assert back.memory_size() == ct.memory_size()
    if target == "buffered":
        assert int(back.fallback_descriptor[2].item()) == 0
        back.free()
        verify_buffer(dst_buffer)
    if source == "buffered":
        ct.free()
        verify_buffer(src_buffer)


def test_reference_format_record_decodes_on_the_gpu():
    """Fields produced by the oracle's restatement of the reference encoder,
    written as lct-v1 on the CPU, load and decode on the GPU."""
    require_gpu()
    bits = _patterns(3 * 65536 + 99, 8)
    ct_cpu, o = _oracle_record(bits.view(np.int16), DIST, (bits.size,))
    assert o.counts[0] > 0
    blob = io.BytesIO()
    save_compressed(ct_cpu, blob)
    blob.seek(0)
    loaded = load_compressed(blob, device="cuda")
    assert np.array_equal(bits_of(decompress(loaded)), bits)


def test_loaded_tensor_takes_a_fused_update():
    require_gpu()
    dist = Distribution(DistType.EMPIRICAL)
    g = torch.Generator().manual_seed(9)
    m = (torch.randn(700, 900, generator=g) * 1e-3).to(torch.bfloat16)
    u = (torch.randn(700, 900, generator=g) * 1e-2).to(torch.bfloat16)
    loaded = _round_trip(compress(m.cuda(), dist))
    alpha = torch.tensor([float(np.float32(0.95))], dtype=torch.float32, device="cuda")
    result = a_compA_add_B(loaded, alpha, u.cuda(), dense_output=False)
    o = oracle_compress(m, dist)
    side, exponents = oracle.pointwise(o, bits_of(u), oracle.OP_SCALAR_MUL_ADD,
                                       float(np.float32(0.95)), policy=1)
    assert_matches_oracle(result, oracle_from_components(side, exponents, dist))
