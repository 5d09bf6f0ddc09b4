"""GPU parity of the batched fused update (``lct_pointwise_update_batch``).

The batched update has no counterpart in the reference, which updates one
tensor per call (``LCT/LCTensor.py:91-99`` -> ``LCT/codec/pointwise.py:262-278``);
each tensor of a batch must store what that call stores.  Each batched result
is checked against the same update made one tensor at a time
(``a_compA_add_B`` / ``a_compA_add_b_B`` with compressed output, themselves
checked against the oracle in ``test_gpu_update.py``) and against
``oracle.apply_array`` on the decoded values:

* every stored field (payload, side bytes, center, shifted decode table,
  totals, block metadata, recorded sample values) and the overflow region's
  lanes | starts | tails at whatever arena offset the reservation got;
* ``a * A + B`` (alpha read and alpha = 1), ``a * A + b * B``, operands with
  and without overflow, a single-block tensor, a ragged tail, both step
  counts (one launch per count) and more than 8 tensors (several launches);
* the buffer's deferred frees are applied before the batch's reservations;
* ``LCTTensor.mul_add_many`` equals ``mul_add_`` tensor by tensor.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import bits_of, require_gpu
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
from losslessly_compressed_tensors_amd.operations import (
    a_compA_add_B, a_compA_add_b_B, a_compA_add_b_B_batch, compress, decompress,
)
from losslessly_compressed_tensors_amd.tensor_buffer import (
    STATUS_EMPTY, STATUS_FREED, STATUS_OK, TensorBuffer, verify_buffer,
)

pytestmark = pytest.mark.gpu

GAUSS = Distribution(DistType.GAUSSIAN)                                 # 256 steps
LAPLACE = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN)   # 128 steps
EMPIRICAL = Distribution(DistType.EMPIRICAL)


def _gaussian(n, seed, std=1.0):
    return (torch.randn(n, generator=torch.Generator().manual_seed(seed)) * std).to(torch.bfloat16)


def _with_patterns(n, seed, std=1.0, count=4096):
    """Gaussian values with ``count`` random bit patterns near the end, so
    that some streams overflow."""
    x = _gaussian(n, seed, std)
    bits = x.view(torch.int16).numpy()
    rng = np.random.default_rng(seed)
    lo = max(0, n - count - 123)
    bits[lo:lo + count] = rng.integers(-32768, 32768, min(count, n - lo), dtype=np.int16)
    return x


def _fields(ct):
    """The stored fields of a buffered record, its overflow region included."""
    B, L, S, W = ct.codec_geometry
    ns = ct.size // B * L
    count, used = int(ct.fallback_count.item()), int(ct.fallback_used.item())
    desc = ct.fallback_descriptor.cpu().numpy()
    status = int(desc[2])
    assert status == (STATUS_OK if count else STATUS_EMPTY), status
    region = ct.buffer.data.cpu().numpy()[int(desc[0]): int(desc[0]) + 2 * count + used]
    return dict(payload=ct.data.cpu().numpy()[: ns * W], side=ct.sign_mantissa.cpu().numpy(),
                center=int(ct.center.item()), table=ct.decode_table.cpu().numpy(),
                totals=(count, used), blocks=ct.fallback_blocks.cpu().numpy(),
                size=int(desc[1]), region=region if count else region[:0],
                samples=ct.sample_values.cpu().numpy())


def _assert_same(batched, single):
    a, b = _fields(batched), _fields(single)
    for key in a:
        assert np.array_equal(np.asarray(a[key]), np.asarray(b[key])), key
    assert batched.memory_size() == single.memory_size()


CASES = [
    ("gauss-ragged", 3 * 65536 - 11, GAUSS, 1.0),
    ("gauss-overflow", 5 * 65536, GAUSS, 1.0),
    ("laplace-one-block", 1000, LAPLACE, 0.02),
    ("laplace-overflow", 9 * 32768 - 5, LAPLACE, 0.02),
    ("empirical", 12 * 65536 + 3, EMPIRICAL, 1e-3),
]


@pytest.fixture(autouse=True)
def _gpu():
    require_gpu()


@pytest.mark.parametrize("form", ["axpy", "axpy-alpha-one", "axpby"])
def test_batch_equals_single_updates(form):
    """Every form of the Muon/SGD weight step, tensor by tensor."""
    print(f"case batched update form={form}", flush=True)
    buffer, single_buffer = (TensorBuffer(256 << 20, device="cuda") for _ in range(2))
    alpha = torch.tensor([0.95], dtype=torch.float32, device="cuda")
    beta = torch.tensor([-0.01], dtype=torch.float32, device="cuda")
    As, Bs, dists = [], [], []
    for k, (name, n, dist, std) in enumerate(CASES):
        x = (_with_patterns if "overflow" in name else _gaussian)(n, 10 + k, std)
        As.append((compress(x.cuda(), dist, buffer=buffer),
                   compress(x.cuda(), dist, buffer=single_buffer), x))
        Bs.append(_gaussian(n, 50 + k, std).cuda())
        dists.append(dist)
    b = beta if form == "axpby" else None
    alpha_is_one = form == "axpy-alpha-one"
    batched = a_compA_add_b_B_batch([a for a, _, _ in As], alpha, Bs, b,
                                    alpha_is_one=alpha_is_one, buffer=buffer)
    for (name, n, dist, _), (_, a_single, x), B, out in zip(CASES, As, Bs, batched):
        print(f"case {name}", flush=True)
        if b is None:
            single = a_compA_add_B(a_single, alpha, B, alpha_is_one=alpha_is_one,
                                   dense_output=False, buffer=single_buffer, distribution=dist)
        else:
            single = a_compA_add_b_B(a_single, alpha, B, b, dense_output=False,
                                     buffer=single_buffer, distribution=dist)
        _assert_same(out, single)
        expected = oracle.apply_array(oracle.OP_SCALAR_MUL_ADD, bits_of(x), bits_of(B),
                                      1.0 if alpha_is_one else 0.95,
                                      -0.01 if b is not None else 1.0,
                                      alpha_is_one=alpha_is_one, beta_is_one=b is None)
        assert np.array_equal(bits_of(decompress(out)), expected), name
    verify_buffer(buffer)


def test_batches_of_more_than_eight_and_deferred_frees():
    """19 tensors (three launches of 8, 8 and 3) after the previous values'
    frees were deferred: the frees ride on the first launch and every result
    equals its single update."""
    buffer, single_buffer = (TensorBuffer(128 << 20, device="cuda") for _ in range(2))
    alpha = torch.tensor([0.9], dtype=torch.float32, device="cuda")
    xs = [_with_patterns(32768 * (1 + k % 4) - 7 * k, 200 + k, 0.02, 512) for k in range(19)]
    Bs = [_gaussian(x.numel(), 300 + k, 0.02).cuda() for k, x in enumerate(xs)]
    # Three earlier tensors with overflow (so each holds an arena region).
    old = [compress(_with_patterns(65536, 100 + k, 0.02, 16384).cuda(), LAPLACE, buffer=buffer)
           for k in range(3)]
    assert [int(ct.fallback_descriptor[2].item()) for ct in old] == [STATUS_OK] * 3
    As = [compress(x.cuda(), LAPLACE, buffer=buffer) for x in xs]
    for ct in old:
        ct.free()                                  # deferred to the next reservation
    assert len(buffer._pending_frees) == 3
    batched = a_compA_add_b_B_batch(As, alpha, Bs, buffer=buffer)
    assert not buffer._pending_frees
    assert [int(ct.fallback_descriptor[2].item()) for ct in old] == [STATUS_FREED] * 3
    for k, (x, B, out) in enumerate(zip(xs, Bs, batched)):
        single = a_compA_add_B(compress(x.cuda(), LAPLACE, buffer=single_buffer), alpha, B,
                               dense_output=False, buffer=single_buffer)
        _assert_same(out, single)
    verify_buffer(buffer)


def test_mul_add_many_equals_mul_add():
    """The Muon weight step of a shape group: LCTTensor.mul_add_many against
    mul_add_ per tensor, two steps in a row (the second reads the first's
    recorded sample values)."""
    weight_dist = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN, zero_prob=0.01)
    buffer, single_buffer = (TensorBuffer(64 << 20, device="cuda") for _ in range(2))
    decay = torch.tensor([1 - 0.05 * 0.01], dtype=torch.float32, device="cuda")
    neg_lr = torch.tensor([-0.05], dtype=torch.float32, device="cuda")
    shapes = [(768, 768)] * 5 + [(768, 3072), (3072, 768)]
    ws = [(torch.randn(*s, generator=torch.Generator().manual_seed(400 + k)) * 0.03)
          .to(torch.bfloat16).cuda() for k, s in enumerate(shapes)]
    batched = [LCTTensor(w, buffer, weight_dist) for w in ws]
    single = [LCTTensor(w, single_buffer, weight_dist) for w in ws]
    for step in range(2):
        updates = [(torch.randn(*s, generator=torch.Generator().manual_seed(500 + 10 * step + k))
                    * 0.1).to(torch.bfloat16).cuda() for k, s in enumerate(shapes)]
        LCTTensor.mul_add_many(batched, decay, updates, beta=neg_lr)
        for t, u in zip(single, updates):
            t.mul_add_(decay, u, beta=neg_lr)
        for t_batched, t_single in zip(batched, single):
            _assert_same(t_batched.x, t_single.x)
    verify_buffer(buffer)
