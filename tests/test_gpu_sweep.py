"""A seeded random sweep of the GPU path against the oracle.

Each case draws a size (1 element to 3 Mi elements, around the codec-block
and center-sample boundaries), a distribution (every family, noise level and
zero probability the layers use), a source (Gaussian at a random scale,
ReLU'd, or with a stretch of random bit patterns that forces escapes and
overflow) and private or buffered storage, then checks one path field for
field against the oracle:

* compress (the one-launch compress) and decompress;
* a fused update with compressed output: A + B, A * B, alpha * A + B and
  alpha * A + beta * B with random FP32 scalars;
* the two-operand update alpha * A + B (both compressed);
* a batched compress of up to 19 tensors (each record's payload and side
  bytes against its own oracle compress, and its decode).
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import (
    assert_matches_oracle, bits_of, oracle_compress, oracle_from_components, require_gpu,
)
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.operations import (
    a_compA_add_b_B, a_compA_add_B, a_compA_add_compB, compA_add_B, compA_mul_B, compress,
    compress_batch, decompress,
)
from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer, verify_buffer

pytestmark = pytest.mark.gpu

SIZES = [1, 7, 64, 1000, 4095, 4096, 4097, 32767, 32768, 65539, 200000, 1 << 20,
         3 * (1 << 20) + 17]
FAMILIES = [DistType.GAUSSIAN, DistType.LAPLACE, DistType.EMPIRICAL]
NOISE = [NoiseLevel.CLEAN, NoiseLevel.MEDIUM, NoiseLevel.HIGH, NoiseLevel.SPARSE]


def _distribution(rng):
    return Distribution(FAMILIES[rng.integers(len(FAMILIES))],
                        zero_prob=float(rng.choice([0.0, 0.0, 0.01, 0.5])),
                        noise_level=NOISE[rng.integers(len(NOISE))])


def _source(rng, n):
    kind = int(rng.integers(5))
    g = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    x = torch.randn(n, generator=g) * float(10.0 ** rng.uniform(-4, 2))
    if kind == 1:
        x = torch.relu(x)
    x = x.to(torch.bfloat16)
    if kind >= 2:   # a stretch of random bit patterns: escapes and overflow
        bits = x.view(torch.int16).numpy()
        k = int(rng.integers(1, max(2, n // (4 if kind == 4 else 50))))
        lo = int(rng.integers(0, max(1, n - k)))
        bits[lo:lo + k] = rng.integers(-32768, 32768, min(k, n - lo), dtype=np.int16)
    return x


def _scalar(rng):
    value = float(np.float32(rng.uniform(-2, 2)))
    return value, torch.tensor([value], dtype=torch.float32, device="cuda")


def _compress_case(rng, n, dist, buf, host):
    x = _source(rng, n)
    ct = compress(x.cuda(), dist, buffer=buf)
    assert_matches_oracle(ct, oracle_compress(x, dist, buffer=host))
    assert np.array_equal(bits_of(decompress(ct)), bits_of(x))


def _update_case(rng, n, dist, buf, host):
    x, b = _source(rng, n), _source(rng, n)
    ct = compress(x.cuda(), dist, buffer=buf)
    o = oracle_compress(x, dist, buffer=host)
    alpha, alpha_t = _scalar(rng)
    beta, beta_t = _scalar(rng)
    op = int(rng.integers(4))
    if op == 0:
        r = compA_add_B(ct, b.cuda(), dense_output=False, buffer=buf)
        args = (oracle.OP_ADD, 1.0, 1.0, False, True)
    elif op == 1:
        r = compA_mul_B(ct, b.cuda(), dense_output=False, buffer=buf)
        args = (oracle.OP_MULTIPLY, 1.0, 1.0, False, True)
    elif op == 2:
        r = a_compA_add_B(ct, alpha_t, b.cuda(), dense_output=False, buffer=buf)
        args = (oracle.OP_SCALAR_MUL_ADD, alpha, 1.0, False, True)
    else:
        r = a_compA_add_b_B(ct, alpha_t, b.cuda(), beta_t, dense_output=False, buffer=buf)
        args = (oracle.OP_SCALAR_MUL_ADD, alpha, beta, False, False)
    side, exponents = oracle.pointwise(o, bits_of(b), *args, policy=1)
    assert_matches_oracle(r, oracle_from_components(side, exponents, dist, buffer=host))


def _dual_case(rng, n, dist, buf, host):
    x, y = _source(rng, n), _source(rng, n)
    ca, cb = compress(x.cuda(), dist, buffer=buf), compress(y.cuda(), dist, buffer=buf)
    oa, ob = oracle_compress(x, dist, buffer=host), oracle_compress(y, dist, buffer=host)
    alpha, alpha_t = _scalar(rng)
    r = a_compA_add_compB(ca, alpha_t, cb, dense_output=False, buffer=buf)
    side, exponents = oracle.dual(oa, ob, alpha, policy=1)
    assert_matches_oracle(r, oracle_from_components(side, exponents, dist, buffer=host))


def _batch_case(rng, n, dist, buf, host):
    xs = [_source(rng, max(1, n // (1 + int(rng.integers(4)))))
          for _ in range(int(rng.integers(1, 20)))]
    buffer = TensorBuffer(128 << 20, max_free_regions=64, device="cuda")
    for x, ct in zip(xs, compress_batch([x.cuda() for x in xs], dist, buffer=buffer)):
        o = oracle_compress(x, dist)
        words = o.encoded.size - 4
        assert np.array_equal(ct.data.cpu().numpy()[:words], o.encoded[:words])
        assert np.array_equal(ct.sign_mantissa.cpu().numpy(), o.side)
        assert np.array_equal(bits_of(decompress(ct)), bits_of(x))
    verify_buffer(buffer)


CASES = [_compress_case, _update_case, _dual_case, _batch_case]


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_random_sweep_matches_the_oracle(seed):
    require_gpu()
    rng = np.random.default_rng(seed)
    for k in range(40):
        case = CASES[int(rng.integers(len(CASES)))]
        n = int(rng.choice(SIZES))
        dist = _distribution(rng)
        buffered = bool(rng.integers(2))
        print(f"case sweep seed={seed} #{k} {case.__name__} n={n} {dist} buffered={buffered}",
              flush=True)
        buf = TensorBuffer(64 << 20, max_free_regions=64, device="cuda") if buffered else None
        host = oracle.Buffer(64 << 20, 64) if buffered else None
        case(rng, n, dist, buf, host)
        if buffered:
            verify_buffer(buf)
