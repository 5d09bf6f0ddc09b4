"""GPU parity of the single-pass compressed-output pointwise path.

``lct_pointwise_sample`` + ``lct_pointwise_encode`` replace the reference's
pointwise COMPRESSED_OUTPUT launch followed by the re-encode of its components
(LCT/codec/pointwise.py:262-278, LCT/codec/encode.py:22-186).  Checks:

* the sampler's per-group exponent sums and counts equal the oracle's result
  at the oracle's sample positions, group by group (a wrong sample changes a
  sum even where the rounded center would not move);
* the public API's compressed output equals, field by field, the oracle's
  re-encode of the oracle's pointwise components, also where the result
  overflows and where n < 4096 (every element sampled);
* the two-pass kernel (``lct_pointwise_dense`` with COMPRESSED_OUTPUT), still
  used by the two-compressed path, writes the oracle's components.
"""
import dataclasses

import numpy as np
import pytest
import torch

import oracle
from gpu_util import (
    assert_matches_oracle,
    bits_of,
    oracle_compress,
    oracle_from_components,
    require_gpu,
)
from losslessly_compressed_tensors_amd.codec.decode import overlay_of, shifted_decode_table
from losslessly_compressed_tensors_amd.comp_format import DistType, Distribution, NoiseLevel
from losslessly_compressed_tensors_amd.compression.huffman_tables import get_distribution_tables
from losslessly_compressed_tensors_amd.kernels import dispatch, hip
from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
from losslessly_compressed_tensors_amd.operations import (
    a_compA_add_B,
    a_compA_add_b_B,
    a_compA_add_compB,
    compA_add_B,
    compA_mul_B,
    compress,
    decompress,
)
from losslessly_compressed_tensors_amd.tensor_buffer import (
    FAIL_INCOMPLETE, STATUS_INCOMPLETE, BufferReservationError, TensorBuffer,
    _free_regions_snapshot, verify_buffer,
)

pytestmark = pytest.mark.gpu

ALPHA = float(np.float32(0.95))
BETA = float(np.float32(-1.25))


def _gaussian(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def _patterns(seed, n=65536):
    """BF16 patterns (all 65536, shuffled, cycled to n): escapes, overflow,
    NaN and infinities."""
    rng = np.random.default_rng(seed)
    bits = np.arange(65536, dtype=np.uint16)
    rng.shuffle(bits)
    bits = np.resize(bits, n)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def _spread(shape, seed):
    """Values whose exponents spread over +-40 binades: results of a multiply
    with them overflow many streams."""
    g = torch.Generator().manual_seed(seed)
    scale = torch.exp2(torch.randint(-40, 40, shape, generator=g).float())
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


# (name, distribution, A, B)
CASES = [
    ("gaussian", Distribution(DistType.GAUSSIAN), lambda: _gaussian((1024, 1024), 0),
     lambda: _gaussian((1024, 1024), 1, 0.5)),
    ("patterns-sparse", Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE),
     lambda: _patterns(2), lambda: _gaussian((65536,), 3)),
    ("ragged-medium", Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM),
     lambda: _gaussian((3, 33333), 4), lambda: _gaussian((3, 33333), 5, 4.0)),
    ("tiny-every-sample", Distribution(DistType.GAUSSIAN), lambda: _gaussian((37, 41), 6),
     lambda: _gaussian((37, 41), 7)),
    ("empirical-high", Distribution(DistType.EMPIRICAL, noise_level=NoiseLevel.HIGH),
     lambda: _patterns(8, 3 * 32768 + 1000), lambda: _spread((3 * 32768 + 1000,), 9)),
    ("empirical-clean", Distribution(DistType.EMPIRICAL), lambda: _gaussian((512, 1100), 10, 1e-3),
     lambda: _gaussian((512, 1100), 11, 1e-2)),
]

# (name, op code, public call, alpha, beta, alpha_is_one, beta_is_one)
OPS = [
    ("add", oracle.OP_ADD, lambda A, B, **kw: compA_add_B(A, B, **kw), 1.0, 1.0, False, True),
    ("mul", oracle.OP_MULTIPLY, lambda A, B, **kw: compA_mul_B(A, B, **kw), 1.0, 1.0, False,
     True),
    ("axpy", oracle.OP_SCALAR_MUL_ADD,
     lambda A, B, **kw: a_compA_add_B(A, _scalar(ALPHA), B, **kw), ALPHA, 1.0, False, True),
    ("axpy-alpha-one", oracle.OP_SCALAR_MUL_ADD,
     lambda A, B, **kw: a_compA_add_B(A, _scalar(ALPHA), B, alpha_is_one=True, **kw),
     ALPHA, 1.0, True, True),
    ("axpby", oracle.OP_SCALAR_MUL_ADD,
     lambda A, B, **kw: a_compA_add_b_B(A, _scalar(ALPHA), B, _scalar(BETA), **kw),
     ALPHA, BETA, False, False),
    ("axpby-alpha-one", oracle.OP_SCALAR_MUL_ADD,
     lambda A, B, **kw: a_compA_add_b_B(A, _scalar(ALPHA), B, _scalar(BETA),
                                        alpha_is_one=True, **kw),
     ALPHA, BETA, True, False),
]


def _scalar(value):
    return torch.tensor([value], dtype=torch.float32, device="cuda")


def _launch_args(ct, op):
    _, code, _, _, _, alpha_is_one, beta_is_one = op
    scaled = code == oracle.OP_SCALAR_MUL_ADD
    B, L, S, W = ct.codec_geometry
    _, _, rare = get_distribution_tables(ct.distribution, ct.data.device)
    return dict(rare_length=rare, logical_numel=ct.logical_numel, block_symbols=B, lanes=L,
                steps=S, fixed_words=W, op=code, alpha_is_one=(not scaled) or alpha_is_one,
                beta_is_one=(not scaled) or beta_is_one, overflow=overlay_of(ct))


def _group_sums(values: np.ndarray, precomputed: bool = False) -> np.ndarray:
    """Per 64-sample group: the kept exponents' sum and count (tables.py:15-49)."""
    raw = values.astype(np.int64) if precomputed else (values.astype(np.int64) >> 7) & 255
    exponents = raw - 127
    keep = exponents >= -120
    groups = -(-values.size // 64)
    padded = np.zeros(groups * 64, dtype=np.int64)
    kept = np.zeros(groups * 64, dtype=np.int64)
    padded[:values.size] = np.where(keep, exponents, 0)
    kept[:values.size] = keep
    return np.stack([padded.reshape(groups, 64).sum(1), kept.reshape(groups, 64).sum(1)], 1)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("op", OPS, ids=[o[0] for o in OPS])
@pytest.mark.parametrize("recorded", [False, True], ids=["streams", "recorded"])
def test_sampler_partials_match_the_oracle(case, op, recorded):
    """The sampler's group sums and its recorded result values, both from A's
    streams and from A's recorded sample values."""
    require_gpu()
    name, dist, make_a, make_b = case
    op_name, code, _, alpha, beta, alpha_is_one, beta_is_one = op
    print(f"case sampler {name} {op_name} recorded={recorded}", flush=True)
    a, b = make_a(), make_b()
    ct = compress(a.cuda(), dist)
    n = ct.logical_numel
    sample_size = min(n, 4096)
    groups = -(-sample_size // 64)
    partials = torch.full((2 * groups,), -7, dtype=torch.int32, device="cuda")
    result_samples = torch.full((sample_size,), -7, dtype=torch.int16, device="cuda")
    args = _launch_args(ct, op)
    assert ct.sample_values is not None and ct.sample_values.numel() == sample_size
    dispatch.pointwise_sample(ct.data, ct.sign_mantissa, shifted_decode_table(ct), ct.center,
                              b.cuda().reshape(-1),
                              None if args["alpha_is_one"] else _scalar(alpha),
                              None if args["beta_is_one"] else _scalar(beta), partials, ct.size,
                              sample_size=sample_size,
                              a_samples=ct.sample_values if recorded else None,
                              result_samples=result_samples, **args)
    o = oracle_compress(a, dist)
    dense = oracle.pointwise(o, bits_of(b), code, alpha, beta, alpha_is_one, beta_is_one)
    expected_values = dense[oracle.sample_positions(n)]
    assert np.array_equal(bits_of(result_samples), expected_values)
    got = partials.cpu().numpy().reshape(groups, 2)
    assert np.array_equal(got, _group_sums(expected_values))


@pytest.mark.parametrize("n", [1, 63, 4095, 4096, 4097, 99999, 1 << 20])
@pytest.mark.parametrize("precomputed", [False, True], ids=["bf16", "exponent-bytes"])
def test_sample_center_and_sampled_encoder(n, precomputed):
    """lct_sample_center's group sums and recorded values, and the center and
    shifted decode table that lct_encode_sampled derives from them, against
    the oracle's sampler (tables.py:15-128)."""
    require_gpu()
    print(f"case sample-center n={n} precomputed={precomputed}", flush=True)
    x = _patterns(30 + n % 7, n) if n < 65536 else _gaussian((n,), 31)
    bits = bits_of(x)
    source = torch.from_numpy(((bits >> 7) & 255).astype(np.uint8)) if precomputed \
        else x.view(torch.int16)
    sample_size = min(n, 4096)
    groups = -(-sample_size // 64)
    partials = torch.full((2 * groups,), -7, dtype=torch.int32, device="cuda")
    values = torch.full((sample_size,), -7, dtype=torch.int16, device="cuda")
    dispatch.sample_center(source.cuda(), n, sample_size, precomputed, partials, values)
    positions = oracle.sample_positions(n)
    sampled = ((bits[positions] >> 7) & 255) if precomputed else bits[positions]
    assert np.array_equal(partials.cpu().numpy().reshape(groups, 2),
                          _group_sums(sampled, precomputed))
    if not precomputed:
        assert np.array_equal(bits_of(values), bits[positions])
    else:
        assert np.all(values.cpu().numpy() == -7), "exponent-byte sources record nothing"
    dist = Distribution(DistType.GAUSSIAN)
    ct = compress(x.cuda(), dist)
    o = oracle_compress(x, dist)
    assert int(ct.center.item()) == o.center == oracle.estimate_center(bits.view(np.int16))
    assert np.array_equal(ct.decode_table.cpu().numpy(), o.shifted_decode)
    assert np.array_equal(bits_of(ct.sample_values), bits[positions])


@pytest.mark.parametrize("case", CASES[:3], ids=[c[0] for c in CASES[:3]])
def test_reference_table_and_encoder_entry_points(case):
    """The one-launch table kernel (dispatch.py:33-48) and the encoder with a
    given shifted table (dispatch.py:294-316), which compress no longer
    sequences, still produce the oracle's center, tables and payload."""
    require_gpu()
    name, dist, make_a, _ = case
    a = make_a()
    bits = bits_of(a)
    o = oracle_compress(a, dist)
    encode_table, decode_table, _ = get_distribution_tables(dist, "cuda")
    n = bits.size
    center = torch.empty(1, dtype=torch.int32, device="cuda")
    shifted_encode = torch.empty(256, dtype=torch.int32, device="cuda")
    shifted_decode = torch.empty(1024, dtype=torch.int32, device="cuda")
    source = a.cuda().reshape(-1).view(torch.int16)
    dispatch.estimate_and_shift_encoding_table(source, center, n, encode_table, shifted_encode,
                                               decode_table, shifted_decode, min(n, 4096), False)
    assert int(center.item()) == o.center
    assert np.array_equal(shifted_decode.cpu().numpy(), o.shifted_decode)
    B, L, S, W = o.geometry
    nb = -(-n // B)
    encoded = torch.empty(nb * L * W + 4, dtype=torch.int32, device="cuda")
    side = torch.empty(nb * B, dtype=torch.uint8, device="cuda")
    extra = torch.empty(nb * L, dtype=torch.uint8, device="cuda")
    summaries = torch.empty(5 * nb + 1, dtype=torch.int32, device="cuda")
    dispatch.encode_kernel(source, side, encoded, shifted_encode, extra, summaries, nb * B,
                           nb * L, precomputed=False, logical_numel=n, block_symbols=B, lanes=L,
                           steps=S, fixed_words=W, write_summary=True)
    assert np.array_equal(encoded.cpu().numpy()[: nb * L * W], o.encoded[: nb * L * W])
    assert np.array_equal(side.cpu().numpy(), o.side)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("op", OPS, ids=[o[0] for o in OPS])
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_single_pass_compressed_output(case, op, buffered):
    require_gpu()
    name, dist, make_a, make_b = case
    op_name, code, call, alpha, beta, alpha_is_one, beta_is_one = op
    print(f"case single-pass {name} {op_name} buffered={buffered}", flush=True)
    a, b = make_a(), make_b()
    buffer = TensorBuffer(8 << 20, max_free_regions=64, device="cuda") if buffered else None
    host = oracle.Buffer(8 << 20, 64) if buffered else None
    ct = compress(a.cuda(), dist, buffer=buffer)
    o = oracle_compress(a, dist, buffer=host)
    result = call(ct, b.cuda(), dense_output=False, buffer=buffer)
    side, exponents = oracle.pointwise(o, bits_of(b), code, alpha, beta, alpha_is_one,
                                       beta_is_one, policy=1)
    expected = oracle_from_components(side, exponents, dist, buffer=host)
    assert_matches_oracle(result, expected)
    dense = oracle.pointwise(o, bits_of(b), code, alpha, beta, alpha_is_one, beta_is_one)
    assert np.array_equal(bits_of(decompress(result)), dense)
    if buffered:
        result.free()
        ct.free()
        verify_buffer(buffer)


def test_cases_exercise_overflow():
    """The overflow branches of the single-pass kernel are reached: A
    overflows in the pattern cases, and so does the multiply's result."""
    require_gpu()
    _, dist, make_a, make_b = CASES[4]
    a, b = make_a(), make_b()
    o = oracle_compress(a, dist)
    assert o.counts[0] > 0
    side, exponents = oracle.pointwise(o, bits_of(b), oracle.OP_MULTIPLY, policy=1)
    assert oracle_from_components(side, exponents, dist).counts[0] > 0


def test_result_distribution_differs_from_the_input():
    """Compressed output under another distribution of the same geometry:
    the result is encoded with that distribution's tables."""
    require_gpu()
    src, out = Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM), \
        Distribution(DistType.LAPLACE, noise_level=NoiseLevel.MEDIUM)
    a, b = _gaussian((700, 900), 12), _gaussian((700, 900), 13, 0.1)
    ct = compress(a.cuda(), src)
    result = a_compA_add_B(ct, _scalar(ALPHA), b.cuda(), dense_output=False, distribution=out)
    o = oracle_compress(a, src)
    side, exponents = oracle.pointwise(o, bits_of(b), oracle.OP_SCALAR_MUL_ADD, ALPHA, policy=1)
    assert_matches_oracle(result, oracle_from_components(side, exponents, out))


@pytest.mark.parametrize("case", CASES[:3], ids=[c[0] for c in CASES[:3]])
def test_two_pass_kernel_components(case):
    """lct_pointwise_dense with COMPRESSED_OUTPUT: side bytes (storage order,
    padding 0) and exponent bytes (logical order) equal the oracle's."""
    require_gpu()
    name, dist, make_a, make_b = case
    print(f"case two-pass components {name}", flush=True)
    a, b = make_a(), make_b()
    ct = compress(a.cuda(), dist)
    op = OPS[4]
    args = _launch_args(ct, op)
    args.pop("sample_size", None)
    side = torch.empty(ct.size, dtype=torch.uint8, device="cuda")
    exponents = torch.empty(ct.logical_numel, dtype=torch.uint8, device="cuda")
    dispatch.pointwise_dense(ct.data, ct.sign_mantissa, b.cuda().reshape(-1), side, exponents,
                             shifted_decode_table(ct), ct.size, ct.center, _scalar(ALPHA),
                             _scalar(BETA), output_policy=1, **args)
    o = oracle_compress(a, dist)
    expect_side, expect_exponents = oracle.pointwise(o, bits_of(b), op[1], ALPHA, BETA, False,
                                                     False, policy=1)
    assert np.array_equal(side.cpu().numpy(), expect_side)
    assert np.array_equal(exponents.cpu().numpy(), expect_exponents)


def test_momentum_sequence_single_pass():
    """Twelve mul_add_ steps on a buffer-backed LCTTensor (the momentum update
    shape of config C4, smaller), each checked against the oracle."""
    require_gpu()
    dist = Distribution(DistType.EMPIRICAL)
    shape = (1024, 1100)
    buffer = TensorBuffer(16 << 20, max_free_regions=64, device="cuda")
    host = oracle.Buffer(16 << 20, 64)
    m0 = _gaussian(shape, 20, 1e-3)
    tensor = LCTTensor(m0.cuda(), buffer, dist)
    state = oracle_compress(m0, dist, buffer=host)
    for step in range(12):
        g = _gaussian(shape, 200 + step, 1e-2)
        tensor.mul_add_(_scalar(ALPHA), g.cuda())
        side, exponents = oracle.pointwise(state, bits_of(g), oracle.OP_SCALAR_MUL_ADD, ALPHA,
                                           policy=1)
        previous = state
        state = oracle_from_components(side, exponents, dist, buffer=host)
        host.free(previous.descriptor)
        assert_matches_oracle(tensor.x, state)
    tensor.free()
    verify_buffer(buffer)


# ---- two compressed operands: alpha * A + B (LCTTensor.add_comp_)

# (name, A's distribution, B's distribution, A, B): the operands share a stream
# geometry; the patterns cases overflow in A, in B or in both.
DUAL_CASES = [
    ("gaussian", Distribution(DistType.GAUSSIAN), Distribution(DistType.GAUSSIAN),
     lambda: _gaussian((1024, 1024), 40), lambda: _gaussian((1024, 1024), 41, 0.5)),
    ("patterns-both", Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE),
     Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE),
     lambda: _patterns(42), lambda: _patterns(43)),
    ("patterns-b-only", Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM),
     Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM),
     lambda: _gaussian((3, 33333), 44), lambda: _patterns(45, 3 * 33333)),
    ("tiny-every-sample", Distribution(DistType.GAUSSIAN, noise_level=NoiseLevel.MEDIUM),
     Distribution(DistType.LAPLACE, noise_level=NoiseLevel.MEDIUM),
     lambda: _gaussian((37, 41), 46), lambda: _gaussian((37, 41), 47)),
    ("empirical-high", Distribution(DistType.EMPIRICAL, noise_level=NoiseLevel.HIGH),
     Distribution(DistType.EMPIRICAL, noise_level=NoiseLevel.HIGH),
     lambda: _spread((3 * 32768 + 1000,), 48), lambda: _patterns(49, 3 * 32768 + 1000)),
]

# Which operands' recorded sample values the sampler is given.
RECORDED = [(False, False), (True, False), (False, True), (True, True)]


def _dual_operands(case, buffer=None, host=None):
    name, dist_a, dist_b, make_a, make_b = case
    a = make_a()
    b = make_b().reshape(a.shape)
    ca, cb = compress(a.cuda(), dist_a, buffer=buffer), compress(b.cuda(), dist_b, buffer=buffer)
    assert ca.codec_geometry == cb.codec_geometry, "dual cases need one stream geometry"
    oa = oracle_compress(a, dist_a, buffer=host)
    ob = oracle_compress(b, dist_b, buffer=host)
    return ca, cb, oa, ob


@pytest.mark.parametrize("case", DUAL_CASES, ids=[c[0] for c in DUAL_CASES])
@pytest.mark.parametrize("recorded", RECORDED, ids=["streams", "a-recorded", "b-recorded",
                                                    "both-recorded"])
def test_dual_sampler_partials_match_the_oracle(case, recorded):
    """lct_dual_sample's group sums and recorded result values, with each
    operand's value taken from its streams or from its recorded samples."""
    require_gpu()
    print(f"case dual sampler {case[0]} recorded={recorded}", flush=True)
    ca, cb, oa, ob = _dual_operands(case)
    n = ca.logical_numel
    sample_size = min(n, 4096)
    groups = -(-sample_size // 64)
    partials = torch.full((2 * groups,), -7, dtype=torch.int32, device="cuda")
    result_samples = torch.full((sample_size,), -7, dtype=torch.int16, device="cuda")
    B, L, S, W = ca.codec_geometry
    _, _, rare = get_distribution_tables(ca.distribution, "cuda")
    dispatch.dual_sample(ca.data, ca.sign_mantissa, shifted_decode_table(ca), ca.center,
                         overlay_of(ca), cb.data, cb.sign_mantissa, shifted_decode_table(cb),
                         cb.center, overlay_of(cb), _scalar(ALPHA), partials, ca.size,
                         rare_length=rare, logical_numel=n, block_symbols=B, lanes=L, steps=S,
                         fixed_words=W, sample_size=sample_size,
                         a_samples=ca.sample_values if recorded[0] else None,
                         b_samples=cb.sample_values if recorded[1] else None,
                         result_samples=result_samples)
    expected_values = oracle.dual(oa, ob, ALPHA)[oracle.sample_positions(n)]
    assert np.array_equal(bits_of(result_samples), expected_values)
    got = partials.cpu().numpy().reshape(groups, 2)
    assert np.array_equal(got, _group_sums(expected_values))


@pytest.mark.parametrize("case", DUAL_CASES, ids=[c[0] for c in DUAL_CASES])
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_dual_single_pass_compressed_output(case, buffered):
    """a_compA_add_compB with compressed output: every stored field equals the
    oracle's re-encode of the oracle's dual components, and the recorded sample
    values are the result's."""
    require_gpu()
    print(f"case dual single-pass {case[0]} buffered={buffered}", flush=True)
    buffer = TensorBuffer(8 << 20, max_free_regions=64, device="cuda") if buffered else None
    host = oracle.Buffer(8 << 20, 64) if buffered else None
    ca, cb, oa, ob = _dual_operands(case, buffer, host)
    result = a_compA_add_compB(ca, _scalar(ALPHA), cb, dense_output=False, buffer=buffer)
    side, exponents = oracle.dual(oa, ob, ALPHA, policy=1)
    expected = oracle_from_components(side, exponents, ca.distribution, buffer=host)
    assert_matches_oracle(result, expected)
    dense = oracle.dual(oa, ob, ALPHA)
    assert np.array_equal(bits_of(decompress(result)), dense)
    assert np.array_equal(bits_of(result.sample_values),
                          dense[oracle.sample_positions(ca.logical_numel)])
    if buffered:
        result.free()
        cb.free()
        ca.free()
        verify_buffer(buffer)


def test_dual_cases_exercise_overflow():
    """The overflow branches of the two-operand kernel are reached: both
    operands overflow in one case, only B in another, and so does a result."""
    require_gpu()
    _, _, oa, ob = _dual_operands(DUAL_CASES[1])
    assert oa.counts[0] > 0 and ob.counts[0] > 0
    _, _, oa, ob = _dual_operands(DUAL_CASES[2])
    assert oa.counts[0] == 0 and ob.counts[0] > 0
    side, exponents = oracle.dual(oa, ob, ALPHA, policy=1)
    assert oracle_from_components(side, exponents, DUAL_CASES[2][1]).counts[0] > 0


def test_weight_update_sequence_single_pass():
    """Eight add_comp_ steps (weight += alpha * compressed update) on a
    buffer-backed LCTTensor, each checked against the oracle; the sampler
    reads both operands' recorded sample values."""
    require_gpu()
    dist = Distribution(DistType.EMPIRICAL)
    shape = (1024, 1100)
    buffer = TensorBuffer(32 << 20, max_free_regions=64, device="cuda")
    host = oracle.Buffer(32 << 20, 64)
    w0 = _gaussian(shape, 50, 0.02)
    tensor = LCTTensor(w0.cuda(), buffer, dist)
    state = oracle_compress(w0, dist, buffer=host)
    for step in range(8):
        u = _gaussian(shape, 500 + step, 1e-3)
        update = LCTTensor(u.cuda(), buffer, dist)
        update_state = oracle_compress(u, dist, buffer=host)
        tensor.add_comp_(update, _scalar(ALPHA))
        side, exponents = oracle.dual(update_state, state, ALPHA, policy=1)
        previous = state
        state = oracle_from_components(side, exponents, dist, buffer=host)
        host.free(previous.descriptor)
        update.free()
        host.free(update_state.descriptor)
        assert_matches_oracle(tensor.x, state)
    tensor.free()
    verify_buffer(buffer)


# The fused updates make their overflow bookkeeping inside the encoder launch
# (lct_pointwise_encode_fused / lct_dual_encode_fused) whenever the block count
# allows; the separate launches (lct_pointwise_encode / lct_dual_encode, then
# lct_allocate_compact or lct_prefix_allocate + lct_compact_extra) serve the
# rest.  Both must store the oracle's tensor.
SEPARATE = [("fused", None), ("separate", 0)]


@pytest.mark.parametrize("case", [CASES[0], CASES[1], CASES[4]],
                         ids=[CASES[0][0], CASES[1][0], CASES[4][0]])
@pytest.mark.parametrize("path", SEPARATE, ids=[p[0] for p in SEPARATE])
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_bookkeeping_paths_store_the_oracle_tensor(case, path, buffered, monkeypatch):
    require_gpu()
    name, dist, make_a, make_b = case
    path_name, limit = path
    print(f"case bookkeeping {name} {path_name} buffered={buffered}", flush=True)
    if limit is not None:
        monkeypatch.setattr(dispatch, "MAX_CODEC_BLOCKS", limit)
    op = OPS[2]
    _, code, call, alpha, beta, alpha_is_one, beta_is_one = op
    a, b = make_a(), make_b()
    buffer = TensorBuffer(8 << 20, max_free_regions=64, device="cuda") if buffered else None
    host = oracle.Buffer(8 << 20, 64) if buffered else None
    ct = compress(a.cuda(), dist, buffer=buffer)
    o = oracle_compress(a, dist, buffer=host)
    # A deferred free rides on the update's reservation on both paths.
    spare = compress(b.cuda(), dist, buffer=buffer)
    spare_oracle = oracle_compress(b, dist, buffer=host)
    spare.free()
    if buffered:
        host.free(spare_oracle.descriptor)
    result = call(ct, b.cuda(), dense_output=False, buffer=buffer)
    side, exponents = oracle.pointwise(o, bits_of(b), code, alpha, beta, alpha_is_one,
                                       beta_is_one, policy=1)
    expected = oracle_from_components(side, exponents, dist, buffer=host)
    assert_matches_oracle(result, expected)
    if buffered:
        result.free()
        ct.free()
        verify_buffer(buffer)


@pytest.mark.parametrize("case", [DUAL_CASES[1], DUAL_CASES[2]],
                         ids=[DUAL_CASES[1][0], DUAL_CASES[2][0]])
@pytest.mark.parametrize("path", SEPARATE, ids=[p[0] for p in SEPARATE])
@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_dual_bookkeeping_paths_store_the_oracle_tensor(case, path, buffered, monkeypatch):
    require_gpu()
    path_name, limit = path
    print(f"case dual bookkeeping {case[0]} {path_name} buffered={buffered}", flush=True)
    if limit is not None:
        monkeypatch.setattr(dispatch, "MAX_CODEC_BLOCKS", limit)
    buffer = TensorBuffer(8 << 20, max_free_regions=64, device="cuda") if buffered else None
    host = oracle.Buffer(8 << 20, 64) if buffered else None
    ca, cb, oa, ob = _dual_operands(case, buffer, host)
    result = a_compA_add_compB(ca, _scalar(ALPHA), cb, dense_output=False, buffer=buffer)
    side, exponents = oracle.dual(oa, ob, ALPHA, policy=1)
    expected = oracle_from_components(side, exponents, ca.distribution, buffer=host)
    assert_matches_oracle(result, expected)
    if buffered:
        result.free()
        cb.free()
        ca.free()
        verify_buffer(buffer)


def _scattered_patterns(n_blocks, block_symbols, seed, std=1.0):
    """A Gaussian tensor of ``n_blocks`` codec blocks (the last one ragged)
    with 4096 random bit patterns in a dozen scattered blocks and in the last
    one, so that streams overflow early, late and at the very end."""
    n = n_blocks * block_symbols - 77
    x = _gaussian((n,), seed, std)
    bits = x.view(torch.int16).numpy()
    rng = np.random.default_rng(seed)
    chosen = sorted(set(rng.choice(n_blocks - 1, 12, replace=False).tolist()) | {n_blocks - 1})
    for k in chosen:
        lo = k * block_symbols + int(rng.integers(0, block_symbols - 8192))
        bits[lo:lo + 4096] = rng.integers(-32768, 32768, 4096, dtype=np.int16)
    return x


@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_fused_update_beyond_one_summary_pass(buffered):
    """lct_pointwise_encode_fused over 3000 codec blocks: workgroup 0 polls the
    block summaries in several passes of 1024 and carries the totals across
    them, with blocks still running when it starts; every stored field equals
    the oracle's."""
    require_gpu()
    print(f"case fused update 3000 blocks buffered={buffered}", flush=True)
    dist = Distribution(DistType.GAUSSIAN)
    a = _scattered_patterns(3000, 32768, 60)
    b = _gaussian((a.numel(),), 61, 0.5)
    buffer = TensorBuffer(32 << 20, max_free_regions=64, device="cuda") if buffered else None
    host = oracle.Buffer(32 << 20, 64) if buffered else None
    ct = compress(a.cuda(), dist, buffer=buffer)
    o = oracle_compress(a, dist, buffer=host)
    assert o.n_blocks == 3000 and o.counts[0] > 0
    result = a_compA_add_B(ct, _scalar(ALPHA), b.cuda(), dense_output=False, buffer=buffer)
    side, exponents = oracle.pointwise(o, bits_of(b), oracle.OP_SCALAR_MUL_ADD, ALPHA, policy=1)
    expected = oracle_from_components(side, exponents, dist, buffer=host)
    assert expected.counts[0] > 0
    assert expected.blocks[expected.n_blocks - 1] > 0, "the last block overflows"
    assert_matches_oracle(result, expected)
    if buffered:
        result.free()
        ct.free()
        verify_buffer(buffer)


@pytest.mark.parametrize("buffered", [False, True], ids=["private", "buffered"])
def test_fused_dual_update_beyond_one_summary_pass(buffered):
    """lct_dual_encode_fused over 3000 codec blocks, both operands overflowing
    in scattered blocks: every stored field equals the oracle's."""
    require_gpu()
    print(f"case fused dual 3000 blocks buffered={buffered}", flush=True)
    dist = Distribution(DistType.GAUSSIAN)
    a = _scattered_patterns(3000, 32768, 62, 1e-3)
    b = _scattered_patterns(3000, 32768, 63, 0.02)
    buffer = TensorBuffer(64 << 20, max_free_regions=64, device="cuda") if buffered else None
    host = oracle.Buffer(64 << 20, 64) if buffered else None
    ca, cb = compress(a.cuda(), dist, buffer=buffer), compress(b.cuda(), dist, buffer=buffer)
    oa, ob = oracle_compress(a, dist, buffer=host), oracle_compress(b, dist, buffer=host)
    assert oa.counts[0] > 0 and ob.counts[0] > 0
    result = a_compA_add_compB(ca, _scalar(ALPHA), cb, dense_output=False, buffer=buffer)
    side, exponents = oracle.dual(oa, ob, ALPHA, policy=1)
    expected = oracle_from_components(side, exponents, dist, buffer=host)
    assert expected.blocks[expected.n_blocks - 1] > 0, "the last block overflows"
    assert_matches_oracle(result, expected)
    if buffered:
        result.free()
        cb.free()
        ca.free()
        verify_buffer(buffer)


@pytest.mark.parametrize("kind", ["pointwise", "dual"])
def test_update_bookkeeping_that_stops_waiting_marks_the_result_incomplete(kind):
    """The fused update's workgroup 0 gives up polling the block summaries (one
    poll round, 3000 blocks: more than the device holds at once, so later
    blocks have not run when workgroup 0 finishes its own): the buffered result
    reads status 7 and raises at memory_size(), its region comes back on free,
    the private form raises at its sync, and with the default bounds both forms
    store the oracle-checked result again."""
    require_gpu()
    print(f"case update incomplete {kind}", flush=True)
    dist = Distribution(DistType.GAUSSIAN)
    g = torch.Generator(device="cuda").manual_seed(52)
    x = torch.randn(3000 * 32768, generator=g, device="cuda").to(torch.bfloat16)
    y = (torch.randn(3000 * 32768, generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    ca = compress(x, dist)
    cb = compress(y, dist) if kind == "dual" else None
    alpha = _scalar(ALPHA)

    def update(buffer):
        if kind == "dual":
            return a_compA_add_compB(ca, alpha, cb, dense_output=False, buffer=buffer)
        return a_compA_add_B(ca, alpha, y, dense_output=False, buffer=buffer)

    expected = decompress(update(None)).view(torch.int16)
    buffer = TensorBuffer(16 << 20, device="cuda")
    before = _free_regions_snapshot(buffer)
    hip.call("lct_set_wait_limits", 0, 1)
    try:
        result = update(buffer)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="gave up"):
            update(None)
    finally:
        hip.call("lct_set_wait_limits", 0, 0)
    assert int(result.fallback_descriptor[2].item()) == STATUS_INCOMPLETE
    with pytest.raises(BufferReservationError, match="status 7"):
        result.memory_size()
    assert buffer.failures() & FAIL_INCOMPLETE
    result.free()
    buffer._flush_frees()
    assert _free_regions_snapshot(buffer) == before
    assert torch.equal(decompress(update(None)).view(torch.int16), expected)
    buffer.reset()
    ok = update(buffer)
    assert torch.equal(decompress(ok).view(torch.int16), expected)
    ok.free()
    verify_buffer(buffer)


def _same_record(x, y):
    """Two compressed tensors store the same fields (private storage; the
    payload's 4 words of padding are never written)."""
    B, L, S, W = x.codec_geometry
    words = x.size // B * L * W
    assert torch.equal(x.data[:words], y.data[:words])
    for field in ("sign_mantissa", "center", "decode_table", "fallback_count",
                  "fallback_used", "fallback_blocks", "fallback_lanes", "fallback_starts",
                  "fallback_buffer"):
        u, v = getattr(x, field), getattr(y, field)
        assert (u is None) == (v is None), field
        if u is not None:
            assert torch.equal(u.cpu(), v.cpu()), field


@pytest.mark.parametrize("case", DUAL_CASES[:4], ids=[c[0] for c in DUAL_CASES[:4]])
def test_dual_in_launch_sampling_equals_the_sampler_launch(case):
    """The weight update with both operands' recorded sample values samples
    the result's center in its encoder launch (its first 64 workgroups; the
    gaussian case has 16 codec blocks, so 48 workgroups only sample; the tiny
    case samples every element, 1517 in 24 groups, in one block): against
    the sampler launch (B's recorded values dropped, so that launch walks B's
    streams) the stored result and its recorded values are the same, and the
    result is the oracle's."""
    require_gpu()
    print(f"case dual in-launch sampling {case[0]}", flush=True)
    ca, cb, oa, ob = _dual_operands(case, None, None)
    assert ca.sample_values is not None and cb.sample_values is not None
    cb_without = dataclasses.replace(cb, sample_values=None)
    first = a_compA_add_compB(ca, _scalar(ALPHA), cb, dense_output=False)
    second = a_compA_add_compB(ca, _scalar(ALPHA), cb_without, dense_output=False)
    _same_record(first, second)
    assert torch.equal(first.sample_values, second.sample_values)
    side, exponents = oracle.dual(oa, ob, ALPHA, policy=1)
    assert_matches_oracle(first, oracle_from_components(side, exponents, ca.distribution))
