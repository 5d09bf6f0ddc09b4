"""Host-side logic (CPU): the reference's selectors, geometry, storage record,
RAW path, module aliases and the loud failure without the GPU library."""
from __future__ import annotations

import importlib

import pytest
import torch

from losslessly_compressed_tensors_amd.codec.geometry import geometry
from losslessly_compressed_tensors_amd.comp_format import (
    Distribution,
    DistType,
    NoiseLevel,
    StorageLayout,
)
from losslessly_compressed_tensors_amd.comp_tensor import CompressedTensor
from losslessly_compressed_tensors_amd.kernels import hip
from losslessly_compressed_tensors_amd.operations import (
    a_compA_add_B,
    a_compA_add_compB,
    compress,
    decompress,
)


# ---- Distribution (comp_format.py:26-74) -------------------------------------


@pytest.mark.parametrize("param, expected", [
    (1.0, 1.0), (0.98, 1.0), (0.1, 0.25), (0.375, 0.5), (0.625, 0.5), (0.875, 1.0),
    (2.2, 2.25), (1e-9, 0.25),
])
def test_param_snaps_to_quarters_with_bankers_rounding(param, expected):
    assert Distribution(DistType.LAPLACE, param).param == expected


@pytest.mark.parametrize("mean, expected", [(0.05, 0.0), (-0.125, 0.0), (0.125, 0.0),
                                            (0.375, 0.5), (-0.3, -0.25), (50.1, 50.0)])
def test_mean_snaps_to_quarters(mean, expected):
    assert Distribution(DistType.GAUSSIAN, 1.0, mean).mean == expected


@pytest.mark.parametrize("zero_prob, expected", [(None, 0.0), (0.123, 0.12), (0.125, 0.12),
                                                 (1.0, 1.0), (0.004, 0.0)])
def test_zero_prob_rounds_to_hundredths(zero_prob, expected):
    assert Distribution(zero_prob=zero_prob).zero_prob == expected


@pytest.mark.parametrize("kwargs, error", [
    ({"family": "gaussian"}, TypeError),
    ({"noise_level": 1}, TypeError),
    ({"param": 0.0}, ValueError),
    ({"param": -1.0}, ValueError),
    ({"param": float("inf")}, ValueError),
    ({"mean": float("nan")}, ValueError),
    ({"zero_prob": 1.5}, ValueError),
    ({"zero_prob": -0.1}, ValueError),
])
def test_distribution_validation(kwargs, error):
    with pytest.raises(error):
        Distribution(**kwargs)


def test_distribution_str():
    assert str(Distribution(DistType.GAUSSIAN)) == "gaussian/std=1.0/mean=0.0/clean"
    assert (str(Distribution(DistType.LAPLACE, 2.0, 0.5, NoiseLevel.SPARSE))
            == "laplace/scale=2.0/mean=0.5/sparse")


# ---- geometry (codec/geometry.py:13-39) ----------------------------------------


@pytest.mark.parametrize("family, noise, expected", [
    (DistType.GAUSSIAN, NoiseLevel.CLEAN, (32768, 256, 128, 12)),
    (DistType.LAPLACE, NoiseLevel.CLEAN, (65536, 256, 256, 25)),
    (DistType.EMPIRICAL, NoiseLevel.CLEAN, (65536, 256, 256, 25)),
    (DistType.GAMMA, NoiseLevel.CLEAN, (65536, 256, 256, 25)),
    (DistType.GAUSSIAN, NoiseLevel.SPARSE, (65536, 256, 256, 20)),
    (DistType.LAPLACE, NoiseLevel.MEDIUM, (32768, 256, 128, 19)),
    (DistType.EMPIRICAL, NoiseLevel.HIGH, (32768, 256, 128, 22)),
])
def test_geometry_table(family, noise, expected):
    assert geometry(Distribution(family, noise_level=noise)) == expected


def test_codec_geometry_fallbacks():
    legacy = CompressedTensor(torch.zeros(4, dtype=torch.int32), 65536,
                              distribution=Distribution(DistType.GAUSSIAN),
                              layout=StorageLayout.COMPRESSED,
                              fallback_blocks=torch.zeros(3, dtype=torch.int32))
    assert legacy.codec_geometry == (65536, 256, 256, 24)   # comp_tensor.py:50-54
    with pytest.raises(ValueError):
        CompressedTensor(torch.zeros(4, dtype=torch.int32), 65536,
                         layout=StorageLayout.COMPRESSED).codec_geometry


# ---- memory_size (comp_tensor.py:57-72) ----------------------------------------


def _record(buffered: bool):
    nb, ns, W, N = 2, 512, 12, 65536
    counts = torch.tensor([3, 40, 0, 0], dtype=torch.int32)
    common = dict(
        data=torch.zeros(ns * W + 4, dtype=torch.int32), size=N,
        sign_mantissa=torch.zeros(N, dtype=torch.uint8),
        fallback_count=counts[0:1], fallback_used=counts[1:2],
        fallback_blocks=torch.zeros(3 * nb, dtype=torch.int32),
        center=torch.zeros(1, dtype=torch.int32),
        decode_table=torch.zeros(1024, dtype=torch.int32),
        distribution=Distribution(DistType.GAUSSIAN), shape=(N,),
        layout=StorageLayout.COMPRESSED, stream_geometry=(32768, 256, 128, W))
    if buffered:
        arena = torch.zeros(1 << 16, dtype=torch.uint8)
        return CompressedTensor(fallback_buffer=arena,
                                fallback_descriptor=torch.tensor([0, 48, 0, 1],
                                                                 dtype=torch.int32),
                                **common)
    return CompressedTensor(fallback_buffer=torch.zeros(40, dtype=torch.uint8),
                            fallback_lanes=torch.zeros(3, dtype=torch.uint8),
                            fallback_starts=torch.zeros(3, dtype=torch.uint8), **common)


def test_memory_size_private():
    fixed = (512 * 12 + 4) * 4 + 65536 + 16 + 24 + 4 + 4096
    assert _record(False).memory_size() == fixed + 3 + 3 + 40


def test_memory_size_buffered_counts_reservation_not_arena():
    fixed = (512 * 12 + 4) * 4 + 65536 + 16 + 24 + 4 + 4096
    # the arena (shared by lanes/starts/tails) is excluded; the 16-byte
    # descriptor and the 48 reserved bytes are counted
    assert _record(True).memory_size() == fixed + 16 + 48


# ---- RAW path and error behaviour ------------------------------------------------


def test_raw_layout_for_tiny_tensors_round_trips_on_host():
    x = torch.randn(3, 5).to(torch.bfloat16)
    ct = compress(x, Distribution(DistType.GAUSSIAN), allow_raw=True)
    assert ct.layout == StorageLayout.RAW
    assert torch.equal(decompress(ct), x)


def test_non_16_bit_input_is_rejected():
    with pytest.raises(TypeError):
        compress(torch.randn(70000), Distribution(DistType.GAUSSIAN))


def test_codec_requires_gpu_tensors():
    with pytest.raises(ValueError, match="GPU"):
        compress(torch.randn(70000).to(torch.bfloat16), Distribution(DistType.GAUSSIAN))


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        hip.load_library(tmp_path / "liblct_hip.so")


def test_scalar_arguments_must_be_tensors():
    ct = _record(False)
    with pytest.raises(TypeError):
        a_compA_add_B(ct, 0.5, torch.zeros(1))
    with pytest.raises(TypeError):
        a_compA_add_compB(ct, 0.5, ct)


# ---- drop-in module paths ------------------------------------------------------------


@pytest.mark.parametrize("name", ["operations", "comp_format", "comp_tensor", "tensor_buffer",
                                  "LCTensor", "codec.encode", "codec.decode",
                                  "compression.huffman_tables"])
def test_reference_module_paths_resolve_to_this_package(name):
    ours = importlib.import_module(f"losslessly_compressed_tensors_amd.{name}")
    assert importlib.import_module(f"LCT.{name}") is ours
    from LCT.operations import compress as lct_compress
    assert lct_compress is compress


class _FakeEvent:
    def __init__(self, log):
        self.log = log

    def record(self, stream):
        self.log.append(("record", stream))


class _FakeStream:
    def __init__(self, log):
        self.log = log

    def wait_event(self, event):
        self.log.append(("wait",))


@pytest.fixture
def deferral(monkeypatch):
    """A TensorBuffer whose device calls are recorded instead of launched:
    ``state.stream`` is the current raw stream; ``log`` collects the frees
    (descriptor, stream), event records and stream waits in order."""
    from losslessly_compressed_tensors_amd import tensor_buffer as tb

    log = []
    state = type("State", (), {"stream": 11})()
    buf = object.__new__(tb.TensorBuffer)
    buf._storage = torch.zeros(64, dtype=torch.uint8)
    buf.max_free_regions = 4
    buf.capacity_bytes = 16
    buf._metadata_bytes = 48
    buf.device = torch.device("cpu")
    buf._pending_frees = []
    buf._pending_stream = 0
    monkeypatch.setattr(tb.TensorBuffer, "_current_stream", lambda self: state.stream)
    monkeypatch.setattr(tb, "_free_now",
                        lambda storage, d, regions, stream=None: log.append(("free", d, stream)))
    monkeypatch.setattr(tb, "_free_many",
                        lambda storage, ds, regions, stream=None: log.append(("free", list(ds),
                                                                              stream)))
    monkeypatch.setattr(tb.torch.cuda, "Event", lambda: _FakeEvent(log))
    monkeypatch.setattr(tb.torch.cuda, "ExternalStream", lambda handle, device=None: handle)
    monkeypatch.setattr(tb.torch.cuda, "current_stream", lambda device=None: _FakeStream(log))
    monkeypatch.setattr(tb.dispatch, "buffer_reset", lambda *a: log.append(("reset",)))
    return buf, state, log


def test_deferred_frees_ride_on_the_next_reservation_in_order(deferral):
    buf, state, log = deferral
    buf._defer_free("d1")
    buf._defer_free("d2")
    buf._defer_free("d3")
    assert log == []                                  # nothing launched yet
    assert buf._take_frees() == ["d1", "d2", "d3"]    # one reservation takes them in order
    assert buf._take_frees() == [] and log == []


def test_a_full_pending_list_is_launched_in_one_batch_before_the_next_free(deferral):
    from losslessly_compressed_tensors_amd.kernels import dispatch
    buf, state, log = deferral
    names = [f"d{i}" for i in range(dispatch.MAX_FREE_BATCH + 1)]
    for name in names:
        buf._defer_free(name)
    # One launch, in order, on the stream the frees were made on.
    assert log == [("free", names[:dispatch.MAX_FREE_BATCH], 11)]
    assert buf._take_frees() == names[dispatch.MAX_FREE_BATCH:]


def test_a_reservation_takes_the_last_frees_and_launches_the_earlier_ones_first(deferral):
    from losslessly_compressed_tensors_amd.kernels import dispatch
    buf, state, log = deferral
    keep = dispatch.MAX_PENDING_FREES
    names = [f"d{i}" for i in range(keep + 5)]
    for name in names:
        buf._defer_free(name)
    assert log == []
    assert buf._take_frees() == names[5:]             # what one reservation applies
    assert log == [("free", names[:5], 11)]           # launched before it, in one batch
    assert buf._take_frees() == []


def test_a_change_of_stream_launches_pending_frees_and_orders_the_new_stream(deferral):
    buf, state, log = deferral
    buf._defer_free("d1")
    state.stream = 22
    assert buf._take_frees() == []                    # not taken on another stream
    assert log == [("free", ["d1"], 11), ("record", 11), ("wait",)]
    log.clear()
    buf._defer_free("d2")                             # now deferred on stream 22
    state.stream = 33
    buf._defer_free("d3")                             # a free on a third stream flushes d2 first
    assert log == [("free", ["d2"], 22), ("record", 22), ("wait",)]
    assert buf._take_frees() == ["d3"]


def test_every_other_buffer_operation_launches_pending_frees_first(deferral):
    buf, state, log = deferral
    buf._defer_free("d1")
    buf.reset()
    assert log == [("free", ["d1"], 11), ("reset",)]  # same stream: no wait needed
    log.clear()
    buf._defer_free("d2")
    buf._flush_frees()
    buf._flush_frees()                                # idempotent
    assert log == [("free", ["d2"], 11)]


def test_frees_taken_by_a_reservation_that_fails_to_launch_stay_pending(deferral, monkeypatch):
    """A reservation whose launch raises (bad arguments, a launch error)
    launches nothing, so the deferred frees it took wait for the next one."""
    from losslessly_compressed_tensors_amd.codec import encode as enc
    from losslessly_compressed_tensors_amd.comp_format import Distribution
    from losslessly_compressed_tensors_amd.kernels import hip

    buf, state, log = deferral

    def failing_launch(*args, **kwargs):
        raise hip.LCTKernelError("lct_allocate_compact failed with code -4")

    monkeypatch.setattr(enc.dispatch, "allocate_compact", failing_launch)
    buf._defer_free("d1")
    buf._defer_free("d2")
    dummy = torch.zeros(8, dtype=torch.int32)
    with pytest.raises(hip.LCTKernelError):
        enc.finish_encode(dummy, dummy, dummy, dummy, dummy, 32768, Distribution(), buf, (32768,),
                          precomputed=False, center=dummy, shifted_decode=dummy,
                          logical_numel=32768)
    assert log == []
    assert buf._take_frees() == ["d1", "d2"]


def test_frees_whose_batch_launch_raises_stay_pending(deferral, monkeypatch):
    """A batched free launch that raises frees nothing, so its frees stay
    deferred, for a flush and for the early frees of a reservation."""
    from losslessly_compressed_tensors_amd import tensor_buffer as tb
    from losslessly_compressed_tensors_amd.kernels import dispatch, hip

    buf, state, log = deferral
    keep = dispatch.MAX_PENDING_FREES
    names = [f"d{i}" for i in range(keep + 3)]
    for name in names:
        buf._defer_free(name)

    def failing_batch(storage, ds, regions, stream=None):
        raise hip.LCTKernelError("lct_buffer_free_batch failed with code -4")

    monkeypatch.setattr(tb, "_free_many", failing_batch)
    with pytest.raises(hip.LCTKernelError):
        buf._take_frees()
    with pytest.raises(hip.LCTKernelError):
        buf._flush_frees()
    assert buf._pending_frees == names and log == []
    monkeypatch.setattr(tb, "_free_many",
                        lambda storage, ds, regions, stream=None: log.append(("free", list(ds),
                                                                              stream)))
    assert buf._take_frees() == names[3:]
    assert log == [("free", names[:3], 11)]


def test_free_batch_checks_descriptor_and_status_sizes_before_launch():
    """``dispatch.buffer_free_batch`` rejects short descriptors and a status
    array shorter than the batch before it touches a device."""
    from losslessly_compressed_tensors_amd.kernels import dispatch

    storage = torch.zeros(64, dtype=torch.int32)
    good = torch.zeros(4, dtype=torch.int32)
    with pytest.raises(ValueError, match="descriptors"):
        dispatch.buffer_free_batch(storage, 4, [good, torch.zeros(3, dtype=torch.int32)])
    with pytest.raises(ValueError, match="descriptors"):
        dispatch.buffer_free_batch(storage, 4, [torch.zeros(4, dtype=torch.int64)])
    with pytest.raises(ValueError, match="status"):
        dispatch.buffer_free_batch(storage, 4, [good, good], torch.zeros(1, dtype=torch.int32))
    with pytest.raises(ValueError, match="GPU tensors"):    # sizes fine: the device check
        dispatch.buffer_free_batch(storage, 4, [good, good], torch.zeros(2, dtype=torch.int32))


def test_a_dense_operand_that_is_not_bfloat16_raises_before_any_launch():
    """The fused pointwise kernels read the dense operand as BF16: a float32
    or int8 operand of the right shape raises TypeError instead of being read
    with the wrong element size."""
    from losslessly_compressed_tensors_amd.codec import pointwise as pw
    from losslessly_compressed_tensors_amd.codec.geometry import geometry
    from losslessly_compressed_tensors_amd.comp_format import Distribution, StorageLayout
    from losslessly_compressed_tensors_amd.comp_tensor import CompressedTensor

    dist = Distribution()
    ct = CompressedTensor(torch.zeros(4, dtype=torch.int32), 65536,
                          torch.zeros(65536, dtype=torch.uint8), distribution=dist,
                          shape=(256, 256), layout=StorageLayout.COMPRESSED,
                          stream_geometry=geometry(dist))
    alpha = torch.ones(1)
    for dtype in (torch.float32, torch.int8):
        other = torch.zeros(256, 256, dtype=dtype)
        with pytest.raises(TypeError, match="bfloat16"):
            pw.pointwise_compressed_dense(ct, other, pw.SCALAR_MUL_ADD, alpha=alpha)
        with pytest.raises(TypeError, match="bfloat16"):
            pw.pointwise_compressed_dense(ct, other, pw.ADD, dense_output=False)


def test_mul_add_many_needs_one_update_per_tensor():
    """A length mismatch raises before any tensor is updated (zip would
    silently leave the extra tensors as they were)."""
    from losslessly_compressed_tensors_amd.LCTensor import LCTTensor

    with pytest.raises(ValueError, match="one update per tensor"):
        LCTTensor.mul_add_many([object(), object()], torch.ones(1), [torch.zeros(1)])


def test_batched_update_needs_one_distribution_per_tensor():
    """zip would drop the tensors past the shorter list: a length mismatch
    raises before any launch."""
    from losslessly_compressed_tensors_amd.comp_format import Distribution
    from losslessly_compressed_tensors_amd.operations import a_compA_add_b_B_batch

    class _A:
        data = torch.zeros(1)
        distribution = Distribution()

    with pytest.raises(ValueError, match="one distribution per compressed A"):
        a_compA_add_b_B_batch([_A(), _A()], torch.ones(1), [torch.zeros(1)] * 2,
                              buffer=None, distributions=[Distribution()])
