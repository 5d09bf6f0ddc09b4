"""ctypes binding of ``liblct_hip.so`` (declared in ``include/lct.h``).

The library is the only compute path: if it is missing, every codec call
raises.  Tensors cross the boundary as raw device pointers, sizes as int64
and the current torch stream as the ``hipStream_t`` argument.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent.parent / "lib" / "liblct_hip.so"

LCT_OP_ADD = 0
LCT_OP_MULTIPLY = 1
LCT_OP_SCALAR_MUL_ADD = 2
LCT_DENSE_OUTPUT = 0
LCT_COMPRESSED_OUTPUT = 1

_c_int32 = ctypes.c_int32
_c_int64 = ctypes.c_int64
_ptr = ctypes.c_void_p


class Geometry(ctypes.Structure):
    """``lct_geometry``: (block_symbols, lanes, steps, fixed_words)."""

    _fields_ = [
        ("block_symbols", _c_int32),
        ("lanes", _c_int32),
        ("steps", _c_int32),
        ("fixed_words", _c_int32),
    ]


class Overflow(ctypes.Structure):
    """``lct_overflow``: one tensor's overflow lanes/starts/tails metadata."""

    _fields_ = [
        ("lanes", _ptr),
        ("starts", _ptr),
        ("tail", _ptr),
        ("blocks", _ptr),
        ("count", _ptr),
        ("descriptor", _ptr),
        ("base", _c_int64),
    ]


MAX_PENDING_FREES = 4   # LCT_MAX_PENDING_FREES


MAX_FREE_BATCH = 32     # LCT_MAX_FREE_BATCH


class PendingFrees(ctypes.Structure):
    """``lct_pending_frees``: descriptors whose frees ride on the next reservation."""

    _fields_ = [
        ("descriptor", _ptr * MAX_PENDING_FREES),
        ("count", _c_int32),
    ]


class Bookkeeping(ctypes.Structure):
    """``lct_bookkeeping``: the in-launch overflow bookkeeping of the fused
    update encoders."""

    _fields_ = [
        ("control", _ptr),
        ("control_words", _c_int64),
        ("epoch", ctypes.c_uint32),
        ("counts", _ptr),
        ("blocks", _ptr),
        ("descriptor", _ptr),
        ("buffer_meta", _ptr),
        ("max_free_regions", _c_int32),
        ("frees", PendingFrees),
        ("a_samples", _ptr),
        ("b_samples", _ptr),
        ("result_samples", _ptr),
    ]


MAX_DECODE_BATCH = 16   # LCT_MAX_DECODE_BATCH


class DecodeJob(ctypes.Structure):
    """``lct_decode_job``: one tensor of a batched decode."""

    _fields_ = [
        ("encoded", _ptr),
        ("side", _ptr),
        ("output", _ptr),
        ("shifted_decode", _ptr),
        ("center", _ptr),
        ("size", _c_int64),
        ("logical_numel", _c_int64),
        ("geometry", Geometry),
        ("rare_length", _c_int32),
        ("has_overflow", _c_int32),
        ("overflow", Overflow),
    ]


MAX_COMPRESS_BATCH = 16   # LCT_MAX_COMPRESS_BATCH


class CompressJob(ctypes.Structure):
    """``lct_compress_job``: one tensor of a batched buffered compress."""

    _fields_ = [
        ("source", _ptr),
        ("side", _ptr),
        ("encoded", _ptr),
        ("base_encode", _ptr),
        ("base_decode", _ptr),
        ("center_out", _ptr),
        ("shifted_decode_out", _ptr),
        ("sample_values", _ptr),
        ("blocks", _ptr),
        ("counts", _ptr),
        ("descriptor", _ptr),
        ("sample_size", _c_int64),
        ("size", _c_int64),
        ("logical_numel", _c_int64),
        ("geometry", Geometry),
    ]


MAX_UPDATE_BATCH = 8   # LCT_MAX_UPDATE_BATCH


class UpdateJob(ctypes.Structure):
    """``lct_update_job``: one tensor of a batched fused update."""

    _fields_ = [
        ("encoded", _ptr),
        ("side", _ptr),
        ("shifted_decode", _ptr),
        ("center", _ptr),
        ("has_overflow", _c_int32),
        ("overflow", Overflow),
        ("a_samples", _ptr),
        ("other", _ptr),
        ("base_encode", _ptr),
        ("base_decode", _ptr),
        ("center_out", _ptr),
        ("shifted_decode_out", _ptr),
        ("side_out", _ptr),
        ("encoded_out", _ptr),
        ("result_samples", _ptr),
        ("exponents", _ptr),
        ("counts", _ptr),
        ("blocks", _ptr),
        ("descriptor", _ptr),
        ("size", _c_int64),
        ("logical_numel", _c_int64),
        ("sample_size", _c_int64),
        ("geometry", Geometry),
        ("rare_length", _c_int32),
    ]


# name -> argument types (all entry points return int32).
_SIGNATURES = {
    "lct_estimate_and_shift_tables": [_ptr, _c_int32, _c_int64, _c_int64, _ptr, _ptr, _ptr, _ptr,
                                      _ptr, _ptr],
    "lct_shift_tables": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr],
    "lct_shift_decoding_table": [_ptr, _ptr, _ptr, _ptr],
    "lct_encode": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _c_int64, _c_int64, Geometry, _c_int32,
                   _c_int32, _ptr],
    "lct_prefix_allocate": [_ptr, _ptr, _ptr, _ptr, _ptr, _c_int64, _c_int32, _c_int32, _ptr],
    "lct_compact_extra": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _c_int64, _ptr, _ptr,
                          _c_int64, _c_int64, Geometry, _c_int32, _c_int32, _ptr],
    "lct_decode": [_ptr, _ptr, _ptr, _ptr, _ptr, _c_int64, _c_int64, Geometry, _c_int32,
                   ctypes.POINTER(Overflow), _ptr],
    "lct_decode_batch": [ctypes.POINTER(DecodeJob), _c_int32, _ptr],
    "lct_pointwise_dense": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _c_int64,
                            _c_int64, Geometry, _c_int32, _c_int32, _c_int32, _c_int32, _c_int32,
                            ctypes.POINTER(Overflow), _ptr],
    "lct_dual": [_ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _ptr, _ptr,
                 ctypes.POINTER(Overflow), _ptr, _ptr, _ptr, _c_int64, _c_int64, Geometry,
                 _c_int32, _c_int32, _ptr],
    "lct_pointwise_sample": [_ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _ptr,
                             _ptr, _c_int64, _c_int64, Geometry, _c_int32, _c_int32, _c_int32,
                             _c_int32, _c_int64, _ptr, _ptr, _ptr],
    "lct_sample_center": [_ptr, _c_int32, _c_int64, _c_int64, _ptr, _ptr, _ptr],
    "lct_encode_sampled": [_ptr, _ptr, _ptr, _ptr, _c_int64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
                           _c_int64, _c_int64, Geometry, _c_int32, _c_int32, _ptr],
    "lct_pointwise_encode": [_ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _ptr,
                             _ptr, _c_int64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
                             _c_int64, _c_int64, Geometry, _c_int32, _c_int32, _c_int32, _c_int32,
                             _ptr],
    "lct_pointwise_encode_fused": [_ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr,
                                   _ptr, _ptr, _c_int64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
                                   _ptr, _ptr, _c_int64, _c_int64, Geometry, _c_int32, _c_int32,
                                   _c_int32, _c_int32, ctypes.POINTER(Bookkeeping), _ptr],
    "lct_dual_sample": [_ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _ptr,
                        _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _c_int64, _c_int64,
                        Geometry, _c_int32, _c_int64, _ptr, _ptr, _ptr],
    "lct_dual_encode": [_ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _ptr,
                        _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _c_int64, _ptr, _ptr, _ptr,
                        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _c_int64, _c_int64, Geometry,
                        _c_int32, _ptr],
    "lct_dual_encode_fused": [_ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr,
                              _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _c_int64, _ptr,
                              _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _c_int64, _c_int64,
                              Geometry, _c_int32, ctypes.POINTER(Bookkeeping), _ptr],
    "lct_allocate_compact": [_ptr, _ptr, _ptr, _ptr, _ptr, _c_int32, _ptr, _ptr, _ptr,
                             ctypes.POINTER(PendingFrees), _ptr, ctypes.c_uint64, _c_int64,
                             _c_int64, Geometry, _c_int32, _ptr],
    "lct_encode_fused": [_ptr, _ptr, _ptr, _c_int64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
                         _ptr, _ptr, _ptr, _c_int64, ctypes.c_uint32, _ptr, _ptr, _c_int32,
                         ctypes.POINTER(PendingFrees), _ptr, _c_int64, _c_int64, Geometry,
                         _c_int32, _ptr],
    "lct_pointwise_update_batch": [ctypes.POINTER(UpdateJob), _c_int32, _c_int32, _c_int32,
                                   _c_int32, _ptr, _ptr, _ptr, _c_int64, _ptr, _c_int64, _ptr,
                                   _c_int64, _ptr, _c_int64, ctypes.c_uint32, _ptr, _c_int32,
                                   _ptr, ctypes.POINTER(PendingFrees), _ptr],
    "lct_compress_batch": [ctypes.POINTER(CompressJob), _c_int32, _ptr, _c_int64, _ptr, _c_int64,
                           _ptr, _c_int64, ctypes.c_uint32, _ptr, _c_int32, _ptr,
                           ctypes.POINTER(PendingFrees), _ptr],
    "lct_count_bad_streams": [_ptr, _ptr, _ptr, _c_int64, _c_int32, _ptr],
    "lct_compact_bad_streams": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _c_int64,
                                _c_int32, _c_int64, _c_int32, _ptr],
    "lct_scatter_fallback": [ctypes.POINTER(Overflow), _ptr, _ptr, _c_int64, _c_int64, Geometry,
                             _ptr],
    "lct_pointwise_fallback": [ctypes.POINTER(Overflow), _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,
                               _c_int64, _c_int64, Geometry, _c_int32, _c_int32, _c_int32,
                               _c_int32, _ptr],
    "lct_dual_maps_init": [_ptr, _ptr, _ptr, _ptr, _c_int64, _c_int32, _ptr],
    "lct_dual_tables_and_maps": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow),
                                 ctypes.POINTER(Overflow), _ptr, _ptr, _ptr, _ptr, _c_int64,
                                 _c_int32, _ptr],
    "lct_dual_mapped": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr,
                        _ptr, _ptr, _ptr, _ptr, ctypes.POINTER(Overflow), _ptr, _ptr, _ptr,
                        _c_int64, _c_int64, Geometry, _c_int32, _c_int32, _ptr],
    "lct_buffer_reset": [_ptr, _c_int32, _c_int32, _ptr],
    "lct_buffer_allocate": [_ptr, _c_int32, _ptr, _ptr, _c_int32, _ptr, _ptr],
    "lct_buffer_free": [_ptr, _c_int32, _ptr, _ptr, _ptr],
    "lct_buffer_free_batch": [_ptr, _c_int32, ctypes.POINTER(_ptr), _c_int32, _ptr, _ptr],
    "lct_set_wait_limits": [_c_int32, _c_int32],
    "lct_set_decoder": [_c_int32],
    "lct_bandwidth_probe": [_c_int32, _ptr, _c_int64, _ptr, _c_int64, _c_int32, _ptr],
    "lct_compress_buffered_noalloc": [_ptr, _c_int64, _c_int64, Geometry, _ptr, _ptr, _ptr, _ptr,
                                      _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _c_int32, _ptr,
                                      ctypes.POINTER(PendingFrees), _ptr],
}

EXPORTED = tuple(_SIGNATURES) + ("lct_version", "lct_error_string")

_lock = threading.Lock()
_library = None


def load_library(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and type the codec library; raise if it is not built."""
    global _library
    with _lock:
        if _library is not None and path is None:
            return _library
        target = Path(path) if path is not None else LIBRARY_PATH
        if not target.exists():
            raise RuntimeError(
                f"LCT HIP library not found at {target}; build it with "
                "`python -m losslessly_compressed_tensors_amd.build`")
        lib = ctypes.CDLL(str(target))
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _c_int32
        lib.lct_version.argtypes = []
        lib.lct_version.restype = ctypes.c_char_p
        lib.lct_error_string.argtypes = [_c_int32]
        lib.lct_error_string.restype = ctypes.c_char_p
        if path is None:
            _library = lib
        return lib


class LCTKernelError(RuntimeError):
    """A codec entry point rejected its arguments or failed to launch."""


_entry_points: dict = {}


def call(name: str, *args) -> None:
    """Invoke entry point ``name`` and raise on a non-zero return code."""
    fn = _entry_points.get(name)
    if fn is None:
        fn = _entry_points[name] = getattr(load_library(), name)
    code = fn(*args)
    if code != 0:
        message = load_library().lct_error_string(code).decode()
        raise LCTKernelError(f"{name} failed with code {code}: {message}")


def geometry(stream_geometry) -> Geometry:
    block_symbols, lanes, steps, fixed_words = stream_geometry
    return Geometry(int(block_symbols), int(lanes), int(steps), int(fixed_words))
