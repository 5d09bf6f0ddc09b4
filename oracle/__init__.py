"""CPU oracle of the LCT codec -- TEST INFRASTRUCTURE, never the product path.

NumPy front end over ``liblct_oracle.so`` (``lct_oracle.c``, a serial C
restatement of the reference's Triton kernels; every function there cites
the reference file:line it follows).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg use it, and
only as the checker or the timed host-core baseline.

Parity pinning of each oracle function (what fixes it besides the reference
text it restates) lives with its tests: golden codebooks from the reference
(``tests/golden/tables.json``), exhaustive round trips over all 65536 BF16
patterns, a naive bit-writer for payload words, brute-force overflow
recounts, exact-rational FMA/rounding checks and an allocator state machine.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

import numpy as np

LIBRARY = Path(__file__).resolve().parent / "liblct_oracle.so"

# (B, L, S, W) per (family, noise level) -- LCT/codec/geometry.py:13-39.
_GAUSSIAN_CLEAN = (32768, 256, 128, 12)
_OTHER_CLEAN = (65536, 256, 256, 25)
_SPARSE = (65536, 256, 256, 20)
_MEDIUM = (32768, 256, 128, 19)
_HIGH = (32768, 256, 128, 22)


def geometry_of(family: str, noise: str) -> tuple[int, int, int, int]:
    noise = noise.lower()
    if noise == "clean":
        return _GAUSSIAN_CLEAN if family.lower() == "gaussian" else _OTHER_CLEAN
    return {"sparse": _SPARSE, "medium": _MEDIUM, "high": _HIGH}[noise]


class _Geometry(ctypes.Structure):
    _fields_ = [("block_symbols", ctypes.c_int32), ("lanes", ctypes.c_int32),
                ("steps", ctypes.c_int32), ("fixed_words", ctypes.c_int32)]


class _Overflow(ctypes.Structure):
    _fields_ = [("lanes", ctypes.c_void_p), ("starts", ctypes.c_void_p),
                ("tail", ctypes.c_void_p), ("blocks", ctypes.c_void_p),
                ("lane_off", ctypes.c_int64), ("start_off", ctypes.c_int64),
                ("tail_off", ctypes.c_int64)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"oracle not built: {LIBRARY} (run python oracle/build.py)")
        _lib = ctypes.CDLL(str(LIBRARY))
        _lib.lcto_estimate_center.restype = ctypes.c_int32
        _lib.lcto_estimate_center.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                              ctypes.c_int]
        _lib.lcto_apply.restype = ctypes.c_uint16
        _lib.lcto_apply.argtypes = [ctypes.c_int, ctypes.c_uint16, ctypes.c_uint16,
                                    ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int]
        _lib.lcto_f32_to_bf16.restype = ctypes.c_uint16
        _lib.lcto_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.lcto_buffer_free.restype = ctypes.c_int32
        _lib.lcto_num_threads.restype = ctypes.c_int32
    return _lib


def _p(array: np.ndarray | None):
    return None if array is None else array.ctypes.data_as(ctypes.c_void_p)


def _geo(g) -> _Geometry:
    return _Geometry(*[int(v) for v in g])


def num_threads() -> int:
    return int(lib().lcto_num_threads())


def set_num_threads(n: int) -> None:
    """Thread count of the oracle's later parallel loops."""
    lib().lcto_set_num_threads(ctypes.c_int32(int(n)))


# ---- allocator ------------------------------------------------------------


class Buffer:
    """Host model of a TensorBuffer: int32 metadata + uint8 arena."""

    def __init__(self, capacity: int, max_free_regions: int = 256):
        self.capacity = int(capacity)
        self.regions = int(max_free_regions)
        self.meta = np.zeros(2 * self.regions + 3, dtype=np.int32)
        self.arena = np.zeros(self.capacity, dtype=np.uint8)
        self.reset()

    def reset(self) -> None:
        lib().lcto_buffer_reset(_p(self.meta), ctypes.c_int32(self.regions),
                                ctypes.c_int32(self.capacity))

    def allocate(self, request: int, items: int = 0, item_bytes: int = 0) -> np.ndarray:
        descriptor = np.zeros(4, dtype=np.int32)
        lib().lcto_buffer_allocate(_p(self.meta), ctypes.c_int32(self.regions),
                                   ctypes.c_int32(request), ctypes.c_int32(items),
                                   ctypes.c_int32(item_bytes), _p(descriptor))
        return descriptor

    def free(self, descriptor: np.ndarray) -> int:
        return int(lib().lcto_buffer_free(_p(self.meta), ctypes.c_int32(self.regions),
                                          _p(descriptor)))

    def free_regions(self) -> list[tuple[int, int]]:
        count = int(self.meta[2 * self.regions])
        return [(int(self.meta[i]), int(self.meta[self.regions + i])) for i in range(count)]


# ---- codec ----------------------------------------------------------------


@dataclass
class Compressed:
    n: int
    size: int
    geometry: tuple[int, int, int, int]
    center: int
    rare_length: int
    shifted_encode: np.ndarray
    shifted_decode: np.ndarray
    encoded: np.ndarray
    side: np.ndarray
    extra_starts: np.ndarray
    summaries: np.ndarray
    counts: np.ndarray
    blocks: np.ndarray
    lanes: np.ndarray
    starts: np.ndarray
    tail: np.ndarray
    lane_off: int = 0
    start_off: int = 0
    tail_off: int = 0
    descriptor: np.ndarray | None = None

    @property
    def n_blocks(self) -> int:
        return self.size // self.geometry[0]

    @property
    def buffered(self) -> bool:
        return self.descriptor is not None

    def overflow(self) -> _Overflow | None:
        if not self.buffered and self.lanes.size == 0:
            return None
        return _Overflow(_p(self.lanes), _p(self.starts), _p(self.tail), _p(self.blocks),
                         self.lane_off, self.start_off, self.tail_off)

    def memory_size(self) -> int:
        """Closed form of CompressedTensor.memory_size (LCT/comp_tensor.py:57-72)."""
        fixed = self.encoded.nbytes + self.side.nbytes + self.blocks.nbytes + 16 + 4 + 4096
        if self.buffered:
            return fixed + 16 + int(self.descriptor[1])
        return fixed + self.lanes.nbytes + self.starts.nbytes + self.tail.nbytes


def shift_tables(base_encode, base_decode, center: int):
    enc = np.zeros(256, dtype=np.int32)
    dec = np.zeros(1024, dtype=np.int32)
    lib().lcto_shift_tables(_p(np.ascontiguousarray(base_encode, dtype=np.int32)),
                            _p(np.ascontiguousarray(base_decode, dtype=np.int32)),
                            ctypes.c_int32(center), _p(enc), _p(dec))
    return enc, dec


def sample_positions(n: int) -> np.ndarray:
    """Logical positions of the center's min(n, 4096) samples."""
    out = np.zeros(min(n, 4096), dtype=np.int64)
    if n:
        lib().lcto_sample_positions(ctypes.c_int64(n), ctypes.c_int64(out.size), _p(out))
    return out


def estimate_center(source: np.ndarray, precomputed: bool = False) -> int:
    n = source.size
    if n == 0:
        return 0
    return int(lib().lcto_estimate_center(_p(source), n, min(n, 4096), int(precomputed)))


def compress(source: np.ndarray, geometry, base_encode, base_decode, rare_length: int, *,
             precomputed: bool = False, side: np.ndarray | None = None,
             buffer: Buffer | None = None, center: int | None = None) -> Compressed:
    """Full compress pipeline (LCT/codec/encode.py:22-218) on the host.

    ``source``: flat int16/uint16 BF16 bits, or uint8 exponent bytes (logical
    order) with ``side`` holding side bytes in storage order if precomputed.
    """
    B, L, S, W = (int(v) for v in geometry)
    source = np.ascontiguousarray(source.reshape(-1))
    if not precomputed:
        source = source.view(np.int16)
    n = source.size
    nb = -(-n // B)
    size = nb * B
    ns = nb * L
    if center is None:
        center = estimate_center(source, precomputed)
    enc, dec = shift_tables(base_encode, base_decode, center)
    encoded = np.zeros(ns * W + 4, dtype=np.int32)
    if precomputed:
        side_out = np.ascontiguousarray(side, dtype=np.uint8).copy()
    else:
        side_out = np.zeros(size, dtype=np.uint8)
    extra = np.full(ns, 255, dtype=np.uint8)
    summaries = np.zeros(4 * nb, dtype=np.int32)
    counts = np.zeros(4, dtype=np.int32)
    g = _geo(geometry)
    if nb:
        lib().lcto_encode(_p(source), int(precomputed), _p(side_out), _p(encoded), _p(enc),
                          _p(extra), _p(summaries), ctypes.c_int64(size), ctypes.c_int64(n), g)
        lib().lcto_prefix(_p(summaries), ctypes.c_int64(nb), _p(counts))
    total_count, total_bytes = int(counts[0]), int(counts[1])
    blocks = np.zeros(3 * nb, dtype=np.int32)
    result = Compressed(n, size, tuple(geometry), int(center), int(rare_length), enc, dec,
                        encoded, side_out, extra, summaries, counts, blocks,
                        np.zeros(0, np.uint8), np.zeros(0, np.uint8), np.zeros(0, np.uint8))
    if buffer is None:
        result.lanes = np.zeros(total_count, dtype=np.uint8)
        result.starts = np.zeros(total_count, dtype=np.uint8)
        result.tail = np.zeros(total_bytes, dtype=np.uint8)
        target = (result.lanes, result.starts, result.tail, 0, 0, 0)
        write = True
    else:
        result.descriptor = buffer.allocate(total_bytes + 2 * total_count)
        base = int(result.descriptor[0])
        result.lanes = result.starts = result.tail = buffer.arena
        result.lane_off, result.start_off = base, base + total_count
        result.tail_off = base + 2 * total_count
        target = (buffer.arena, buffer.arena, buffer.arena, result.lane_off,
                  result.start_off, result.tail_off)
        write = int(result.descriptor[2]) == 0
    if nb:
        if write:
            lib().lcto_compact_extra(_p(source), int(precomputed), _p(extra), _p(summaries),
                                     ctypes.c_int64(nb), ctypes.c_int64(size), ctypes.c_int64(n),
                                     g, _p(target[0]), _p(target[1]), _p(target[2]),
                                     ctypes.c_int64(target[3]), ctypes.c_int64(target[4]),
                                     ctypes.c_int64(target[5]), _p(blocks))
        else:
            blocks[:nb] = summaries[:nb]
            blocks[nb:2 * nb] = summaries[2 * nb:3 * nb]
            blocks[2 * nb:] = summaries[3 * nb:]
    return result


def decompress(c: Compressed) -> np.ndarray:
    """BF16 bits (uint16[n]) of a compressed tensor (LCT/codec/decode.py:54-82)."""
    out = np.zeros(c.n, dtype=np.int16)
    if c.n:
        ov = c.overflow()
        if c.buffered and int(c.descriptor[2]) != 0:
            ov = None
        lib().lcto_decode(_p(c.encoded), _p(c.side), _p(out), _p(c.shifted_decode),
                          ctypes.c_int32(c.center), ctypes.c_int32(c.rare_length),
                          ctypes.c_int64(c.size), ctypes.c_int64(c.n), _geo(c.geometry),
                          None if ov is None else ctypes.byref(ov))
    return out.view(np.uint16)


OP_ADD, OP_MULTIPLY, OP_SCALAR_MUL_ADD = 0, 1, 2


def pointwise(c: Compressed, other_bits: np.ndarray, op: int, alpha: float = 1.0,
              beta: float = 1.0, alpha_is_one: bool = False, beta_is_one: bool = True,
              policy: int = 0):
    """Fused op with a dense BF16 operand (LCT/kernels/generic/pointwise.py).

    policy 0 returns uint16[n] BF16 bits; policy 1 returns (side uint8[size],
    exponent uint8[n]) components.
    """
    other = np.ascontiguousarray(other_bits.reshape(-1)).view(np.uint16)
    ov = c.overflow()
    if policy == 0:
        out = np.zeros(c.n, dtype=np.uint16)
        aux = None
    else:
        out = np.zeros(c.size, dtype=np.uint8)
        aux = np.zeros(c.size, dtype=np.uint8)
    lib().lcto_pointwise(_p(c.encoded), _p(c.side), _p(c.shifted_decode),
                         ctypes.c_int32(c.center), ctypes.c_int32(c.rare_length),
                         ctypes.c_int64(c.size), ctypes.c_int64(c.n), _geo(c.geometry),
                         None if ov is None else ctypes.byref(ov), _p(other), int(op),
                         ctypes.c_float(alpha), ctypes.c_float(beta), int(alpha_is_one),
                         int(beta_is_one), int(policy), _p(out), _p(aux))
    return out if policy == 0 else (out, aux[: c.n])


def dual(a: Compressed, b: Compressed, alpha: float, policy: int = 0):
    """Fused alpha*A + B of two compressed operands."""
    a_ov, b_ov = a.overflow(), b.overflow()
    if policy == 0:
        out = np.zeros(a.n, dtype=np.uint16)
        aux = None
    else:
        out = np.zeros(a.size, dtype=np.uint8)
        aux = np.zeros(a.size, dtype=np.uint8)
    lib().lcto_dual(_p(a.encoded), _p(a.side), _p(a.shifted_decode), ctypes.c_int32(a.center),
                    None if a_ov is None else ctypes.byref(a_ov),
                    _p(b.encoded), _p(b.side), _p(b.shifted_decode), ctypes.c_int32(b.center),
                    None if b_ov is None else ctypes.byref(b_ov),
                    ctypes.c_int32(a.rare_length), ctypes.c_int64(a.size), ctypes.c_int64(a.n),
                    _geo(a.geometry), ctypes.c_float(alpha), int(policy), _p(out), _p(aux))
    return out if policy == 0 else (out, aux[: a.n])


def apply(op: int, left: int, right: int, alpha: float = 1.0, beta: float = 1.0,
          alpha_is_one: bool = False, beta_is_one: bool = True) -> int:
    return int(lib().lcto_apply(int(op), int(left), int(right), alpha, beta,
                                int(alpha_is_one), int(beta_is_one)))


def apply_array(op: int, left_bits: np.ndarray, right_bits: np.ndarray, alpha: float = 1.0,
                beta: float = 1.0, alpha_is_one: bool = False,
                beta_is_one: bool = True) -> np.ndarray:
    """``apply`` elementwise over two equal-length BF16 bit arrays."""
    left = np.ascontiguousarray(left_bits.reshape(-1)).view(np.uint16)
    right = np.ascontiguousarray(right_bits.reshape(-1)).view(np.uint16)
    if left.size != right.size:
        raise ValueError("operands differ in length")
    out = np.zeros(left.size, dtype=np.uint16)
    lib().lcto_apply_n(int(op), _p(left), _p(right), ctypes.c_int64(left.size),
                       ctypes.c_float(alpha), ctypes.c_float(beta), int(alpha_is_one),
                       int(beta_is_one), _p(out))
    return out


def f32_to_bf16(value: float) -> int:
    return int(lib().lcto_f32_to_bf16(value))
