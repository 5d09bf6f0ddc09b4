"""The C-ABI boundary (CPU): header, library exports and argument checks.

``include/lct.h`` declares the entry points that replace the reference's
operator boundary (LCT/kernels/dispatch.py).  The built library must export
exactly those symbols, the ctypes binding must agree with the declared
argument counts, and every entry point must reject bad arguments before it
touches the GPU (these calls launch nothing).
"""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import ROOT
from losslessly_compressed_tensors_amd.kernels import hip

HEADER = ROOT / "include" / "lct.h"
LCT_E_NULL, LCT_E_GEOMETRY, LCT_E_SIZE, LCT_E_ARG = -1, -2, -3, -4


def _declarations() -> dict[str, int]:
    """name -> number of parameters, from the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for match in re.finditer(r"(?:int32_t|const char \*)\s*(lct_\w+)\s*\(([^)]*)\)\s*;", text):
        params = match.group(2).strip()
        out[match.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    if not hip.LIBRARY_PATH.exists():
        pytest.skip("liblct_hip.so not built (python -m losslessly_compressed_tensors_amd.build)")
    return hip.load_library()


def test_header_declares_every_binding():
    declared = _declarations()
    assert set(declared) == set(hip.EXPORTED)
    for name, argtypes in hip._SIGNATURES.items():
        assert declared[name] == len(argtypes), name


def test_library_exports_exactly_the_header(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(hip.LIBRARY_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines()
                if line.split() and line.split()[-1].startswith("lct_")}
    assert exported == set(_declarations())


def test_version_and_error_strings(lib):
    assert lib.lct_version().decode().startswith("lct-hip-gfx950")
    for code in (LCT_E_NULL, LCT_E_GEOMETRY, LCT_E_SIZE, LCT_E_ARG):
        assert lib.lct_error_string(code)


def _nulls(name):
    """Arguments for ``name`` with every pointer NULL and plain scalars."""
    args = []
    for argtype in hip._SIGNATURES[name]:
        if argtype is hip.Geometry:
            args.append(hip.Geometry(32768, 256, 128, 12))
        elif argtype in (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64):
            args.append(argtype(1))
        else:
            args.append(None)
    return args


# Entry points that take no pointer.
_NO_POINTERS = {"lct_set_wait_limits", "lct_set_decoder"}


@pytest.mark.parametrize("name", sorted(set(hip._SIGNATURES) - _NO_POINTERS))
def test_null_pointers_are_rejected(lib, name):
    assert getattr(lib, name)(*_nulls(name)) == LCT_E_NULL


def test_wait_limits_reject_negative_bounds_and_restore_defaults(lib):
    assert lib.lct_set_wait_limits(-1, 0) == LCT_E_ARG
    assert lib.lct_set_wait_limits(0, -1) == LCT_E_ARG
    assert lib.lct_set_wait_limits(16, 16) == 0
    assert lib.lct_set_wait_limits(0, 0) == 0   # the defaults again


def test_decoder_choice_accepts_only_its_modes(lib):
    assert lib.lct_set_decoder(3) == LCT_E_ARG
    assert lib.lct_set_decoder(-1) == LCT_E_ARG
    for mode in (1, 2, 0):   # ends on the default (automatic)
        assert lib.lct_set_decoder(mode) == 0


def test_bad_geometry_is_rejected_before_launch(lib):
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced: geometry fails first
    for geometry in [hip.Geometry(32768, 256, 100, 12), hip.Geometry(32768, 128, 256, 12),
                     hip.Geometry(32768, 256, 128, 1), hip.Geometry(32768, 256, 128, 65)]:
        code = lib.lct_decode(fake, fake, fake, fake, fake, 32768, 32768, geometry, 8, None, None)
        assert code == LCT_E_GEOMETRY
        code = lib.lct_encode(fake, fake, fake, fake, fake, fake, 32768, 32768, geometry, 0, 1,
                              None)
        assert code == LCT_E_GEOMETRY


def test_call_raises_on_error_code(lib):
    with pytest.raises(hip.LCTKernelError, match="lct_decode failed with code -1"):
        hip.call("lct_decode", *_nulls("lct_decode"))


def test_allocate_compact_rejects_bad_frees_and_ready_before_launch(lib):
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced: the checks fail first
    geometry = hip.Geometry(32768, 256, 128, 12)

    def call(frees, ready=fake):
        return lib.lct_allocate_compact(fake, fake, fake, fake, fake, 256, fake, fake, fake,
                                        frees, ready, 1, 32768, 32768, geometry, 0, None)

    too_many = hip.PendingFrees()
    too_many.count = hip.MAX_PENDING_FREES + 1
    assert call(ctypes.byref(too_many)) == -4          # LCT_E_ARG
    missing = hip.PendingFrees()
    missing.count = 1                                  # descriptor[0] is NULL
    assert call(ctypes.byref(missing)) == LCT_E_NULL
    assert call(None, ready=ctypes.c_void_p((1 << 20) + 4)) == -4   # ready not 8-byte aligned
    bad_regions = lib.lct_allocate_compact(fake, fake, fake, fake, fake, 100, fake, fake, fake,
                                           None, fake, 1, 32768, 32768, geometry, 0, None)
    assert bad_regions == -4


def test_free_batch_rejects_bad_counts_and_null_descriptors_before_launch(lib):
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced: the checks fail first
    array = (ctypes.c_void_p * hip.MAX_FREE_BATCH)(*([1 << 20] * hip.MAX_FREE_BATCH))

    def call(count, regions=256, descriptors=array):
        return lib.lct_buffer_free_batch(fake, regions, descriptors, count, None, None)

    assert call(0) == LCT_E_ARG
    assert call(-1) == LCT_E_ARG
    assert call(hip.MAX_FREE_BATCH + 1) == LCT_E_ARG
    assert call(1, regions=100) == LCT_E_ARG            # not a power of two
    holes = (ctypes.c_void_p * 3)(1 << 20, None, 1 << 20)
    assert call(3, descriptors=holes) == LCT_E_NULL


def test_no_alloc_compress_rejects_tensors_beyond_its_array(lib):
    """More than 8192 codec blocks exceed the file-scope working array: rejected
    before anything is launched (the fake pointers are never dereferenced)."""
    fake = ctypes.c_void_p(1 << 20)
    geometry = hip.Geometry(32768, 256, 128, 12)

    def call(blocks):
        size = blocks * 32768
        return lib.lct_compress_buffered_noalloc(fake, size, size, geometry, fake, fake, fake,
                                                 fake, fake, fake, None, fake, fake, fake, fake,
                                                 256, fake, None, None)

    assert call(8193) == -5   # LCT_E_SCRATCH
    assert lib.lct_error_string(-5).decode().startswith("tensor larger than")
    bad_size = lib.lct_compress_buffered_noalloc(fake, 10, 32768 * 2, geometry, fake, fake, fake,
                                                 fake, fake, fake, None, fake, fake, fake, fake,
                                                 256, fake, None, None)
    assert bad_size == LCT_E_SIZE   # a whole empty block of padding


def test_encode_fused_rejects_bad_arguments_before_launch(lib):
    """lct_encode_fused checks its epoch, control array, sample count, buffer
    and frees before anything is launched (the fake pointers are never
    dereferenced)."""
    fake = ctypes.c_void_p(1 << 20)
    geometry = hip.Geometry(32768, 256, 128, 12)
    size = 4 * 32768

    def call(sample_size=4096, control=fake, words=64 + 4, epoch=7, meta=None,
             regions=256, frees=None, logical=size, host_totals=None):
        return lib.lct_encode_fused(fake, fake, fake, sample_size, fake, fake, fake, fake, None,
                                    fake, fake, fake, fake, control, words, epoch, fake, meta,
                                    regions, frees, host_totals, size, logical, geometry, 0,
                                    None)

    assert call(epoch=0) == LCT_E_ARG                       # 0 matches a fresh array
    assert call(meta=fake, host_totals=fake) == LCT_E_ARG   # host totals: private only
    assert call(host_totals=ctypes.c_void_p((1 << 20) + 4)) == LCT_E_ARG   # not 8-byte aligned
    assert call(words=64 + 3) == LCT_E_SIZE                 # no word for the last block
    assert call(control=ctypes.c_void_p((1 << 20) + 4)) == LCT_E_ARG   # not 8-byte aligned
    assert call(sample_size=3000) == LCT_E_ARG              # neither n nor a power of two
    assert call(sample_size=8192) == LCT_E_SIZE             # more than 4096 samples
    assert call(logical=size - 32768) == LCT_E_SIZE         # a whole block of padding
    assert call(meta=fake, regions=100) == LCT_E_ARG        # not a power of two
    too_many = hip.PendingFrees()
    too_many.count = hip.MAX_PENDING_FREES + 1
    assert call(meta=fake, frees=ctypes.byref(too_many)) == LCT_E_ARG
    missing = hip.PendingFrees()
    missing.count = 1
    assert call(meta=fake, frees=ctypes.byref(missing)) == LCT_E_NULL


def test_compress_batch_rejects_bad_jobs_before_launch(lib):
    """lct_compress_batch checks the job count, every job and the working
    arrays' sizes before anything is launched (the fake pointers are never
    dereferenced)."""
    base = 1 << 20

    def job(steps=128, words=12, blocks=4, logical=None, source=base, side=base, sample=4096):
        size = blocks * 256 * steps
        return hip.CompressJob(source, side, base, base, base, base, base, None, base, base,
                               base, sample, size, size if logical is None else logical,
                               hip.Geometry(256 * steps, 256, steps, words))

    def call(jobs, extra=1 << 20, summaries=1 << 20, control=1 << 20, epoch=7, regions=256,
             frees=None, control_address=base):
        array = (hip.CompressJob * max(len(jobs), 1))(*jobs)
        return lib.lct_compress_batch(array, len(jobs), base, extra, base, summaries,
                                      control_address, control, epoch, base, regions, base,
                                      frees, None)

    two = [job(), job(blocks=9, logical=9 * 32768 - 5)]
    assert call([]) == LCT_E_ARG                                       # no job
    assert call([job()] * (hip.MAX_COMPRESS_BATCH + 1)) == LCT_E_ARG   # more than the table
    assert call(two, epoch=0) == LCT_E_ARG                             # 0 matches a fresh array
    assert call(two, control_address=base + 4) == LCT_E_ARG            # not 8-byte aligned
    assert call(two, regions=100) == LCT_E_ARG                         # not a power of two
    assert call([job(), job(steps=256, words=25)]) == LCT_E_ARG        # two step counts
    assert call([job(), job(source=base + 2)]) == LCT_E_ARG            # not 16-byte aligned
    assert call([job(), job(side=None)]) == LCT_E_NULL                 # a missing array
    assert call([job(), job(sample=3000)]) == LCT_E_ARG                # neither n nor 2^k
    assert call([job(), job(logical=3 * 32768)]) == LCT_E_SIZE         # a block of padding
    assert call([job(), job(words=1)]) == LCT_E_GEOMETRY
    # Working arrays: 256 extra starts per block, 5 nb + 1 summary words per
    # job, a gate word and 64 + nb control words per job.
    assert call(two, extra=13 * 256 - 1) == LCT_E_SIZE
    assert call(two, summaries=5 * 13 + 2 - 1) == LCT_E_SIZE
    assert call(two, control=1 + 2 * 64 + 13 - 1) == LCT_E_SIZE
    too_many = hip.PendingFrees()
    too_many.count = hip.MAX_PENDING_FREES + 1
    assert call(two, frees=ctypes.byref(too_many)) == LCT_E_ARG
    missing = hip.PendingFrees()
    missing.count = 1
    assert call(two, frees=ctypes.byref(missing)) == LCT_E_NULL


def test_update_batch_rejects_bad_jobs_before_launch(lib):
    """lct_pointwise_update_batch checks the job count, the operation, every
    job and the working arrays' sizes before anything is launched (the fake
    pointers are never dereferenced)."""
    base = 1 << 20

    def job(steps=128, words=12, blocks=4, logical=None, side_out=base, sample=4096, rare=5):
        size = blocks * 256 * steps
        j = hip.UpdateJob()
        j.encoded = j.side = j.shifted_decode = j.center = base
        j.other = j.base_encode = j.base_decode = j.center_out = j.shifted_decode_out = base
        j.side_out = side_out
        j.encoded_out = j.exponents = j.counts = j.blocks = j.descriptor = base
        j.size, j.logical_numel = size, size if logical is None else logical
        j.sample_size = sample
        j.geometry = hip.Geometry(256 * steps, 256, steps, words)
        j.rare_length = rare
        return j

    def call(jobs, op=2, alpha_is_one=1, beta_is_one=1, partials=1 << 20, extra=1 << 20,
             summaries=1 << 20, control=1 << 20, epoch=7, regions=256, frees=None):
        array = (hip.UpdateJob * max(len(jobs), 1))(*jobs)
        return lib.lct_pointwise_update_batch(array, len(jobs), op, alpha_is_one, beta_is_one,
                                              None, None, base, partials, base, extra, base,
                                              summaries, base, control, epoch, base, regions,
                                              base, frees, None)

    two = [job(), job(blocks=9, logical=9 * 32768 - 5)]
    assert call([]) == LCT_E_ARG                                      # no job
    assert call([job()] * (hip.MAX_UPDATE_BATCH + 1)) == LCT_E_ARG    # more than the table
    assert call(two, op=3) == LCT_E_ARG                               # no such operation
    assert call(two, alpha_is_one=0) == LCT_E_NULL                    # alpha needed, absent
    assert call(two, epoch=0) == LCT_E_ARG                            # 0 matches a fresh array
    assert call(two, regions=100) == LCT_E_ARG                        # not a power of two
    assert call([job(), job(steps=256, words=25)]) == LCT_E_ARG       # two step counts
    assert call([job(), job(side_out=base + 4)]) == LCT_E_ARG         # not 16-byte aligned
    assert call([job(), job(sample=3000)]) == LCT_E_ARG               # neither n nor 2^k
    assert call([job(), job(rare=9)]) == LCT_E_ARG                    # rare length above 8
    assert call([job(), job(logical=3 * 32768)]) == LCT_E_SIZE        # a block of padding
    assert call([job(), job(words=1)]) == LCT_E_GEOMETRY
    # Working arrays: 2 partial words per 64 samples, 256 extra starts per
    # block, 5 nb + 1 summary words per job, a gate word and 64 + nb control
    # words per job.
    assert call(two, partials=2 * 64 * 2 - 1) == LCT_E_SIZE
    assert call(two, extra=13 * 256 - 1) == LCT_E_SIZE
    assert call(two, summaries=5 * 13 + 2 - 1) == LCT_E_SIZE
    assert call(two, control=1 + 2 * 64 + 13 - 1) == LCT_E_SIZE
    too_many = hip.PendingFrees()
    too_many.count = hip.MAX_PENDING_FREES + 1
    assert call(two, frees=ctypes.byref(too_many)) == LCT_E_ARG


def test_fused_update_encoders_reject_bad_bookkeeping_before_launch(lib):
    """lct_pointwise_encode_fused and lct_dual_encode_fused check their
    bookkeeping record (control array, epoch, buffer, frees) before anything
    is launched (the fake pointers are never dereferenced)."""
    fake = ctypes.c_void_p(1 << 20)
    geometry = hip.Geometry(65536, 256, 256, 25)
    size = 4 * 65536

    def record(words=64 + 4, epoch=7, control=1 << 20, meta=None, regions=256, frees=0):
        r = hip.Bookkeeping()
        r.control = control
        r.control_words = words
        r.epoch = epoch
        r.counts = 1 << 20
        r.blocks = 1 << 20
        r.descriptor = 1 << 20
        r.buffer_meta = meta
        r.max_free_regions = regions
        r.frees.count = frees
        return r

    def pointwise(r):
        return lib.lct_pointwise_encode_fused(
            fake, fake, fake, fake, None, fake, None, None, fake, 4096, fake, fake, fake, fake,
            fake, fake, fake, fake, fake, size, size, geometry, 5, 0, 0, 1,
            None if r is None else ctypes.byref(r), None)

    def dual(r):
        return lib.lct_dual_encode_fused(
            fake, fake, fake, fake, None, fake, fake, fake, fake, None, fake, fake, 4096, fake,
            fake, fake, fake, fake, fake, fake, fake, fake, size, size, geometry, 5,
            None if r is None else ctypes.byref(r), None)

    for call in (pointwise, dual):
        assert call(None) == LCT_E_NULL                                  # no record
        assert call(record(epoch=0)) == LCT_E_ARG                        # 0 matches a fresh array
        assert call(record(words=64 + 3)) == LCT_E_SIZE                  # no word for the last block
        assert call(record(control=(1 << 20) + 4)) == LCT_E_ARG          # not 8-byte aligned
        assert call(record(meta=1 << 20, regions=100)) == LCT_E_ARG      # not a power of two
        assert call(record(meta=1 << 20, frees=hip.MAX_PENDING_FREES + 1)) == LCT_E_ARG
        assert call(record(meta=1 << 20, frees=1)) == LCT_E_NULL         # a missing descriptor
