/* C ABI of the MI355X (gfx950) LCT codec library, liblct_hip.so.
 *
 * Each entry point replaces one kernel-launch function of the reference's
 * operator boundary, LCT/kernels/dispatch.py (cited per function; paths are
 * relative to the reference repository root).  Conventions:
 *
 *  - every pointer argument is a device pointer unless documented otherwise;
 *    sizes are element counts; nothing is allocated, synchronised or thrown;
 *  - work is enqueued on `stream` (NULL = the default stream);
 *  - the return value is LCT_OK, a negative LCT_E* argument error (nothing
 *    was launched), or a positive hipError_t from the launch;
 *  - device-side failures (allocator) are reported through the allocator
 *    descriptor/status words, as in the reference.
 *
 * Storage format (identical to the reference's): a tensor of n BF16 values is
 * padded to N = nb*B storage elements in nb blocks of L=256 lanes x S steps.
 * Storage (block k, step t, lane l) holds logical element
 * (k*S+t)*256 + (l ^ ((k*S+t) & 254)).  Each lane's exponents form one Huffman
 * stream whose first W 32-bit words live at encoded[w*nb*256 + k*256 + l];
 * sign+mantissa bytes are stored separately in storage order.
 */
#ifndef LCT_H
#define LCT_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LCT_OK 0
#define LCT_E_NULL (-1)        /* a required pointer is NULL */
#define LCT_E_GEOMETRY (-2)    /* geometry not (B, 256, B/256, W) with even S, 2 <= W <= 64 */
#define LCT_E_SIZE (-3)        /* sizes inconsistent or out of the supported range */
#define LCT_E_ARG (-4)         /* another argument out of range */
#define LCT_E_SCRATCH (-5)     /* larger than lct_compress_buffered_noalloc's working array */

/* Stream geometry (B, L, S, W): LCT/codec/geometry.py:13-39. */
typedef struct {
    int32_t block_symbols; /* B = L * S */
    int32_t lanes;         /* L, always 256 */
    int32_t steps;         /* S, even */
    int32_t fixed_words;   /* W, 32-bit payload words per stream */
} lct_geometry;

/* Overflow (fallback) storage of one compressed tensor, as
 * LCT/kernels/backends.py:36-50 (FallbackStorage) + decode.py:195-240 read it.
 * Private layout: lanes/starts/tail are separate arrays, `base` is the tail
 * base (CompressedTensor.fallback_base).  Buffered layout: lanes, starts and
 * tail all point at the TensorBuffer arena; entries sit at descriptor[0],
 * starts at descriptor[0]+count, tails at descriptor[0]+2*count. */
typedef struct {
    const uint8_t *lanes;
    const uint8_t *starts;
    const uint8_t *tail;
    const int32_t *blocks;     /* int32[3*nb]: count, first entry, tail byte base */
    const int32_t *count;      /* int32[1]: total entries (buffered offsets) */
    const int32_t *descriptor; /* int32[4] TensorBuffer descriptor, or NULL = private */
    int64_t base;              /* private tail base */
} lct_overflow;

/* Frees a caller deferred to its next arena reservation (at most
 * LCT_MAX_PENDING_FREES descriptors of the same TensorBuffer, applied in
 * order). */
#define LCT_MAX_PENDING_FREES 4
typedef struct {
    int32_t *descriptor[LCT_MAX_PENDING_FREES];
    int32_t count;
} lct_pending_frees;

/* The overflow bookkeeping an encoder launch can do in its own workgroup 0
 * after that workgroup's block (lct_pointwise_encode_fused,
 * lct_dual_encode_fused), with the arrays of lct_encode_fused's:
 * control: uint64[control_words >= 64 + nb], one array per stream, zeroed once
 * when created and never again; epoch: a value != 0 that no earlier call with
 * this control array used; counts: int32[4]; blocks: int32[3 * nb];
 * buffer_meta: the TensorBuffer's metadata, or NULL for private storage;
 * descriptor: int32[4] (buffered); max_free_regions: the buffer's R; frees:
 * deferred frees applied first, as lct_allocate_compact applies them.
 * a_samples, b_samples (lct_dual_encode_fused; lct_pointwise_encode_fused
 * does not read them): both operands' values at the center's sample
 * positions, as lct_dual_sample takes them, or NULL.  When both are given the
 * launch takes the result's center itself, as lct_encode_fused does: its
 * first ceil(sample_size / 64) workgroups compute the result at the sample
 * positions, publish their partial sums in control[0, 64) and write the
 * result's values to result_samples (NULL: not recorded); `partials` is then
 * not read and may be NULL.  The outputs equal those of lct_dual_sample
 * followed by this launch with `partials`. */
typedef struct {
    uint64_t *control;
    int64_t control_words;
    uint32_t epoch;
    int32_t *counts;
    int32_t *blocks;
    int32_t *descriptor;
    int32_t *buffer_meta;
    int32_t max_free_regions;
    lct_pending_frees frees;
    const uint16_t *a_samples;
    const uint16_t *b_samples;
    uint16_t *result_samples;
} lct_bookkeeping;

/* Pointwise operation selectors: LCT/codec/pointwise.py:289-304. */
#define LCT_OP_ADD 0
#define LCT_OP_MULTIPLY 1
#define LCT_OP_SCALAR_MUL_ADD 2
/* Output policies: LCT/kernels/generic/pointwise.py:14-15. */
#define LCT_DENSE_OUTPUT 0
#define LCT_COMPRESSED_OUTPUT 1

/* Library version string (host pointer, static storage). */
const char *lct_version(void);

/* Human-readable text for an LCT_* or hipError_t return code. */
const char *lct_error_string(int32_t code);

/* ---- tables: replaces dispatch.py:33-48 (estimate_and_shift_encoding_table)
 * Sample min(logical_numel, 4096)=sample_size exponents of `source` (int16 BF16
 * bits, or uint8 exponent bytes if `precomputed`), store their rounded mean in
 * center[0], and build the center-shifted tables: shifted_encode int32[256]
 * indexed by raw exponent byte, shifted_decode int32[1024] holding
 * len | exponent<<8.  base_encode/base_decode are the distribution's tables. */
int32_t lct_estimate_and_shift_tables(const void *source, int32_t precomputed,
                                      int64_t logical_numel, int64_t sample_size,
                                      const int32_t *base_encode,
                                      const int32_t *base_decode,
                                      int32_t *center, int32_t *shifted_encode,
                                      int32_t *shifted_decode, hipStream_t stream);

/* ---- the sampling half of dispatch.py:33-48 spread over many workgroups:
 * sample min(logical_numel, 4096) = sample_size exponents of `source` (as
 * lct_estimate_and_shift_tables) and write each group of 64 samples' kept
 * exponent sum and count to partials[2*g], partials[2*g+1]
 * (int32[2*ceil(sample_size/64)]).  sample_values: NULL, or uint16[
 * sample_size] that receives the sampled BF16 bits (ignored if precomputed).
 * lct_encode_sampled turns the partials into the center and tables. */
int32_t lct_sample_center(const void *source, int32_t precomputed,
                          int64_t logical_numel, int64_t sample_size,
                          int32_t *partials, uint16_t *sample_values,
                          hipStream_t stream);

/* ---- replaces dispatch.py:16-30 (shift_encoding_table): same tables for a
 * given device-resident center. */
int32_t lct_shift_tables(const int32_t *base_encode, const int32_t *center,
                         int32_t *shifted_encode, const int32_t *base_decode,
                         int32_t *shifted_decode, hipStream_t stream);

/* ---- replaces dispatch.py:51-62 (shift_decoding_table). */
int32_t lct_shift_decoding_table(const int32_t *base_decode,
                                 const int32_t *center, int32_t *shifted_decode,
                                 hipStream_t stream);

/* ---- encoder: replaces dispatch.py:294-316 (encode_kernel).
 * source: int16 BF16 bits [logical_numel] or, if precomputed, uint8 exponent
 * bytes [logical_numel] (logical order).  side: uint8[size] sign+mantissa in
 * storage order -- written here unless precomputed (padding is written as 0).
 * encoded: int32[nb*256*W + 4]; every one of the first nb*256*W words is
 * written (words a stream does not use are 0).  extra_starts: uint8[nb*256],
 * the first overflowing (even) step of each stream or 255.  summaries: the
 * per-block overflow count and tail bytes go to its first 2*nb entries when
 * write_summary, else unused.  size = nb*B.  source, side and encoded must be
 * 16-byte aligned. */
int32_t lct_encode(const void *source, uint8_t *side, int32_t *encoded,
                   const int32_t *shifted_encode, uint8_t *extra_starts,
                   int32_t *summaries, int64_t size, int64_t logical_numel,
                   lct_geometry geometry, int32_t precomputed,
                   int32_t write_summary, hipStream_t stream);

/* ---- lct_encode with the table step of dispatch.py:33-48 folded in: every
 * workgroup reduces `partials` (lct_sample_center, same sample_size) to the
 * center and shifts base_encode by it; center_out[1] and
 * shifted_decode_out[1024] receive the center and the shifted decode table
 * (as lct_estimate_and_shift_tables writes them).  Other arguments and
 * outputs as lct_encode. */
int32_t lct_encode_sampled(const void *source, uint8_t *side, int32_t *encoded,
                           const int32_t *partials, int64_t sample_size,
                           const int32_t *base_encode, const int32_t *base_decode,
                           int32_t *center_out, int32_t *shifted_decode_out,
                           uint8_t *extra_starts, int32_t *summaries, int64_t size,
                           int64_t logical_numel, lct_geometry geometry,
                           int32_t precomputed, int32_t write_summary,
                           hipStream_t stream);

/* ---- replaces dispatch.py:70-85 (prefix_allocate) and the block-metadata
 * part of compact_extra: summaries is int32[5*nb + 1] whose first 2*nb
 * entries the encoder filled; writes the exclusive scans of the per-block
 * overflow counts/bytes into summaries[2nb..4nb), the list of blocks with
 * overflow into summaries[4nb..) and its length into summaries[5nb];
 * blocks[3*nb] = {count, first, byte_base}; counts[4] = {total_count,
 * total_bytes, 0, 0}; if buffered, reserves align16(total_bytes +
 * 2*total_count) bytes from the TensorBuffer whose metadata starts at
 * buffer_meta (int32 free_starts[R] | free_sizes[R] | count | lock |
 * generation) and writes descriptor[4] = {offset, size, status, gen}.
 * Any n_blocks up to 65535 (fewer than 2^31 storage elements: the format's
 * offsets are int32); blocks are scanned in chunks of 8192 with running
 * totals, so entries keep block order at every size (the reference's path
 * above 8192 blocks, LCT/kernels/autotune.py:54, orders them by atomics). */
int32_t lct_prefix_allocate(int32_t *summaries, int32_t *counts,
                            int32_t *descriptor, int32_t *buffer_meta,
                            int32_t *blocks, int64_t n_blocks, int32_t buffered,
                            int32_t max_free_regions, hipStream_t stream);

/* ---- replaces the buffered sequence dispatch.py:70-85 (prefix_allocate)
 * + dispatch.py:113-130 (compact_extra), LCT/codec/encode.py:77-170, with
 * TensorBuffer.free (LCT/tensor_buffer.py:121-128) of up to
 * LCT_MAX_PENDING_FREES earlier allocations folded in: one launch.
 * Workgroup 0 takes the arena lock, applies `frees` in order (each as
 * lct_buffer_free would; statuses are not reported, a freed descriptor gets
 * status 5), then does what lct_prefix_allocate does with buffered = 1 and
 * stores `epoch` to *ready.  Every other workgroup waits (bounded) until
 * *ready == epoch and then writes the entries and tails of the listed blocks,
 * as lct_compact_extra with buffered = 1 (lanes, starts and tails in `arena`).
 * summaries: int32[5*nb + 1] as for lct_prefix_allocate, except that the
 * exclusive scans [2*nb, 4*nb) are not written (blocks holds them).  ready: a device
 * uint64 whose value before the launch differs from `epoch` and from ~epoch
 * (use a value no earlier call used).  The result (counts, descriptor, blocks,
 * arena bytes) equals lct_buffer_free on each pending descriptor followed by
 * lct_prefix_allocate and lct_compact_extra.  A compacting workgroup whose
 * bounded wait ends first writes nothing and leaves ~epoch in *ready; the
 * reservation then gets status 7 (LCT_STATUS_INCOMPLETE).  A failed reservation
 * of a non-empty request (status 1, 6 or 7) also sets a bit of the buffer's
 * failure word (LCT_FAIL_*). */
int32_t lct_allocate_compact(const void *source, int32_t *summaries, int32_t *counts,
                             int32_t *descriptor, int32_t *buffer_meta,
                             int32_t max_free_regions, uint8_t *arena, int32_t *blocks,
                             const uint8_t *extra_starts, const lct_pending_frees *frees,
                             uint64_t *ready, uint64_t epoch, int64_t size,
                             int64_t logical_numel, lct_geometry g, int32_t precomputed,
                             hipStream_t stream);

/* ---- replaces, for one tensor, the sequence dispatch.py:33-48 (center +
 * tables), :294-316 (encoder) and :70-85 (prefix + allocate) that
 * LCT/codec/encode.py:22-186 runs, in one launch of one workgroup per codec
 * block (the first 64 also sample the center before they encode; workgroup 0
 * does the bookkeeping after its block).  Its outputs equal those of
 * lct_sample_center (sample_values) -> lct_encode_sampled (side, encoded,
 * center_out, shifted_decode_out, extra_starts) -> lct_prefix_allocate
 * (counts, blocks, and the overflow-block list summaries[4*nb .. 5*nb]; the
 * other summary entries are not written).  With buffer_meta != NULL the
 * bookkeeping workgroup first applies `frees` (as lct_allocate_compact) and
 * then makes the reservation of lct_prefix_allocate with buffered = 1 into
 * descriptor; lct_compact_extra (buffered = 1, or into exact-size private
 * arrays after the host reads counts; summaries NULL or as written here) then
 * writes the entries and tails.
 * control: uint64[control_words >= 64 + nb], one array per stream, zeroed once
 * when created and never again; epoch: a value != 0 that no earlier call with
 * this control array used (the launch's cross-workgroup words carry it).
 * sample_size as lct_sample_center; sample_values may be NULL.  A bounded
 * device-side wait that gives up marks the tensor incomplete instead of
 * hanging: counts[3] = 1 and, with a buffer, status 7 and the failure word's
 * LCT_FAIL_INCOMPLETE bit.  source, side and encoded 16-byte aligned.
 * host_totals (private storage only, else NULL): uint64[2] in pinned host
 * memory, 8-byte aligned.  Once the bookkeeping has the totals, word 0
 * becomes epoch << 32 | entries | incomplete << 31 and word 1 epoch << 32 |
 * tail bytes (system-scope stores), so a host that sizes the exact overflow
 * arrays (the reference's sync on counts, LCT/codec/encode.py:137-171) can
 * poll them instead of waiting for the launch to end. */
int32_t lct_encode_fused(const void *source, uint8_t *side, int32_t *encoded,
                         int64_t sample_size, const int32_t *base_encode,
                         const int32_t *base_decode, int32_t *center_out,
                         int32_t *shifted_decode_out, uint16_t *sample_values,
                         uint8_t *extra_starts, int32_t *summaries, int32_t *blocks,
                         int32_t *counts, uint64_t *control, int64_t control_words,
                         uint32_t epoch, int32_t *descriptor, int32_t *buffer_meta,
                         int32_t max_free_regions, const lct_pending_frees *frees,
                         uint64_t *host_totals, int64_t size, int64_t logical_numel,
                         lct_geometry g, int32_t precomputed, hipStream_t stream);

/* ---- lct_encode_fused with a buffer, then lct_compact_extra (buffered = 1),
 * for up to LCT_MAX_COMPRESS_BATCH BF16 tensors in two launches: one fused
 * compress whose workgroups are the jobs' single-launch grids laid end to
 * end, and one compaction of every job's blocks.  No counterpart in the
 * reference, which compresses one tensor per call (LCT/codec/encode.py:189-218):
 * a tensor of a few codec blocks (a layer's activations, a weight's optimizer
 * state) is bound by one block's latency, so one launch serves several.
 * Each job's outputs are those of its own lct_encode_fused +
 * lct_compact_extra, except where in the arena its overflow region lies
 * (the jobs reserve in the order their bookkeeping takes the arena lock).
 * `frees` are applied before any job's reservation.  All jobs share
 * geometry.steps.  Working arrays, shared by the jobs and partitioned in job
 * order: extra_starts uint8[sum nb*256], summaries int32[sum (5*nb + 1)],
 * control uint64[1 + sum (64 + nb)] (the array of lct_encode_fused, with the
 * same zeroing and epoch rules).  arena: the buffer's payload arena (the
 * descriptors' offsets index into it).  A bounded wait that gives up marks
 * its tensor incomplete (status 7), as in lct_encode_fused. */
#define LCT_MAX_COMPRESS_BATCH 16
typedef struct {
    const void *source;          /* BF16 bits, logical_numel, 16-byte aligned */
    uint8_t *side;               /* uint8[size], 16-byte aligned */
    int32_t *encoded;            /* int32[nb*256*W + 4], 16-byte aligned */
    const int32_t *base_encode;
    const int32_t *base_decode;
    int32_t *center_out;         /* int32[1] */
    int32_t *shifted_decode_out; /* int32[1024] */
    uint16_t *sample_values;     /* uint16[sample_size], or NULL */
    int32_t *blocks;             /* int32[3*nb] */
    int32_t *counts;             /* int32[4] */
    int32_t *descriptor;         /* int32[4] */
    int64_t sample_size;
    int64_t size;
    int64_t logical_numel;
    lct_geometry geometry;
} lct_compress_job;
int32_t lct_compress_batch(const lct_compress_job *jobs, int32_t n_jobs,
                           uint8_t *extra_starts, int64_t extra_bytes, int32_t *summaries,
                           int64_t summary_words, uint64_t *control, int64_t control_words,
                           uint32_t epoch, int32_t *buffer_meta, int32_t max_free_regions,
                           uint8_t *arena, const lct_pending_frees *frees, hipStream_t stream);

/* ---- replaces dispatch.py:88-95 (count_bad_streams, the atomic path's
 * totals, LCT/kernels/generic/compaction.py:31-51): adds the number of
 * overflowing streams (extra_starts[s] != 255) to count[0] and their tail
 * bytes (steps - start) to total[0] with device atomics; the caller zeroes
 * both first. */
int32_t lct_count_bad_streams(const uint8_t *extra_starts, int32_t *count,
                              int32_t *total, int64_t n_streams, int32_t steps,
                              hipStream_t stream);

/* ---- replaces dispatch.py:98-110 (compact_bad_streams, compaction.py:54-96):
 * one workgroup per codec block reserves its entry slots and tail bytes with
 * atomics on bad_count[0] / fallback_total[0] (zeroed by the caller), writes
 * blocks[3*nb] = {count, first, byte_base} (0, 0, 0 for blocks without
 * overflow) and its entries (lane, start; lanes ascending) at first.. .
 * Buffered: lanes/starts point at the arena, entries at descriptor[0] and
 * starts at descriptor[0] + final_counts[0]; a failed reservation (status
 * != 0) gets no entries.  The order of the blocks' slices follows the
 * atomics; lct_compact_extra with summaries = NULL then writes the tails. */
int32_t lct_compact_bad_streams(const uint8_t *extra_starts, uint8_t *lanes,
                                uint8_t *starts, const int32_t *descriptor,
                                int32_t *blocks, const int32_t *final_counts,
                                int32_t *bad_count, int32_t *fallback_total,
                                int64_t n_streams, int32_t steps, int64_t n_blocks,
                                int32_t buffered, hipStream_t stream);

/* ---- replaces dispatch.py:113-130 (compact_extra): for the blocks listed by
 * lct_prefix_allocate (summaries path), or for every block with overflow
 * when summaries is NULL (block metadata from lct_compact_bad_streams,
 * BUILD_META=False, or from lct_encode_fused; one workgroup per block, which
 * needs no list), write the overflowing streams' lane and start bytes
 * (ascending lane) at entries blocks[nb+k].. and their exponent tails
 * int8(e-127) for steps start..S-1 from byte blocks[2nb+k].  Private:
 * lanes/starts/tail are exact-size arrays, tails at tail + base.  Buffered:
 * all three point at the arena; offsets from descriptor and count as in
 * lct_overflow.  A buffered allocation whose status is not 0 gets no entries
 * or tails written. */
int32_t lct_compact_extra(const void *source, uint8_t *lanes, uint8_t *starts,
                          uint8_t *tail, const int32_t *descriptor,
                          const int32_t *count, const int32_t *blocks, int64_t base,
                          const uint8_t *extra_starts, const int32_t *summaries,
                          int64_t size, int64_t logical_numel,
                          lct_geometry geometry, int32_t precomputed,
                          int32_t buffered, hipStream_t stream);

/* ---- decoder: replaces dispatch.py:319-361 (decode_kernel), with the
 * overflow overlay fused (overflow != NULL) as _decode_overflow_kernel does.
 * output: int16[logical_numel] BF16 bits in logical order. */
int32_t lct_decode(const int32_t *encoded, const uint8_t *side, int16_t *output,
                   const int32_t *shifted_decode, const int32_t *center,
                   int64_t size, int64_t logical_numel, lct_geometry geometry,
                   int32_t rare_length, const lct_overflow *overflow,
                   hipStream_t stream);

/* ---- several lct_decode calls in one launch: each job's arguments mean what
 * lct_decode's do (overflow: has_overflow != 0), and each job's output equals
 * its lct_decode's.  No counterpart in the reference, which decodes one tensor
 * per launch (dispatch.py:319-361): for tensors of a few codec blocks (a
 * layer's weights), whose decodes are bound by one block's latency, one launch
 * serves them all.  At most LCT_MAX_DECODE_BATCH jobs, 2^31 - 1 blocks in
 * all; the outputs must not overlap. */
#define LCT_MAX_DECODE_BATCH 16
typedef struct {
    const int32_t *encoded;
    const uint8_t *side;
    int16_t *output;
    const int32_t *shifted_decode;
    const int32_t *center;
    int64_t size;
    int64_t logical_numel;
    lct_geometry geometry;
    int32_t rare_length;
    int32_t has_overflow;
    lct_overflow overflow;
} lct_decode_job;
int32_t lct_decode_batch(const lct_decode_job *jobs, int32_t n_jobs, hipStream_t stream);

/* ---- replaces dispatch.py:146-165 (scatter_fallback,
 * LCT/kernels/generic/compaction.py:238-306): after a decode without the
 * overlay, rebuilds every overflow tail byte into BF16 with its side byte
 * and writes it at its logical position of output (int16[logical_numel]). */
int32_t lct_scatter_fallback(const lct_overflow *overflow, const uint8_t *side,
                             void *output, int64_t size, int64_t logical_numel,
                             lct_geometry geometry, hipStream_t stream);

/* ---- fused pointwise, one compressed + one dense operand: replaces
 * dispatch.py:168-187 (pointwise_dense); with overflow != NULL the overflow
 * rows are overlaid in the same pass (what dispatch.py:190-212,
 * pointwise_fallback, does as a second launch; see lct_pointwise_fallback).
 * other: bf16[logical_numel].  alpha/beta: float32[1] device scalars, read
 * only for LCT_OP_SCALAR_MUL_ADD when !alpha_is_one / !beta_is_one.
 * Dense policy: output bf16[logical_numel]; auxiliary unused.  Compressed
 * policy: output uint8[size] side bytes (storage order, padding 0) and
 * auxiliary uint8[>= logical_numel] exponent bytes (logical order). */
int32_t lct_pointwise_dense(const int32_t *encoded, const uint8_t *side,
                            const void *other, void *output, uint8_t *auxiliary,
                            const int32_t *shifted_decode, const int32_t *center,
                            const float *alpha, const float *beta,
                            int64_t size, int64_t logical_numel,
                            lct_geometry geometry, int32_t rare_length,
                            int32_t op, int32_t alpha_is_one,
                            int32_t beta_is_one, int32_t output_policy,
                            const lct_overflow *overflow, hipStream_t stream);

/* ---- replaces dispatch.py:190-212 (pointwise_fallback,
 * LCT/kernels/generic/pointwise.py:265-340): after lct_pointwise_dense
 * without the overlay, recomputes op(A, other) at every overflow tail byte
 * of A and stores it as lct_pointwise_dense does (dense BF16 at logical
 * positions, or side byte at the storage position, 0 for padding, and
 * exponent byte at the logical position). */
int32_t lct_pointwise_fallback(const lct_overflow *overflow, const uint8_t *side,
                               const void *other, void *output, uint8_t *auxiliary,
                               const float *alpha, const float *beta, int64_t size,
                               int64_t logical_numel, lct_geometry geometry, int32_t op,
                               int32_t alpha_is_one, int32_t beta_is_one,
                               int32_t output_policy, hipStream_t stream);

/* ---- fused alpha*A + B with both operands compressed (same geometry):
 * replaces dispatch.py:215-286 (dual_maps_init + dual_tables_and_maps +
 * dual_mapped) with one launch, the maps built per block in the prologue; a_shifted/b_shifted are each operand's
 * shifted decode table.  Outputs as lct_pointwise_dense. */
int32_t lct_dual(const int32_t *a_encoded, const uint8_t *a_side,
                 const int32_t *a_shifted_decode, const int32_t *a_center,
                 const lct_overflow *a_overflow, const int32_t *b_encoded,
                 const uint8_t *b_side, const int32_t *b_shifted_decode,
                 const int32_t *b_center, const lct_overflow *b_overflow,
                 const float *alpha, void *output, uint8_t *auxiliary,
                 int64_t size, int64_t logical_numel, lct_geometry geometry,
                 int32_t rare_length, int32_t output_policy,
                 hipStream_t stream);

/* ---- the reference's three-launch form of the fused dual, for callers that
 * sequence it themselves.  lct_dual_maps_init replaces dispatch.py:215-225
 * (dual_maps_init): both operands' per-stream maps int32[n_streams] get
 * start = steps and offset 0. */
int32_t lct_dual_maps_init(int32_t *a_stream_starts, int32_t *a_stream_offsets,
                           int32_t *b_stream_starts, int32_t *b_stream_offsets,
                           int64_t n_streams, int32_t steps, hipStream_t stream);

/* ---- replaces dispatch.py:228-252 (dual_tables_and_maps): shifts both base
 * decode tables (int32[1024]) by their centers into a/b_shifted_decode and
 * writes, for every overflowing stream of either operand, its start step and
 * tail byte offset (from the tail base: descriptor[0] + 2*count when
 * buffered, overflow->base when private) into that operand's maps.  An
 * operand with overflow = NULL, or a buffered one whose reservation failed,
 * writes no map entries. */
int32_t lct_dual_tables_and_maps(const int32_t *a_base_decode, const int32_t *a_center,
                                 int32_t *a_shifted_decode, const int32_t *b_base_decode,
                                 const int32_t *b_center, int32_t *b_shifted_decode,
                                 const lct_overflow *a_overflow, const lct_overflow *b_overflow,
                                 int32_t *a_stream_starts, int32_t *a_stream_offsets,
                                 int32_t *b_stream_starts, int32_t *b_stream_offsets,
                                 int64_t n_blocks, int32_t steps, hipStream_t stream);

/* ---- replaces dispatch.py:255-286 (dual_mapped): lct_dual with each
 * operand's overlay read from its per-stream maps instead of its compact
 * list (the overflow struct then supplies only the tail bytes). */
int32_t lct_dual_mapped(const int32_t *a_encoded, const uint8_t *a_side,
                        const int32_t *a_shifted_decode, const int32_t *a_center,
                        const int32_t *a_stream_starts, const int32_t *a_stream_offsets,
                        const lct_overflow *a_overflow, const int32_t *b_encoded,
                        const uint8_t *b_side, const int32_t *b_shifted_decode,
                        const int32_t *b_center, const int32_t *b_stream_starts,
                        const int32_t *b_stream_offsets, const lct_overflow *b_overflow,
                        const float *alpha, void *output, uint8_t *auxiliary, int64_t size,
                        int64_t logical_numel, lct_geometry geometry, int32_t rare_length,
                        int32_t output_policy, hipStream_t stream);

/* ---- single-pass compressed-output pointwise, step 1 of 2: replaces the
 * center estimate that dispatch.py:33-48 (estimate_and_shift_encoding_table)
 * makes over the exponent bytes written by dispatch.py:168-187
 * (pointwise_dense, COMPRESSED_OUTPUT), as LCT/codec/pointwise.py:262-278
 * sequences them.  Computes op(A, other) only at the center's sample
 * positions (sample_size = min(logical_numel, 4096), a power of two or
 * logical_numel) and writes each group of 64 samples' exponent sum and count
 * to partials[2*g], partials[2*g+1] (int32[2*ceil(sample_size/64)]).  A is
 * given as for lct_pointwise_dense; op/alpha/beta/flags as there.
 * a_samples: NULL, or A's BF16 values at the sample positions (uint16[
 * sample_size], as lct_sample_center or this function records them); with it
 * A's streams are not read.  result_samples: NULL, or uint16[sample_size] that
 * receives the result's values at the sample positions. */
int32_t lct_pointwise_sample(const int32_t *encoded, const uint8_t *side,
                             const int32_t *shifted_decode, const int32_t *center,
                             const lct_overflow *overflow, const void *a_samples,
                             const void *other, const float *alpha, const float *beta,
                             int64_t size, int64_t logical_numel, lct_geometry geometry,
                             int32_t rare_length, int32_t op, int32_t alpha_is_one,
                             int32_t beta_is_one, int64_t sample_size,
                             int32_t *partials, void *result_samples, hipStream_t stream);

/* ---- single-pass compressed-output pointwise, step 2 of 2: replaces
 * dispatch.py:168-187 (pointwise_dense, COMPRESSED_OUTPUT) followed by the
 * table shift of dispatch.py:16-30 and dispatch.py:294-316 (encode_kernel,
 * precomputed) in one pass.  Reduces `partials` (from lct_pointwise_sample,
 * same sample_size) to the result's center, shifts the result distribution's
 * base_encode/base_decode by it, decodes A, applies op with `other` and
 * encodes the result.  Writes center_out[1], shifted_decode_out[1024] (as
 * lct_estimate_and_shift_tables), and side_out[size], encoded_out,
 * extra_starts and summaries[0..2nb) exactly as lct_encode does for the
 * result; for every overflowing stream, the result's exponent bytes of steps
 * extra_start..S-1 go to exponents (uint8[logical_numel], logical order; no
 * other byte of it is written), from where lct_compact_extra
 * (precomputed = 1) reads the tails.  The result geometry is A's.  encoded,
 * side and side_out must be 16-byte aligned. */
int32_t lct_pointwise_encode(const int32_t *encoded, const uint8_t *side,
                             const int32_t *shifted_decode, const int32_t *center,
                             const lct_overflow *overflow, const void *other,
                             const float *alpha, const float *beta,
                             const int32_t *partials, int64_t sample_size,
                             const int32_t *base_encode, const int32_t *base_decode,
                             int32_t *center_out, int32_t *shifted_decode_out,
                             uint8_t *side_out, int32_t *encoded_out,
                             uint8_t *extra_starts, int32_t *summaries,
                             uint8_t *exponents, int64_t size, int64_t logical_numel,
                             lct_geometry geometry, int32_t rare_length, int32_t op,
                             int32_t alpha_is_one, int32_t beta_is_one,
                             hipStream_t stream);

/* ---- lct_pointwise_encode with the overflow bookkeeping of
 * LCT/codec/encode.py:77-170 (dispatch.py:70-85, prefix + allocate) in the
 * same launch: outputs as lct_pointwise_encode followed by
 * lct_prefix_allocate (counts, blocks, and the overflow-block list
 * summaries[4nb .. 5nb]; summaries[0 .. 4nb) are not written) or, with a
 * buffer, by lct_allocate_compact's frees and reservation (descriptor); then
 * lct_compact_extra (summaries NULL, precomputed = 1, source = exponents)
 * writes the entries and tails.  A bounded wait that gives up marks the
 * tensor incomplete as lct_encode_fused does (counts[3] = 1; status 7).
 * summaries: int32[5*nb + 1]; encoded_out 16-byte aligned. */
int32_t lct_pointwise_encode_fused(const int32_t *encoded, const uint8_t *side,
                                   const int32_t *shifted_decode, const int32_t *center,
                                   const lct_overflow *overflow, const void *other,
                                   const float *alpha, const float *beta,
                                   const int32_t *partials, int64_t sample_size,
                                   const int32_t *base_encode, const int32_t *base_decode,
                                   int32_t *center_out, int32_t *shifted_decode_out,
                                   uint8_t *side_out, int32_t *encoded_out,
                                   uint8_t *extra_starts, int32_t *summaries,
                                   uint8_t *exponents, int64_t size, int64_t logical_numel,
                                   lct_geometry geometry, int32_t rare_length, int32_t op,
                                   int32_t alpha_is_one, int32_t beta_is_one,
                                   const lct_bookkeeping *bookkeeping, hipStream_t stream);

/* ---- several fused updates of one operation with compressed output into one
 * TensorBuffer, in three launches: the samplers of up to LCT_MAX_UPDATE_BATCH
 * tensors (lct_pointwise_sample), their encoders with the in-launch
 * bookkeeping (lct_pointwise_encode_fused, buffered) and their compactions
 * (lct_compact_extra, buffered, precomputed = 1, source = exponents).  No
 * counterpart in the reference, which updates one tensor per call
 * (LCT/LCTensor.py:91-99 -> codec/pointwise.py:262-278): an update of a few
 * codec blocks (a layer's weight) is bound by one block's latency per launch.
 * Each job's outputs are those of its own sequence, except where in the
 * arena its overflow region lies (the jobs reserve in the order their
 * bookkeeping takes the arena lock); `frees` are applied before any job's
 * reservation.  op/alpha/beta/flags as lct_pointwise_sample, shared by the
 * jobs.  Working arrays, partitioned in job order: partials int32[sum 2 *
 * ceil(sample_size / 64)], extra_starts uint8[sum nb*256], summaries
 * int32[sum (5*nb + 1)], control uint64[1 + sum (64 + nb)] (the array of
 * lct_encode_fused, with its zeroing and epoch rules).  All jobs share
 * geometry.steps.  A bounded wait that gives up marks its tensor incomplete
 * (status 7). */
#define LCT_MAX_UPDATE_BATCH 8
typedef struct {
    const int32_t *encoded;        /* A, 16-byte aligned */
    const uint8_t *side;           /* 16-byte aligned */
    const int32_t *shifted_decode;
    const int32_t *center;
    int32_t has_overflow;
    lct_overflow overflow;
    const void *a_samples;         /* A's BF16 values at the sample positions, or NULL */
    const void *other;             /* B: bf16[logical_numel] */
    const int32_t *base_encode;    /* the result distribution's tables */
    const int32_t *base_decode;
    int32_t *center_out;           /* int32[1] */
    int32_t *shifted_decode_out;   /* int32[1024] */
    uint8_t *side_out;             /* uint8[size], 16-byte aligned */
    int32_t *encoded_out;          /* int32[nb*256*W + 4] */
    void *result_samples;          /* uint16[sample_size], or NULL */
    uint8_t *exponents;            /* uint8[logical_numel] */
    int32_t *counts;               /* int32[4] */
    int32_t *blocks;               /* int32[3*nb] */
    int32_t *descriptor;           /* int32[4] */
    int64_t size;
    int64_t logical_numel;
    int64_t sample_size;
    lct_geometry geometry;
    int32_t rare_length;
} lct_update_job;
int32_t lct_pointwise_update_batch(const lct_update_job *jobs, int32_t n_jobs, int32_t op,
                                   int32_t alpha_is_one, int32_t beta_is_one,
                                   const float *alpha, const float *beta, int32_t *partials,
                                   int64_t partial_words, uint8_t *extra_starts,
                                   int64_t extra_bytes, int32_t *summaries,
                                   int64_t summary_words, uint64_t *control,
                                   int64_t control_words, uint32_t epoch,
                                   int32_t *buffer_meta, int32_t max_free_regions,
                                   uint8_t *arena, const lct_pending_frees *frees,
                                   hipStream_t stream);

/* ---- single-pass compressed-output alpha*A + B over two compressed
 * operands, step 1 of 2: replaces the center estimate that dispatch.py:33-48
 * makes over the exponent bytes written by dispatch.py:215-286 (dual_mapped,
 * COMPRESSED_OUTPUT), as LCT/codec/pointwise.py:159-210 sequences them for
 * LCT/LCTensor.py:91-99 (add_comp_).  As lct_pointwise_sample, with the
 * result fma(a, alpha[0], b) rounded to BF16: A and B as for lct_dual;
 * a_samples / b_samples: NULL, or that operand's values at the sample
 * positions (then its streams are not read). */
int32_t lct_dual_sample(const int32_t *a_encoded, const uint8_t *a_side,
                        const int32_t *a_shifted_decode, const int32_t *a_center,
                        const lct_overflow *a_overflow, const void *a_samples,
                        const int32_t *b_encoded, const uint8_t *b_side,
                        const int32_t *b_shifted_decode, const int32_t *b_center,
                        const lct_overflow *b_overflow, const void *b_samples,
                        const float *alpha, int64_t size, int64_t logical_numel,
                        lct_geometry geometry, int32_t rare_length, int64_t sample_size,
                        int32_t *partials, void *result_samples, hipStream_t stream);

/* ---- single-pass compressed-output alpha*A + B over two compressed
 * operands, step 2 of 2: replaces dispatch.py:215-286 (dual_mapped,
 * COMPRESSED_OUTPUT) followed by the table shift of dispatch.py:16-30 and
 * dispatch.py:294-316 (encode_kernel, precomputed) in one pass.  Outputs as
 * lct_pointwise_encode; partials from lct_dual_sample with the same
 * sample_size.  a_encoded, b_encoded, a_side, b_side and side_out must be
 * 16-byte aligned. */
int32_t lct_dual_encode(const int32_t *a_encoded, const uint8_t *a_side,
                        const int32_t *a_shifted_decode, const int32_t *a_center,
                        const lct_overflow *a_overflow, const int32_t *b_encoded,
                        const uint8_t *b_side, const int32_t *b_shifted_decode,
                        const int32_t *b_center, const lct_overflow *b_overflow,
                        const float *alpha, const int32_t *partials, int64_t sample_size,
                        const int32_t *base_encode, const int32_t *base_decode,
                        int32_t *center_out, int32_t *shifted_decode_out, uint8_t *side_out,
                        int32_t *encoded_out, uint8_t *extra_starts, int32_t *summaries,
                        uint8_t *exponents, int64_t size, int64_t logical_numel,
                        lct_geometry geometry, int32_t rare_length, hipStream_t stream);

/* ---- lct_dual_encode with the overflow bookkeeping in the same launch, as
 * lct_pointwise_encode_fused adds it to lct_pointwise_encode. */
int32_t lct_dual_encode_fused(const int32_t *a_encoded, const uint8_t *a_side,
                              const int32_t *a_shifted_decode, const int32_t *a_center,
                              const lct_overflow *a_overflow, const int32_t *b_encoded,
                              const uint8_t *b_side, const int32_t *b_shifted_decode,
                              const int32_t *b_center, const lct_overflow *b_overflow,
                              const float *alpha, const int32_t *partials, int64_t sample_size,
                              const int32_t *base_encode, const int32_t *base_decode,
                              int32_t *center_out, int32_t *shifted_decode_out,
                              uint8_t *side_out, int32_t *encoded_out, uint8_t *extra_starts,
                              int32_t *summaries, uint8_t *exponents, int64_t size,
                              int64_t logical_numel, lct_geometry geometry, int32_t rare_length,
                              const lct_bookkeeping *bookkeeping, hipStream_t stream);

/* ---- TensorBuffer allocator kernels: replace LCT/tensor_buffer.py:130-136
 * (_reset_kernel launch), :93-120 (_allocate_kernel launches) and
 * LCT/kernels/tensor_buffer_ops.py:5-15 (_free_storage_kernel launch).
 * meta: the int32 metadata block at the start of the buffer's storage,
 * free_starts[R] | free_sizes[R] | count | lock | generation | failures (the
 * failure word sits in the padding the reference leaves after generation).
 * requested/item_count: device int32[1]; item_count may be NULL when
 * item_bytes == 0.  descriptor: int32[4] {offset, size, status, generation};
 * status 0 ok, 1 no fit, 2 empty request, 5 freed, 6 lock not acquired,
 * 7 reserved but the compaction into it did not complete (freeable).
 * free writes status_out[0]: 0 ok, 3 free list full, 4 invalid descriptor,
 * 6 lock not acquired.  reset also clears the failure word. */
#define LCT_STATUS_INCOMPLETE 7
/* Bits of the failure word: a codec reservation (lct_prefix_allocate buffered,
 * lct_allocate_compact) of a non-empty request found no fit, could not take
 * the lock, or its compaction did not complete.  Sticky until reset. */
#define LCT_FAIL_NO_FIT 1
#define LCT_FAIL_LOCK 2
#define LCT_FAIL_INCOMPLETE 4
int32_t lct_buffer_reset(int32_t *meta, int32_t max_free_regions,
                         int32_t capacity_bytes, hipStream_t stream);
int32_t lct_buffer_allocate(int32_t *meta, int32_t max_free_regions,
                            const int32_t *requested, const int32_t *item_count,
                            int32_t item_bytes, int32_t *descriptor,
                            hipStream_t stream);
int32_t lct_buffer_free(int32_t *meta, int32_t max_free_regions,
                        int32_t *descriptor, int32_t *status_out,
                        hipStream_t stream);

/* ---- several frees of one TensorBuffer in one launch.  No counterpart in
 * the reference, which launches _free_storage_kernel once per descriptor
 * (LCT/kernels/tensor_buffer_ops.py:5-15); it is for callers that free many
 * compressed tensors between two reservations (a training step's saved
 * activations and replaced optimizer state).  descriptors: `count` (1 to
 * LCT_MAX_FREE_BATCH) device descriptor pointers.  One workgroup takes the
 * arena lock once and frees them in order, each as lct_buffer_free would (a
 * descriptor listed twice is freed once; the second gets status 4); the free
 * list and descriptors end as after lct_buffer_free on each in turn.
 * status_out: device int32[count] ({0, 3, 4, 6} as lct_buffer_free), or
 * NULL. */
#define LCT_MAX_FREE_BATCH 32
int32_t lct_buffer_free_batch(int32_t *meta, int32_t max_free_regions,
                              int32_t *const *descriptors, int32_t count,
                              int32_t *status_out, hipStream_t stream);

/* ---- buffered compress that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * It enqueues what compress() with a shared TensorBuffer enqueues --
 * lct_sample_center, lct_encode_sampled and lct_allocate_compact -- and its
 * outputs are theirs, byte for byte: side, encoded, center_out,
 * shifted_decode_out, sample_values (NULL: not recorded), blocks, counts,
 * descriptor, the TensorBuffer's free list and the arena region, with `frees`
 * (NULL or pending frees) applied first.  The working arrays (partial sums,
 * block summaries, extra starts, ready word) live in a file-scope device array
 * of 2.2 MiB that each GPU holds until the process ends; the call allocates
 * nothing.  Tensors of more than 8192 codec blocks are rejected with
 * LCT_E_SCRATCH before anything is launched.  Every call on a GPU uses that
 * GPU's one array: calls that overlap on one GPU (different streams without
 * ordering) race; calls ordered on one stream do not.  The current device must
 * be the stream's. */
int32_t lct_compress_buffered_noalloc(const void *source, int64_t logical_numel, int64_t size,
                                      lct_geometry geometry, const int32_t *base_encode,
                                      const int32_t *base_decode, uint8_t *side,
                                      int32_t *encoded, int32_t *center_out,
                                      int32_t *shifted_decode_out, uint16_t *sample_values,
                                      int32_t *blocks, int32_t *counts, int32_t *descriptor,
                                      int32_t *buffer_meta, int32_t max_free_regions,
                                      uint8_t *arena, const lct_pending_frees *frees,
                                      hipStream_t stream);

/* ---- bounds of the device-side waits, in polls: the arena lock (every
 * allocator entry point, default 2^20) and lct_allocate_compact's wait for its
 * reservation (default 2^22); 0 restores a default.  Applies to launches made
 * after the call.  No counterpart in the reference (its lock wait is
 * unbounded, LCT/kernels/tensor_buffer.py:7-15): tests lower the bounds to
 * drive the give-up paths from the host without long waits. */
int32_t lct_set_wait_limits(int32_t lock_polls, int32_t ready_polls);

/* ---- which decoder kernel lct_decode launches: LCT_DECODER_AUTO (the
 * default: the wide-tile kernel, or the compact one when only it holds the
 * whole grid at once), LCT_DECODER_WIDE or LCT_DECODER_COMPACT.  Both write
 * the same output.  Applies to launches made after the call.  No counterpart
 * in the reference: tests pin each kernel on the same inputs. */
#define LCT_DECODER_AUTO 0
#define LCT_DECODER_WIDE 1
#define LCT_DECODER_COMPACT 2
int32_t lct_set_decoder(int32_t mode);

/* ---- attainable HBM bandwidth with the codec kernels' access shape (16-byte
 * non-temporal buffer accesses, `workgroups` workgroups of 256 threads each
 * walking 16 KiB passes).  kind 0: copy src -> dst (src_bytes = dst_bytes);
 * 1: read src (dst: at least 4 KiB, scratch); 2: write dst (src unused, may
 * be NULL); 3: read src and write dst together, each pass covering the same
 * fraction of both (0 < src_bytes <= dst_bytes).  Sizes are multiples of 16,
 * at most 2^31; dst at least 4 KiB; pointers 16-byte aligned.  No counterpart
 * in the reference: bench.py reports these ceilings beside the roofline
 * fractions. */
int32_t lct_bandwidth_probe(int32_t kind, const void *src, int64_t src_bytes, void *dst,
                            int64_t dst_bytes, int32_t workgroups, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
