// Job tables of the batched buffered compress (lct_compress_batch): the fused
// compress of several tensors in one launch (compress.hip), then the
// compaction of their overflow entries in one more (compaction.hip), which
// the batched fused update (lct_pointwise_update_batch) uses too.  The
// tables travel in the kernel arguments; workgroup w works for the last job
// whose first workgroup is at most w.
#pragma once

#include "lct_device.h"

namespace lct {

// One tensor of a batched compress: lct_encode_fused's per-tensor arguments,
// with its slices of the shared working arrays already resolved.
struct CompressBatchJob {
    const void *source;
    uint8_t *side;
    int32_t *encoded;
    const int32_t *base_encode;
    const int32_t *base_decode;
    int32_t *center_out;
    int32_t *shifted_decode_out;
    uint16_t *sample_values;
    uint8_t *extra_starts;
    int32_t *summaries;
    int32_t *blocks;
    int32_t *counts;
    int32_t *descriptor;
    uint64_t *control;
    int64_t sample_size;
    int64_t logical_numel;
    int32_t n_groups;
    int32_t n_blocks;
    int32_t fixed_words;
};

struct CompressBatch {
    int32_t n_jobs;
    int32_t first_group[LCT_MAX_COMPRESS_BATCH + 1];
    CompressBatchJob jobs[LCT_MAX_COMPRESS_BATCH];
    int32_t *buffer_meta;
    int32_t max_free_regions;
    lct_pending_frees frees;   // job 0 applies them
    uint64_t *gate;            // job 0's "frees applied" word, nullptr without frees
    uint32_t epoch;
    int32_t steps;   // every job's S (the side-store policy is chosen by it)
    int32_t lock_spins;
    int32_t polls;
};

// One tensor's compaction into its reservation (compact_blocks_kernel with
// buffered = 1).
struct CompactBatchJob {
    const void *source;
    const int32_t *blocks;
    const int32_t *counts;
    const int32_t *descriptor;
    const uint8_t *extra_starts;
    int64_t n_blocks;
    int64_t logical_numel;
};

struct CompactBatch {
    int32_t n_jobs;
    int32_t first_block[LCT_MAX_COMPRESS_BATCH + 1];
    CompactBatchJob jobs[LCT_MAX_COMPRESS_BATCH];
    uint8_t *arena;
    int32_t steps;
    int32_t precomputed;   // sources are exponent bytes (fused updates), else BF16
};

// Launchers (the kernels live in their files' anonymous namespaces).
hipError_t launch_compress_batch(const CompressBatch &batch, uint32_t grid, size_t lds,
                                 hipStream_t stream);
hipError_t launch_compact_batch(const CompactBatch &batch, uint32_t grid, hipStream_t stream);

}  // namespace lct
