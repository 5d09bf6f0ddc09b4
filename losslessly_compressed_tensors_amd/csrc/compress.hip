// Fused compress: center sampling, field split + encoder, and the overflow
// bookkeeping (block scans, overflow-block list, block metadata and, for a
// shared TensorBuffer, the arena reservation after the buffer's deferred
// frees) in one launch.  Only the compaction of the overflowing streams
// (lct_compact_extra) stays a launch of its own: it reads the extra starts
// that other workgroups wrote, which a kernel boundary makes visible.
//
// Replaces, for one tensor, the sequence LCT/kernels/dispatch.py:33-48
// (center + tables), :294-316 (encoder) and :70-85 (prefix + allocate) that
// LCT/codec/encode.py:22-186 runs; the results are those of
// lct_sample_center -> lct_encode_sampled -> lct_prefix_allocate (or, with a
// buffer, the reservation of lct_allocate_compact), value for value.
//
// One workgroup per codec block (and, for tensors of fewer blocks than
// center-sample groups, one per group), in dispatch order; no workgroup is
// only a helper, so a grid that fills the device runs in whole rounds:
//  * workgroup g < G (G = ceil(samples / 64) <= 64): wave 0 first samples
//    center group g (64 positions) and publishes its partial sum; it waits
//    for nothing before that;
//  * every workgroup b < nb then polls the G partial sums (its first input
//    chunk in flight meanwhile), encodes block b as lct_encode_sampled does
//    and publishes its overflow count and tail bytes;
//  * workgroup 0, after its own block, does the bookkeeping: with a buffer it
//    takes the arena lock, reads the free list into LDS and applies the
//    deferred frees, then polls every block's summary, scans them into the
//    metadata and the overflow-block list and reserves the tensor's overflow
//    region (request = tail bytes + 2 x entries).  Only the last summary's
//    arrival, the scan's last pass and the reservation follow the last block.
// Every wait is for words that workgroups dispatched no later than the waiter
// publish before they wait for anything, and every poll is bounded; a summary
// or partial sum that does not arrive within the bound marks the tensor
// incomplete (counts[3] = 1; with a buffer, status 7 and the buffer's failure
// word) instead of hanging.  (Helper workgroups of their own -- a bookkeeping
// workgroup and 64 samplers in front of the encoders -- pushed the last of
// 1024 blocks of 256 steps, four per CU, into a second round: 55 us against
// the 43 us in which the other blocks had finished.)
//
// Cross-workgroup values travel in a control array of 64-bit words tagged with
// the call's epoch (lct_device.h), one array per stream, never cleared: a word
// is current exactly when its tag is this call's epoch.
#include "batch.h"
#include "encode_core.h"
#include "reserve.h"

namespace lct {
namespace {

// Workgroup `group` of one tensor's fused compress (the launch layout above):
// the single launch runs it for blockIdx.x, the batched launch for its job's
// share of the grid.  gate: GatedReserve's word (batched launches only).
template <int kSidePolicy, bool kPrecomputed>
__device__ __forceinline__ void compress_group(
    const void *__restrict__ source, uint8_t *__restrict__ side, int32_t *__restrict__ encoded,
    const int32_t *__restrict__ base_encode, const int32_t *__restrict__ base_decode,
    int32_t *__restrict__ center_out, int32_t *__restrict__ shifted_decode_out,
    uint16_t *__restrict__ sample_values, int64_t sample_size, int32_t n_groups,
    uint8_t *__restrict__ extra_starts, int32_t *__restrict__ summaries,
    int32_t *__restrict__ blocks, int32_t *__restrict__ counts, uint64_t *__restrict__ control,
    uint32_t epoch, int32_t *__restrict__ descriptor, int32_t *__restrict__ buffer_meta,
    int32_t max_free_regions, const lct_pending_frees &frees, uint64_t *host_totals,
    int32_t n_blocks, int64_t logical_numel, int S, int W, int32_t lock_spins, int32_t polls,
    int64_t group, uint64_t *gate, bool post_gate, uint32_t *stage) {
    __shared__ uint2 table[256];
    __shared__ __attribute__((aligned(16))) uint8_t slices[kWavesPerBlock * kSliceBytes];
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t shared[2];

    if (group < n_groups && threadIdx.x < kWave) {
        // Samples group * 64 + lane (tables.py:15-49): the kept exponents' sum
        // and count; a BF16 source's sampled bits also go to sample_values.
        const int t = threadIdx.x;
        const int64_t i = group * kSampleGroup + t;
        const bool active = i < sample_size;
        const int shift = __builtin_ctzll(static_cast<uint64_t>(sample_size));
        int32_t exp = -127;
        if (active) {
            const int64_t pos = sample_position(i, logical_numel, sample_size, shift);
            if (kPrecomputed) {
                exp = static_cast<int32_t>(static_cast<const uint8_t *>(source)[pos]) - 127;
            } else {
                const uint32_t bits = static_cast<const uint16_t *>(source)[pos];
                exp = static_cast<int32_t>((bits >> 7) & 0xFFu) - 127;
                if (sample_values != nullptr) sample_values[i] = static_cast<uint16_t>(bits);
            }
        }
        const bool keep = active && exp >= -120;
        const int32_t sum = wave_sum(keep ? exp : 0);      // |sum| <= 64 * 128
        const int32_t kept = wave_sum(keep ? 1 : 0);
        if (t == 0) {
            const uint32_t value = (static_cast<uint32_t>(static_cast<uint16_t>(sum)) << 16)
                                   | static_cast<uint32_t>(kept);
            control_store(control + group, tagged_word(epoch, value));
        }
    }
    if (group >= n_blocks) return;   // a sample group past the last block

    const int64_t block = group;
    const TableSource tables{nullptr, nullptr, n_groups, base_encode, base_decode, center_out,
                             shifted_decode_out, control, epoch, polls};
    const EncodeLds lds{stage, table, slices, scratch, shared};
    const BlockSummary s = encode_codec_block<kSidePolicy>(source, side, encoded, tables,
                                                           extra_starts, block, n_blocks,
                                                           logical_numel, S, W, kPrecomputed,
                                                           true, lds);
    if (threadIdx.x == 0) {
        // count <= 256 and bytes <= 256 * 256 fit 9 and 17 bits.
        const uint32_t value = s.failed ? (kFailedBlock << 17)
                                        : (static_cast<uint32_t>(s.count) << 17)
                                              | static_cast<uint32_t>(s.bytes);
        control_store(control + kControlPartials + block, tagged_word(epoch, value));
    }
    if (block != 0) return;

    // The bookkeeping.  The stage's last readers passed the summary's
    // barriers, so it can hold the free list.
    PolledSummaries polled{control, epoch, n_blocks, polls, false};
    if (buffer_meta != nullptr) {
        GatedReserve reserve{
            LdsReserve<false>{AllocatorMeta(buffer_meta, max_free_regions, lock_spins),
                              descriptor, frees, reinterpret_cast<int32_t *>(stage), {}, -1,
                              kStatusOk},
            gate, post_gate, epoch, polls, false};
        scan_allocate<false>(polled, summaries, counts, blocks, n_blocks, reserve);
    } else {
        NoReserve reserve;
        const ScanTotals totals =
            scan_allocate<false>(polled, summaries, counts, blocks, n_blocks, reserve);
        if (host_totals != nullptr && threadIdx.x == 0) {
            // The totals a private compress sizes its overflow arrays by, for
            // a host waiting on this word instead of on the launch's end.
            host_word_store(host_totals,
                            tagged_word(epoch, static_cast<uint32_t>(totals.entries)
                                                   | (totals.incomplete ? 0x80000000u : 0u)));
            host_word_store(host_totals + 1,
                            tagged_word(epoch, static_cast<uint32_t>(totals.bytes)));
        }
    }
}

// One kernel per input kind (BF16 bits or precomputed exponent bytes), so
// each carries one encoder variant and its registers.
template <int kSidePolicy, bool kPrecomputed>
__global__ __launch_bounds__(kLanes) void compress_kernel(
    const void *__restrict__ source, uint8_t *__restrict__ side, int32_t *__restrict__ encoded,
    const int32_t *__restrict__ base_encode, const int32_t *__restrict__ base_decode,
    int32_t *__restrict__ center_out, int32_t *__restrict__ shifted_decode_out,
    uint16_t *__restrict__ sample_values, int64_t sample_size, int32_t n_groups,
    uint8_t *__restrict__ extra_starts, int32_t *__restrict__ summaries,
    int32_t *__restrict__ blocks, int32_t *__restrict__ counts, uint64_t *__restrict__ control,
    uint32_t epoch, int32_t *__restrict__ descriptor, int32_t *__restrict__ buffer_meta,
    int32_t max_free_regions, lct_pending_frees frees, uint64_t *host_totals, int32_t n_blocks,
    int64_t logical_numel, int S, int W, int32_t lock_spins, int32_t polls) {
    extern __shared__ uint32_t stage[];   // (W + 2) rows x 256 lanes, or the free list
    compress_group<kSidePolicy, kPrecomputed>(
        source, side, encoded, base_encode, base_decode, center_out, shifted_decode_out,
        sample_values, sample_size, n_groups, extra_starts, summaries, blocks, counts, control,
        epoch, descriptor, buffer_meta, max_free_regions, frees, host_totals, n_blocks,
        logical_numel, S, W, lock_spins, polls, blockIdx.x, nullptr, false, stage);
}

// Several BF16 tensors into one TensorBuffer: job j takes workgroups
// [first_group[j], first_group[j + 1]) and runs the single launch's layout
// over them with its own control words.  Every wait stays inside one job
// (plus the gate on job 0, dispatched first), so each job's waits end as in
// its own launch.
template <int kSidePolicy>
__global__ __launch_bounds__(kLanes) void compress_batch_kernel(CompressBatch batch) {
    extern __shared__ uint32_t stage[];
    const int32_t w = static_cast<int32_t>(blockIdx.x);
    int j = 0;
    for (int k = 1; k < batch.n_jobs; ++k)
        if (w >= batch.first_group[k]) j = k;
    const CompressBatchJob &job = batch.jobs[j];
    lct_pending_frees frees = batch.frees;
    if (j != 0) frees.count = 0;
    compress_group<kSidePolicy, false>(
        job.source, job.side, job.encoded, job.base_encode, job.base_decode, job.center_out,
        job.shifted_decode_out, job.sample_values, job.sample_size, job.n_groups,
        job.extra_starts, job.summaries, job.blocks, job.counts, job.control, batch.epoch,
        job.descriptor, batch.buffer_meta, batch.max_free_regions, frees, nullptr, job.n_blocks,
        job.logical_numel, batch.steps, job.fixed_words, batch.lock_spins, batch.polls,
        w - batch.first_group[j], batch.gate, j == 0, stage);
}

}  // namespace

hipError_t launch_compress_batch(const CompressBatch &batch, uint32_t grid, size_t lds,
                                 hipStream_t stream) {
    const auto kernel = batch.steps == 128 ? compress_batch_kernel<kStreaming>
                                     : compress_batch_kernel<0>;
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(kernel), lds)) return e;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kLanes), lds, stream, batch);
    return hipGetLastError();
}

}  // namespace lct

using namespace lct;

extern "C" int32_t lct_encode_fused(
    const void *source, uint8_t *side, int32_t *encoded, int64_t sample_size,
    const int32_t *base_encode, const int32_t *base_decode, int32_t *center_out,
    int32_t *shifted_decode_out, uint16_t *sample_values, uint8_t *extra_starts,
    int32_t *summaries, int32_t *blocks, int32_t *counts, uint64_t *control,
    int64_t control_words, uint32_t epoch, int32_t *descriptor, int32_t *buffer_meta,
    int32_t max_free_regions, const lct_pending_frees *frees, uint64_t *host_totals,
    int64_t size, int64_t logical_numel, lct_geometry g, int32_t precomputed,
    hipStream_t stream) {
    if (!source || !side || !encoded || !base_encode || !base_decode || !center_out
        || !shifted_decode_out || !extra_starts || !summaries || !blocks || !counts || !control)
        return LCT_E_NULL;
    const bool buffered = buffer_meta != nullptr;
    if (buffered && !descriptor) return LCT_E_NULL;
    if (host_totals != nullptr && (buffered || (reinterpret_cast<uintptr_t>(host_totals) & 7) != 0))
        return LCT_E_ARG;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (logical_numel <= 0 || size <= 0 || size % g.block_symbols != 0
        || logical_numel > size || logical_numel <= size - g.block_symbols)
        return LCT_E_SIZE;
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > kMaxBlocks) return LCT_E_SIZE;
    if (sample_size <= 0 || sample_size > kMaxSamples || sample_size > logical_numel)
        return LCT_E_SIZE;
    if (sample_size != logical_numel && (sample_size & (sample_size - 1)) != 0)
        return LCT_E_ARG;
    if (control_words < kControlPartials + n_blocks) return LCT_E_SIZE;
    // Epoch 0 would match a control array's initial zeros.
    if (epoch == 0) return LCT_E_ARG;
    if (((reinterpret_cast<uintptr_t>(encoded) | reinterpret_cast<uintptr_t>(source)
          | reinterpret_cast<uintptr_t>(side)) & 15) != 0
        || (reinterpret_cast<uintptr_t>(control) & 7) != 0)
        return LCT_E_ARG;
    lct_pending_frees pending{};
    if (buffered) {
        if (max_free_regions <= 0 || max_free_regions > 4096
            || (max_free_regions & (max_free_regions - 1)) != 0)
            return LCT_E_ARG;
        if (frees != nullptr) {
            if (frees->count < 0 || frees->count > LCT_MAX_PENDING_FREES) return LCT_E_ARG;
            for (int i = 0; i < frees->count; ++i)
                if (frees->descriptor[i] == nullptr) return LCT_E_NULL;
            pending = *frees;
        }
    }
    const int32_t n_groups = sample_groups(sample_size);
    // The encoders' stage, or workgroup 0's LDS copy of the free list.
    size_t lds = static_cast<size_t>(g.fixed_words + 2) * kLanes * 4;
    if (buffered && static_cast<size_t>(max_free_regions) * 8 > lds)
        lds = static_cast<size_t>(max_free_regions) * 8;
    // Side bytes: non-temporal stores for 128-step blocks, the default policy
    // for 256-step blocks (the encoder's side-byte comment has the figures).
    const auto kernel = g.steps == 128
                            ? (precomputed ? compress_kernel<kStreaming, true>
                                           : compress_kernel<kStreaming, false>)
                            : (precomputed ? compress_kernel<0, true> : compress_kernel<0, false>);
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(kernel), lds))
        return static_cast<int32_t>(e);
    const uint32_t grid = static_cast<uint32_t>(n_blocks > n_groups ? n_blocks : n_groups);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kLanes), lds, stream, source, side,
                       encoded, base_encode, base_decode, center_out, shifted_decode_out,
                       precomputed ? nullptr : sample_values, sample_size, n_groups,
                       extra_starts, summaries, blocks, counts, control, epoch,
                       buffered ? descriptor : nullptr, buffer_meta, max_free_regions, pending,
                       host_totals, static_cast<int32_t>(n_blocks), logical_numel, g.steps,
                       g.fixed_words,
                       lock_spins(), ready_polls());
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_compress_batch(const lct_compress_job *jobs, int32_t n_jobs,
                                      uint8_t *extra_starts, int64_t extra_bytes,
                                      int32_t *summaries, int64_t summary_words,
                                      uint64_t *control, int64_t control_words, uint32_t epoch,
                                      int32_t *buffer_meta, int32_t max_free_regions,
                                      uint8_t *arena, const lct_pending_frees *frees,
                                      hipStream_t stream) {
    if (!jobs || !extra_starts || !summaries || !control || !buffer_meta || !arena)
        return LCT_E_NULL;
    if (n_jobs <= 0 || n_jobs > LCT_MAX_COMPRESS_BATCH) return LCT_E_ARG;
    if (epoch == 0 || (reinterpret_cast<uintptr_t>(control) & 7) != 0) return LCT_E_ARG;
    if (max_free_regions <= 0 || max_free_regions > 4096
        || (max_free_regions & (max_free_regions - 1)) != 0)
        return LCT_E_ARG;
    CompressBatch batch{};
    CompactBatch compact{};
    batch.n_jobs = compact.n_jobs = n_jobs;
    batch.buffer_meta = buffer_meta;
    batch.max_free_regions = max_free_regions;
    if (frees != nullptr) {
        if (frees->count < 0 || frees->count > LCT_MAX_PENDING_FREES) return LCT_E_ARG;
        for (int i = 0; i < frees->count; ++i)
            if (frees->descriptor[i] == nullptr) return LCT_E_NULL;
        batch.frees = *frees;
    }
    batch.epoch = epoch;
    batch.steps = compact.steps = jobs[0].geometry.steps;
    compact.precomputed = 0;
    batch.lock_spins = lock_spins();
    batch.polls = ready_polls();
    // Word 0 of the control array is the frees' gate; job j's words follow
    // those of jobs before it.
    batch.gate = batch.frees.count > 0 ? control : nullptr;
    int64_t groups = 0, blocks_total = 0, extra_used = 0, summary_used = 0, control_used = 1;
    size_t lds = static_cast<size_t>(max_free_regions) * 8;
    for (int j = 0; j < n_jobs; ++j) {
        const lct_compress_job &in = jobs[j];
        const lct_geometry &g = in.geometry;
        if (!in.source || !in.side || !in.encoded || !in.base_encode || !in.base_decode
            || !in.center_out || !in.shifted_decode_out || !in.blocks || !in.counts
            || !in.descriptor)
            return LCT_E_NULL;
        if (!geometry_ok(g)) return LCT_E_GEOMETRY;
        if (g.steps != batch.steps) return LCT_E_ARG;
        if (in.logical_numel <= 0 || in.size <= 0 || in.size % g.block_symbols != 0
            || in.logical_numel > in.size || in.logical_numel <= in.size - g.block_symbols)
            return LCT_E_SIZE;
        const int64_t nb = in.size / g.block_symbols;
        if (nb > kMaxBlocks) return LCT_E_SIZE;
        if (in.sample_size <= 0 || in.sample_size > kMaxSamples
            || in.sample_size > in.logical_numel)
            return LCT_E_SIZE;
        if (in.sample_size != in.logical_numel && (in.sample_size & (in.sample_size - 1)) != 0)
            return LCT_E_ARG;
        if (((reinterpret_cast<uintptr_t>(in.encoded) | reinterpret_cast<uintptr_t>(in.source)
              | reinterpret_cast<uintptr_t>(in.side)) & 15) != 0)
            return LCT_E_ARG;
        const int32_t n_groups = sample_groups(in.sample_size);
        CompressBatchJob &job = batch.jobs[j];
        job.source = in.source;
        job.side = in.side;
        job.encoded = in.encoded;
        job.base_encode = in.base_encode;
        job.base_decode = in.base_decode;
        job.center_out = in.center_out;
        job.shifted_decode_out = in.shifted_decode_out;
        job.sample_values = in.sample_values;
        job.extra_starts = extra_starts + extra_used;
        job.summaries = summaries + summary_used;
        job.blocks = in.blocks;
        job.counts = in.counts;
        job.descriptor = in.descriptor;
        job.control = control + control_used;
        job.sample_size = in.sample_size;
        job.logical_numel = in.logical_numel;
        job.n_groups = n_groups;
        job.n_blocks = static_cast<int32_t>(nb);
        job.fixed_words = g.fixed_words;
        CompactBatchJob &c = compact.jobs[j];
        c.source = in.source;
        c.blocks = in.blocks;
        c.counts = in.counts;
        c.descriptor = in.descriptor;
        c.extra_starts = job.extra_starts;
        c.n_blocks = nb;
        c.logical_numel = in.logical_numel;
        batch.first_group[j] = static_cast<int32_t>(groups);
        compact.first_block[j] = static_cast<int32_t>(blocks_total);
        groups += nb > n_groups ? nb : n_groups;
        blocks_total += nb;
        extra_used += nb * kLanes;
        summary_used += 5 * nb + 1;
        control_used += kControlPartials + nb;
        const size_t stage = static_cast<size_t>(g.fixed_words + 2) * kLanes * 4;
        if (stage > lds) lds = stage;
    }
    if (extra_used > extra_bytes || summary_used > summary_words || control_used > control_words)
        return LCT_E_SIZE;
    batch.first_group[n_jobs] = static_cast<int32_t>(groups);
    compact.first_block[n_jobs] = static_cast<int32_t>(blocks_total);
    compact.arena = arena;
    if (hipError_t e = launch_compress_batch(batch, static_cast<uint32_t>(groups), lds, stream))
        return static_cast<int32_t>(e);
    return static_cast<int32_t>(
        launch_compact_batch(compact, static_cast<uint32_t>(blocks_total), stream));
}
