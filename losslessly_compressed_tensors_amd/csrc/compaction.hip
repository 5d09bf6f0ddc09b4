// Overflow bookkeeping after the encoder: block prefix scans, block metadata
// and arena allocation (one workgroup), then compaction of the overflowing
// streams of the blocks that have any.
//
// Follows LCT/kernels/generic/metadata.py:13-38 and
// LCT/kernels/generic/compaction.py:99-235 (summaries path).  The compact list
// is stored per codec block: the block's overflowing lanes in ascending order
// at entries [first, first+count), their exponent tails int8(e-127) for steps
// start..S-1 concatenated from byte_base, and blocks[3*nb] = {count, first,
// byte_base} so every reader walks the list one block at a time.
#include "batch.h"
#include "overflow_walk.h"
#include "reserve.h"

namespace lct {
namespace {

constexpr int kCompactGrid = 2048;                   // workgroups walking the overflow-block list

__global__ __launch_bounds__(kLanes) void prefix_allocate_kernel(
    int32_t *__restrict__ summaries, int32_t *__restrict__ counts,
    int32_t *__restrict__ descriptor, int32_t *__restrict__ buffer_meta,
    int32_t *__restrict__ blocks, int32_t n_blocks, int32_t buffered,
    int32_t max_free_regions, int32_t lock_spins) {
    __shared__ int32_t flag;
    RegisterReserve reserve{AllocatorMeta(buffer_meta, max_free_regions, lock_spins), descriptor,
                            &flag, buffered != 0, {}};
    SummaryLoads source(summaries, n_blocks);
    scan_allocate<true>(source, summaries, counts, blocks, n_blocks, reserve);
}

// One codec block's overflow entries and tails (compaction.py:137-228), in
// two halves.  rank_block needs nothing from the reservation: it ranks the
// block's overflowing lanes (ascending) and puts each one's tail offset, start
// and lane in LDS.  write_block then stores the entries at `first` and the
// tails at `byte_base`: tail byte i belongs to the overflowing lane whose local
// byte range holds i (binary search over the offsets in LDS), so every byte is
// an independent load and the tail stores are contiguous.
struct BlockEntries {
    int32_t start;   // this lane's first overflow step (255: none)
    int32_t rank;    // this lane's entry index in the block, if it overflows
    int32_t count;   // entries of the block (uniform)
    int32_t bytes;   // tail bytes of the block (uniform)
    int32_t first_tail;   // tail byte threadIdx.x of the block (if < bytes)
};

// The block's source elements (BF16 bits, or exponent bytes when
// precomputed) as a buffer resource over the part inside the tensor: loads
// past the tensor's end return 0, which both kinds map to int8(0 - 127) = -127,
// the tail byte of a padding position.  Buffer accesses cannot alias LDS, so
// the compiler keeps them in flight across the entry arrays' LDS accesses (the
// generic pointers they replace made every load wait for the LDS stores
// before it, one load latency per tail byte).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_source(const void *__restrict__ source,
                                                               int64_t block, int S,
                                                               int64_t logical_numel,
                                                               int precomputed) {
    const int64_t first = block * S * kLanes;
    const int64_t left = logical_numel - first;
    const int64_t valid = left < int64_t{S} * kLanes ? (left > 0 ? left : 0) : int64_t{S} * kLanes;
    const int64_t elem = precomputed ? 1 : 2;
    return make_rsrc(static_cast<const uint8_t *>(source) + first * elem,
                     static_cast<uint32_t>(valid * elem));
}

// int8(e - 127) of the element at `offset` within the block.
__device__ __forceinline__ int32_t tail_value(__amdgpu_buffer_rsrc_t src, uint32_t offset,
                                              int precomputed) {
    if (precomputed)
        return static_cast<int32_t>(__builtin_amdgcn_raw_buffer_load_b8(src, offset, 0, 0)) - 127;
    const uint32_t bits = __builtin_amdgcn_raw_buffer_load_b16(src, offset * 2u, 0, 0);
    return static_cast<int32_t>((bits >> 7) & 255u) - 127;
}

// Tail byte i of the block: int8(e - 127) of the exponent at its logical
// position (-127 past the tensor's end), from the entries in LDS.
__device__ __forceinline__ int32_t tail_byte(__amdgpu_buffer_rsrc_t src, int32_t i,
                                             int32_t count, int64_t block, int S,
                                             int precomputed, const int32_t *entry_offset,
                                             const int32_t *entry_start,
                                             const int32_t *entry_lane) {
    // Last entry whose offset is <= i.
    int32_t lo = 0, hi = count - 1;
    while (lo < hi) {
        const int32_t mid = (lo + hi + 1) >> 1;
        if (entry_offset[mid] <= i) lo = mid;
        else hi = mid - 1;
    }
    const int64_t row_base = block * S;
    const int32_t row = entry_start[lo] + (i - entry_offset[lo]);
    const uint32_t offset = static_cast<uint32_t>(row) * kLanes
        + static_cast<uint32_t>(entry_lane[lo] ^ static_cast<int32_t>((row_base + row) & 254));
    return tail_value(src, offset, precomputed);
}

// With `source` given, the block's first 256 tail bytes are also read here
// (they depend on the ranking only), one per thread.
__device__ __forceinline__ BlockEntries rank_block_start(int32_t start, int64_t block, int S,
                                                         int32_t *scratch, int32_t *entry_offset,
                                                         int32_t *entry_start, int32_t *entry_lane,
                                                         const void *__restrict__ source,
                                                         int64_t logical_numel, int precomputed) {
    const int t = threadIdx.x;
    BlockEntries e;
    e.start = start;
    const bool bad = e.start != 255;
    // One scan of both counts: tail bytes in bits 0..19 (at most 256 x 256),
    // entries from bit 20 (at most 256).
    int32_t totals;
    const int32_t packed = block_exclusive_scan(bad ? (S - e.start) | (1 << 20) : 0, scratch,
                                                &totals);
    const int32_t local = packed & 0xFFFFF;
    e.rank = packed >> 20;
    e.bytes = totals & 0xFFFFF;
    e.count = totals >> 20;
    if (bad) {
        entry_offset[e.rank] = local;
        entry_start[e.rank] = e.start;
        entry_lane[e.rank] = t;
    }
    __syncthreads();
    e.first_tail = source != nullptr && t < e.bytes
                       ? tail_byte(block_source(source, block, S, logical_numel, precomputed), t,
                                   e.count, block, S, precomputed, entry_offset, entry_start,
                                   entry_lane)
                       : 0;
    return e;
}

// The same, loading this lane's extra start.
__device__ __forceinline__ BlockEntries rank_block(const uint8_t *__restrict__ extra_starts,
                                                   int64_t block, int S, int32_t *scratch,
                                                   int32_t *entry_offset, int32_t *entry_start,
                                                   int32_t *entry_lane,
                                                   const void *__restrict__ source = nullptr,
                                                   int64_t logical_numel = 0,
                                                   int precomputed = 0) {
    return rank_block_start(extra_starts[block * kLanes + threadIdx.x], block, S, scratch,
                            entry_offset, entry_start, entry_lane, source, logical_numel,
                            precomputed);
}

// Tail bytes of a block with many of them, through LDS: the overflowing rows
// are staged 64 at a time as exponent bytes (each logical row read whole and
// contiguous, each byte put at its storage lane: lane l of row r holds logical
// column l ^ (r & 254)), and then each wave writes whole entries' runs for
// those rows, one contiguous store of up to 64 bytes per entry and tile, lane j
// taking row j of the tile.  The staged rows are 260 bytes apart, so the 64
// lanes' reads of one column fall in 64 different banks.  The search path
// below costs about one LDS round trip per search step (8 for 256 entries) per
// byte and thread, and its loads and stores touch one cache line per byte:
// with 52 KB of tails in one block of 32768 elements it took the compaction to
// 153 us.
constexpr int kTileRows = 64;
constexpr int kTileStride = kLanes + 4;
constexpr int kStagedTailBytesPerStep = 16;   // take this path from 16 x S tail bytes on

__device__ __forceinline__ void write_tails_staged(__amdgpu_buffer_rsrc_t src,
                                                   __amdgpu_buffer_rsrc_t dst,
                                                   const BlockEntries &e,
                                                   const int32_t *entry_offset,
                                                   const int32_t *entry_start,
                                                   const int32_t *entry_lane, int64_t block,
                                                   int S, int precomputed, uint32_t valid) {
    __shared__ uint8_t tile[kTileRows * kTileStride];
    __shared__ int32_t wave_first[kWavesPerBlock];
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    // The first row any entry overflows at (entries <= 256: one per thread).
    const int32_t mine = wave_min(t < e.count ? entry_start[t] : S);
    if (lane == 0) wave_first[wave] = mine;
    __syncthreads();
    int32_t first_row = wave_first[0];
    for (int w = 1; w < kWavesPerBlock; ++w) first_row = min(first_row, wave_first[w]);
    const int64_t row_base = block * S;
    for (int t0 = first_row & ~(kTileRows - 1); t0 < S; t0 += kTileRows) {
        // Stage rows t0 .. t0 + 63: thread t takes elements 4t .. 4t + 3 of
        // each 1024-element quarter of the tile (4 rows), 16 quarters.
        // All sixteen loads of a thread in flight at once.
#pragma unroll
        for (int q = 0; q < kTileRows / 4; ++q) {
            const int r_local = q * 4 + (t >> 6);
            const uint32_t mask = static_cast<uint32_t>((row_base + t0 + r_local) & 254);
            const uint32_t col = static_cast<uint32_t>(t & 63) * 4u;
            const uint32_t offset = static_cast<uint32_t>(t0 + r_local) * kLanes + col;
            // Four elements: 8 bytes of BF16 or 4 exponent bytes (0 past the
            // tensor's end, which gives -127 as in tail_value).  A wide access
            // that straddles the resource's end reads as 0 whole, so the four
            // that hold the tensor's last element load one by one.
            uint32_t e4[4];
            if (offset < valid && offset + 4 > valid) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    e4[k] = static_cast<uint32_t>(tail_value(src, offset + k, precomputed));
            } else if (precomputed) {
                const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(src, offset, 0, 0);
#pragma unroll
                for (int k = 0; k < 4; ++k) e4[k] = ((w >> (8 * k)) & 255u) - 127u;
            } else {
                using u32x2 = __attribute__((ext_vector_type(2))) uint32_t;
                const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(src, offset * 2u, 0, 0);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    e4[k] = ((w[k >> 1] >> (16 * (k & 1) + 7)) & 255u) - 127u;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
                tile[r_local * kTileStride + ((col + k) ^ mask)] = static_cast<uint8_t>(e4[k]);
        }
        __syncthreads();
        // Wave w writes entries w, w + 4, ...: lane j takes row t0 + j; four
        // entries at a time, so their LDS reads overlap.
        const int32_t row = t0 + lane;
        for (int k0 = wave; k0 < e.count; k0 += 4 * kWavesPerBlock) {
            int32_t start[4], offset[4];
            uint32_t value[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int k = k0 + u * kWavesPerBlock;
                const bool present = k < e.count;
                start[u] = present ? entry_start[k] : S;   // S: no row of this tile
                offset[u] = present ? entry_offset[k] : 0;
                value[u] = tile[lane * kTileStride + (present ? entry_lane[k] : 0)];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                __builtin_amdgcn_raw_buffer_store_b8(
                    static_cast<uint8_t>(value[u]), dst,
                    row >= start[u] && row < S ? static_cast<uint32_t>(offset[u] + (row - start[u]))
                                               : 0x80000000u,
                    0, 0);
        }
        __syncthreads();   // the tile is restaged next
    }
}

__device__ __forceinline__ void write_block(
    const void *__restrict__ source, uint8_t *__restrict__ lanes, uint8_t *__restrict__ starts,
    uint8_t *__restrict__ tail, int64_t lane_off, int64_t start_off, int64_t tail_off,
    int32_t first, int32_t byte_base, const BlockEntries &e, int64_t block,
    int64_t logical_numel, int S, int precomputed, const int32_t *entry_offset,
    const int32_t *entry_start, const int32_t *entry_lane, bool prefetched = false) {
    const int t = threadIdx.x;
    if (e.start != 255) {
        lanes[lane_off + first + e.rank] = static_cast<uint8_t>(t);
        starts[start_off + first + e.rank] = static_cast<uint8_t>(e.start);
    }
    uint8_t *out = tail + tail_off + byte_base;
    const __amdgpu_buffer_rsrc_t src = block_source(source, block, S, logical_numel, precomputed);
    const __amdgpu_buffer_rsrc_t dst = make_rsrc(out, static_cast<uint32_t>(e.bytes));
    if (e.bytes >= kStagedTailBytesPerStep * S) {
        // Many tail bytes: staged rows and whole runs per entry (above), so
        // no byte needs the entry search.
        const int64_t left = logical_numel - block * S * kLanes;
        write_tails_staged(src, dst, e, entry_offset, entry_start, entry_lane, block, S,
                           precomputed,
                           static_cast<uint32_t>(left < int64_t{S} * kLanes ? left
                                                                            : int64_t{S} * kLanes));
        return;
    }
    // Byte t may have been read by rank_block already (prefetched).  The rest
    // go kTailBatch per thread at a time, every load issued before the batch's
    // stores, so a block with many tail bytes waits for one load latency per
    // batch instead of one per byte.
    int32_t i = t;
    if (prefetched) {
        __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(e.first_tail), dst,
                                             i < e.bytes ? static_cast<uint32_t>(i) : 0x80000000u,
                                             0, 0);
        i += kLanes;
    }
    constexpr int kTailBatch = 4;
    for (; i < e.bytes; i += kTailBatch * kLanes) {
        int32_t x[kTailBatch];
#pragma unroll
        for (int k = 0; k < kTailBatch; ++k) {
            const int32_t j = i + k * kLanes;
            x[k] = j < e.bytes ? tail_byte(src, j, e.count, block, S, precomputed, entry_offset,
                                           entry_start, entry_lane)
                               : 0;
        }
#pragma unroll
        for (int k = 0; k < kTailBatch; ++k) {
            const int32_t j = i + k * kLanes;
            __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(x[k]), dst,
                                                 j < e.bytes ? static_cast<uint32_t>(j)
                                                             : 0x80000000u,
                                                 0, 0);
        }
    }
    __syncthreads();   // the entry arrays are reused by the next block
}

__global__ __launch_bounds__(kLanes) void compact_extra_kernel(
    const void *__restrict__ source, uint8_t *__restrict__ lanes,
    uint8_t *__restrict__ starts, uint8_t *__restrict__ tail,
    const int32_t *__restrict__ descriptor, const int32_t *__restrict__ count_total,
    const int32_t *__restrict__ blocks, int64_t base, const uint8_t *__restrict__ extra_starts,
    const int32_t *__restrict__ summaries, int64_t n_blocks, int64_t logical_numel,
    int S, int precomputed, int buffered) {
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t entry_offset[kLanes], entry_start[kLanes], entry_lane[kLanes];
    const int32_t *list = summaries + 4 * n_blocks;
    // The reservation, the list's length and this workgroup's first list entry
    // are loaded together -- the entry speculatively (blockIdx.x < n_blocks by
    // the grid's size, and the list has n_blocks entries), used only if it is
    // listed -- so one memory round trip precedes the first block's extra
    // starts instead of three.
    const int32_t status = buffered ? descriptor[2] : kStatusOk;
    const int64_t arena = buffered ? descriptor[0] : 0;
    const int64_t total = buffered ? count_total[0] : 0;
    const int64_t listed = summaries[5 * n_blocks];
    int64_t i = blockIdx.x;
    int64_t block = list[i];
    if (status != kStatusOk) return;   // failed allocation: write nothing
    const int64_t lane_off = buffered ? arena : 0;
    const int64_t start_off = buffered ? arena + total : 0;
    const int64_t tail_off = buffered ? arena + 2 * total : base;
    for (; i < listed; i += gridDim.x) {
        if (i != blockIdx.x) block = list[i];
        // The block's first 256 tail bytes are read with the ranking.
        const BlockEntries e = rank_block(extra_starts, block, S, scratch, entry_offset,
                                          entry_start, entry_lane, source, logical_numel,
                                          precomputed);
        write_block(source, lanes, starts, tail, lane_off, start_off, tail_off,
                    blocks[n_blocks + block], blocks[2 * n_blocks + block], e, block,
                    logical_numel, S, precomputed, entry_offset, entry_start, entry_lane, true);
    }
}

// compact_extra's form without summaries (every block's metadata written
// before the launch: lct_compact_bad_streams, or the one-launch compress's
// bookkeeping): one workgroup per codec block loads the block's metadata, the
// reservation and its lanes' extra starts at once -- one memory round trip
// before the ranking -- and leaves if the block has no overflow.  The entries
// a block rewrites are the ones already there.
// Entries and tails of codec block `block`, at the offsets the block
// metadata holds (one workgroup).
__device__ __forceinline__ void compact_block(
    const void *__restrict__ source, uint8_t *__restrict__ lanes,
    uint8_t *__restrict__ starts, uint8_t *__restrict__ tail,
    const int32_t *__restrict__ descriptor, const int32_t *__restrict__ count_total,
    const int32_t *__restrict__ blocks, int64_t base, const uint8_t *__restrict__ extra_starts,
    int64_t n_blocks, int64_t logical_numel, int S, int precomputed, int buffered,
    int64_t block) {
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t entry_offset[kLanes], entry_start[kLanes], entry_lane[kLanes];
    const int32_t count = blocks[block];
    const int32_t first = blocks[n_blocks + block];
    const int32_t byte_base = blocks[2 * n_blocks + block];
    const int32_t start = extra_starts[block * kLanes + threadIdx.x];
    const int32_t status = buffered ? descriptor[2] : kStatusOk;
    const int64_t arena = buffered ? descriptor[0] : 0;
    const int64_t total = buffered ? count_total[0] : 0;
    if (count == 0 || status != kStatusOk) return;   // uniform
    const int64_t lane_off = buffered ? arena : 0;
    const int64_t start_off = buffered ? arena + total : 0;
    const int64_t tail_off = buffered ? arena + 2 * total : base;
    const BlockEntries e = rank_block_start(start, block, S, scratch, entry_offset, entry_start,
                                            entry_lane, source, logical_numel, precomputed);
    write_block(source, lanes, starts, tail, lane_off, start_off, tail_off, first, byte_base, e,
                block, logical_numel, S, precomputed, entry_offset, entry_start, entry_lane,
                true);
}

__global__ __launch_bounds__(kLanes) void compact_blocks_kernel(
    const void *__restrict__ source, uint8_t *__restrict__ lanes,
    uint8_t *__restrict__ starts, uint8_t *__restrict__ tail,
    const int32_t *__restrict__ descriptor, const int32_t *__restrict__ count_total,
    const int32_t *__restrict__ blocks, int64_t base, const uint8_t *__restrict__ extra_starts,
    int64_t n_blocks, int64_t logical_numel, int S, int precomputed, int buffered) {
    compact_block(source, lanes, starts, tail, descriptor, count_total, blocks, base,
                  extra_starts, n_blocks, logical_numel, S, precomputed, buffered, blockIdx.x);
}

// The compaction of a batched compress: workgroup w compacts block
// w - first_block[j] of job j into job j's reservation.
__global__ __launch_bounds__(kLanes) void compact_batch_kernel(CompactBatch batch) {
    const int32_t w = static_cast<int32_t>(blockIdx.x);
    int j = 0;
    for (int k = 1; k < batch.n_jobs; ++k)
        if (w >= batch.first_block[k]) j = k;
    const CompactBatchJob &job = batch.jobs[j];
    compact_block(job.source, batch.arena, batch.arena, batch.arena, job.descriptor, job.counts,
                  job.blocks, 0, job.extra_starts, job.n_blocks, job.logical_numel, batch.steps,
                  batch.precomputed, 1, w - batch.first_block[j]);
}

// Waits of the compacting workgroups for workgroup 0's reservation: polls of
// the ready word with a sleep between them, about 4 s at most with the default
// limit (workgroup 0's own wait for the arena lock is bounded well below that,
// and it publishes in every case).  A workgroup that gives up writes nothing:
// it replaces the ready word's old value with ~epoch, and workgroup 0, which
// publishes with an exchange, then finds ~epoch and marks the reservation
// incomplete (status 7, failure bit 4).  Had workgroup 0 published first, the
// replacement fails, the waiter sees epoch and goes on as usual.
// Compacting workgroups of one launch (each owns every 2047th block): 2047
// measured best on gfx950 at 4096 blocks (694 with overflow: 12.6 us with a
// pending free) and at 1024 blocks (all with overflow: 11.9 us), against 511
// (16.3, 14.7 us), 1023 and 4095.  Workgroups that do not fit on the device
// at once start as others leave; those whose blocks have no overflow leave
// at once.
constexpr int64_t kAllocateCompactWaiters = 2047;

// A value workgroup 0 wrote in this launch: an agent-scope load, which reads
// the coherent copy (workgroup 0 released its writes before the ready word).
// An agent-scope acquire fence instead would invalidate the whole L2 once per
// wave; measured on gfx950 that made the launch 22 us against 15 us for the
// two launches it replaces.
__device__ __forceinline__ int32_t published(const int32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Scan + reservation (workgroup 0, deferred frees first) and compaction
// (workgroups 1..G-1) in one launch.  Workgroup 0 publishes its writes with an
// agent-scope release and then stores `epoch` to *ready.  Compacting
// workgroup w owns blocks w - 1 + k (G - 1): it ranks its first overflowing
// block's lanes before waiting, then polls *ready, reads the offsets workgroup
// 0 wrote with agent-scope loads and writes its blocks' entries and tails; a
// workgroup whose blocks have no overflow exits at once.  Workgroup 0 is
// dispatched first and waits for nothing but the arena lock, so every wait
// ends.
__global__ __launch_bounds__(kLanes) void allocate_compact_kernel(
    const void *__restrict__ source, int32_t *__restrict__ summaries,
    int32_t *__restrict__ counts, int32_t *__restrict__ descriptor,
    int32_t *__restrict__ buffer_meta, int32_t max_free_regions, uint8_t *__restrict__ arena,
    int32_t *__restrict__ blocks, const uint8_t *__restrict__ extra_starts,
    lct_pending_frees frees, uint64_t *__restrict__ ready, uint64_t epoch, int32_t n_blocks,
    int64_t logical_numel, int S, int precomputed, int32_t lock_spins, int32_t ready_limit) {
    extern __shared__ int32_t free_list[];   // 2 * max_free_regions ints (workgroup 0)
    const uint64_t gave_up = ~epoch;
    if (blockIdx.x == 0) {
        LdsReserve<true> reserve{AllocatorMeta(buffer_meta, max_free_regions, lock_spins), descriptor,
                           frees, free_list, {}, -1, kStatusOk};
        SummaryLoads loads(summaries, n_blocks);
        scan_allocate<false>(loads, summaries, counts, blocks, n_blocks, reserve);
        // finish() released every write of the workgroup at agent scope.
        if (threadIdx.x == 0) {
            const uint64_t before = __hip_atomic_exchange(ready, epoch, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT);
            if (before == gave_up && reserve.status == kStatusOk) {
                // Some compacting workgroup left without writing its blocks.
                __hip_atomic_store(descriptor + 2, kStatusIncomplete, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                record_failure(reserve.meta, kFailIncomplete);
            }
        }
        return;
    }
    __shared__ int32_t go;
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t entry_offset[kLanes], entry_start[kLanes], entry_lane[kLanes];
    __shared__ uint64_t mine[kWavesPerBlock];
    // This workgroup's blocks are blockIdx.x - 1 + k * stride; the encoder's
    // per-block counts (summaries[0, nb), written before this launch) say which
    // of them overflow, one load per thread (at most 33 blocks per workgroup:
    // n_blocks <= 65535 and stride = min(n_blocks, 2047)).
    const int64_t nb = n_blocks;
    const int64_t stride = gridDim.x - 1;
    const int64_t own = blockIdx.x - 1;
    const int64_t k_count = (nb - own + stride - 1) / stride;
    const int t = threadIdx.x;
    const bool has = t < k_count && summaries[own + t * stride] > 0;
    const uint64_t has_mask = __ballot(has);
    if ((t & (kWave - 1)) == 0) mine[t / kWave] = has_mask;
    __syncthreads();
    int wave = 0;
    uint64_t pending = mine[0];
    auto next_block = [&]() -> int64_t {   // uniform; -1 when none is left
        while (pending == 0) {
            if (++wave == kWavesPerBlock) return -1;
            pending = mine[wave];
        }
        const int k = __builtin_ctzll(pending);
        pending &= pending - 1;
        return own + static_cast<int64_t>(wave * kWave + k) * stride;
    };
    int64_t block = next_block();
    if (block < 0) return;   // no overflow here: nothing to wait for
    // Ranking needs nothing from workgroup 0, so the first block's is done
    // while workgroup 0 works.
    BlockEntries e = rank_block(extra_starts, block, S, scratch, entry_offset, entry_start,
                                entry_lane, source, logical_numel, precomputed);
    if (t == 0) {
        uint64_t value = 0;
        for (int i = 0; i < ready_limit; ++i) {
            value = __hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (value == epoch) break;
            __builtin_amdgcn_s_sleep(8);
        }
        // Giving up: leave ~epoch in the ready word for workgroup 0 to find,
        // unless it published meanwhile (the value can change at most twice:
        // to epoch, or to ~epoch by another waiter).
        while (value != epoch && value != gave_up) {
            uint64_t expected = value;
            if (__hip_atomic_compare_exchange_strong(ready, &expected, gave_up,
                                                     __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT))
                value = gave_up;
            else
                value = expected;
        }
        go = value == epoch ? 1 : 0;
    }
    __syncthreads();
    if (go == 0) return;
    // All of the reservation's values at once (reading them is harmless when
    // it failed), then the status.
    const int32_t status = published(descriptor + 2);
    const int64_t total = published(counts);
    const int64_t lane_off = published(descriptor);
    int32_t first = published(blocks + nb + block);
    int32_t byte_base = published(blocks + 2 * nb + block);
    if (status != kStatusOk) return;   // failed reservation: write nothing
    const int64_t start_off = lane_off + total;
    const int64_t tail_off = lane_off + 2 * total;
    bool prefetched = true;
    for (;;) {
        write_block(source, arena, arena, arena, lane_off, start_off, tail_off, first,
                    byte_base, e, block, logical_numel, S, precomputed, entry_offset,
                    entry_start, entry_lane, prefetched);
        block = next_block();
        if (block < 0) break;
        e = rank_block(extra_starts, block, S, scratch, entry_offset, entry_start, entry_lane);
        first = published(blocks + nb + block);
        byte_base = published(blocks + 2 * nb + block);
        prefetched = false;
    }
}

// Totals of the overflowing streams and their tail bytes, added atomically to
// count[0] and total[0] (compaction.py:31-51: the atomic path's counts; the
// caller zeroes both).  Each thread reads 16 streams' extra starts.
__global__ __launch_bounds__(kLanes) void count_bad_streams_kernel(
    const uint8_t *__restrict__ extra_starts, int32_t *__restrict__ count,
    int32_t *__restrict__ total, int64_t n_streams, int S) {
    __shared__ int32_t scratch[kWavesPerBlock];
    const int64_t first = (static_cast<int64_t>(blockIdx.x) * kLanes + threadIdx.x) * 16;
    int32_t bad = 0, bytes = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int64_t s = first + k;
        const int32_t start = s < n_streams ? extra_starts[s] : 255;
        bad += start != 255 ? 1 : 0;
        bytes += start != 255 ? S - start : 0;
    }
    bad = block_sum(bad, scratch);
    bytes = block_sum(bytes, scratch);
    if (threadIdx.x == 0) {
        if (bad != 0)
            __hip_atomic_fetch_add(count, bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (bytes != 0)
            __hip_atomic_fetch_add(total, bytes, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// One workgroup per codec block (compaction.py:54-96): the block reserves its
// entry slots and tail bytes with two atomics on bad_count / fallback_total
// (which start at 0), records {count, first, byte_base} and writes its
// entries, lanes ascending.  Slot order across blocks follows the atomics;
// every reader locates a block's slice through its own metadata.  Blocks
// without overflow record first = byte_base = 0.  A buffered reservation that
// failed (descriptor status != 0) gets its metadata but no entries.
__global__ __launch_bounds__(kLanes) void compact_bad_streams_kernel(
    const uint8_t *__restrict__ extra_starts, uint8_t *__restrict__ lanes,
    uint8_t *__restrict__ starts, const int32_t *__restrict__ descriptor,
    int32_t *__restrict__ blocks, const int32_t *__restrict__ final_counts,
    int32_t *__restrict__ bad_count, int32_t *__restrict__ fallback_total, int64_t n_streams,
    int64_t n_blocks, int S, int buffered) {
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t reserved[2];
    const int t = threadIdx.x;
    const int64_t block = blockIdx.x;
    const int64_t stream = block * kLanes + t;
    const int32_t start = stream < n_streams ? extra_starts[stream] : 255;
    const bool bad = start != 255;
    int32_t count;
    const int32_t rank = block_exclusive_scan(bad ? 1 : 0, scratch, &count);
    const int32_t bytes = block_sum(bad ? S - start : 0, scratch);
    if (t == 0) {
        reserved[0] = count != 0 ? __hip_atomic_fetch_add(bad_count, count, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                 : 0;
        reserved[1] = bytes != 0 ? __hip_atomic_fetch_add(fallback_total, bytes,
                                                          __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                 : 0;
        blocks[block] = count;
        blocks[n_blocks + block] = reserved[0];
        blocks[2 * n_blocks + block] = reserved[1];
    }
    __syncthreads();
    if (!bad) return;
    int64_t lane_off = 0, start_off = 0;
    if (buffered) {
        if (descriptor[2] != kStatusOk) return;
        lane_off = descriptor[0];
        start_off = lane_off + final_counts[0];
    }
    const int64_t pos = reserved[0] + rank;
    lanes[lane_off + pos] = static_cast<uint8_t>(t);
    starts[start_off + pos] = static_cast<uint8_t>(start);
}

// Overflow rows of a decode made without the overlay (compaction.py:238-306):
// every tail byte of every block, rebuilt into BF16 with its side byte and
// written at its logical position.  A grid-stride loop over blocks.
__global__ __launch_bounds__(kLanes) void scatter_fallback_kernel(
    lct_overflow ov, const uint8_t *__restrict__ side, uint16_t *__restrict__ output,
    int64_t n_blocks, int64_t logical_numel, int S) {
    __shared__ TailEntries entries;
    for (int64_t block = blockIdx.x; block < n_blocks; block += gridDim.x) {
        const TailWalk w = stage_block_entries(ov, block, n_blocks, S, entries);
        if (w.count == 0) continue;   // uniform
        for (int32_t i = threadIdx.x; i < w.bytes; i += kLanes) {
            int32_t step, lane;
            tail_position(w, entries, i, step, lane);
            const int64_t row = block * S + step;
            const int64_t logical = row * kLanes + (lane ^ static_cast<int32_t>(row & 254));
            if (logical < logical_numel)
                output[logical] = static_cast<uint16_t>(pack_tail(w.tail[i], side[row * kLanes + lane]));
        }
        __syncthreads();   // the entries are restaged for the next block
    }
}

}  // namespace

hipError_t launch_compact_batch(const CompactBatch &batch, uint32_t grid, hipStream_t stream) {
    hipLaunchKernelGGL(compact_batch_kernel, dim3(grid), dim3(kLanes), 0, stream, batch);
    return hipGetLastError();
}

}  // namespace lct

using namespace lct;

extern "C" int32_t lct_prefix_allocate(int32_t *summaries, int32_t *counts,
                                       int32_t *descriptor, int32_t *buffer_meta,
                                       int32_t *blocks, int64_t n_blocks, int32_t buffered,
                                       int32_t max_free_regions, hipStream_t stream) {
    if (!summaries || !counts || !blocks) return LCT_E_NULL;
    if (buffered && (!descriptor || !buffer_meta)) return LCT_E_NULL;
    // 5*nb + 1 summary entries and the int32 tail offsets bound the block count.
    if (n_blocks <= 0 || n_blocks > kMaxBlocks) return LCT_E_SIZE;
    if (buffered && (max_free_regions <= 0 || max_free_regions > 4096
                     || (max_free_regions & (max_free_regions - 1)) != 0))
        return LCT_E_ARG;
    hipLaunchKernelGGL(prefix_allocate_kernel, dim3(1), dim3(kLanes), 0, stream, summaries,
                       counts, descriptor, buffer_meta, blocks, static_cast<int32_t>(n_blocks),
                       buffered, max_free_regions, lock_spins());
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_compact_extra(const void *source, uint8_t *lanes, uint8_t *starts,
                                     uint8_t *tail, const int32_t *descriptor,
                                     const int32_t *count, const int32_t *blocks, int64_t base,
                                     const uint8_t *extra_starts, const int32_t *summaries,
                                     int64_t size, int64_t logical_numel, lct_geometry g,
                                     int32_t precomputed, int32_t buffered,
                                     hipStream_t stream) {
    if (!source || !blocks || !extra_starts) return LCT_E_NULL;
    if (buffered && (!descriptor || !count || !tail)) return LCT_E_NULL;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (size <= 0 || size % g.block_symbols != 0 || logical_numel <= 0 || logical_numel > size)
        return LCT_E_SIZE;
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > 0x7FFFFFFF) return LCT_E_SIZE;
    if (summaries == nullptr) {
        hipLaunchKernelGGL(compact_blocks_kernel, dim3(static_cast<uint32_t>(n_blocks)),
                           dim3(kLanes), 0, stream, source, lanes, starts, tail, descriptor, count,
                           blocks, base, extra_starts, n_blocks, logical_numel, g.steps,
                           precomputed, buffered);
        return static_cast<int32_t>(hipGetLastError());
    }
    const uint32_t grid = static_cast<uint32_t>(n_blocks < kCompactGrid ? n_blocks : kCompactGrid);
    hipLaunchKernelGGL(compact_extra_kernel, dim3(grid), dim3(kLanes), 0, stream, source, lanes,
                       starts, tail, descriptor, count, blocks, base, extra_starts, summaries,
                       n_blocks, logical_numel, g.steps, precomputed, buffered);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_allocate_compact(const void *source, int32_t *summaries,
                                        int32_t *counts, int32_t *descriptor,
                                        int32_t *buffer_meta, int32_t max_free_regions,
                                        uint8_t *arena, int32_t *blocks,
                                        const uint8_t *extra_starts,
                                        const lct_pending_frees *frees, uint64_t *ready,
                                        uint64_t epoch, int64_t size, int64_t logical_numel,
                                        lct_geometry g, int32_t precomputed,
                                        hipStream_t stream) {
    if (!source || !summaries || !counts || !descriptor || !buffer_meta || !arena || !blocks
        || !extra_starts || !ready)
        return LCT_E_NULL;
    if ((reinterpret_cast<uintptr_t>(ready) & 7) != 0) return LCT_E_ARG;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (size <= 0 || size % g.block_symbols != 0 || logical_numel <= 0 || logical_numel > size)
        return LCT_E_SIZE;
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > kMaxBlocks) return LCT_E_SIZE;
    if (max_free_regions <= 0 || max_free_regions > 4096
        || (max_free_regions & (max_free_regions - 1)) != 0)
        return LCT_E_ARG;
    lct_pending_frees pending{};
    if (frees != nullptr) {
        if (frees->count < 0 || frees->count > LCT_MAX_PENDING_FREES) return LCT_E_ARG;
        for (int i = 0; i < frees->count; ++i)
            if (frees->descriptor[i] == nullptr) return LCT_E_NULL;
        pending = *frees;
    }
    // Workgroup 0 plus up to kAllocateCompactWaiters compacting workgroups.
    const uint32_t grid = 1u + static_cast<uint32_t>(
        n_blocks < kAllocateCompactWaiters ? n_blocks : kAllocateCompactWaiters);
    const size_t lds = static_cast<size_t>(max_free_regions) * 8;
    hipLaunchKernelGGL(allocate_compact_kernel, dim3(grid), dim3(kLanes), lds, stream, source,
                       summaries, counts, descriptor, buffer_meta, max_free_regions, arena,
                       blocks, extra_starts, pending, ready, epoch,
                       static_cast<int32_t>(n_blocks), logical_numel, g.steps, precomputed,
                       lock_spins(), ready_polls());
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_count_bad_streams(const uint8_t *extra_starts, int32_t *count,
                                         int32_t *total, int64_t n_streams, int32_t steps,
                                         hipStream_t stream) {
    if (!extra_starts || !count || !total) return LCT_E_NULL;
    if (n_streams <= 0 || n_streams > kMaxBlocks * kLanes) return LCT_E_SIZE;
    if (steps != 128 && steps != 256) return LCT_E_GEOMETRY;
    const int64_t per_group = 16 * kLanes;
    const uint32_t grid = static_cast<uint32_t>((n_streams + per_group - 1) / per_group);
    hipLaunchKernelGGL(count_bad_streams_kernel, dim3(grid), dim3(kLanes), 0, stream,
                       extra_starts, count, total, n_streams, static_cast<int>(steps));
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_compact_bad_streams(const uint8_t *extra_starts, uint8_t *lanes,
                                           uint8_t *starts, const int32_t *descriptor,
                                           int32_t *blocks, const int32_t *final_counts,
                                           int32_t *bad_count, int32_t *fallback_total,
                                           int64_t n_streams, int32_t steps, int64_t n_blocks,
                                           int32_t buffered, hipStream_t stream) {
    if (!extra_starts || !lanes || !starts || !blocks || !bad_count || !fallback_total)
        return LCT_E_NULL;
    if (buffered && (!descriptor || !final_counts)) return LCT_E_NULL;
    if (n_blocks <= 0 || n_blocks > kMaxBlocks || n_streams <= 0 || n_streams > n_blocks * kLanes)
        return LCT_E_SIZE;
    if (steps != 128 && steps != 256) return LCT_E_GEOMETRY;
    hipLaunchKernelGGL(compact_bad_streams_kernel, dim3(static_cast<uint32_t>(n_blocks)),
                       dim3(kLanes), 0, stream, extra_starts, lanes, starts, descriptor, blocks,
                       final_counts, bad_count, fallback_total, n_streams, n_blocks,
                       static_cast<int>(steps), buffered);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_scatter_fallback(const lct_overflow *overflow, const uint8_t *side,
                                        void *output, int64_t size, int64_t logical_numel,
                                        lct_geometry g, hipStream_t stream) {
    if (!overflow || !side || !output) return LCT_E_NULL;
    if (!overflow->lanes || !overflow->starts || !overflow->tail || !overflow->blocks)
        return LCT_E_NULL;
    if (overflow->descriptor != nullptr && overflow->count == nullptr) return LCT_E_NULL;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (size <= 0 || size % g.block_symbols != 0 || logical_numel <= 0 || logical_numel > size)
        return LCT_E_SIZE;
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > kMaxBlocks) return LCT_E_SIZE;
    const uint32_t grid = static_cast<uint32_t>(n_blocks < kCompactGrid ? n_blocks : kCompactGrid);
    hipLaunchKernelGGL(scatter_fallback_kernel, dim3(grid), dim3(kLanes), 0, stream, *overflow,
                       side, static_cast<uint16_t *>(output), n_blocks, logical_numel, g.steps);
    return static_cast<int32_t>(hipGetLastError());
}
