// Overflow bookkeeping after the encoder: block prefix scans + arena
// allocation (one workgroup), then per-block compaction of overflowing streams.
//
// Follows LCT/kernels/generic/metadata.py:13-38 and
// LCT/kernels/generic/compaction.py:99-235 (summaries path).  The compact list
// is stored per codec block: the block's overflowing lanes in ascending order
// at entries [first, first+count), their exponent tails int8(e-127) for steps
// start..S-1 concatenated from byte_base, and blocks[3*nb] = {count, first,
// byte_base} so every reader walks the list one block at a time.
#include "allocator.h"

namespace lct {
namespace {

constexpr int kPrefixPerThread = 32;   // 256 x 32 = 8192 blocks

__global__ __launch_bounds__(kLanes) void prefix_allocate_kernel(
    int32_t *__restrict__ summaries, int32_t *__restrict__ counts,
    int32_t *__restrict__ descriptor, int32_t *__restrict__ buffer_meta,
    int32_t n_blocks, int32_t buffered, int32_t max_free_regions) {
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t flag;
    const int t = threadIdx.x;
    // Thread t owns the contiguous run [t*per, t*per + per) and keeps it in
    // registers between the load, the block scan and the store.
    const int per = (n_blocks + kLanes - 1) / kLanes;
    const int begin = t * per;
    int32_t counts_local[kPrefixPerThread], bytes_local[kPrefixPerThread];
    int32_t local_count = 0, local_bytes = 0;
#pragma unroll
    for (int j = 0; j < kPrefixPerThread; ++j) {
        const int b = begin + j;
        const bool in = j < per && b < n_blocks;
        counts_local[j] = in ? summaries[b] : 0;
        bytes_local[j] = in ? summaries[n_blocks + b] : 0;
        local_count += counts_local[j];
        local_bytes += bytes_local[j];
    }
    int32_t total_count, total_bytes;
    int32_t count_run = block_exclusive_scan(local_count, scratch, &total_count);
    int32_t byte_run = block_exclusive_scan(local_bytes, scratch, &total_bytes);
#pragma unroll
    for (int j = 0; j < kPrefixPerThread; ++j) {
        const int b = begin + j;
        if (j < per && b < n_blocks) {
            summaries[2 * n_blocks + b] = count_run;
            summaries[3 * n_blocks + b] = byte_run;
        }
        count_run += counts_local[j];
        byte_run += bytes_local[j];
    }
    if (t == 0) {
        counts[0] = total_count;
        counts[1] = total_bytes;
        counts[2] = 0;
        counts[3] = 0;
    }
    if (buffered) {
        // Two metadata bytes per overflowing stream: lane, then start step.
        const AllocatorMeta meta(buffer_meta, max_free_regions);
        allocator_allocate(meta, total_bytes + 2 * total_count, descriptor, scratch, &flag);
    }
}

__global__ __launch_bounds__(kLanes) void compact_extra_kernel(
    const void *__restrict__ source, uint8_t *__restrict__ lanes,
    uint8_t *__restrict__ starts, uint8_t *__restrict__ tail,
    const int32_t *__restrict__ descriptor, const int32_t *__restrict__ count_total,
    int32_t *__restrict__ blocks, int64_t base, const uint8_t *__restrict__ extra_starts,
    const int32_t *__restrict__ summaries, int64_t n_blocks, int64_t logical_numel,
    int S, int precomputed, int buffered) {
    __shared__ int32_t scratch[kWavesPerBlock];
    const int t = threadIdx.x;
    const int64_t block = blockIdx.x;
    const int32_t count = summaries[block];
    const int32_t first = summaries[2 * n_blocks + block];
    const int32_t byte_base = summaries[3 * n_blocks + block];
    if (t == 0) {
        blocks[block] = count;
        blocks[n_blocks + block] = first;
        blocks[2 * n_blocks + block] = byte_base;
    }
    if (count == 0) return;
    int64_t lane_off = 0, start_off = 0, tail_off = base;
    if (buffered) {
        if (descriptor[2] != kStatusOk) return;   // failed allocation: write nothing
        const int64_t arena = descriptor[0];
        const int64_t total = count_total[0];
        lane_off = arena;
        start_off = arena + total;
        tail_off = arena + 2 * total;
    }
    const int32_t start = extra_starts[block * kLanes + t];
    const bool bad = start != 255;
    int32_t ignored;
    const int32_t local = block_exclusive_scan(bad ? S - start : 0, scratch, &ignored);
    const int32_t rank = block_exclusive_scan(bad ? 1 : 0, scratch, &ignored);
    if (!bad) return;
    lanes[lane_off + first + rank] = static_cast<uint8_t>(t);
    starts[start_off + first + rank] = static_cast<uint8_t>(start);
    uint8_t *out = tail + tail_off + byte_base + local;
    const int64_t row_base = block * S;
    for (int row = start; row < S; ++row) {
        const int64_t logical = (row_base + row) * kLanes
            + (t ^ static_cast<int32_t>((row_base + row) & 254));
        int32_t e = -127;
        if (logical < logical_numel) {
            if (precomputed) {
                e = static_cast<int32_t>(static_cast<const uint8_t *>(source)[logical]) - 127;
            } else {
                const int32_t bits = static_cast<const uint16_t *>(source)[logical];
                e = ((bits >> 7) & 255) - 127;
            }
        }
        out[row - start] = static_cast<uint8_t>(e);
    }
}

}  // namespace
}  // namespace lct

using namespace lct;

extern "C" int32_t lct_prefix_allocate(int32_t *summaries, int32_t *counts,
                                       int32_t *descriptor, int32_t *buffer_meta,
                                       int64_t n_blocks, int32_t buffered,
                                       int32_t max_free_regions, hipStream_t stream) {
    if (!summaries || !counts) return LCT_E_NULL;
    if (buffered && (!descriptor || !buffer_meta)) return LCT_E_NULL;
    if (n_blocks <= 0 || n_blocks > kLanes * kPrefixPerThread) return LCT_E_SIZE;
    if (buffered && (max_free_regions <= 0 || max_free_regions > 4096
                     || (max_free_regions & (max_free_regions - 1)) != 0))
        return LCT_E_ARG;
    hipLaunchKernelGGL(prefix_allocate_kernel, dim3(1), dim3(kLanes), 0, stream, summaries,
                       counts, descriptor, buffer_meta, static_cast<int32_t>(n_blocks),
                       buffered, max_free_regions);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_compact_extra(const void *source, uint8_t *lanes, uint8_t *starts,
                                     uint8_t *tail, const int32_t *descriptor,
                                     const int32_t *count, int32_t *blocks, int64_t base,
                                     const uint8_t *extra_starts, const int32_t *summaries,
                                     int64_t size, int64_t logical_numel, lct_geometry g,
                                     int32_t precomputed, int32_t buffered,
                                     hipStream_t stream) {
    if (!source || !blocks || !extra_starts || !summaries) return LCT_E_NULL;
    if (buffered && (!descriptor || !count || !tail)) return LCT_E_NULL;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (size <= 0 || size % g.block_symbols != 0 || logical_numel <= 0 || logical_numel > size)
        return LCT_E_SIZE;
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > 0x7FFFFFFF) return LCT_E_SIZE;
    hipLaunchKernelGGL(compact_extra_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes),
                       0, stream, source, lanes, starts, tail, descriptor, count, blocks, base,
                       extra_starts, summaries, n_blocks, logical_numel, g.steps, precomputed,
                       buffered);
    return static_cast<int32_t>(hipGetLastError());
}
