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
#include <algorithm>

#include "allocator.h"

namespace lct {
namespace {

constexpr int kPrefixChunk = 8192;      // blocks per LDS pass: 3 x 8192 int32 of LDS
constexpr int kCompactGrid = 2048;     // workgroups walking the overflow-block list

// summaries layout (int32[5*nb + 1]): per-block overflow counts | tail bytes |
// exclusive count scan | exclusive byte scan | list of blocks with overflow |
// list length.  The encoder writes the first two; this kernel the rest.
// Blocks are scanned in chunks of kPrefixChunk with the running totals carried
// from chunk to chunk, so any block count gives the same deterministic layout
// (entries in block order, lanes ascending within a block).
__global__ __launch_bounds__(kLanes) void prefix_allocate_kernel(
    int32_t *__restrict__ summaries, int32_t *__restrict__ counts,
    int32_t *__restrict__ descriptor, int32_t *__restrict__ buffer_meta,
    int32_t *__restrict__ blocks, int32_t n_blocks, int32_t buffered,
    int32_t max_free_regions) {
    // LDS per chunk: counts | tail bytes (then byte scan) | count scan.
    extern __shared__ int32_t lds[];
    const int chunk_cap = min(n_blocks, kPrefixChunk);
    int32_t *c_lds = lds;
    int32_t *v_lds = lds + chunk_cap;
    int32_t *cp_lds = lds + 2 * chunk_cap;
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t flag;
    const int t = threadIdx.x;
    int32_t *list = summaries + 4 * static_cast<int64_t>(n_blocks);
    int32_t carry_count = 0, carry_bytes = 0, carry_listed = 0;
    for (int base = 0; base < n_blocks; base += kPrefixChunk) {
        const int m = min(kPrefixChunk, n_blocks - base);
        // Coalesced loads into LDS, all issued before the first LDS write.
        constexpr int kRows = kPrefixChunk / kLanes;
        int32_t c_reg[kRows], v_reg[kRows];
#pragma unroll
        for (int j = 0; j < kRows; ++j) {
            const int b = j * kLanes + t;
            c_reg[j] = b < m ? summaries[base + b] : 0;
            v_reg[j] = b < m ? summaries[n_blocks + base + b] : 0;
        }
#pragma unroll
        for (int j = 0; j < kRows; ++j) {
            const int b = j * kLanes + t;
            if (b < m) {
                c_lds[b] = c_reg[j];
                v_lds[b] = v_reg[j];
            }
        }
        __syncthreads();
        // Thread t scans the contiguous run [t*per, t*per + per) of the chunk.
        const int per = (m + kLanes - 1) / kLanes;
        const int begin = min(t * per, m);
        const int end = min(begin + per, m);
        int32_t run_count = 0, run_bytes = 0, run_listed = 0;
        for (int b = begin; b < end; ++b) {
            run_count += c_lds[b];
            run_bytes += v_lds[b];
            run_listed += c_lds[b] > 0 ? 1 : 0;
        }
        int32_t chunk_count, chunk_bytes, chunk_listed;
        int32_t count_before = carry_count + block_exclusive_scan(run_count, scratch, &chunk_count);
        int32_t byte_before = carry_bytes + block_exclusive_scan(run_bytes, scratch, &chunk_bytes);
        int32_t list_before =
            carry_listed + block_exclusive_scan(run_listed, scratch, &chunk_listed);
        for (int b = begin; b < end; ++b) {
            const int32_t count = c_lds[b];
            const int32_t bytes = v_lds[b];
            cp_lds[b] = count_before;
            v_lds[b] = byte_before;
            if (count > 0) list[list_before++] = base + b;
            count_before += count;
            byte_before += bytes;
        }
        __syncthreads();
        // Coalesced stores of the scans and the block metadata.
        for (int b = t; b < m; b += kLanes) {
            const int32_t count = c_lds[b], first = cp_lds[b], byte_base = v_lds[b];
            const int64_t k = static_cast<int64_t>(base) + b;
            summaries[2 * static_cast<int64_t>(n_blocks) + k] = first;
            summaries[3 * static_cast<int64_t>(n_blocks) + k] = byte_base;
            blocks[k] = count;
            blocks[n_blocks + k] = first;
            blocks[2 * static_cast<int64_t>(n_blocks) + k] = byte_base;
        }
        carry_count += chunk_count;
        carry_bytes += chunk_bytes;
        carry_listed += chunk_listed;
        __syncthreads();   // the next chunk overwrites the LDS arrays
    }
    if (t == 0) {
        counts[0] = carry_count;
        counts[1] = carry_bytes;
        counts[2] = 0;
        counts[3] = 0;
        summaries[5 * static_cast<int64_t>(n_blocks)] = carry_listed;
    }
    if (buffered) {
        // Two metadata bytes per overflowing stream: lane, then start step.
        const AllocatorMeta meta(buffer_meta, max_free_regions);
        allocator_allocate(meta, carry_bytes + 2 * carry_count, descriptor, scratch, &flag);
    }
}

// One codec block's overflow entries and tails (compaction.py:137-228).  The
// block's tail bytes are produced one per thread: tail byte i belongs to the
// overflowing lane whose local byte range holds i (binary search over the
// lanes' offsets in LDS), so every byte is an independent load and the tail
// stores are contiguous.
__device__ __forceinline__ void compact_block(
    const void *__restrict__ source, uint8_t *__restrict__ lanes, uint8_t *__restrict__ starts,
    uint8_t *__restrict__ tail, int64_t lane_off, int64_t start_off, int64_t tail_off,
    const int32_t *__restrict__ blocks, const uint8_t *__restrict__ extra_starts,
    int64_t block, int64_t n_blocks, int64_t logical_numel, int S, int precomputed,
    int32_t *scratch, int32_t *entry_offset, int32_t *entry_start, int32_t *entry_lane) {
    const int t = threadIdx.x;
    const int32_t count = blocks[block];
    const int32_t first = blocks[n_blocks + block];
    const int32_t byte_base = blocks[2 * n_blocks + block];
    const int32_t start = extra_starts[block * kLanes + t];
    const bool bad = start != 255;
    int32_t block_bytes, ignored;
    const int32_t local = block_exclusive_scan(bad ? S - start : 0, scratch, &block_bytes);
    const int32_t rank = block_exclusive_scan(bad ? 1 : 0, scratch, &ignored);
    if (bad) {
        lanes[lane_off + first + rank] = static_cast<uint8_t>(t);
        starts[start_off + first + rank] = static_cast<uint8_t>(start);
        entry_offset[rank] = local;
        entry_start[rank] = start;
        entry_lane[rank] = t;
    }
    __syncthreads();
    uint8_t *out = tail + tail_off + byte_base;
    const int64_t row_base = block * S;
    for (int32_t i = t; i < block_bytes; i += kLanes) {
        // Last entry whose offset is <= i.
        int32_t lo = 0, hi = count - 1;
        while (lo < hi) {
            const int32_t mid = (lo + hi + 1) >> 1;
            if (entry_offset[mid] <= i) lo = mid;
            else hi = mid - 1;
        }
        const int32_t row = entry_start[lo] + (i - entry_offset[lo]);
        const int64_t logical = (row_base + row) * kLanes
            + (entry_lane[lo] ^ static_cast<int32_t>((row_base + row) & 254));
        int32_t e = -127;
        if (logical < logical_numel) {
            if (precomputed) {
                e = static_cast<int32_t>(static_cast<const uint8_t *>(source)[logical]) - 127;
            } else {
                const int32_t bits = static_cast<const uint16_t *>(source)[logical];
                e = ((bits >> 7) & 255) - 127;
            }
        }
        out[i] = static_cast<uint8_t>(e);
    }
    __syncthreads();   // entry arrays are reused by the next listed block
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
    int64_t lane_off = 0, start_off = 0, tail_off = base;
    if (buffered) {
        if (descriptor[2] != kStatusOk) return;   // failed allocation: write nothing
        const int64_t arena = descriptor[0];
        const int64_t total = count_total[0];
        lane_off = arena;
        start_off = arena + total;
        tail_off = arena + 2 * total;
    }
    const int32_t *list = summaries + 4 * n_blocks;
    const int32_t listed = summaries[5 * n_blocks];
    for (int32_t i = blockIdx.x; i < listed; i += gridDim.x)
        compact_block(source, lanes, starts, tail, lane_off, start_off, tail_off, blocks,
                      extra_starts, list[i], n_blocks, logical_numel, S, precomputed, scratch,
                      entry_offset, entry_start, entry_lane);
}

}  // namespace
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
    const size_t lds = 3 * static_cast<size_t>(std::min<int64_t>(n_blocks, kPrefixChunk))
        * sizeof(int32_t);
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(prefix_allocate_kernel),
                                           lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(prefix_allocate_kernel, dim3(1), dim3(kLanes), lds, stream, summaries,
                       counts, descriptor, buffer_meta, blocks, static_cast<int32_t>(n_blocks),
                       buffered, max_free_regions);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_compact_extra(const void *source, uint8_t *lanes, uint8_t *starts,
                                     uint8_t *tail, const int32_t *descriptor,
                                     const int32_t *count, const int32_t *blocks, int64_t base,
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
    const uint32_t grid = static_cast<uint32_t>(n_blocks < kCompactGrid ? n_blocks : kCompactGrid);
    hipLaunchKernelGGL(compact_extra_kernel, dim3(grid), dim3(kLanes), 0, stream, source, lanes, starts, tail, descriptor, count, blocks, base,
                       extra_starts, summaries, n_blocks, logical_numel, g.steps, precomputed,
                       buffered);
    return static_cast<int32_t>(hipGetLastError());
}
