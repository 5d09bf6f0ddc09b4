// One codec block's overflow tail, walked one byte per thread.
//
// The compact overflow list (LCT/kernels/generic/compaction.py:3-16) stores a
// block's overflowing lanes in ascending order at entries [first,
// first+count), with their tail bytes (steps start..S-1) concatenated from
// byte_base.  The restore kernels (compaction.py:238-306,
// LCT/kernels/generic/pointwise.py:265-340) visit every tail byte; here the
// block's entries are staged in LDS with each entry's first byte offset, and
// tail byte i belongs to the last entry whose offset is <= i (a binary search
// over at most 256 entries), so each thread handles independent bytes and the
// tail reads are contiguous.
#pragma once

#include "lct_device.h"

namespace lct {

struct TailWalk {
    int32_t count;        // the block's entries; 0 = nothing to walk
    int32_t bytes;        // the block's tail bytes
    const uint8_t *tail;  // the block's first tail byte
};

// LDS arrays of the staged entries (kLanes each) plus scan scratch.
struct TailEntries {
    int32_t offset[kLanes];
    int32_t start[kLanes];
    int32_t lane[kLanes];
    int32_t scratch[kWavesPerBlock];
};

// Stage block `block`'s entries.  Every thread of the workgroup must call it;
// the result is uniform across the workgroup.  A buffered tensor whose
// reservation failed (descriptor status != 0) has no tails.  Contains
// barriers, including one after the staging.
__device__ __forceinline__ TailWalk stage_block_entries(const lct_overflow &ov, int64_t block,
                                                        int64_t n_blocks, int S,
                                                        TailEntries &e) {
    TailWalk w{0, 0, nullptr};
    if (ov.descriptor != nullptr && ov.descriptor[2] != 0) return w;
    const int32_t count = ov.blocks[block];
    if (count <= 0) return w;
    int64_t lane_off = 0, start_off = 0, tail_base = ov.base;
    if (ov.descriptor != nullptr) {
        const int64_t arena = ov.descriptor[0];
        const int64_t total = ov.count[0];
        lane_off = arena;
        start_off = arena + total;
        tail_base = arena + 2 * total;
    }
    const int32_t first = ov.blocks[n_blocks + block];
    const int32_t byte_base = ov.blocks[2 * n_blocks + block];
    const int t = threadIdx.x;
    const bool valid = t < count;
    const int32_t start = valid ? static_cast<int32_t>(ov.starts[start_off + first + t]) : S;
    const int32_t lane = valid ? static_cast<int32_t>(ov.lanes[lane_off + first + t]) : 0;
    int32_t bytes;
    const int32_t local = block_exclusive_scan(valid ? S - start : 0, e.scratch, &bytes);
    if (valid) {
        e.offset[t] = local;
        e.start[t] = start;
        e.lane[t] = lane;
    }
    __syncthreads();
    w.count = count;
    w.bytes = bytes;
    w.tail = ov.tail + tail_base + byte_base;
    return w;
}

// Storage step and lane of the block's tail byte i.
__device__ __forceinline__ void tail_position(const TailWalk &w, const TailEntries &e, int32_t i,
                                              int32_t &step, int32_t &lane) {
    int32_t lo = 0, hi = w.count - 1;
    while (lo < hi) {
        const int32_t mid = (lo + hi + 1) >> 1;
        if (e.offset[mid] <= i) lo = mid;
        else hi = mid - 1;
    }
    step = e.start[lo] + (i - e.offset[lo]);
    lane = e.lane[lo];
}

// BF16 bits of a tail byte int8(e - 127) with its side byte
// (LCT/kernels/primitives.py:7-36, pack_bf16).
__device__ __forceinline__ uint32_t pack_tail(uint32_t tail_byte, uint32_t sm) {
    return (((tail_byte + 127u) & 255u) << 7) | (sm & 0x7Fu) | ((sm & 0x80u) << 8);
}

}  // namespace lct
