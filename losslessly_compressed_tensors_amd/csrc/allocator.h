// Device-resident first-fit free-list allocator (one workgroup of 256 threads).
//
// Follows LCT/kernels/tensor_buffer.py:7-192.  Metadata is int32
// free_starts[R] | free_sizes[R] | free_count | lock | generation, with the free
// regions sorted by start and coalesced.  Allocation takes the first region
// that fits the 16-byte-aligned request; free re-inserts a region, merging it
// with its neighbours, and rejects stale or already-freed descriptors.
//
// The lock is taken with an agent-scope compare-and-swap by one thread; unlike
// the reference's unbounded spin, the wait is bounded, and an allocator call
// that cannot take the lock reports status LCT_STATUS_LOCK and changes nothing.
#pragma once

#include "lct_device.h"

namespace lct {

constexpr int32_t kAlignment = 16;
constexpr int32_t kStatusOk = 0;
constexpr int32_t kStatusNoFit = 1;
constexpr int32_t kStatusEmpty = 2;
constexpr int32_t kStatusFreeListFull = 3;
constexpr int32_t kStatusInvalid = 4;
constexpr int32_t kStatusFreed = 5;
constexpr int32_t kStatusLock = 6;
constexpr int kLockSpinLimit = 1 << 20;

struct AllocatorMeta {
    int32_t *starts;
    int32_t *sizes;
    int32_t *count;
    int32_t *lock;
    int32_t *generation;
    int32_t regions;

    __device__ explicit AllocatorMeta(int32_t *meta, int32_t r)
        : starts(meta), sizes(meta + r), count(meta + 2 * r), lock(meta + 2 * r + 1),
          generation(meta + 2 * r + 2), regions(r) {}
};

// Returns true in every thread if the lock was taken.  Contains barriers.
__device__ __forceinline__ bool allocator_lock(int32_t *lock, int32_t *flag) {
    if (threadIdx.x == 0) {
        int32_t got = 0;
        for (int i = 0; i < kLockSpinLimit; ++i) {
            int32_t expected = 0;
            if (__hip_atomic_compare_exchange_strong(lock, &expected, 1, __ATOMIC_ACQUIRE,
                                                     __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)) {
                got = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        *flag = got;
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return *flag != 0;
}

// Publishes every thread's metadata writes, then releases.  Contains barriers.
__device__ __forceinline__ void allocator_unlock(int32_t *lock) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(lock, 0, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide minimum; scratch holds kWavesPerBlock ints.  Contains barriers.
__device__ __forceinline__ int32_t block_min(int32_t v, int32_t *scratch) {
    v = wave_min(v);
    if (wave_lane() == 0) scratch[threadIdx.x / kWave] = v;
    __syncthreads();
    int32_t m = scratch[0];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) m = min(m, scratch[w]);
    __syncthreads();
    return m;
}

// Shift entries [from, to) of both arrays by `delta` (+1 or -1).  All reads
// finish before any write.  Contains barriers.
__device__ __forceinline__ void allocator_shift(const AllocatorMeta &m, int32_t from,
                                                int32_t to, int32_t delta) {
    constexpr int kPerThread = 16;   // up to 4096 regions
    int32_t s[kPerThread], z[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int32_t i = from + static_cast<int32_t>(threadIdx.x) + j * kLanes;
        if (i < to) {
            s[j] = m.starts[i];
            z[j] = m.sizes[i];
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int32_t i = from + static_cast<int32_t>(threadIdx.x) + j * kLanes;
        if (i < to) {
            m.starts[i + delta] = s[j];
            m.sizes[i + delta] = z[j];
        }
    }
    __syncthreads();
}

// tensor_buffer.py:37-91.  `request` already includes item bytes.
__device__ __forceinline__ void allocator_allocate(const AllocatorMeta &m, int32_t request,
                                                   int32_t *descriptor, int32_t *scratch,
                                                   int32_t *flag) {
    if (!allocator_lock(m.lock, flag)) {
        if (threadIdx.x == 0) {
            descriptor[0] = -1;
            descriptor[1] = 0;
            descriptor[2] = kStatusLock;
            descriptor[3] = -1;
        }
        return;
    }
    const int32_t generation = *m.generation;
    const int32_t count = *m.count;
    const int32_t size = ((request + kAlignment - 1) / kAlignment) * kAlignment;
    int32_t candidate = m.regions;
    for (int32_t i = threadIdx.x; i < count; i += kLanes)
        if (m.sizes[i] >= size) candidate = min(candidate, i);
    const int32_t slot = block_min(candidate, scratch);
    const bool success = request > 0 && slot < count;
    int32_t start = 0, region = 0;
    if (success) {
        start = m.starts[slot];
        region = m.sizes[slot];
    }
    __syncthreads();
    if (success && region == size) {
        allocator_shift(m, slot + 1, count, -1);
        if (threadIdx.x == 0) *m.count = count - 1;
    } else if (success && threadIdx.x == 0) {
        m.starts[slot] = start + size;
        m.sizes[slot] = region - size;
    }
    if (threadIdx.x == 0) {
        descriptor[0] = success ? start : -1;
        descriptor[1] = success ? size : 0;
        descriptor[2] = request <= 0 ? kStatusEmpty : (success ? kStatusOk : kStatusNoFit);
        descriptor[3] = generation;
    }
    allocator_unlock(m.lock);
}

// tensor_buffer.py:94-179.  Returns the status in every thread.
__device__ __forceinline__ int32_t allocator_free(const AllocatorMeta &m, int32_t *descriptor,
                                                  int32_t *scratch, int32_t *flag) {
    if (!allocator_lock(m.lock, flag)) return kStatusLock;
    const int32_t offset = descriptor[0];
    const int32_t size = descriptor[1];
    const int32_t status = descriptor[2];
    const int32_t generation = descriptor[3];
    const int32_t count = *m.count;
    const bool valid = status == kStatusOk && generation == *m.generation && offset >= 0
        && size > 0;
    int32_t result = kStatusInvalid;
    if (valid) {
        int32_t below = 0;
        for (int32_t i = threadIdx.x; i < count; i += kLanes) below += m.starts[i] < offset ? 1 : 0;
        const int32_t insert = block_sum(below, scratch);
        const bool has_prev = insert > 0, has_next = insert < count;
        const int32_t prev_start = has_prev ? m.starts[insert - 1] : 0;
        const int32_t prev_size = has_prev ? m.sizes[insert - 1] : 0;
        const int32_t next_start = has_next ? m.starts[insert] : 0;
        const int32_t next_size = has_next ? m.sizes[insert] : 0;
        const bool merge_prev = has_prev && prev_start + prev_size == offset;
        const bool merge_next = has_next && offset + size == next_start;
        __syncthreads();
        result = kStatusOk;
        if (merge_prev && merge_next) {
            if (threadIdx.x == 0) m.sizes[insert - 1] = prev_size + size + next_size;
            allocator_shift(m, insert + 1, count, -1);
            if (threadIdx.x == 0) *m.count = count - 1;
        } else if (merge_prev) {
            if (threadIdx.x == 0) m.sizes[insert - 1] = prev_size + size;
        } else if (merge_next) {
            if (threadIdx.x == 0) {
                m.starts[insert] = offset;
                m.sizes[insert] = next_size + size;
            }
        } else if (count < m.regions) {
            allocator_shift(m, insert, count, +1);
            if (threadIdx.x == 0) {
                m.starts[insert] = offset;
                m.sizes[insert] = size;
                *m.count = count + 1;
            }
        } else {
            result = kStatusFreeListFull;
        }
        if (result == kStatusOk && threadIdx.x == 0) descriptor[2] = kStatusFreed;
    }
    allocator_unlock(m.lock);
    return result;
}

}  // namespace lct
