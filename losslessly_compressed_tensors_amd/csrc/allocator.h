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

// The free list held in registers: thread t owns entries t + k*256.
constexpr int kRegionsPerThread = 16;   // up to 4096 regions

struct RegionRegs {
    int32_t start[kRegionsPerThread];
    int32_t size[kRegionsPerThread];
};

// Load every entry below `regions` (the caller masks by the live count).
__device__ __forceinline__ void load_regions(const AllocatorMeta &m, RegionRegs &r) {
#pragma unroll
    for (int k = 0; k < kRegionsPerThread; ++k) {
        const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kLanes;
        r.start[k] = i < m.regions ? m.starts[i] : 0;
        r.size[k] = i < m.regions ? m.sizes[i] : 0;
    }
}

// Write entries i in [from, to) to index i + delta.
__device__ __forceinline__ void shift_regions(const AllocatorMeta &m, const RegionRegs &r,
                                              int32_t from, int32_t to, int32_t delta) {
#pragma unroll
    for (int k = 0; k < kRegionsPerThread; ++k) {
        const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kLanes;
        if (i >= from && i < to) {
            m.starts[i + delta] = r.start[k];
            m.sizes[i + delta] = r.size[k];
        }
    }
}

// Value of entry `index` from whichever thread holds it; contains barriers.
__device__ __forceinline__ void fetch_region(const RegionRegs &r, int32_t index, int32_t *shared2,
                                             int32_t &start, int32_t &size) {
#pragma unroll
    for (int k = 0; k < kRegionsPerThread; ++k) {
        if (static_cast<int32_t>(threadIdx.x) + k * kLanes == index) {
            shared2[0] = r.start[k];
            shared2[1] = r.size[k];
        }
    }
    __syncthreads();
    start = shared2[0];
    size = shared2[1];
    __syncthreads();
}

// An allocation in two halves, so a caller can take the lock and fetch the
// free list before it knows the request size (the prefix scan overlaps this
// latency with its own work).  allocator_begin returns whether the lock was
// taken; allocator_finish must follow in every case.  Both contain barriers.
struct AllocatorSnapshot {
    RegionRegs r;
    int32_t generation;
    int32_t count;
    bool locked;
};

__device__ __forceinline__ void allocator_begin(const AllocatorMeta &m, AllocatorSnapshot &snap,
                                                int32_t *flag) {
    snap.locked = allocator_lock(m.lock, flag);
    snap.generation = 0;
    snap.count = 0;
    if (!snap.locked) return;
    snap.generation = *m.generation;
    snap.count = *m.count;
    load_regions(m, snap.r);
}

// tensor_buffer.py:37-91.  `request` already includes item bytes.
__device__ __forceinline__ void allocator_finish(const AllocatorMeta &m,
                                                 const AllocatorSnapshot &snap, int32_t request,
                                                 int32_t *descriptor, int32_t *scratch) {
    __shared__ int32_t shared2[2];
    if (!snap.locked) {
        if (threadIdx.x == 0) {
            descriptor[0] = -1;
            descriptor[1] = 0;
            descriptor[2] = kStatusLock;
            descriptor[3] = -1;
        }
        return;
    }
    const RegionRegs &r = snap.r;
    const int32_t count = snap.count;
    const int32_t size = ((request + kAlignment - 1) / kAlignment) * kAlignment;
    int32_t candidate = m.regions;
#pragma unroll
    for (int k = kRegionsPerThread - 1; k >= 0; --k) {
        const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kLanes;
        if (i < count && r.size[k] >= size) candidate = i;
    }
    const int32_t slot = block_min(candidate, scratch);
    const bool success = request > 0 && slot < count;
    int32_t start = 0, region = 0;
    if (success) fetch_region(r, slot, shared2, start, region);
    if (success && region == size) {
        shift_regions(m, r, slot + 1, count, -1);
        if (threadIdx.x == 0) *m.count = count - 1;
    } else if (success && threadIdx.x == 0) {
        m.starts[slot] = start + size;
        m.sizes[slot] = region - size;
    }
    if (threadIdx.x == 0) {
        descriptor[0] = success ? start : -1;
        descriptor[1] = success ? size : 0;
        descriptor[2] = request <= 0 ? kStatusEmpty : (success ? kStatusOk : kStatusNoFit);
        descriptor[3] = snap.generation;
    }
    allocator_unlock(m.lock);
}

__device__ __forceinline__ void allocator_allocate(const AllocatorMeta &m, int32_t request,
                                                   int32_t *descriptor, int32_t *scratch,
                                                   int32_t *flag) {
    AllocatorSnapshot snap;
    allocator_begin(m, snap, flag);
    allocator_finish(m, snap, request, descriptor, scratch);
}

// tensor_buffer.py:94-179 with the lock already held.  Returns the status in
// every thread.  Contains barriers; the free list in memory is updated (and
// visible to the whole workgroup) when it returns.
__device__ __forceinline__ int32_t allocator_free_locked(const AllocatorMeta &m,
                                                         int32_t *descriptor, int32_t *scratch) {
    __shared__ int32_t shared2[2];
    const int32_t offset = descriptor[0];
    const int32_t size = descriptor[1];
    const int32_t status = descriptor[2];
    const int32_t generation = descriptor[3];
    const int32_t count = *m.count;
    const int32_t current_generation = *m.generation;
    RegionRegs r;
    load_regions(m, r);
    const bool valid = status == kStatusOk && generation == current_generation && offset >= 0
        && size > 0;
    int32_t result = kStatusInvalid;
    if (valid) {
        int32_t below = 0;
#pragma unroll
        for (int k = 0; k < kRegionsPerThread; ++k) {
            const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kLanes;
            below += (i < count && r.start[k] < offset) ? 1 : 0;
        }
        const int32_t insert = block_sum(below, scratch);
        const bool has_prev = insert > 0, has_next = insert < count;
        int32_t prev_start = 0, prev_size = 0, next_start = 0, next_size = 0;
        fetch_region(r, has_prev ? insert - 1 : -1, shared2, prev_start, prev_size);
        if (!has_prev) prev_start = prev_size = 0;
        fetch_region(r, has_next ? insert : -1, shared2, next_start, next_size);
        if (!has_next) next_start = next_size = 0;
        const bool merge_prev = has_prev && prev_start + prev_size == offset;
        const bool merge_next = has_next && offset + size == next_start;
        result = kStatusOk;
        if (merge_prev && merge_next) {
            if (threadIdx.x == 0) {
                m.sizes[insert - 1] = prev_size + size + next_size;
                *m.count = count - 1;
            }
            shift_regions(m, r, insert + 1, count, -1);
        } else if (merge_prev) {
            if (threadIdx.x == 0) m.sizes[insert - 1] = prev_size + size;
        } else if (merge_next) {
            if (threadIdx.x == 0) {
                m.starts[insert] = offset;
                m.sizes[insert] = next_size + size;
            }
        } else if (count < m.regions) {
            shift_regions(m, r, insert, count, +1);
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
    __syncthreads();   // metadata writes visible to the next reader in the workgroup
    return result;
}

// tensor_buffer.py:94-179.  Returns the status in every thread.
__device__ __forceinline__ int32_t allocator_free(const AllocatorMeta &m, int32_t *descriptor,
                                                  int32_t *scratch, int32_t *flag) {
    if (!allocator_lock(m.lock, flag)) return kStatusLock;
    const int32_t result = allocator_free_locked(m, descriptor, scratch);
    allocator_unlock(m.lock);
    return result;
}

// allocator_begin that first returns the caller's deferred frees, in order,
// under the same lock (each exactly as allocator_free would, its status
// discarded), so the allocation that follows sees the free list those frees
// leave.  Contains barriers.
__device__ __forceinline__ void allocator_begin_after_frees(const AllocatorMeta &m,
                                                            AllocatorSnapshot &snap,
                                                            const lct_pending_frees &frees,
                                                            int32_t *flag, int32_t *scratch) {
    snap.locked = allocator_lock(m.lock, flag);
    snap.generation = 0;
    snap.count = 0;
    if (!snap.locked) return;
    for (int i = 0; i < frees.count; ++i) allocator_free_locked(m, frees.descriptor[i], scratch);
    snap.generation = *m.generation;
    snap.count = *m.count;
    load_regions(m, snap.r);
}

}  // namespace lct
