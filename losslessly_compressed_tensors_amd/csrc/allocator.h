// Device-resident first-fit free-list allocator (one workgroup of 256 threads).
//
// Follows LCT/kernels/tensor_buffer.py:7-192.  Metadata is int32
// free_starts[R] | free_sizes[R] | free_count | lock | generation, with the free
// regions sorted by start and coalesced.  Allocation takes the first region
// that fits the 16-byte-aligned request; free re-inserts a region, merging it
// with its neighbours, and rejects stale or already-freed descriptors.
//
// The lock word is versioned: even = free, odd = held; the holder that took
// it at value v releases it with v + 2 (the reference's lock is 0/1,
// LCT/kernels/tensor_buffer.py:7-15).  It is taken with an agent-scope
// compare-and-swap by one thread; unlike the reference's unbounded spin, the
// wait is bounded, and an allocator call that cannot take the lock reports
// status LCT_STATUS_LOCK and changes nothing.  The version lets a caller read
// the free list before it owns the lock: a snapshot read after the lock was
// seen free at v is exactly current if the compare-and-swap v -> v + 1 then
// succeeds (no holder came and went in between).
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
// A codec reservation that succeeded but whose compaction did not complete
// (a compacting workgroup stopped waiting for the reservation and wrote none
// of its blocks' entries or tails).  The region is held like a status-0 one
// and is freed the same way; decoding treats the tensor as failed.
constexpr int32_t kStatusIncomplete = 7;
// Bounded waits: polls of the arena lock, and of lct_allocate_compact's ready
// word.  The host passes the limits to every kernel that waits
// (lct_set_wait_limits lowers them for tests of the give-up paths).
constexpr int kLockSpinLimit = 1 << 20;
constexpr int kReadyPollLimit = 1 << 22;

// The limits in force (host side; tensor_buffer.hip).
int32_t lock_spins();
int32_t ready_polls();

// Bits of the buffer's failure word (int32 at metadata index 2R + 3, in the
// padding after the generation): set, and kept until the next reset, when a
// compressed tensor's overflow reservation fails (no fit, lock not taken) or
// its compaction does not complete.  The host reads it at its sync points.
constexpr int32_t kFailNoFit = 1;
constexpr int32_t kFailLock = 2;
constexpr int32_t kFailIncomplete = 4;

// Whether a descriptor holds a live region (freeable).
__device__ __forceinline__ bool holds_region(int32_t status) {
    return status == kStatusOk || status == kStatusIncomplete;
}

struct AllocatorMeta {
    int32_t *starts;
    int32_t *sizes;
    int32_t *count;
    int32_t *lock;
    int32_t *generation;
    int32_t *failures;
    int32_t regions;
    int32_t spins;   // bound of the lock wait, in polls

    __device__ explicit AllocatorMeta(int32_t *meta, int32_t r, int32_t lock_spins)
        : starts(meta), sizes(meta + r), count(meta + 2 * r), lock(meta + 2 * r + 1),
          generation(meta + 2 * r + 2), failures(meta + 2 * r + 3), regions(r),
          spins(lock_spins) {}
};

// Records a codec reservation's failure (status 1 or 6 for a non-empty
// request, or an incomplete compaction) in the buffer's failure word.
__device__ __forceinline__ void record_failure(const AllocatorMeta &m, int32_t bits) {
    __hip_atomic_fetch_or(m.failures, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int32_t failure_bits(int32_t status, int32_t request) {
    if (request <= 0) return 0;
    return status == kStatusNoFit ? kFailNoFit : status == kStatusLock ? kFailLock : 0;
}

// A value another workgroup wrote (or may be writing) in this launch: an
// agent-scope load reads the coherent copy, where a plain load could hit a
// stale line of this XCD's L2.
__device__ __forceinline__ int32_t coherent_load(const int32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0's bounded wait for the lock; returns the version taken (even), or
// -1.  `seen` is a value of the lock word already read, or -1.
__device__ __forceinline__ int32_t take_lock_thread0(int32_t *lock, int32_t seen,
                                                     int32_t spins) {
    int32_t v = seen;
    for (int i = 0; i < spins; ++i) {
        if (v >= 0 && (v & 1) == 0) {
            int32_t expected = v;
            if (__hip_atomic_compare_exchange_strong(lock, &expected, v + 1, __ATOMIC_ACQUIRE,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                return v;
            v = expected;
            if ((v & 1) == 0) continue;
        }
        __builtin_amdgcn_s_sleep(2);
        v = coherent_load(lock);
    }
    return -1;
}

// Returns the version taken (>= 0) in every thread, or -1 if the lock was not
// taken.  flag: one LDS int.  Contains barriers.
__device__ __forceinline__ int32_t allocator_lock(int32_t *lock, int32_t *flag, int32_t spins) {
    if (threadIdx.x == 0) *flag = take_lock_thread0(lock, coherent_load(lock), spins);
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return *flag;
}

// Publishes every thread's metadata writes, then releases the version `held`
// took.  Contains barriers.
__device__ __forceinline__ void allocator_unlock(int32_t *lock, int32_t held) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(lock, held + 2, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
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
    int32_t held;   // version the lock was taken at
    bool locked;
};

__device__ __forceinline__ void allocator_begin(const AllocatorMeta &m, AllocatorSnapshot &snap,
                                                int32_t *flag) {
    snap.held = allocator_lock(m.lock, flag, m.spins);
    snap.locked = snap.held >= 0;
    snap.generation = 0;
    snap.count = 0;
    if (!snap.locked) return;
    snap.generation = *m.generation;
    snap.count = *m.count;
    load_regions(m, snap.r);
}

// tensor_buffer.py:37-91.  `request` already includes item bytes.  A codec
// reservation (`codec`) records its failure in the buffer's failure word.
__device__ __forceinline__ void allocator_finish(const AllocatorMeta &m,
                                                 const AllocatorSnapshot &snap, int32_t request,
                                                 int32_t *descriptor, int32_t *scratch,
                                                 bool codec = false) {
    __shared__ int32_t shared2[2];
    if (!snap.locked) {
        if (threadIdx.x == 0) {
            descriptor[0] = -1;
            descriptor[1] = 0;
            descriptor[2] = kStatusLock;
            descriptor[3] = -1;
            if (codec && request > 0) record_failure(m, kFailLock);
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
        if (codec && request > 0 && !success) record_failure(m, kFailNoFit);
    }
    allocator_unlock(m.lock, snap.held);
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
    const bool valid = holds_region(status) && generation == current_generation && offset >= 0
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
    const int32_t held = allocator_lock(m.lock, flag, m.spins);
    if (held < 0) return kStatusLock;
    const int32_t result = allocator_free_locked(m, descriptor, scratch);
    allocator_unlock(m.lock, held);
    return result;
}


// ---- The free list on an LDS copy (one workgroup holding the lock): frees
// and a first-fit reservation with no memory round trip, then one write-back.
// The algorithms are those of allocator_free_locked and allocator_finish.
struct LdsFreeList {
    int32_t *start;   // LDS int32[regions]
    int32_t *size;    // LDS int32[regions]
    int32_t regions;
    int32_t count;        // uniform in every thread
    int32_t generation;   // uniform in every thread
};

// Entries [from, to) move by delta (+1 or -1), 256 at a time: a +1 shift
// walks the chunks from the last, a -1 shift from the first, so no entry is
// overwritten before it is read, and a thread holds one entry at a time (the
// LDS copy serves kernels whose registers the encoder's path bounds).
// Contains barriers (none when the range is empty; from and to are uniform).
__device__ __forceinline__ void lds_shift(LdsFreeList &f, int32_t from, int32_t to,
                                          int32_t delta) {
    const int32_t chunks = to > from ? (to - from + kLanes - 1) / kLanes : 0;
    for (int32_t k = 0; k < chunks; ++k) {
        const int32_t chunk = delta > 0 ? chunks - 1 - k : k;
        const int32_t i = from + chunk * kLanes + static_cast<int32_t>(threadIdx.x);
        const bool mine = i < to;
        int32_t start = 0, size = 0;
        if (mine) {
            start = f.start[i];
            size = f.size[i];
        }
        __syncthreads();
        if (mine) {
            f.start[i + delta] = start;
            f.size[i + delta] = size;
        }
        __syncthreads();
    }
}

// tensor_buffer.py:94-179 on the LDS list for descriptor values d
// {offset, size, status, generation}; returns the status in every thread.
// Contains barriers.
__device__ __forceinline__ int32_t lds_free(LdsFreeList &f, const int32_t (&d)[4],
                                            int32_t *scratch) {
    const int32_t offset = d[0], size = d[1];
    if (!(holds_region(d[2]) && d[3] == f.generation && offset >= 0 && size > 0))
        return kStatusInvalid;
    const int32_t count = f.count;
    int32_t below = 0;
#pragma unroll
    for (int k = 0; k < kRegionsPerThread; ++k) {
        const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kLanes;
        below += (i < count && f.start[i] < offset) ? 1 : 0;
    }
    const int32_t insert = block_sum(below, scratch);
    const bool has_prev = insert > 0, has_next = insert < count;
    const int32_t prev_start = has_prev ? f.start[insert - 1] : 0;
    const int32_t prev_size = has_prev ? f.size[insert - 1] : 0;
    const int32_t next_start = has_next ? f.start[insert] : 0;
    const int32_t next_size = has_next ? f.size[insert] : 0;
    const bool merge_prev = has_prev && prev_start + prev_size == offset;
    const bool merge_next = has_next && offset + size == next_start;
    __syncthreads();   // every thread has read its neighbours before any write
    if (merge_prev && merge_next) {
        if (threadIdx.x == 0) f.size[insert - 1] = prev_size + size + next_size;
        __syncthreads();
        lds_shift(f, insert + 1, count, -1);
        f.count = count - 1;
    } else if (merge_prev) {
        if (threadIdx.x == 0) f.size[insert - 1] = prev_size + size;
        __syncthreads();
    } else if (merge_next) {
        if (threadIdx.x == 0) {
            f.start[insert] = offset;
            f.size[insert] = next_size + size;
        }
        __syncthreads();
    } else if (count < f.regions) {
        lds_shift(f, insert, count, +1);
        if (threadIdx.x == 0) {
            f.start[insert] = offset;
            f.size[insert] = size;
        }
        __syncthreads();
        f.count = count + 1;
    } else {
        return kStatusFreeListFull;
    }
    return kStatusOk;
}

// tensor_buffer.py:37-91 on the LDS list: the first region that holds the
// 16-byte-aligned request.  Writes {offset, size, status} (uniform) to out.
// Contains barriers.
__device__ __forceinline__ void lds_reserve(LdsFreeList &f, int32_t request, int32_t *scratch,
                                            int32_t (&out)[3]) {
    const int32_t count = f.count;
    const int32_t size = ((request + kAlignment - 1) / kAlignment) * kAlignment;
    int32_t candidate = f.regions;
#pragma unroll
    for (int k = kRegionsPerThread - 1; k >= 0; --k) {
        const int32_t i = static_cast<int32_t>(threadIdx.x) + k * kLanes;
        if (i < count && f.size[i] >= size) candidate = i;
    }
    const int32_t slot = block_min(candidate, scratch);
    const bool success = request > 0 && slot < count;
    int32_t start = 0;
    if (success) {
        start = f.start[slot];
        const int32_t region = f.size[slot];
        __syncthreads();
        if (region == size) {
            lds_shift(f, slot + 1, count, -1);
            f.count = count - 1;
        } else {
            if (threadIdx.x == 0) {
                f.start[slot] = start + size;
                f.size[slot] = region - size;
            }
            __syncthreads();
        }
    }
    out[0] = success ? start : -1;
    out[1] = success ? size : 0;
    out[2] = request <= 0 ? kStatusEmpty : (success ? kStatusOk : kStatusNoFit);
}

// Entries [0, count) and the count back to the buffer's metadata.
__device__ __forceinline__ void lds_write_back(const LdsFreeList &f, const AllocatorMeta &m) {
    for (int32_t i = threadIdx.x; i < f.count; i += kLanes) {
        m.starts[i] = f.start[i];
        m.sizes[i] = f.size[i];
    }
    if (threadIdx.x == 0) *m.count = f.count;
}

// The same with agent-scope atomic stores, which are coherent across the XCDs
// once complete: the next lock holder reads them with coherent loads.
__device__ __forceinline__ void lds_write_back_coherent(const LdsFreeList &f,
                                                        const AllocatorMeta &m) {
    for (int32_t i = threadIdx.x; i < f.count; i += kLanes) {
        __hip_atomic_store(m.starts + i, f.start[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(m.sizes + i, f.size[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(m.count, f.count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace lct
