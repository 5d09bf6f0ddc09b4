// TensorBuffer allocator kernels: reset, allocate, free (one workgroup each).
//
// Launch-for-launch replacements of LCT/kernels/tensor_buffer.py:18-34
// (_reset_kernel), :37-91 (_allocate_kernel) and :182-192
// (_free_storage_kernel), plus several frees in one launch; the algorithms
// live in allocator.h.
#include <atomic>

#include "allocator.h"

namespace lct {
namespace {

__global__ __launch_bounds__(kLanes) void buffer_reset_kernel(int32_t *__restrict__ meta,
                                                              int32_t regions,
                                                              int32_t capacity) {
    const AllocatorMeta m(meta, regions, 0);
    for (int32_t i = threadIdx.x; i < regions; i += kLanes) {
        m.starts[i] = 0;
        m.sizes[i] = i == 0 ? capacity : 0;
    }
    if (threadIdx.x == 0) {
        *m.count = 1;
        // The next free version (the reference stores 0): a free-list snapshot
        // taken before the reset cannot validate against the lock afterwards.
        const int32_t version = coherent_load(m.lock);
        __hip_atomic_store(m.lock, (version | 1) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *m.generation = *m.generation + 1;
        *m.failures = 0;
    }
}

__global__ __launch_bounds__(kLanes) void buffer_allocate_kernel(
    int32_t *__restrict__ meta, int32_t regions, const int32_t *__restrict__ requested,
    const int32_t *__restrict__ item_count, int32_t item_bytes,
    int32_t *__restrict__ descriptor, int32_t lock_spins) {
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t flag;
    int32_t request = requested[0];
    if (item_bytes) request += item_count[0] * item_bytes;
    allocator_allocate(AllocatorMeta(meta, regions, lock_spins), request, descriptor, scratch,
                       &flag);
}

__global__ __launch_bounds__(kLanes) void buffer_free_kernel(int32_t *__restrict__ meta,
                                                             int32_t regions,
                                                             int32_t *__restrict__ descriptor,
                                                             int32_t *__restrict__ status_out,
                                                             int32_t lock_spins) {
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t flag;
    const int32_t status = allocator_free(AllocatorMeta(meta, regions, lock_spins), descriptor,
                                          scratch, &flag);
    if (threadIdx.x == 0) status_out[0] = status;
}

// Descriptors of one lct_buffer_free_batch launch (kernel arguments).
struct FreeBatch {
    int32_t count;
    int32_t *descriptor[LCT_MAX_FREE_BATCH];
};

// The frees of lct_buffer_free in order under one hold of the lock: each
// allocator_free_locked ends with a barrier after its metadata writes, and the
// workgroup shares one vector L1, so the next free reads the updated list.
__global__ __launch_bounds__(kLanes) void buffer_free_batch_kernel(int32_t *__restrict__ meta,
                                                                   int32_t regions,
                                                                   FreeBatch batch,
                                                                   int32_t *__restrict__ status_out,
                                                                   int32_t lock_spins) {
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t flag;
    const AllocatorMeta m(meta, regions, lock_spins);
    const int32_t held = allocator_lock(m.lock, &flag, m.spins);
    for (int32_t j = 0; j < batch.count; ++j) {
        const int32_t status =
            held < 0 ? kStatusLock : allocator_free_locked(m, batch.descriptor[j], scratch);
        if (threadIdx.x == 0 && status_out != nullptr) status_out[j] = status;
    }
    if (held >= 0) allocator_unlock(m.lock, held);
}

bool regions_ok(int32_t r) { return r > 0 && r <= 4096 && (r & (r - 1)) == 0; }

}  // namespace

// Bounds of the device-side waits (in polls), passed to every kernel that waits.
std::atomic<int32_t> g_lock_spins{kLockSpinLimit};
std::atomic<int32_t> g_ready_polls{kReadyPollLimit};

int32_t lock_spins() { return g_lock_spins.load(std::memory_order_relaxed); }
int32_t ready_polls() { return g_ready_polls.load(std::memory_order_relaxed); }

}  // namespace lct

using namespace lct;

extern "C" int32_t lct_buffer_reset(int32_t *meta, int32_t max_free_regions,
                                    int32_t capacity_bytes, hipStream_t stream) {
    if (!meta) return LCT_E_NULL;
    if (!regions_ok(max_free_regions) || capacity_bytes < 0) return LCT_E_ARG;
    hipLaunchKernelGGL(buffer_reset_kernel, dim3(1), dim3(kLanes), 0, stream, meta,
                       max_free_regions, capacity_bytes);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_buffer_allocate(int32_t *meta, int32_t max_free_regions,
                                       const int32_t *requested, const int32_t *item_count,
                                       int32_t item_bytes, int32_t *descriptor,
                                       hipStream_t stream) {
    if (!meta || !requested || !descriptor) return LCT_E_NULL;
    if (item_bytes != 0 && !item_count) return LCT_E_NULL;
    if (!regions_ok(max_free_regions) || item_bytes < 0) return LCT_E_ARG;
    hipLaunchKernelGGL(buffer_allocate_kernel, dim3(1), dim3(kLanes), 0, stream, meta,
                       max_free_regions, requested, item_count, item_bytes, descriptor,
                       lock_spins());
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_buffer_free(int32_t *meta, int32_t max_free_regions,
                                   int32_t *descriptor, int32_t *status_out,
                                   hipStream_t stream) {
    if (!meta || !descriptor || !status_out) return LCT_E_NULL;
    if (!regions_ok(max_free_regions)) return LCT_E_ARG;
    hipLaunchKernelGGL(buffer_free_kernel, dim3(1), dim3(kLanes), 0, stream, meta,
                       max_free_regions, descriptor, status_out, lock_spins());
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_buffer_free_batch(int32_t *meta, int32_t max_free_regions,
                                         int32_t *const *descriptors, int32_t count,
                                         int32_t *status_out, hipStream_t stream) {
    if (!meta || !descriptors) return LCT_E_NULL;
    if (!regions_ok(max_free_regions) || count < 1 || count > LCT_MAX_FREE_BATCH)
        return LCT_E_ARG;
    FreeBatch batch{};
    batch.count = count;
    for (int32_t j = 0; j < count; ++j) {
        if (!descriptors[j]) return LCT_E_NULL;
        batch.descriptor[j] = descriptors[j];
    }
    hipLaunchKernelGGL(buffer_free_batch_kernel, dim3(1), dim3(kLanes), 0, stream, meta,
                       max_free_regions, batch, status_out, lock_spins());
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_set_wait_limits(int32_t lock_polls, int32_t ready_wait_polls) {
    if (lock_polls < 0 || ready_wait_polls < 0) return LCT_E_ARG;
    g_lock_spins.store(lock_polls == 0 ? kLockSpinLimit : lock_polls,
                       std::memory_order_relaxed);
    g_ready_polls.store(ready_wait_polls == 0 ? kReadyPollLimit : ready_wait_polls,
                        std::memory_order_relaxed);
    return LCT_OK;
}

extern "C" const char *lct_version(void) { return "lct-hip-gfx950 0.1"; }

extern "C" const char *lct_error_string(int32_t code) {
    switch (code) {
        case LCT_OK: return "ok";
        case LCT_E_NULL: return "a required pointer is NULL";
        case LCT_E_GEOMETRY: return "unsupported stream geometry";
        case LCT_E_SIZE: return "sizes inconsistent or out of range";
        case LCT_E_ARG: return "argument out of range";
        case LCT_E_SCRATCH:
            return "tensor larger than the no-allocation entry point serves (8192 codec blocks)";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "unknown error";
}
