// Buffered compress with no device allocation, for callers that cannot call
// hipMalloc (code under HIP graph capture, tight serving loops, harnesses that
// forbid it).  It runs the public compress sequence of a shared TensorBuffer:
// lct_sample_center -> lct_encode_sampled -> lct_allocate_compact, with the
// working arrays those launches need (the sampler's partial sums, the
// per-block summaries and overflow-block list, the per-stream extra starts and
// the ready word) in one file-scope device array instead of caller- or
// library-allocated memory.  Outputs are the caller's, as for the sequence.
#include <mutex>

#include "lct_device.h"

namespace lct {
namespace {

// Largest tensor served: 8192 codec blocks (2^28 elements at B = 32768, 2^29
// at 65536), which bounds the array at about 2.2 MiB per GPU.
constexpr int64_t kNoAllocMaxBlocks = 8192;

constexpr size_t round_up_256(size_t bytes) { return (bytes + 255) / 256 * 256; }

// Layout of the array: the ready word, the partial sums (int32[2 * 64]: a
// kept-exponent sum and a count per 64-sample group), the summaries
// (int32[5 * nb + 1]) and the extra starts (uint8[nb * 256]), each at a
// 256-byte boundary and each sized for its largest use, so that no region's
// writes reach another's (the encoders read the partial sums while finished
// blocks store their summaries).
constexpr size_t kReadyBytes = round_up_256(sizeof(uint64_t));
constexpr size_t kPartialsBytes = round_up_256(2 * kControlPartials * sizeof(int32_t));
constexpr size_t kSummariesBytes = round_up_256((5 * kNoAllocMaxBlocks + 1) * sizeof(int32_t));
constexpr size_t kExtraBytes = round_up_256(kNoAllocMaxBlocks * kLanes);
constexpr size_t kReadyOffset = 0;
constexpr size_t kPartialsOffset = kReadyOffset + kReadyBytes;
constexpr size_t kSummariesOffset = kPartialsOffset + kPartialsBytes;
constexpr size_t kExtraOffset = kSummariesOffset + kSummariesBytes;
constexpr size_t kScratchBytes = kExtraOffset + kExtraBytes;

static_assert(kMaxSamples / kSampleGroup <= kControlPartials,
              "the sampler writes two int32 per group for at most kControlPartials groups");
static_assert(kPartialsOffset - kReadyOffset >= sizeof(uint64_t), "ready word");
static_assert(kSummariesOffset - kPartialsOffset >= 2 * kControlPartials * sizeof(int32_t),
              "partial sums");
static_assert(kExtraOffset - kSummariesOffset >= (5 * kNoAllocMaxBlocks + 1) * sizeof(int32_t),
              "summaries");
static_assert(kScratchBytes - kExtraOffset >= kNoAllocMaxBlocks * kLanes, "extra starts");
static_assert(kPartialsOffset % 256 == 0 && kSummariesOffset % 256 == 0
                  && kExtraOffset % 256 == 0,
              "regions start at 256-byte boundaries");

}  // namespace

// Held by every GPU the library runs on until the process ends.  In host code
// this name is a host-side stand-in: only the address hipGetSymbolAddress
// returns for the current device may be passed to kernels or copies.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

// The device address of each GPU's copy, looked up once per device with that
// device current.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
uint8_t *g_scratch[kMaxDevices] = {};

// The ready word is cleared at the start of every call (a fill kernel, so a
// captured graph clears it on every replay too), so one constant epoch serves
// every call: lct_allocate_compact needs only that the word differs from the
// epoch and from its complement when it starts.
constexpr uint64_t kEpoch = 1;

__global__ __launch_bounds__(64) void clear_ready_kernel(uint64_t *ready) {
    if (threadIdx.x == 0) ready[0] = 0;
}

int32_t device_scratch(uint8_t **out) {
    int device = 0;
    if (hipError_t e = hipGetDevice(&device)) return static_cast<int32_t>(e);
    if (device < 0 || device >= kMaxDevices) return LCT_E_ARG;
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (g_scratch[device] == nullptr) {
        void *address = nullptr;
        if (hipError_t e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)))
            return static_cast<int32_t>(e);
        if (address == nullptr) return static_cast<int32_t>(hipErrorInvalidSymbol);
        g_scratch[device] = static_cast<uint8_t *>(address);
    }
    *out = g_scratch[device];
    return LCT_OK;
}

}  // namespace
}  // namespace lct

using namespace lct;

extern "C" int32_t lct_compress_buffered_noalloc(
    const void *source, int64_t logical_numel, int64_t size, lct_geometry g,
    const int32_t *base_encode, const int32_t *base_decode, uint8_t *side, int32_t *encoded,
    int32_t *center_out, int32_t *shifted_decode_out, uint16_t *sample_values,
    int32_t *blocks, int32_t *counts, int32_t *descriptor, int32_t *buffer_meta,
    int32_t max_free_regions, uint8_t *arena, const lct_pending_frees *frees,
    hipStream_t stream) {
    // Every check of the three launches, before the first one.
    if (!source || !base_encode || !base_decode || !side || !encoded || !center_out
        || !shifted_decode_out || !blocks || !counts || !descriptor || !buffer_meta || !arena)
        return LCT_E_NULL;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (logical_numel <= 0 || size <= 0 || size % g.block_symbols != 0
        || logical_numel > size || logical_numel <= size - g.block_symbols)
        return LCT_E_SIZE;
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > kNoAllocMaxBlocks) return LCT_E_SCRATCH;
    if (((reinterpret_cast<uintptr_t>(encoded) | reinterpret_cast<uintptr_t>(source)
          | reinterpret_cast<uintptr_t>(side)) & 15) != 0)
        return LCT_E_ARG;
    if (max_free_regions <= 0 || max_free_regions > 4096
        || (max_free_regions & (max_free_regions - 1)) != 0)
        return LCT_E_ARG;
    if (frees != nullptr) {
        if (frees->count < 0 || frees->count > LCT_MAX_PENDING_FREES) return LCT_E_ARG;
        for (int i = 0; i < frees->count; ++i)
            if (frees->descriptor[i] == nullptr) return LCT_E_NULL;
    }
    uint8_t *base = nullptr;
    if (int32_t e = device_scratch(&base)) return e;
    uint64_t *ready = reinterpret_cast<uint64_t *>(base + kReadyOffset);
    int32_t *partials = reinterpret_cast<int32_t *>(base + kPartialsOffset);
    int32_t *summaries = reinterpret_cast<int32_t *>(base + kSummariesOffset);
    uint8_t *extra_starts = base + kExtraOffset;
    const int64_t sample_size = logical_numel < kMaxSamples ? logical_numel : kMaxSamples;

    hipLaunchKernelGGL(clear_ready_kernel, dim3(1), dim3(64), 0, stream, ready);
    if (hipError_t e = hipGetLastError()) return static_cast<int32_t>(e);
    if (int32_t e = lct_sample_center(source, 0, logical_numel, sample_size, partials,
                                      sample_values, stream))
        return e;
    if (int32_t e = lct_encode_sampled(source, side, encoded, partials, sample_size, base_encode,
                                       base_decode, center_out, shifted_decode_out,
                                       extra_starts, summaries, size, logical_numel, g, 0, 1,
                                       stream))
        return e;
    return lct_allocate_compact(source, summaries, counts, descriptor, buffer_meta,
                                max_free_regions, arena, blocks, extra_starts, frees, ready,
                                kEpoch, size, logical_numel, g, 0, stream);
}
