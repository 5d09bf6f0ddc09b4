// Device-side helpers shared by the gfx950 codec kernels.
//
// Format facts used throughout (LCT/kernels/generic/layout.py:15-18,
// LCT/kernels/primitives.py:7-36, LCT/kernels/common/tables.py:53-118):
//  * storage row r = k*S + t, lane l  <->  logical r*256 + (l ^ (r & 254));
//    rows 2j and 2j+1 share the XOR mask, so one step pair uses one column;
//  * a BF16 value b splits into exponent byte (b >> 7) & 255 and side byte
//    (b & 0x7F) | ((b >> 8) & 0x80);
//  * Huffman table index 0 is exact zero; other indices are centred exponent
//    deltas with the zero delta removed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lct.h"

namespace lct {

constexpr int kLanes = 256;     // streams per codec block (= threads per workgroup)
constexpr int kWave = 64;
constexpr int kWavesPerBlock = kLanes / kWave;
constexpr int kMaxWords = 64;   // largest fixed payload per stream accepted
constexpr int kEscapeLength = 31;  // decode-table length field marking an escape

// Buffer resource word 3 for gfx9-family raw buffers.
constexpr int32_t kBufferConfig = 0x00020000;

// A raw buffer resource over `bytes` bytes from `base`: accesses are 32-bit
// offsets from an SGPR base, and those at or past `bytes` read 0 / are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes),
                                             kBufferConfig);
}

// 16-byte buffer store with the whole offset in the VGPR and soffset 0.
// A store of more than 8 bytes reads its data VGPRs after issue, and a VALU
// write to them must wait one cycle; the compiler inserts that wait only when
// soffset is a constant (it treats an SGPR soffset as hazard-free).  On gfx950
// the hazard does occur with an SGPR soffset: with two or more workgroups per
// CU, a 16-byte store followed at once by a VALU write of its first data
// register wrote the new value.  16-byte buffer stores pass soffset 0, directly
// or through this helper.
template <int kAux>
__device__ __forceinline__ void store_b128(uint4 q, __amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
    __builtin_amdgcn_raw_buffer_store_b128(
        __builtin_bit_cast(__attribute__((ext_vector_type(4))) uint32_t, q), rsrc, offset, 0,
        kAux);
}

// Unbiased exponent of Huffman table index `symbol` under `center`
// (tables.py:109-116, primitives.py:29-35).
__device__ __forceinline__ int32_t index_to_exponent(int32_t symbol, int32_t center) {
    const int32_t zero_delta = (-127 - center) & 255;
    int32_t delta = symbol - (symbol <= zero_delta ? 1 : 0);
    delta = delta >= 128 ? delta - 256 : delta;
    return symbol == 0 ? -127 : delta + center;
}

// Table index of a raw exponent byte under `center` (tables.py:53-67).
__device__ __forceinline__ int32_t byte_to_index(int32_t raw, int32_t center) {
    const int32_t zero_delta = (-127 - center) & 255;
    const int32_t exp = raw - 127;
    const int32_t delta = (exp - center) & 255;
    return exp == -127 ? 0 : delta + (delta < zero_delta ? 1 : 0);
}

// Entry of the center-shifted decode table: len | exponent << 8, or 0 for a
// continuation entry (tables.py:102-118).
__device__ __forceinline__ int32_t shifted_decode_entry(int32_t packed, int32_t center) {
    const int32_t length = packed & 255;
    const int32_t exponent = index_to_exponent((packed >> 8) & 255, center);
    return length == 0 ? 0
                       : static_cast<int32_t>(static_cast<uint32_t>(length)
                                              | (static_cast<uint32_t>(exponent) << 8));
}

// Side byte -> its bits in BF16 position: sign to bit 15, mantissa to 0..6.
// sm * 257 copies the byte into bits 8..15; the mask keeps bit 15 and 0..6.
__device__ __forceinline__ uint32_t side_bits(uint32_t sm) {
    return (sm * 257u) & 0x807Fu;
}

// BF16 bits from an exponent field already at bits 7..14 and a side byte.
__device__ __forceinline__ uint32_t join_bf16(uint32_t exponent_field, uint32_t sm) {
    return (exponent_field & 0x7F80u) | side_bits(sm);
}

__device__ __forceinline__ uint32_t side_byte_of(uint32_t bits) {
    return (bits & 0x7Fu) | ((bits >> 8) & 0x80u);
}

__device__ __forceinline__ float bf16_to_float(uint32_t bits) {
    return __uint_as_float(bits << 16);
}

// FP32 -> BF16, round to nearest even; NaN becomes the canonical 0x7FFF.
__device__ __forceinline__ uint32_t float_to_bf16(float value) {
    uint32_t u = __float_as_uint(value);
    const bool nan = (u & 0x7FFFFFFFu) > 0x7F800000u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return nan ? 0x7FFFu : (u >> 16);
}

// Center sampling (tables.py:15-49): sample i of M = min(n, 4096) lies in
// region [i*n/M, (i+1)*n/M) at a hashed offset.  M is either n itself (one
// element per region, offset 0) or a power of two (the entry points reject any
// other M), so no 64-bit division is needed; `shift` = log2(M).
constexpr int kMaxSamples = 4096;

__device__ __forceinline__ int64_t sample_position(int64_t i, int64_t n, int64_t m, int shift) {
    if (m == n) return i;
    const uint32_t hashed = static_cast<uint32_t>(i) * 0x9E3779B9u;
    const int64_t start = (i * n) >> shift;
    const int64_t end = ((i + 1) * n) >> shift;
    const uint64_t jitter =
        (static_cast<uint64_t>(hashed) * static_cast<uint64_t>(end - start)) >> 32;
    return start + static_cast<int64_t>(jitter);
}

// The center from the kept samples' exponent sum and count: the mean rounded
// half away from zero, clamped to [-128, 127]; 0 without samples
// (tables.py:40-49).
__device__ __forceinline__ int32_t center_of(int32_t total, int32_t count) {
    if (count <= 0) return 0;
    const int32_t c = total >= 0 ? (total + count / 2) / count : -((-total + count / 2) / count);
    return min(max(c, -128), 127);
}

__device__ __forceinline__ int wave_lane() { return threadIdx.x & (kWave - 1); }

__device__ __forceinline__ int32_t wave_sum(int32_t v) {
#pragma unroll
    for (int offset = kWave / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
    return v;
}

__device__ __forceinline__ int32_t wave_min(int32_t v) {
#pragma unroll
    for (int offset = kWave / 2; offset > 0; offset >>= 1) v = min(v, __shfl_xor(v, offset, kWave));
    return v;
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ int32_t wave_inclusive_scan(int32_t v) {
    const int lane = wave_lane();
#pragma unroll
    for (int offset = 1; offset < kWave; offset <<= 1) {
        const int32_t other = __shfl_up(v, offset, kWave);
        if (lane >= offset) v += other;
    }
    return v;
}

// Exclusive prefix sum over the 256 threads of a block; returns the total in
// *total.  `scratch` holds kWavesPerBlock ints of LDS.  Contains barriers.
__device__ __forceinline__ int32_t block_exclusive_scan(int32_t v, int32_t *scratch, int32_t *total) {
    const int wave = threadIdx.x / kWave;
    const int32_t inclusive = wave_inclusive_scan(v);
    if (wave_lane() == kWave - 1) scratch[wave] = inclusive;
    __syncthreads();
    int32_t before = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
        const int32_t s = scratch[w];
        before += w < wave ? s : 0;
        sum += s;
    }
    __syncthreads();
    *total = sum;
    return before + inclusive - v;
}

__device__ __forceinline__ int32_t block_sum(int32_t v, int32_t *scratch) {
    int32_t total;
    block_exclusive_scan(v, scratch, &total);
    return total;
}

// The center's samples are taken by workgroups of one wave, one sample per
// lane; each group writes its kept exponents' sum and count to partials[2g],
// partials[2g + 1] (at most kMaxSamples / kSampleGroup = 64 groups).
constexpr int kSampleGroup = 64;

// The center from those partial sums, computed by wave 0 of the block into
// *shared (visible to the block after its next barrier).
__device__ __forceinline__ void center_from_partials(const int32_t *__restrict__ partials,
                                                     int32_t n_groups, int32_t *shared) {
    if (threadIdx.x < kWave) {
        const int t = threadIdx.x;
        const int32_t sum = wave_sum(t < n_groups ? partials[2 * t] : 0);
        const int32_t kept = wave_sum(t < n_groups ? partials[2 * t + 1] : 0);
        if (t == 0) *shared = center_of(sum, kept);
    }
}

// The fused compress's control array (one per stream, reused by every call on
// it): 64-bit words that carry the call's 32-bit epoch in their high half, so a
// word an earlier call wrote never reads as current and no call has to clear
// the array.  Words [0, 64) are the center samplers' partial sums (low half:
// the kept exponents' sum as int16 in bits 16..31, their count in bits 0..15);
// words [64, 64 + nb) the encoders' per-block overflow summaries (low half:
// count << 17 | tail bytes; a count field of kFailedBlock marks a block that
// could not read its center).  Every word is written with one agent-scope
// atomic store and read with agent-scope atomic loads, so it is read whole and
// coherently across the XCDs.
constexpr int kControlPartials = 64;
constexpr uint32_t kFailedBlock = 0x1FFu;

__device__ __forceinline__ uint64_t tagged_word(uint32_t epoch, uint32_t value) {
    return (static_cast<uint64_t>(epoch) << 32) | value;
}

__device__ __forceinline__ bool tagged_with(uint64_t word, uint32_t epoch) {
    return static_cast<uint32_t>(word >> 32) == epoch;
}

__device__ __forceinline__ uint64_t control_load(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void control_store(uint64_t *p, uint64_t value) {
    __hip_atomic_store(p, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A word for the host, in pinned host memory: one system-scope store of the
// whole 64-bit word (no fence: the host reads only this word, which carries
// its call's epoch in the high half, so it is current exactly when the tag
// matches).
__device__ __forceinline__ void host_word_store(uint64_t *p, uint64_t value) {
    __hip_atomic_store(p, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The center from the partial sums the sampling workgroups of the same launch
// publish in control[0, n_groups), computed by wave 0 of the block: lane g
// polls word g until it carries `epoch` (at most `polls` times).  Writes the
// center to shared[0] and whether some word did not arrive to shared[1]
// (center 0 then), visible to the block after its next barrier.
__device__ __forceinline__ void center_from_control(const uint64_t *__restrict__ control,
                                                    int32_t n_groups, uint32_t epoch,
                                                    int32_t polls, int32_t *shared) {
    if (threadIdx.x < kWave) {
        const int t = threadIdx.x;
        int32_t sum = 0, kept = 0;
        bool arrived = true;
        if (t < n_groups) {
            uint64_t word = control_load(control + t);
            for (int i = 0; !tagged_with(word, epoch) && i < polls; ++i) {
                __builtin_amdgcn_s_sleep(2);
                word = control_load(control + t);
            }
            arrived = tagged_with(word, epoch);
            sum = static_cast<int16_t>(static_cast<uint16_t>(word >> 16));
            kept = static_cast<int32_t>(word & 0xFFFFu);
        }
        const bool missing = __ballot(!arrived) != 0;
        sum = wave_sum(sum);
        kept = wave_sum(kept);
        if (t == 0) {
            shared[0] = missing ? 0 : center_of(sum, kept);
            shared[1] = missing ? 1 : 0;
        }
    }
}

// Number of sampling groups for sample_size samples.
__host__ __device__ constexpr int32_t sample_groups(int64_t sample_size) {
    return static_cast<int32_t>((sample_size + kSampleGroup - 1) / kSampleGroup);
}

// Largest codec block count of one tensor: overflow offsets and tail byte
// counts are int32 in the storage format, so a tensor stays below 2^31 storage
// elements (65535 blocks of 32768).
constexpr int64_t kMaxBlocks = 65535;

// Geometry check shared by every entry point.
inline bool geometry_ok(const lct_geometry &g) {
    // Every geometry of LCT/codec/geometry.py:13-39 (and the legacy layout of
    // LCT/comp_tensor.py:50-54) has 128 or 256 steps.
    return g.lanes == kLanes && (g.steps == 128 || g.steps == 256)
        && g.block_symbols == g.lanes * g.steps && g.fixed_words >= 2
        && g.fixed_words <= kMaxWords;
}

// Lift a kernel's dynamic LDS limit above the 64 KiB default when a launch
// needs more (the device allows 160 KiB per workgroup).
inline hipError_t reserve_dynamic_lds(const void *kernel, size_t bytes) {
    if (bytes <= 65536) return hipSuccess;
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(bytes));
}

}  // namespace lct
