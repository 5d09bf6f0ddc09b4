// Center estimation and center-shifted Huffman tables (one workgroup).
//
// Follows LCT/kernels/common/tables.py:9-128: the center is the mean unbiased
// exponent of min(n, 4096) hashed sample positions (one jittered position per
// equal-width region, exponents below -120 excluded), rounded half away from
// zero and clamped to [-128, 127]; the encode table is re-indexed by raw
// exponent byte and the decode table stores exponents instead of indices.
#include "lct_device.h"

namespace lct {
namespace {

__global__ __launch_bounds__(kLanes) void tables_kernel(
    const void *__restrict__ source, int32_t precomputed, int64_t logical_numel,
    int64_t sample_size, const int32_t *__restrict__ base_encode,
    const int32_t *__restrict__ base_decode, int32_t *__restrict__ center_io,
    int32_t estimate, int32_t *__restrict__ shifted_encode,
    int32_t *__restrict__ shifted_decode) {
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t shared_center;
    const int t = threadIdx.x;
    int32_t center;
    if (estimate) {
        const int shift = __builtin_ctzll(static_cast<uint64_t>(sample_size));
        // All of a thread's (at most 16) samples are loaded before any is used.
        constexpr int kPerThread = kMaxSamples / kLanes;
        int32_t raw[kPerThread];
#pragma unroll
        for (int k = 0; k < kPerThread; ++k) {
            const int64_t i = t + k * kLanes;
            raw[k] = 0x7FFFFFFF;
            if (i < sample_size) {
                const int64_t pos = sample_position(i, logical_numel, sample_size, shift);
                raw[k] = precomputed ? static_cast<int32_t>(static_cast<const uint8_t *>(source)[pos])
                                     : static_cast<int32_t>(static_cast<const int16_t *>(source)[pos]);
            }
        }
        int32_t sum = 0, kept = 0;
#pragma unroll
        for (int k = 0; k < kPerThread; ++k) {
            if (raw[k] == 0x7FFFFFFF) continue;
            const int32_t exp = (precomputed ? raw[k] : (raw[k] >> 7) & 0xFF) - 127;
            if (exp >= -120) {
                sum += exp;
                kept += 1;
            }
        }
        const int32_t total = block_sum(sum, scratch);
        const int32_t count = block_sum(kept, scratch);
        if (t == 0) {
            const int32_t c = center_of(total, count);
            center_io[0] = c;
            shared_center = c;
        }
        __syncthreads();
        center = shared_center;
    } else {
        center = center_io[0];
    }

    if (shifted_encode != nullptr) {
        shifted_encode[t] = base_encode[byte_to_index(t, center)];
    }
    if (shifted_decode != nullptr) {
#pragma unroll
        for (int i = t; i < 1024; i += kLanes)
            shifted_decode[i] = shifted_decode_entry(base_decode[i], center);
    }
}

// One sample per lane (tables.py:15-49 split over 64-sample groups): the
// group's kept exponent sum and count go to partials; the sampled BF16 bits
// also go to sample_values[i] when given (never for exponent-byte sources).
__global__ __launch_bounds__(kSampleGroup) void sample_center_kernel(
    const void *__restrict__ source, int32_t precomputed, int64_t logical_numel,
    int64_t sample_size, int32_t *__restrict__ partials, uint16_t *__restrict__ sample_values) {
    const int t = threadIdx.x;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kSampleGroup + t;
    const bool active = i < sample_size;
    const int shift = __builtin_ctzll(static_cast<uint64_t>(sample_size));
    int32_t exp = -127;
    if (active) {
        const int64_t pos = sample_position(i, logical_numel, sample_size, shift);
        if (precomputed) {
            exp = static_cast<int32_t>(static_cast<const uint8_t *>(source)[pos]) - 127;
        } else {
            const uint32_t bits = static_cast<const uint16_t *>(source)[pos];
            exp = static_cast<int32_t>((bits >> 7) & 0xFFu) - 127;
            if (sample_values != nullptr) sample_values[i] = static_cast<uint16_t>(bits);
        }
    }
    const bool keep = active && exp >= -120;
    const int32_t sum = wave_sum(keep ? exp : 0);
    const int32_t kept = wave_sum(keep ? 1 : 0);
    if (t == 0) {
        partials[2 * blockIdx.x] = sum;
        partials[2 * blockIdx.x + 1] = kept;
    }
}

}  // namespace
}  // namespace lct

using namespace lct;

extern "C" int32_t lct_sample_center(const void *source, int32_t precomputed,
                                     int64_t logical_numel, int64_t sample_size,
                                     int32_t *partials, uint16_t *sample_values,
                                     hipStream_t stream) {
    if (!source || !partials) return LCT_E_NULL;
    if (logical_numel <= 0 || sample_size <= 0 || sample_size > kMaxSamples
        || sample_size > logical_numel)
        return LCT_E_SIZE;
    if (sample_size != logical_numel && (sample_size & (sample_size - 1)) != 0)
        return LCT_E_ARG;
    hipLaunchKernelGGL(sample_center_kernel, dim3(sample_groups(sample_size)), dim3(kSampleGroup),
                       0, stream, source, precomputed, logical_numel, sample_size, partials,
                       precomputed ? nullptr : sample_values);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_estimate_and_shift_tables(
    const void *source, int32_t precomputed, int64_t logical_numel,
    int64_t sample_size, const int32_t *base_encode, const int32_t *base_decode,
    int32_t *center, int32_t *shifted_encode, int32_t *shifted_decode,
    hipStream_t stream) {
    if (!source || !base_encode || !base_decode || !center || !shifted_encode || !shifted_decode)
        return LCT_E_NULL;
    if (logical_numel <= 0 || sample_size <= 0 || sample_size > kMaxSamples
        || sample_size > logical_numel)
        return LCT_E_SIZE;
    if (sample_size != logical_numel && (sample_size & (sample_size - 1)) != 0)
        return LCT_E_ARG;
    hipLaunchKernelGGL(tables_kernel, dim3(1), dim3(kLanes), 0, stream, source,
                       precomputed, logical_numel, sample_size, base_encode,
                       base_decode, center, 1, shifted_encode, shifted_decode);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_shift_tables(const int32_t *base_encode, const int32_t *center,
                                    int32_t *shifted_encode, const int32_t *base_decode,
                                    int32_t *shifted_decode, hipStream_t stream) {
    if (!base_encode || !center || !shifted_encode || !base_decode || !shifted_decode)
        return LCT_E_NULL;
    hipLaunchKernelGGL(tables_kernel, dim3(1), dim3(kLanes), 0, stream, nullptr, 0,
                       int64_t{0}, int64_t{0}, base_encode, base_decode,
                       const_cast<int32_t *>(center), 0, shifted_encode, shifted_decode);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_shift_decoding_table(const int32_t *base_decode,
                                            const int32_t *center,
                                            int32_t *shifted_decode,
                                            hipStream_t stream) {
    if (!base_decode || !center || !shifted_decode) return LCT_E_NULL;
    hipLaunchKernelGGL(tables_kernel, dim3(1), dim3(kLanes), 0, stream, nullptr, 0,
                       int64_t{0}, int64_t{0}, nullptr, base_decode,
                       const_cast<int32_t *>(center), 0, nullptr, shifted_decode);
    return static_cast<int32_t>(hipGetLastError());
}
