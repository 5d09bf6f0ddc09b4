// Attainable-bandwidth probes: the HBM ceiling the codec kernels are judged
// against.  Plain streaming kernels with the codec's access shape (16-byte
// non-temporal buffer loads and stores, four in flight per thread, each
// workgroup pass covering 16 KiB): a copy, a read-only pass, a write-only
// pass, and a mix of reads and writes in a given proportion (the decoder's at
// NS: 185 MB read, 268 MB written per launch).  bench.py reports them beside
// the roofline fractions, which stay relative to the 8 TB/s peak.
#include "decode_core.h"   // kStreaming: the non-temporal cache policy

namespace lct {
namespace {

using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

constexpr int kUnroll = 4;                                // 16-byte accesses in flight
constexpr uint32_t kPassBytes = kLanes * kUnroll * 16;    // bytes per workgroup pass

// A 32-bit buffer resource covers at most 4 GiB; the probes take buffers of
// up to 2 GiB.
constexpr int64_t kMaxProbeBytes = int64_t{1} << 31;

enum ProbeKind { kCopy = 0, kReadOnly = 1, kWriteOnly = 2, kMix = 3 };

// Pass p covers [p * kPassBytes, (p + 1) * kPassBytes) of the primary buffer
// (src for kReadOnly, dst otherwise); kMix reads [p * read_pass, (p + 1) *
// read_pass) of src in the same pass, read_pass = kPassBytes * src / dst.
// Loaded values feed an accumulator that decides one (practically never
// taken) store per thread, so no load is dead.
template <int kKind>
__global__ __launch_bounds__(kLanes) void bandwidth_kernel(const uint8_t *__restrict__ src,
                                                           uint32_t src_bytes,
                                                           uint8_t *__restrict__ dst,
                                                           uint32_t dst_bytes,
                                                           uint32_t read_pass) {
    const __amdgpu_buffer_rsrc_t in = make_rsrc(src, src_bytes);
    const __amdgpu_buffer_rsrc_t out = make_rsrc(dst, dst_bytes);
    const uint32_t lane_off = threadIdx.x * 16u;
    uint32_t acc = 0u;
    const uint32_t primary = kKind == kReadOnly ? src_bytes : dst_bytes;
    const uint32_t passes = (primary + kPassBytes - 1) / kPassBytes;
    for (uint32_t pass = blockIdx.x; pass < passes; pass += gridDim.x) {
        const uint32_t base = pass * kPassBytes;
        if (kKind == kWriteOnly || kKind == kMix) {
            const u32x4 fill = {pass, threadIdx.x, acc, ~acc};
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
                __builtin_amdgcn_raw_buffer_store_b128(fill, out,
                                                       base + u * (kLanes * 16u) + lane_off, 0,
                                                       kStreaming);
        }
        if (kKind == kWriteOnly) continue;
        const uint32_t read_base = kKind == kMix ? pass * read_pass : base;
        u32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint32_t within = u * (kLanes * 16u) + lane_off;
            // kMix reads only its pass's share (the resource drops the rest).
            const uint32_t off =
                kKind == kMix && within >= read_pass ? 0xFFFFFFF0u : read_base + within;
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(in, off, 0, kStreaming);
        }
        if (kKind == kCopy) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
                __builtin_amdgcn_raw_buffer_store_b128(v[u], out,
                                                       base + u * (kLanes * 16u) + lane_off, 0,
                                                       kStreaming);
        } else {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) acc += v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        }
    }
    if (kKind != kCopy && acc == 0x9E3779B9u)
        __builtin_amdgcn_raw_buffer_store_b32(acc, out, lane_off, 0, 0);
}

}  // namespace
}  // namespace lct

using namespace lct;

extern "C" int32_t lct_bandwidth_probe(int32_t kind, const void *src, int64_t src_bytes,
                                       void *dst, int64_t dst_bytes, int32_t workgroups,
                                       hipStream_t stream) {
    if (!dst || (kind != kWriteOnly && !src)) return LCT_E_NULL;
    if (kind < kCopy || kind > kMix || workgroups <= 0) return LCT_E_ARG;
    if (src_bytes < 0 || dst_bytes < kLanes * 16 || src_bytes > kMaxProbeBytes
        || dst_bytes > kMaxProbeBytes || src_bytes % 16 != 0 || dst_bytes % 16 != 0)
        return LCT_E_SIZE;
    if (kind == kCopy && src_bytes != dst_bytes) return LCT_E_SIZE;
    if (kind == kMix && (src_bytes == 0 || src_bytes > dst_bytes)) return LCT_E_SIZE;
    if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) != 0)
        return LCT_E_ARG;
    const auto *s = static_cast<const uint8_t *>(src);
    auto *d = static_cast<uint8_t *>(dst);
    const uint32_t sb = static_cast<uint32_t>(src_bytes), db = static_cast<uint32_t>(dst_bytes);
    const uint32_t read_pass = kind == kMix ? static_cast<uint32_t>(
        (static_cast<uint64_t>(kPassBytes) * sb / db) & ~15ull) : 0u;
    const dim3 grid(static_cast<uint32_t>(workgroups)), block(kLanes);
    switch (kind) {
    case kCopy:
        hipLaunchKernelGGL(bandwidth_kernel<kCopy>, grid, block, 0, stream, s, sb, d, db,
                           read_pass);
        break;
    case kReadOnly:
        hipLaunchKernelGGL(bandwidth_kernel<kReadOnly>, grid, block, 0, stream, s, sb, d, db,
                           read_pass);
        break;
    case kWriteOnly:
        hipLaunchKernelGGL(bandwidth_kernel<kWriteOnly>, grid, block, 0, stream, s, sb, d, db,
                           read_pass);
        break;
    default:
        hipLaunchKernelGGL(bandwidth_kernel<kMix>, grid, block, 0, stream, s, sb, d, db,
                           read_pass);
        break;
    }
    return static_cast<int32_t>(hipGetLastError());
}
