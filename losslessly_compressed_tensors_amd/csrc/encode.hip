// Encoder launches: the field split + fixed-payload Huffman encoder of
// encode_core.h, one workgroup per codec block, with the table step either
// done before (lct_encode) or folded into each workgroup's prologue from the
// sampler's partial sums (lct_encode_sampled).
// Follows LCT/kernels/generic/encode.py:10-169 and LCT/kernels/dispatch.py:294-316.
#include "encode_core.h"

namespace lct {
namespace {

// One kernel per input kind (BF16 bits or precomputed exponent bytes), so
// each carries one encoder variant and its registers.
template <bool kPrecomputed>
__global__ __launch_bounds__(kLanes) void encode_kernel(
    const void *__restrict__ source, uint8_t *__restrict__ side,
    int32_t *__restrict__ encoded, TableSource tables,
    uint8_t *__restrict__ extra_starts, int32_t *__restrict__ summaries,
    int64_t n_blocks, int64_t logical_numel, int S, int W, int write_summary) {
    extern __shared__ uint32_t stage[];   // (W + 2) rows x 256 lanes
    __shared__ uint2 table[256];
    __shared__ __attribute__((aligned(16))) uint8_t slices[kWavesPerBlock * kSliceBytes];
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t shared[2];
    const EncodeLds lds{stage, table, slices, scratch, shared};
    const int64_t block = blockIdx.x;
    const BlockSummary s = encode_codec_block(source, side, encoded, tables, extra_starts, block,
                                              n_blocks, logical_numel, S, W, kPrecomputed,
                                              write_summary != 0, lds);
    if (write_summary && threadIdx.x == 0) {
        summaries[block] = s.count;
        summaries[n_blocks + block] = s.bytes;
    }
}

}  // namespace
}  // namespace lct

using namespace lct;

namespace {

int32_t launch_encode(const void *source, uint8_t *side, int32_t *encoded,
                      const TableSource &tables, uint8_t *extra_starts, int32_t *summaries,
                      int64_t size, int64_t logical_numel, const lct_geometry &g,
                      int32_t precomputed, int32_t write_summary, hipStream_t stream) {
    if (!source || !side || !encoded || !extra_starts) return LCT_E_NULL;
    if (write_summary && !summaries) return LCT_E_NULL;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (logical_numel <= 0 || size <= 0 || size % g.block_symbols != 0
        || logical_numel > size || logical_numel <= size - g.block_symbols)
        return LCT_E_SIZE;
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > 0x7FFFFFFF) return LCT_E_SIZE;
    // 16-byte vector access to the source, side bytes and payload.
    if (((reinterpret_cast<uintptr_t>(encoded) | reinterpret_cast<uintptr_t>(source)
          | reinterpret_cast<uintptr_t>(side)) & 15) != 0)
        return LCT_E_ARG;
    const size_t lds = static_cast<size_t>(g.fixed_words + 2) * kLanes * 4;
    const auto kernel = precomputed ? encode_kernel<true> : encode_kernel<false>;
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes),
                       lds, stream, source, side, encoded, tables,
                       extra_starts, summaries, n_blocks, logical_numel, g.steps,
                       g.fixed_words, write_summary);
    return static_cast<int32_t>(hipGetLastError());
}

}  // namespace

extern "C" int32_t lct_encode(const void *source, uint8_t *side, int32_t *encoded,
                              const int32_t *shifted_encode, uint8_t *extra_starts,
                              int32_t *summaries, int64_t size, int64_t logical_numel,
                              lct_geometry g, int32_t precomputed,
                              int32_t write_summary, hipStream_t stream) {
    if (!shifted_encode) return LCT_E_NULL;
    const TableSource tables{shifted_encode, nullptr, 0, nullptr, nullptr, nullptr, nullptr};
    return launch_encode(source, side, encoded, tables, extra_starts, summaries, size,
                         logical_numel, g, precomputed, write_summary, stream);
}

extern "C" int32_t lct_encode_sampled(const void *source, uint8_t *side, int32_t *encoded,
                                      const int32_t *partials, int64_t sample_size,
                                      const int32_t *base_encode, const int32_t *base_decode,
                                      int32_t *center_out, int32_t *shifted_decode_out,
                                      uint8_t *extra_starts, int32_t *summaries, int64_t size,
                                      int64_t logical_numel, lct_geometry g,
                                      int32_t precomputed, int32_t write_summary,
                                      hipStream_t stream) {
    if (!partials || !base_encode || !base_decode || !center_out || !shifted_decode_out)
        return LCT_E_NULL;
    if (sample_size <= 0 || sample_size > kMaxSamples || sample_size > logical_numel)
        return LCT_E_SIZE;
    const TableSource tables{nullptr, partials, sample_groups(sample_size), base_encode,
                             base_decode, center_out, shifted_decode_out};
    return launch_encode(source, side, encoded, tables, extra_starts, summaries, size,
                         logical_numel, g, precomputed, write_summary, stream);
}
