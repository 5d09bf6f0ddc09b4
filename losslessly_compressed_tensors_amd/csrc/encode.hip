// Field split + fixed-payload Huffman encoder for gfx950.
//
// One workgroup per codec block, one thread per lane (= one Huffman stream),
// as the format requires (LCT/kernels/generic/encode.py:10-169).  Per step
// pair a lane reads two BF16 values at the swizzled logical offsets (one
// column for both rows), writes their side bytes in storage order, looks the
// exponent bytes up in an LDS copy of the shifted encode table and appends the
// concatenated pair code to its bit position `pos`.
//
// Instead of masked, scattered word-major global stores the payload is built
// in LDS: every pair writes the lane's current partial word to stage row
// pos/32 (conflict-free: row stride 256 words, lane-contiguous), so the final
// contents of each row are the completed words; after the loop the block
// copies rows 0..W-1 to `encoded` with 16-byte coalesced stores.  Row W is a
// pad row that absorbs writes of overflowed lanes.
//
// Overflow rule (encode.py:73-90): a pair overflows when pos + len > 32W; the
// first overflowing pair's even step is the stream's extra_start and word W-1
// keeps only the bits before that pair.  The first-overflow bookkeeping runs in
// a wave-uniform branch that is skipped unless some lane of the wave overflows.
#include "lct_device.h"

namespace lct {
namespace {

// Encode-table entry repacked for the kernel: reversed code (<= 16 bits) in
// bits 0..15, code length in bits 16..20.
__device__ __forceinline__ uint32_t repack_encode_entry(uint32_t packed) {
    return (packed & 0xFFFFu) | ((packed >> 20) << 16);
}

// S is a template parameter so the pair loop can be unrolled: the
// wave-uniform branch inside it is convergent, which rules out unrolling a
// loop with a run-time trip count.
template <bool kFull, bool kPrecomputed, int S>
__device__ __forceinline__ void encode_block(
    const void *__restrict__ source, uint8_t *__restrict__ side,
    const uint32_t *__restrict__ table, uint32_t *__restrict__ stage,
    int64_t block, int64_t logical_numel, int W, uint32_t &pos_out,
    bool &overflow_out, int &extra_out) {
    const uint32_t lane = threadIdx.x;
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;   // also the storage base k*B
    uint8_t *side_block = side + logical_base;
    const uint32_t limit = static_cast<uint32_t>(W) * 32u;
    const uint32_t pad_slot = static_cast<uint32_t>(W) * kLanes + lane;

    uint32_t pos = 0, word_value = 0;
    bool overflow = false;
    int extra = S;
#pragma unroll 4
    for (int step = 0; step < S; step += 2) {
        const uint32_t col = lane ^ static_cast<uint32_t>((row_base + step) & 254);
        const uint32_t off0 = static_cast<uint32_t>(step) * kLanes + col;
        const uint32_t off1 = off0 + kLanes;
        bool valid0 = true, valid1 = true;
        if (!kFull) {
            valid0 = logical_base + off0 < logical_numel;
            valid1 = logical_base + off1 < logical_numel;
        }
        uint32_t e0, e1;
        if (kPrecomputed) {
            const uint8_t *src = static_cast<const uint8_t *>(source) + logical_base;
            e0 = valid0 ? src[off0] : 0u;
            e1 = valid1 ? src[off1] : 0u;
        } else {
            const uint16_t *src = static_cast<const uint16_t *>(source) + logical_base;
            const uint32_t v0 = valid0 ? src[off0] : 0u;
            const uint32_t v1 = valid1 ? src[off1] : 0u;
            e0 = (v0 >> 7) & 0xFFu;
            e1 = (v1 >> 7) & 0xFFu;
            const uint32_t slot = static_cast<uint32_t>(step) * kLanes + lane;
            side_block[slot] = static_cast<uint8_t>(side_byte_of(v0));
            side_block[slot + kLanes] = static_cast<uint8_t>(side_byte_of(v1));
        }
        uint32_t p0 = table[e0], p1 = table[e1];
        if (!kFull) {
            p0 = valid0 ? p0 : 0u;
            p1 = valid1 ? p1 : 0u;
        }
        const uint32_t len0 = p0 >> 16;
        const uint32_t code = (p0 & 0xFFFFu) | ((p1 & 0xFFFFu) << len0);
        const uint32_t len = len0 + (p1 >> 16);

        const uint32_t shift = pos & 31u;
        const uint64_t placed = static_cast<uint64_t>(code) << shift;
        const uint32_t new_word = word_value | static_cast<uint32_t>(placed);
        const uint32_t carry = static_cast<uint32_t>(placed >> 32);
        const uint32_t row = pos >> 5;
        const uint32_t pos_after = pos + len;
        const bool overflow_now = pos_after > limit;
        stage[overflow_now ? pad_slot : row * kLanes + lane] = new_word;
        const bool first = overflow_now && !overflow;
        if (__any(first)) {
            // This pair is the stream's first that does not fit: keep the
            // bits before it in its current word (row <= W).
            if (first) {
                extra = step;
                stage[row * kLanes + lane] = word_value;
            }
        }
        overflow = overflow_now;
        word_value = (pos_after >> 5) != row ? carry : new_word;
        pos = pos_after;
    }
    if (!overflow) stage[(pos >> 5) * kLanes + lane] = word_value;
    pos_out = pos;
    overflow_out = overflow;
    extra_out = extra;
}

__global__ __launch_bounds__(kLanes) void encode_kernel(
    const void *__restrict__ source, uint8_t *__restrict__ side,
    int32_t *__restrict__ encoded, const int32_t *__restrict__ shifted_encode,
    uint8_t *__restrict__ extra_starts, int32_t *__restrict__ summaries,
    int64_t n_blocks, int64_t logical_numel, int S, int W, int precomputed,
    int write_summary) {
    extern __shared__ uint32_t stage[];   // (W + 1) rows x 256 lanes
    __shared__ uint32_t table[256];
    __shared__ int32_t scratch[kWavesPerBlock];
    const int t = threadIdx.x;
    const int64_t block = blockIdx.x;

    table[t] = repack_encode_entry(static_cast<uint32_t>(shifted_encode[t]));
    for (int i = t; i < (W + 1) * kLanes; i += kLanes) stage[i] = 0u;
    __syncthreads();

    uint32_t pos;
    bool overflow;
    int extra;
    const bool full = (block + 1) * static_cast<int64_t>(S) * kLanes <= logical_numel;
#define LCT_ENCODE_CASE(FULL, PRE)                                                           \
    if (S == 128)                                                                            \
        encode_block<FULL, PRE, 128>(source, side, table, stage, block, logical_numel, W,    \
                                     pos, overflow, extra);                                  \
    else                                                                                     \
        encode_block<FULL, PRE, 256>(source, side, table, stage, block, logical_numel, W,    \
                                     pos, overflow, extra);
    if (precomputed) {
        if (full) { LCT_ENCODE_CASE(true, true) } else { LCT_ENCODE_CASE(false, true) }
    } else {
        if (full) { LCT_ENCODE_CASE(true, false) } else { LCT_ENCODE_CASE(false, false) }
    }
#undef LCT_ENCODE_CASE
    (void)pos;

    const int64_t n_streams = n_blocks * kLanes;
    extra_starts[block * kLanes + t] = static_cast<uint8_t>(overflow ? extra : 255);
    __syncthreads();

    // Copy the W payload rows out, 16 bytes per thread per store.
    const int chunks = W * (kLanes / 4);
    for (int c = t; c < chunks; c += kLanes) {
        const int row = c / (kLanes / 4);
        const int quad = c % (kLanes / 4);
        const uint4 value = reinterpret_cast<const uint4 *>(stage + row * kLanes)[quad];
        uint4 *dst = reinterpret_cast<uint4 *>(encoded + row * n_streams + block * kLanes);
        dst[quad] = value;
    }

    if (write_summary) {
        const int32_t count = block_sum(overflow ? 1 : 0, scratch);
        const int32_t bytes = block_sum(overflow ? S - extra : 0, scratch);
        if (t == 0) {
            summaries[block] = count;
            summaries[n_blocks + block] = bytes;
        }
    }
}

}  // namespace
}  // namespace lct

using namespace lct;

extern "C" int32_t lct_encode(const void *source, uint8_t *side, int32_t *encoded,
                              const int32_t *shifted_encode, uint8_t *extra_starts,
                              int32_t *summaries, int64_t size, int64_t logical_numel,
                              lct_geometry g, int32_t precomputed,
                              int32_t write_summary, hipStream_t stream) {
    if (!source || !side || !encoded || !shifted_encode || !extra_starts) return LCT_E_NULL;
    if (write_summary && !summaries) return LCT_E_NULL;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (logical_numel <= 0 || size <= 0 || size % g.block_symbols != 0
        || logical_numel > size || logical_numel <= size - g.block_symbols)
        return LCT_E_SIZE;
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > 0x7FFFFFFF) return LCT_E_SIZE;
    if ((reinterpret_cast<uintptr_t>(encoded) & 15) != 0) return LCT_E_ARG;
    const size_t lds = static_cast<size_t>(g.fixed_words + 1) * kLanes * sizeof(uint32_t);
    hipLaunchKernelGGL(encode_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes),
                       lds, stream, source, side, encoded, shifted_encode,
                       extra_starts, summaries, n_blocks, logical_numel, g.steps,
                       g.fixed_words, precomputed, write_summary);
    return static_cast<int32_t>(hipGetLastError());
}
