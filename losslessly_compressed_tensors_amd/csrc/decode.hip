// Decoder with fused overflow overlay (gfx950).
//
// Replaces LCT/kernels/generic/decode.py:174-308 (_decode_kernel and
// _decode_overflow_kernel).  One workgroup per codec block: stage the block's
// payload and tables in LDS, expand its overflow list, then every lane walks
// its stream two symbols per iteration, joining each exponent with its side
// byte and storing the BF16 bits at the swizzled logical offset.  Steps at or
// past a stream's overflow start take their exponent from the tail bytes and
// consume no payload bits.
#include "decode_core.h"

namespace lct {
namespace {

// S is a template parameter so the pair loop (which holds convergent
// wave-uniform branches) can be unrolled.
template <bool kFull, int S>
__device__ __forceinline__ void decode_rows(const StreamCursor &cursor_in, const LaneOverlay &lane,
                                            const uint8_t *__restrict__ side_block,
                                            uint16_t *__restrict__ out_block, int64_t row_base,
                                            int64_t valid_in_block) {
    StreamCursor cursor = cursor_in;
    const uint32_t t = threadIdx.x;
#pragma unroll 2
    for (int step = 0; step < S; step += 2) {
        uint32_t f0, len0, f1, len1;
        cursor.next_pair(f0, len0, f1, len1);
        const uint32_t slot = static_cast<uint32_t>(step) * kLanes + t;
        const uint32_t sm0 = side_block[slot];
        const uint32_t sm1 = side_block[slot + kLanes];
        if (step >= lane.wave_start) {
            if (step >= lane.start) {
                const uint8_t *src = lane.tail + lane.offset + (step - lane.start);
                f0 = tail_field(src[0]);
                f1 = tail_field(src[1]);
                len0 = 0;
                len1 = 0;
            }
        }
        const uint32_t col = t ^ static_cast<uint32_t>((row_base + step) & 254);
        const uint32_t off0 = static_cast<uint32_t>(step) * kLanes + col;
        const uint32_t off1 = off0 + kLanes;
        const uint16_t out0 = static_cast<uint16_t>(join_bf16(f0, sm0));
        const uint16_t out1 = static_cast<uint16_t>(join_bf16(f1, sm1));
        if (kFull) {
            out_block[off0] = out0;
            out_block[off1] = out1;
        } else {
            const bool v0 = off0 < valid_in_block;
            const bool v1 = off1 < valid_in_block;
            if (v0) out_block[off0] = out0;
            if (v1) out_block[off1] = out1;
            len0 = v0 ? len0 : 0u;
            len1 = v1 ? len1 : 0u;
        }
        cursor.pos += len0 + len1;
    }
}

__global__ __launch_bounds__(kLanes) void decode_kernel(
    const int32_t *__restrict__ encoded, const uint8_t *__restrict__ side,
    uint16_t *__restrict__ output, const int32_t *__restrict__ shifted_decode,
    const int32_t *__restrict__ center_ptr, int64_t n_blocks, int64_t logical_numel, int S,
    int W, int rare, lct_overflow ov, int has_overlay) {
    extern __shared__ uint32_t stage[];   // (W + 2) rows x 256
    __shared__ DecodeTables tb;
    __shared__ int32_t map_start[kLanes], map_offset[kLanes], scratch[kWavesPerBlock];
    const int64_t block = blockIdx.x;
    const int32_t center = center_ptr[0];
    build_decode_tables(tb, shifted_decode, center);
    stage_payload(stage, encoded, n_blocks * kLanes, block, W);
    const LaneOverlay lane = build_overlay(ov, has_overlay != 0, block, n_blocks, S, map_start,
                                           map_offset, scratch);
    __syncthreads();

    const StreamCursor cursor{stage + threadIdx.x, &tb, 0u, static_cast<uint32_t>(W), rare};
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    const uint8_t *side_block = side + logical_base;
    uint16_t *out_block = output + logical_base;
    const int64_t valid = logical_numel - logical_base;
    const bool full = valid >= static_cast<int64_t>(S) * kLanes;
#define LCT_DECODE_CASE(FULL)                                                          \
    if (S == 128)                                                                      \
        decode_rows<FULL, 128>(cursor, lane, side_block, out_block, row_base, valid);  \
    else                                                                               \
        decode_rows<FULL, 256>(cursor, lane, side_block, out_block, row_base, valid);
    if (full) { LCT_DECODE_CASE(true) } else { LCT_DECODE_CASE(false) }
#undef LCT_DECODE_CASE
}

}  // namespace
}  // namespace lct

using namespace lct;

extern "C" int32_t lct_decode(const int32_t *encoded, const uint8_t *side, int16_t *output,
                              const int32_t *shifted_decode, const int32_t *center,
                              int64_t size, int64_t logical_numel, lct_geometry g,
                              int32_t rare_length, const lct_overflow *overflow,
                              hipStream_t stream) {
    if (!encoded || !side || !output || !shifted_decode || !center) return LCT_E_NULL;
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (logical_numel <= 0 || size <= 0 || size % g.block_symbols != 0
        || logical_numel > size || logical_numel <= size - g.block_symbols)
        return LCT_E_SIZE;
    if (rare_length < 0 || rare_length > 8) return LCT_E_ARG;
    if ((reinterpret_cast<uintptr_t>(encoded) & 15) != 0) return LCT_E_ARG;
    lct_overflow ov{};
    if (overflow != nullptr) {
        if (!overflow->lanes || !overflow->starts || !overflow->tail || !overflow->blocks)
            return LCT_E_NULL;
        if (overflow->descriptor != nullptr && overflow->count == nullptr) return LCT_E_NULL;
        ov = *overflow;
    }
    const int64_t n_blocks = size / g.block_symbols;
    if (n_blocks > 0x7FFFFFFF) return LCT_E_SIZE;
    const size_t lds = static_cast<size_t>(g.fixed_words + 2) * kLanes * sizeof(uint32_t);
    hipLaunchKernelGGL(decode_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes), lds,
                       stream, encoded, side, reinterpret_cast<uint16_t *>(output),
                       shifted_decode, center, n_blocks, logical_numel, g.steps, g.fixed_words,
                       rare_length, ov, overflow != nullptr ? 1 : 0);
    return static_cast<int32_t>(hipGetLastError());
}
