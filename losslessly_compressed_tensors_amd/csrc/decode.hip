// Decoder with fused overflow overlay (gfx950).
//
// Replaces LCT/kernels/generic/decode.py:174-308 (_decode_kernel and
// _decode_overflow_kernel).  One workgroup per codec block: stage the block's
// payload and tables in LDS, expand its overflow list, then every lane walks
// its stream two symbols per iteration, joining each exponent with its side
// byte and storing the BF16 bits at the swizzled logical offset.  Steps at or
// past a stream's overflow start take their exponent from the tail bytes and
// consume no payload bits.
//
// The step loop runs in 32-step chunks: while a chunk is decoded from the
// wave's LDS side slice, the next chunk's side bytes are already in flight,
// and the overflow check is only compiled into chunks that reach the wave's
// first overflow start.
#include "decode_core.h"

namespace lct {
namespace {

template <bool kFull, bool kOverlay>
__device__ __forceinline__ void decode_chunk(StreamCursor &cursor, const LaneOverlay &lane,
                                             const uint8_t *slice, __amdgpu_buffer_rsrc_t out,
                                             int first_step, int64_t row_base,
                                             uint32_t valid_in_block) {
    const uint32_t t2 = threadIdx.x * 2u;
#pragma unroll
    for (int j = 0; j < kChunkSteps; j += 2) {
        const int step = first_step + j;
        uint32_t f0, len0, f1, len1;
        cursor.next_pair(f0, len0, f1, len1);
        if (kOverlay) overlay_pair(lane, step, f0, len0, f1, len1);
        // Byte offset of the lane's logical column within its row; rows step
        // and step+1 share the swizzle mask.
        const uint32_t col2 = t2 ^ (static_cast<uint32_t>((row_base + step) & 254) * 2u);
        const uint32_t out0 = join_bf16(f0, side_byte(slice, j));
        const uint32_t out1 = join_bf16(f1, side_byte(slice, j + 1));
        const int row_bytes = step * kLanes * 2;
        if (kFull) {
            __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(out0), out, col2, row_bytes, 0);
            __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(out1), out, col2,
                                                  row_bytes + kLanes * 2, 0);
        } else {
            const uint32_t off0 = static_cast<uint32_t>(step) * kLanes + (col2 >> 1);
            const bool v0 = off0 < valid_in_block;
            const bool v1 = off0 + kLanes < valid_in_block;
            if (v0)
                __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(out0), out, col2,
                                                      row_bytes, 0);
            if (v1)
                __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(out1), out, col2,
                                                      row_bytes + kLanes * 2, 0);
            len0 = v0 ? len0 : 0u;
            len1 = v1 ? len1 : 0u;
        }
        cursor.pos += len0 + len1;
    }
}

// S is a template parameter so the chunk loop has a fixed trip count.
// `next` holds the side bytes of chunk 0, fetched by the caller.
template <bool kFull, int S>
__device__ __forceinline__ void decode_rows(StreamCursor cursor, const LaneOverlay &lane,
                                            uint8_t *slice, __amdgpu_buffer_rsrc_t side,
                                            SideChunk next, __amdgpu_buffer_rsrc_t out,
                                            int64_t row_base, uint32_t valid_in_block) {
    static_assert(S % kChunkSteps == 0, "whole chunks");
    const uint32_t voffset = side_fetch_offset();
#pragma unroll 1
    for (int c = 0; c < S; c += kChunkSteps) {
        store_side_chunk(slice, next);
        if (c + kChunkSteps < S) next = fetch_side_chunk(side, voffset, c + kChunkSteps);
        if (c + kChunkSteps > lane.wave_start)
            decode_chunk<kFull, true>(cursor, lane, slice, out, c, row_base, valid_in_block);
        else
            decode_chunk<kFull, false>(cursor, lane, slice, out, c, row_base, valid_in_block);
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
    __shared__ __attribute__((aligned(16))) uint8_t side_slices[kWavesPerBlock][kChunkSteps * kWave];
    const int64_t block = blockIdx.x;
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    const uint32_t block_elems = static_cast<uint32_t>(S) * kLanes;
    const int64_t remaining = logical_numel - logical_base;
    const uint32_t valid = remaining < block_elems ? static_cast<uint32_t>(remaining) : block_elems;
    const __amdgpu_buffer_rsrc_t side_rsrc = make_rsrc(side + logical_base, block_elems);
    const __amdgpu_buffer_rsrc_t out_rsrc = make_rsrc(output + logical_base, 2u * valid);
    // The first side chunk is in flight while the prologue stages the payload.
    const SideChunk first = fetch_side_chunk(side_rsrc, side_fetch_offset(), 0);

    const int32_t center = center_ptr[0];
    build_decode_tables(tb, shifted_decode, center);
    stage_payload(stage, encoded, n_blocks * kLanes, block, W);
    const LaneOverlay lane = build_overlay(ov, has_overlay != 0, block, n_blocks, S, map_start,
                                           map_offset, scratch);
    wait_memory();
    __syncthreads();

    const StreamCursor cursor{stage + threadIdx.x, &tb, 0u, static_cast<uint32_t>(W), rare};
    uint8_t *slice = side_slices[threadIdx.x / kWave];
    if (valid == block_elems) {
        if (S == 128)
            decode_rows<true, 128>(cursor, lane, slice, side_rsrc, first, out_rsrc, row_base, valid);
        else
            decode_rows<true, 256>(cursor, lane, slice, side_rsrc, first, out_rsrc, row_base, valid);
    } else {
        if (S == 128)
            decode_rows<false, 128>(cursor, lane, slice, side_rsrc, first, out_rsrc, row_base, valid);
        else
            decode_rows<false, 256>(cursor, lane, slice, side_rsrc, first, out_rsrc, row_base, valid);
    }
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
