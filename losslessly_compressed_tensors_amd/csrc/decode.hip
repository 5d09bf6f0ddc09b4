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
// The step loop runs in 16-step chunks, each in two phases.  The decode
// phase walks the 16 steps using only LDS (payload, tables, overflow tails)
// and keeps the exponent fields in registers.  The store phase then waits for
// the chunk's side bytes, which were fetched one chunk earlier, issues the next
// chunk's fetch and writes the 16 BF16 values.  On gfx9 loads and stores share
// one counter, so a wait for a load also waits for every older store: with the
// decode phase between a chunk's stores and the next wait, those stores have
// drained by the time the wave waits.  The overflow check is only compiled into
// chunks that reach the wave's first overflow start.
#include "decode_core.h"

namespace lct {
namespace {

// Store phase.  Lanes j and j^1 hold adjacent columns (c, c+1) of the same
// two rows: the swizzle mask is even, so it never changes bit 0 of a column.
// In a full block the pair swaps one value over DPP so that the even lane
// stores row `step` and the odd lane row `step + 1`, each as one 4-byte
// non-temporal store of both columns: a wave writes 2 x 128 contiguous bytes
// per instruction, which gfx950 streams to HBM markedly faster than 2-byte
// stores.  The last block masks positions past the tensor's end with 2-byte
// stores.  `first_step` and the block's first row are multiples of 8, so the
// column of row first_step + j (j < 8) is the first row's column XOR 2j.
// `first_step` is the first step of these entries; `slice_step` its index in
// the side slice (0 or kHalfSteps).
template <bool kFull>
__device__ __forceinline__ void store_fields(const uint32_t (&f)[kHalfSteps], const uint8_t *slice,
                                             int slice_step, __amdgpu_buffer_rsrc_t out,
                                             int first_step, int64_t row_base,
                                             uint32_t valid_in_block) {
    const uint32_t chunk_col2 = logical_col2(row_base, first_step);
    // Byte form of the swizzle mask of the chunk's first row pair.
    const uint32_t chunk_mask2 = static_cast<uint32_t>((row_base + first_step) & 254) * 2u;
    const bool odd = (threadIdx.x & 1u) != 0;
    // Byte selectors of v_perm_b32(recv, keep, sel): even lanes keep column
    // c in the low half, odd lanes column c+1 in the high half.
    const uint32_t select = odd ? 0x01000504u : 0x05040100u;
    // Even lane: row step, column c; odd lane: row step+1, column c (= its
    // own column - 1).  The swizzle only touches bits 2..8 of this offset.
    const uint32_t pair_offset = ((threadIdx.x * 2u) & ~3u) | (odd ? kLanes * 2u : 0u);
#pragma unroll
    for (int j = 0; j < kHalfSteps; j += 2) {
        const int step = first_step + j;
        const uint32_t out0 = join_entry(f[j], side_byte(slice, slice_step + j));
        const uint32_t out1 = join_entry(f[j + 1], side_byte(slice, slice_step + j + 1));
        const int row_bytes = step * kLanes * 2;
        if (kFull) {
            const uint32_t send = odd ? out0 : out1;
            const uint32_t keep = odd ? out1 : out0;
            // quad_perm [1, 0, 3, 2]: exchange with the neighbouring lane.
            const uint32_t recv = static_cast<uint32_t>(
                __builtin_amdgcn_mov_dpp(static_cast<int>(send), 0xB1, 0xF, 0xF, false));
            const uint32_t word = __builtin_amdgcn_perm(recv, keep, select);
            const uint32_t offset = pair_offset ^ chunk_mask2 ^ static_cast<uint32_t>(2 * j);
            __builtin_amdgcn_raw_buffer_store_b32(word, out, offset, row_bytes, kStreaming);
        } else {
            const uint32_t col2 = chunk_col2 ^ static_cast<uint32_t>(2 * j);
            const uint32_t off0 = static_cast<uint32_t>(step) * kLanes + (col2 >> 1);
            if (off0 < valid_in_block)
                __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(out0), out, col2,
                                                      row_bytes, kStreaming);
            if (off0 + kLanes < valid_in_block)
                __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(out1), out, col2,
                                                      row_bytes + kLanes * 2, kStreaming);
        }
    }
}

// Chunks [c_begin, c_end) with one overlay variant.  `side_next` holds the side
// bytes of chunk c_begin on entry and of chunk c_end on exit.
template <bool kFull, Overlay kOverlay, int S>
__device__ __forceinline__ void decode_chunks(StreamCursor &cursor, const LaneOverlay &lane,
                                              const uint8_t *tail_lds, uint8_t *slice,
                                              __amdgpu_buffer_rsrc_t side, SideChunk &side_next,
                                              __amdgpu_buffer_rsrc_t out, int64_t row_base,
                                              uint32_t valid_in_block, int c_begin, int c_end) {
    const uint32_t voffset = side_fetch_offset();
#pragma unroll 1
    for (int c = c_begin; c < c_end; c += kChunkSteps) {
        uint32_t f[kHalfSteps];
        decode_fields<kFull, kOverlay>(cursor, lane, tail_lds, c, row_base, valid_in_block, f);
        store_side_chunk(slice, side_next);
        if (c + kChunkSteps < S) side_next = fetch_side_chunk(side, voffset, c + kChunkSteps);
        store_fields<kFull>(f, slice, 0, out, c, row_base, valid_in_block);
        decode_fields<kFull, kOverlay>(cursor, lane, tail_lds, c + kHalfSteps, row_base,
                                       valid_in_block, f);
        store_fields<kFull>(f, slice, kHalfSteps, out, c + kHalfSteps, row_base, valid_in_block);
    }
}

// S is a template parameter so the chunk loops have fixed bounds.  Chunks that
// end at or before the wave's first overflow start skip the overlay check.
template <bool kFull, int S>
__device__ __forceinline__ void decode_rows(StreamCursor cursor, const LaneOverlay &lane,
                                            const uint8_t *tail_lds, uint8_t *slice,
                                            __amdgpu_buffer_rsrc_t side, SideChunk side_next,
                                            __amdgpu_buffer_rsrc_t out, int64_t row_base,
                                            uint32_t valid_in_block) {
    static_assert(S % kChunkSteps == 0, "whole chunks");
    const int split = min(S, lane.wave_start & ~(kChunkSteps - 1));
    decode_chunks<kFull, kNoOverlay, S>(cursor, lane, tail_lds, slice, side, side_next, out,
                                        row_base, valid_in_block, 0, split);
    if (split == S) return;
    if (lane.lds)
        decode_chunks<kFull, kLdsOverlay, S>(cursor, lane, tail_lds, slice, side, side_next, out,
                                             row_base, valid_in_block, split, S);
    else
        decode_chunks<kFull, kHbmOverlay, S>(cursor, lane, tail_lds, slice, side, side_next, out,
                                             row_base, valid_in_block, split, S);
}

__global__ __launch_bounds__(kLanes) void decode_kernel(
    const int32_t *__restrict__ encoded, const uint8_t *__restrict__ side,
    uint16_t *__restrict__ output, const int32_t *__restrict__ shifted_decode,
    const int32_t *__restrict__ center_ptr, int64_t n_blocks, int64_t logical_numel, int S,
    int W, int rare, lct_overflow ov, int has_overlay) {
    extern __shared__ uint32_t stage[];   // stage_bytes(W)
    __shared__ DecodeTables tb;
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ uint8_t tail_lds[kTailLds];
    // The overflow maps (2 KiB) are only used before the first side chunk is
    // stored, so they share the side slices' LDS.
    __shared__ __attribute__((aligned(16))) uint8_t side_slices[kWavesPerBlock][kChunkSteps * kWave];
    int32_t *map_start = reinterpret_cast<int32_t *>(&side_slices[0][0]);
    int32_t *map_offset = map_start + kLanes;
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
                                           map_offset, scratch, tail_lds, kTailLds);
    wait_memory();
    __syncthreads();   // payload and tails visible; overflow maps no longer read

    StreamCursor cursor;
    cursor.init(stage + threadIdx.x, &tb, static_cast<uint32_t>(W), rare);
    uint8_t *slice = side_slices[threadIdx.x / kWave];
    if (valid == block_elems) {
        if (S == 128)
            decode_rows<true, 128>(cursor, lane, tail_lds, slice, side_rsrc, first, out_rsrc,
                                   row_base, valid);
        else
            decode_rows<true, 256>(cursor, lane, tail_lds, slice, side_rsrc, first, out_rsrc,
                                   row_base, valid);
    } else {
        if (S == 128)
            decode_rows<false, 128>(cursor, lane, tail_lds, slice, side_rsrc, first, out_rsrc,
                                    row_base, valid);
        else
            decode_rows<false, 256>(cursor, lane, tail_lds, slice, side_rsrc, first, out_rsrc,
                                    row_base, valid);
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
    const size_t lds = static_cast<size_t>(stage_bytes(g.fixed_words));
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(&decode_kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(decode_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes), lds,
                       stream, encoded, side, reinterpret_cast<uint16_t *>(output),
                       shifted_decode, center, n_blocks, logical_numel, g.steps, g.fixed_words,
                       rare_length, ov, overflow != nullptr ? 1 : 0);
    return static_cast<int32_t>(hipGetLastError());
}
