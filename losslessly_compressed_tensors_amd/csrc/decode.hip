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
// chunk's fetch and writes the 16 BF16 values through a wave-private LDS tile
// as 16-byte stores (81.8 -> 78.2 us at 4096 blocks on gfx950 against 4-byte
// stores of lane pairs).  Each stream's first three payload words start in
// registers and only rows 3..W-1 are staged, which keeps the workgroup at
// 19.5 KiB of LDS with the tile; 64 VGPRs keep 8 waves per SIMD.  On gfx9 loads and stores share
// one counter, so a wait for a load also waits for every older store: with the
// decode phase between a chunk's stores and the next wait, those stores have
// drained by the time the wave waits.  The overflow check is only compiled into
// chunks that reach the wave's first overflow start.
#include "decode_core.h"

namespace lct {
namespace {

// Store phase of a full block.  The 8 rows' values go through a wave-private
// 1 KiB LDS tile (8 rows x the wave's 64 columns x 2 bytes) in column order,
// and each lane then stores 16 bytes (8 columns of one row): a wave store
// covers 8 whole 128-byte lines, where a direct store from the decoding lanes
// could only write 2 bytes (or 4, pairing lanes over DPP) per lane.  A wave's
// 64 lanes hold the 64 columns of one aligned group of a row: lane l of the
// wave holds column G + (l ^ (m & 63)) of group G = 64 * wave ^ (m & 192),
// m = the row's swizzle mask.  `first_step` and the block's first row are
// multiples of 8, so rows first_step + j and first_step + j + 1 (j even) share
// mask m0 ^ j, m0 = the mask of row first_step.
__device__ __forceinline__ void store_fields_tile(const uint32_t (&f)[kHalfSteps],
                                                  const uint8_t *slice, int slice_step,
                                                  uint16_t *tile, __amdgpu_buffer_rsrc_t out,
                                                  int first_step, int64_t row_base) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t m0 = static_cast<uint32_t>((row_base + first_step) & 254);
#pragma unroll
    for (int j = 0; j < kHalfSteps; j += 2) {
        const uint32_t pos = lane ^ ((m0 ^ static_cast<uint32_t>(j)) & (kWave - 1));
        tile[j * kWave + pos] =
            static_cast<uint16_t>(join_entry(f[j], side_byte(slice, slice_step + j)));
        tile[(j + 1) * kWave + pos] =
            static_cast<uint16_t>(join_entry(f[j + 1], side_byte(slice, slice_step + j + 1)));
    }
    // Lane l stores row r = first_step + (l >> 3), columns (l & 7) * 8.. of
    // the row's group.
    const uint4 q = reinterpret_cast<const uint4 *>(tile)[lane];
    const uint32_t r = lane >> 3;
    const uint32_t mask = m0 ^ (r & 6u);
    const uint32_t group = ((threadIdx.x & ~(kWave - 1u)) ^ (mask & 192u));
    const uint32_t offset = (group + (lane & 7u) * 8u) * 2u + r * (kLanes * 2u);
    store_b128<kStreaming>(q, out, offset + static_cast<uint32_t>(first_step) * (kLanes * 2));
}

// Store phase of the last, partial block: 2-byte stores of the positions
// inside the tensor.
__device__ __forceinline__ void store_fields_partial(const uint32_t (&f)[kHalfSteps],
                                                     const uint8_t *slice, int slice_step,
                                                     __amdgpu_buffer_rsrc_t out, int first_step,
                                                     int64_t row_base, uint32_t valid_in_block) {
    const uint32_t chunk_col2 = logical_col2(row_base, first_step);
#pragma unroll
    for (int j = 0; j < kHalfSteps; j += 2) {
        const int step = first_step + j;
        const uint32_t out0 = join_entry(f[j], side_byte(slice, slice_step + j));
        const uint32_t out1 = join_entry(f[j + 1], side_byte(slice, slice_step + j + 1));
        const int row_bytes = step * kLanes * 2;
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

template <bool kFull>
__device__ __forceinline__ void store_fields(const uint32_t (&f)[kHalfSteps], const uint8_t *slice,
                                             int slice_step, uint16_t *tile,
                                             __amdgpu_buffer_rsrc_t out, int first_step,
                                             int64_t row_base, uint32_t valid_in_block) {
    if (kFull)
        store_fields_tile(f, slice, slice_step, tile, out, first_step, row_base);
    else
        store_fields_partial(f, slice, slice_step, out, first_step, row_base, valid_in_block);
}

// Chunks [c_begin, c_end) with one overlay variant.  `side_next` holds the side
// bytes of chunk c_begin on entry and of chunk c_end on exit.
template <bool kFull, Overlay kOverlay, int S>
__device__ __forceinline__ void decode_chunks(StreamCursor &cursor, const LaneOverlay &lane,
                                              const uint8_t *tail_lds, uint8_t *slice,
                                              uint16_t *tile,
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
        store_fields<kFull>(f, slice, 0, tile, out, c, row_base, valid_in_block);
        decode_fields<kFull, kOverlay>(cursor, lane, tail_lds, c + kHalfSteps, row_base,
                                       valid_in_block, f);
        store_fields<kFull>(f, slice, kHalfSteps, tile, out, c + kHalfSteps, row_base,
                            valid_in_block);
    }
}

// S is a template parameter so the chunk loops have fixed bounds.  Chunks that
// end at or before the wave's first overflow start skip the overlay check.
template <bool kFull, int S>
__device__ __forceinline__ void decode_rows(StreamCursor cursor, const LaneOverlay &lane,
                                            const uint8_t *tail_lds, uint8_t *slice,
                                            uint16_t *tile,
                                            __amdgpu_buffer_rsrc_t side, SideChunk side_next,
                                            __amdgpu_buffer_rsrc_t out, int64_t row_base,
                                            uint32_t valid_in_block) {
    static_assert(S % kChunkSteps == 0, "whole chunks");
    const int split = min(S, lane.wave_start & ~(kChunkSteps - 1));
    decode_chunks<kFull, kNoOverlay, S>(cursor, lane, tail_lds, slice, tile, side, side_next,
                                        out, row_base, valid_in_block, 0, split);
    if (split == S) return;
    if (lane.lds)
        decode_chunks<kFull, kLdsOverlay, S>(cursor, lane, tail_lds, slice, tile, side,
                                             side_next, out, row_base, valid_in_block, split, S);
    else
        decode_chunks<kFull, kHbmOverlay, S>(cursor, lane, tail_lds, slice, tile, side,
                                             side_next, out, row_base, valid_in_block, split, S);
}

// 8 waves per SIMD: the compiler keeps to 64 VGPRs (65 unconstrained).
__global__ __launch_bounds__(kLanes, 8) void decode_kernel(
    const int32_t *__restrict__ encoded, const uint8_t *__restrict__ side,
    uint16_t *__restrict__ output, const int32_t *__restrict__ shifted_decode,
    const int32_t *__restrict__ center_ptr, int64_t n_blocks, int64_t logical_numel, int S,
    int W, int rare, lct_overflow ov, int has_overlay) {
    extern __shared__ uint32_t stage[];   // register_stage_bytes(W): rows 3..W-1
    __shared__ DecodeTables tb;
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ uint8_t tail_lds[kTailLds];
    __shared__ __attribute__((aligned(16))) uint16_t out_tiles[kWavesPerBlock][kHalfSteps * kWave];
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

    uint32_t words[kRegisterRows];
    load_register_rows(encoded, n_blocks * kLanes, block, words);

    const int32_t center = center_ptr[0];
    build_decode_tables(tb, shifted_decode, center);
    stage_payload_rows(stage, encoded, n_blocks * kLanes, block, kRegisterRows, W);
    const LaneOverlay lane = build_overlay(ov, has_overlay != 0, block, n_blocks, S, map_start,
                                           map_offset, scratch, tail_lds, kTailLds);
    wait_memory();
    __syncthreads();   // payload and tails visible; overflow maps no longer read

    StreamCursor cursor;
    cursor.init_registers(stage + threadIdx.x, &tb, static_cast<uint32_t>(W), rare, words[0],
                          words[1], words[2]);
    uint8_t *slice = side_slices[threadIdx.x / kWave];
    uint16_t *tile = out_tiles[threadIdx.x / kWave];
    if (valid == block_elems) {
        if (S == 128)
            decode_rows<true, 128>(cursor, lane, tail_lds, slice, tile, side_rsrc, first,
                                   out_rsrc, row_base, valid);
        else
            decode_rows<true, 256>(cursor, lane, tail_lds, slice, tile, side_rsrc, first,
                                   out_rsrc, row_base, valid);
    } else {
        if (S == 128)
            decode_rows<false, 128>(cursor, lane, tail_lds, slice, tile, side_rsrc, first,
                                    out_rsrc, row_base, valid);
        else
            decode_rows<false, 256>(cursor, lane, tail_lds, slice, tile, side_rsrc, first,
                                    out_rsrc, row_base, valid);
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
    // Rows 0..2 of every stream start in registers (W = 2 or 3 never occurs in
    // a reference geometry).
    if (g.fixed_words <= kRegisterRows) return LCT_E_GEOMETRY;
    const size_t lds = static_cast<size_t>(register_stage_bytes(g.fixed_words));
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(&decode_kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(decode_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes), lds,
                       stream, encoded, side, reinterpret_cast<uint16_t *>(output),
                       shifted_decode, center, n_blocks, logical_numel, g.steps, g.fixed_words,
                       rare_length, ov, overflow != nullptr ? 1 : 0);
    return static_cast<int32_t>(hipGetLastError());
}
