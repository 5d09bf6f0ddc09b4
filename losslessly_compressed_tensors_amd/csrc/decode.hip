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
#include <atomic>

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
// Codec block `block` of one tensor, by the workgroup.
__device__ __forceinline__ void decode_block_wide(
    const int32_t *__restrict__ encoded, const uint8_t *__restrict__ side,
    uint16_t *__restrict__ output, const int32_t *__restrict__ shifted_decode,
    const int32_t *__restrict__ center_ptr, int64_t n_blocks, int64_t logical_numel, int S,
    int W, int rare, const lct_overflow &ov, int has_overlay, int64_t block) {
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

__global__ __launch_bounds__(kLanes, 8) void decode_kernel(
    const int32_t *__restrict__ encoded, const uint8_t *__restrict__ side,
    uint16_t *__restrict__ output, const int32_t *__restrict__ shifted_decode,
    const int32_t *__restrict__ center_ptr, int64_t n_blocks, int64_t logical_numel, int S,
    int W, int rare, lct_overflow ov, int has_overlay) {
    decode_block_wide(encoded, side, output, shifted_decode, center_ptr, n_blocks, logical_numel,
                      S, W, rare, ov, has_overlay, blockIdx.x);
}

// Several tensors in one launch (LCT_MAX_DECODE_BATCH at most): workgroup b
// decodes block b - first_block[j] of job j, the last job whose first block
// is at most b.  For tensors of a few codec blocks each (a layer's weights),
// whose decodes are bound by one block's latency, one launch replaces one per
// tensor.  The job table travels in the kernel arguments.
struct DecodeBatchJob {
    const int32_t *encoded;
    const uint8_t *side;
    uint16_t *output;
    const int32_t *shifted_decode;
    const int32_t *center;
    int64_t n_blocks;
    int64_t logical_numel;
    int32_t steps;
    int32_t fixed_words;
    int32_t rare;
    int32_t has_overlay;
    lct_overflow ov;
};

struct DecodeBatch {
    int32_t n_jobs;
    int32_t first_block[LCT_MAX_DECODE_BATCH + 1];
    DecodeBatchJob jobs[LCT_MAX_DECODE_BATCH];
};

__global__ __launch_bounds__(kLanes, 8) void decode_batch_kernel(DecodeBatch batch) {
    const int32_t b = static_cast<int32_t>(blockIdx.x);
    int j = 0;
    for (int k = 1; k < batch.n_jobs; ++k)
        if (b >= batch.first_block[k]) j = k;
    const DecodeBatchJob &job = batch.jobs[j];
    decode_block_wide(job.encoded, job.side, job.output, job.shifted_decode, job.center,
                      job.n_blocks, job.logical_numel, job.steps, job.fixed_words, job.rare,
                      job.ov, job.has_overlay, b - batch.first_block[j]);
}

// ---- the compact decoder: 8 workgroups per CU for payloads of 13 to 19 words
//
// The kernel above keeps 10 KiB of LDS beside its payload stage (the tables,
// the tails, a 1 KiB side slice and a 1 KiB output tile per wave), so from
// W = 13 on it holds more than 20 KiB and fewer than 8 workgroups fit on a CU
// (C2's W = 19: 26 KiB, 6 per CU, so 2048 blocks ran in 1.33 rounds).  This
// variant keeps 3.5 KiB beside the stage (19.5 KiB at W = 19):
//  * side bytes move in 8-step halves, 8 bytes per lane, through a 512-byte
//    region per wave, which then also serves as a 4-row output tile: a lane
//    reads its 8 side bytes before any lane writes the tile (a wave's LDS
//    accesses complete in program order), and each 4-row tile leaves with one
//    8-byte store per lane (4 whole 128-byte lines per wave store);
//  * the escape table is not kept: an escaped literal's exponent field is
//    computed from the center (escapes are rare and take a wave-uniform
//    branch);
//  * the overflow maps (2 KiB) share the four regions before the first half.
// Side bytes are fetched two halves (one 16-step chunk) ahead, as above.

struct CompactDecodeTables {
    uint16_t entry[256];

    __device__ __forceinline__ uint32_t escaped(uint32_t literal, int32_t center) const {
        return static_cast<uint32_t>(
                   (index_to_exponent(static_cast<int32_t>(literal), center) + 127) & 255)
            << 7;
    }
    static __device__ __forceinline__ uint32_t tail(uint32_t byte) {
        return DecodeTables::tail(byte);
    }
};

using CompactCursor = StreamCursorT<kLanes, CompactDecodeTables>;

constexpr int kRegionBytes = kHalfSteps * kWave;   // 512: 8 side rows, or a 4-row tile

// Buffer offset of this lane's 8 bytes within an 8-step half: row j >> 3,
// columns (j & 7) * 8 .. + 8 of the wave's 64-column segment.
__device__ __forceinline__ uint32_t side_half_offset() {
    const uint32_t j = threadIdx.x & (kWave - 1);
    return (j >> 3) * kLanes + (threadIdx.x / kWave) * kWave + (j & 7) * 8;
}

__device__ __forceinline__ uint2 fetch_side_half(__amdgpu_buffer_rsrc_t side, uint32_t voffset,
                                                 int first_step) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                         side, voffset, first_step * kLanes, 0));
}

// The half's entries f joined with its side bytes (q: this lane's 8 fetched
// bytes), stored at their logical positions: full blocks through two 4-row
// tiles in `region`, the last block with 2-byte stores of the positions
// inside the tensor.
template <bool kFull>
__device__ __forceinline__ void store_half_compact(const uint32_t (&f)[kHalfSteps], uint2 q,
                                                   uint8_t *region, __amdgpu_buffer_rsrc_t out,
                                                   int first_step, int64_t row_base,
                                                   uint32_t valid_in_block) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    reinterpret_cast<uint2 *>(region)[lane] = q;   // byte s * 64 + column: step s
    uint32_t v[kHalfSteps];
#pragma unroll
    for (int j = 0; j < kHalfSteps; ++j) v[j] = join_entry(f[j], region[j * kWave + lane]);
    if (!kFull) {
        const uint32_t chunk_col2 = logical_col2(row_base, first_step);
#pragma unroll
        for (int j = 0; j < kHalfSteps; j += 2) {
            const int step = first_step + j;
            const int row_bytes = step * kLanes * 2;
            const uint32_t col2 = chunk_col2 ^ static_cast<uint32_t>(2 * j);
            const uint32_t off0 = static_cast<uint32_t>(step) * kLanes + (col2 >> 1);
            if (off0 < valid_in_block)
                __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(v[j]), out, col2,
                                                      row_bytes, kStreaming);
            if (off0 + kLanes < valid_in_block)
                __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(v[j + 1]), out, col2,
                                                      row_bytes + kLanes * 2, kStreaming);
        }
        return;
    }
    // Tile rows r = 0..3 hold half rows 4t + r; lane l of the wave holds
    // column l ^ (m & 63) of the row's group (m: the row's swizzle mask), and
    // then stores 8 bytes: columns (l & 15) * 4 .. + 4 of tile row l >> 4.
    // first_step and the block's first row are multiples of 8, so half row r
    // has mask m0 ^ (r & 6).
    uint16_t *tile = reinterpret_cast<uint16_t *>(region);
    const uint32_t m0 = static_cast<uint32_t>((row_base + first_step) & 254);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t row = static_cast<uint32_t>(4 * t + r);
            tile[r * kWave + (lane ^ ((m0 ^ (row & 6u)) & (kWave - 1)))] =
                static_cast<uint16_t>(v[4 * t + r]);
        }
        const uint2 d = reinterpret_cast<const uint2 *>(tile)[lane];
        const uint32_t row = 4u * t + (lane >> 4);
        const uint32_t mask = m0 ^ (row & 6u);
        const uint32_t group = (threadIdx.x & ~(kWave - 1u)) ^ (mask & 192u);
        const uint32_t offset = (group + (lane & 15u) * 4u) * 2u
            + (static_cast<uint32_t>(first_step) + row) * (kLanes * 2u);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(
                                                  __attribute__((ext_vector_type(2))) uint32_t, d),
                                              out, offset, 0, kStreaming);
    }
}

// Halves [h_begin, h_end) (in steps) with one overlay variant.  On entry
// `ahead0` and `ahead1` hold the side bytes of halves h_begin and h_begin + 8;
// on exit those of h_end and h_end + 8.
template <bool kFull, Overlay kOverlay, int S>
__device__ __forceinline__ void decode_halves_compact(CompactCursor &cursor,
                                                      const LaneOverlay &lane,
                                                      const uint8_t *tail_lds, uint8_t *region,
                                                      __amdgpu_buffer_rsrc_t side, uint2 &ahead0,
                                                      uint2 &ahead1, __amdgpu_buffer_rsrc_t out,
                                                      int64_t row_base, uint32_t valid_in_block,
                                                      int h_begin, int h_end) {
    const uint32_t voffset = side_half_offset();
#pragma unroll 1
    for (int h = h_begin; h < h_end; h += kHalfSteps) {
        uint32_t f[kHalfSteps];
        decode_fields<kFull, kOverlay>(cursor, lane, tail_lds, h, row_base, valid_in_block, f);
        const uint2 q = ahead0;
        ahead0 = ahead1;
        if (h + 2 * kHalfSteps < S)
            ahead1 = fetch_side_half(side, voffset, h + 2 * kHalfSteps);
        store_half_compact<kFull>(f, q, region, out, h, row_base, valid_in_block);
    }
}

template <bool kFull, int S>
__device__ __forceinline__ void decode_rows_compact(CompactCursor cursor, const LaneOverlay &lane,
                                                    const uint8_t *tail_lds, uint8_t *region,
                                                    __amdgpu_buffer_rsrc_t side, uint2 ahead0,
                                                    uint2 ahead1, __amdgpu_buffer_rsrc_t out,
                                                    int64_t row_base, uint32_t valid_in_block) {
    const int split = min(S, lane.wave_start & ~(kHalfSteps - 1));
    decode_halves_compact<kFull, kNoOverlay, S>(cursor, lane, tail_lds, region, side, ahead0,
                                                ahead1, out, row_base, valid_in_block, 0, split);
    if (split == S) return;
    if (lane.lds)
        decode_halves_compact<kFull, kLdsOverlay, S>(cursor, lane, tail_lds, region, side,
                                                     ahead0, ahead1, out, row_base,
                                                     valid_in_block, split, S);
    else
        decode_halves_compact<kFull, kHbmOverlay, S>(cursor, lane, tail_lds, region, side,
                                                     ahead0, ahead1, out, row_base,
                                                     valid_in_block, split, S);
}

// LDS beside the payload stage: the entry table, scan scratch, the tails and
// the four regions.
constexpr int32_t kCompactStaticLds = 512 + 16 + kTailLds + kWavesPerBlock * kRegionBytes;
static_assert(register_stage_bytes(19) + kCompactStaticLds <= 20 * 1024,
              "MEDIUM's payload (W = 19) keeps 8 workgroups per CU");

__global__ __launch_bounds__(kLanes, 8) void decode_kernel_compact(
    const int32_t *__restrict__ encoded, const uint8_t *__restrict__ side,
    uint16_t *__restrict__ output, const int32_t *__restrict__ shifted_decode,
    const int32_t *__restrict__ center_ptr, int64_t n_blocks, int64_t logical_numel, int S,
    int W, int rare, lct_overflow ov, int has_overlay) {
    extern __shared__ uint32_t stage[];   // register_stage_bytes(W): rows 3..W-1
    __shared__ CompactDecodeTables tb;
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ uint8_t tail_lds[kTailLds];
    __shared__ __attribute__((aligned(16))) uint8_t regions[kWavesPerBlock][kRegionBytes];
    static_assert(sizeof(regions) >= 2 * kLanes * sizeof(int32_t), "the overflow maps fit");
    int32_t *map_start = reinterpret_cast<int32_t *>(&regions[0][0]);
    int32_t *map_offset = map_start + kLanes;
    const int64_t block = blockIdx.x;
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    const uint32_t block_elems = static_cast<uint32_t>(S) * kLanes;
    const int64_t remaining = logical_numel - logical_base;
    const uint32_t valid = remaining < block_elems ? static_cast<uint32_t>(remaining) : block_elems;
    const __amdgpu_buffer_rsrc_t side_rsrc = make_rsrc(side + logical_base, block_elems);
    const __amdgpu_buffer_rsrc_t out_rsrc = make_rsrc(output + logical_base, 2u * valid);
    // The first two side halves are in flight while the prologue stages the
    // payload.
    const uint32_t voffset = side_half_offset();
    const uint2 ahead0 = fetch_side_half(side_rsrc, voffset, 0);
    const uint2 ahead1 = fetch_side_half(side_rsrc, voffset, kHalfSteps);

    uint32_t words[kRegisterRows];
    load_register_rows(encoded, n_blocks * kLanes, block, words);

    const int32_t center = center_ptr[0];
    {
        const int32_t packed = shifted_decode[threadIdx.x];
        const int32_t length = packed & 255;
        const uint32_t field = static_cast<uint32_t>(((packed >> 8) + 127) & 255) << 7;
        tb.entry[threadIdx.x] = static_cast<uint16_t>(
            (length >= 1 && length <= 8) ? (static_cast<uint32_t>(length) | field)
                                         : static_cast<uint32_t>(kEscapeLength));
    }
    stage_payload_rows(stage, encoded, n_blocks * kLanes, block, kRegisterRows, W);
    const LaneOverlay lane = build_overlay(ov, has_overlay != 0, block, n_blocks, S, map_start,
                                           map_offset, scratch, tail_lds, kTailLds);
    wait_memory();
    __syncthreads();   // payload and tails visible; overflow maps no longer read

    CompactCursor cursor;
    cursor.init_registers(stage + threadIdx.x, &tb, static_cast<uint32_t>(W), rare, words[0],
                          words[1], words[2], center);
    uint8_t *region = regions[threadIdx.x / kWave];
    if (valid == block_elems) {
        if (S == 128)
            decode_rows_compact<true, 128>(cursor, lane, tail_lds, region, side_rsrc, ahead0,
                                           ahead1, out_rsrc, row_base, valid);
        else
            decode_rows_compact<true, 256>(cursor, lane, tail_lds, region, side_rsrc, ahead0,
                                           ahead1, out_rsrc, row_base, valid);
    } else {
        if (S == 128)
            decode_rows_compact<false, 128>(cursor, lane, tail_lds, region, side_rsrc, ahead0,
                                            ahead1, out_rsrc, row_base, valid);
        else
            decode_rows_compact<false, 256>(cursor, lane, tail_lds, region, side_rsrc, ahead0,
                                            ahead1, out_rsrc, row_base, valid);
    }
}

// Workgroups of each decoder that the current device holds at once for W
// payload words (CUs x workgroups per CU at that kernel's LDS), looked up once
// per device and W.
constexpr int kSlotDevices = 64;
std::atomic<int64_t> g_decoder_slots[kSlotDevices][kMaxWords + 1];

// lct_set_decoder's choice (LCT_DECODER_*).
std::atomic<int32_t> g_decoder_mode{LCT_DECODER_AUTO};

int32_t decoder_slots(int W, int32_t *wide, int32_t *compact) {
    int device = 0;
    if (hipError_t e = hipGetDevice(&device)) return static_cast<int32_t>(e);
    if (device < 0 || device >= kSlotDevices || W < 0 || W > kMaxWords) return LCT_E_ARG;
    int64_t cached = g_decoder_slots[device][W].load(std::memory_order_relaxed);
    if (cached == 0) {
        int cus = 0, per_wide = 0, per_compact = 0;
        const size_t lds = static_cast<size_t>(register_stage_bytes(W));
        if (hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                                                 device))
            return static_cast<int32_t>(e);
        if (hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_wide, reinterpret_cast<const void *>(decode_kernel), kLanes, lds))
            return static_cast<int32_t>(e);
        if (hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_compact, reinterpret_cast<const void *>(decode_kernel_compact), kLanes,
                lds))
            return static_cast<int32_t>(e);
        cached = (static_cast<int64_t>(cus) * per_wide << 32)
                 | static_cast<uint32_t>(cus * per_compact);
        g_decoder_slots[device][W].store(cached, std::memory_order_relaxed);
    }
    *wide = static_cast<int32_t>(cached >> 32);
    *compact = static_cast<int32_t>(cached & 0xFFFFFFFF);
    return LCT_OK;
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
    int32_t wide_slots = 0, compact_slots = 0;
    if (int32_t e = decoder_slots(g.fixed_words, &wide_slots, &compact_slots)) return e;
    // The wide-tile kernel, unless the whole grid fits the device at once only
    // with the compact one (C2: 2048 blocks at W = 19 take 1.33 rounds of the
    // wide kernel, one of the compact; 51.5 -> 44.8 us).  With the same number
    // of rounds the wide kernel's 16-byte stores are faster (W = 25: 81 against
    // 90 us at 2048 blocks, 347 against 366 us at 8192; C3: 40 against 44 us).
    const int32_t mode = g_decoder_mode.load(std::memory_order_relaxed);
    const bool compact = mode == LCT_DECODER_AUTO
                             ? n_blocks > wide_slots && n_blocks <= compact_slots
                             : mode == LCT_DECODER_COMPACT;
    const auto kernel = compact ? decode_kernel_compact : decode_kernel;
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes), lds,
                       stream, encoded, side, reinterpret_cast<uint16_t *>(output),
                       shifted_decode, center, n_blocks, logical_numel, g.steps, g.fixed_words,
                       rare_length, ov, overflow != nullptr ? 1 : 0);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_set_decoder(int32_t mode) {
    if (mode != LCT_DECODER_AUTO && mode != LCT_DECODER_WIDE && mode != LCT_DECODER_COMPACT)
        return LCT_E_ARG;
    g_decoder_mode.store(mode, std::memory_order_relaxed);
    return LCT_OK;
}

extern "C" int32_t lct_decode_batch(const lct_decode_job *jobs, int32_t n_jobs,
                                    hipStream_t stream) {
    if (!jobs) return LCT_E_NULL;
    if (n_jobs <= 0 || n_jobs > LCT_MAX_DECODE_BATCH) return LCT_E_ARG;
    DecodeBatch batch{};
    batch.n_jobs = n_jobs;
    int64_t total = 0;
    size_t lds = 0;
    for (int32_t j = 0; j < n_jobs; ++j) {
        const lct_decode_job &in = jobs[j];
        if (!in.encoded || !in.side || !in.output || !in.shifted_decode || !in.center)
            return LCT_E_NULL;
        const lct_geometry &g = in.geometry;
        if (!geometry_ok(g)) return LCT_E_GEOMETRY;
        if (in.logical_numel <= 0 || in.size <= 0 || in.size % g.block_symbols != 0
            || in.logical_numel > in.size || in.logical_numel <= in.size - g.block_symbols)
            return LCT_E_SIZE;
        if (in.rare_length < 0 || in.rare_length > 8) return LCT_E_ARG;
        if ((reinterpret_cast<uintptr_t>(in.encoded) & 15) != 0) return LCT_E_ARG;
        if (g.fixed_words <= kRegisterRows) return LCT_E_GEOMETRY;
        if (in.has_overflow) {
            const lct_overflow &o = in.overflow;
            if (!o.lanes || !o.starts || !o.tail || !o.blocks) return LCT_E_NULL;
            if (o.descriptor != nullptr && o.count == nullptr) return LCT_E_NULL;
        }
        const int64_t n_blocks = in.size / g.block_symbols;
        batch.first_block[j] = static_cast<int32_t>(total);
        total += n_blocks;
        if (total > 0x7FFFFFFF) return LCT_E_SIZE;
        DecodeBatchJob &out = batch.jobs[j];
        out.encoded = in.encoded;
        out.side = in.side;
        out.output = reinterpret_cast<uint16_t *>(in.output);
        out.shifted_decode = in.shifted_decode;
        out.center = in.center;
        out.n_blocks = n_blocks;
        out.logical_numel = in.logical_numel;
        out.steps = g.steps;
        out.fixed_words = g.fixed_words;
        out.rare = in.rare_length;
        out.has_overlay = in.has_overflow ? 1 : 0;
        out.ov = in.has_overflow ? in.overflow : lct_overflow{};
        const size_t job_lds = static_cast<size_t>(register_stage_bytes(g.fixed_words));
        lds = job_lds > lds ? job_lds : lds;
    }
    batch.first_block[n_jobs] = static_cast<int32_t>(total);
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(&decode_batch_kernel),
                                           lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(decode_batch_kernel, dim3(static_cast<uint32_t>(total)), dim3(kLanes), lds,
                       stream, batch);
    return static_cast<int32_t>(hipGetLastError());
}
