// Fused pointwise operations on compressed BF16 operands (gfx950).
//
// lct_pointwise_dense: decode one compressed operand, combine it with a dense
// BF16 operand and emit dense BF16 or the split components a re-encode
// consumes (LCT/kernels/generic/pointwise.py:84-337).  The reference runs a
// second "fallback" kernel over overflow rows; here the overflow tails are
// overlaid during the same pass, which gives identical results.
//
// lct_dual: alpha * A + B with both operands compressed in the same geometry
// (LCT/kernels/generic/pointwise_scalar_dual.py:17-346); the reference's
// per-stream map kernels are folded into each workgroup's prologue.
//
// Arithmetic (pointwise.py:340-363, _store_result :43-65): operands are
// widened to FP32; add and multiply round once; scalar_mul_add uses FP32
// fma(a, alpha, b) (b pre-scaled by beta in FP32 when beta is given, or
// fma(b, beta, a) when alpha is one); the result is rounded to BF16 to
// nearest-even.  Compressed output: side byte at the storage offset (0 for
// padding), exponent byte at the logical offset.
#include "overflow_walk.h"
#include "pointwise_ops.h"

namespace lct {
namespace {

// Emits one result.  Dense: bf16 at the logical offset.  Compressed: side byte
// at the storage slot (0 when the position is padding) and exponent byte at
// the logical offset.
template <int kPolicy>
__device__ __forceinline__ void store_result(uint32_t bits, bool logical_valid, uint32_t slot,
                                             uint32_t logical, uint16_t *dense_block,
                                             uint8_t *side_out_block, uint8_t *exp_out_block) {
    if (kPolicy == LCT_DENSE_OUTPUT) {
        if (logical_valid) dense_block[logical] = static_cast<uint16_t>(bits);
    } else {
        bits = logical_valid ? bits : 0u;
        side_out_block[slot] = static_cast<uint8_t>(side_byte_of(bits));
        if (logical_valid) exp_out_block[logical] = static_cast<uint8_t>((bits >> 7) & 0xFFu);
    }
}

// Per-workgroup view of the pointwise operands and outputs of one block.
struct PointwiseIo {
    __amdgpu_buffer_rsrc_t side;       // A's side bytes (storage order)
    __amdgpu_buffer_rsrc_t other;      // B, BF16 in logical order
    __amdgpu_buffer_rsrc_t dense;      // dense output (policy 0)
    __amdgpu_buffer_rsrc_t side_out;   // result side bytes (policy 1, storage order)
    __amdgpu_buffer_rsrc_t exp_out;    // result exponent bytes (policy 1, logical order)
};

// One half chunk (8 steps from first_step, entries f) of a full block: B is
// read as one 4-byte word per lane per step pair (lane pairs), the results
// go out as one 4-byte word (dense) or 2 exponent bytes (compressed) per lane
// per pair; compressed side bytes replace A's side bytes in the wave's slice.
template <int kPolicy>
__device__ __forceinline__ void pointwise_half_full(const uint32_t (&f)[kHalfSteps],
                                                    const uint32_t (&bw)[kHalfSteps / 2],
                                                    uint8_t *slice, int slice_step,
                                                    const PointwiseIo &io, const LanePair &lp,
                                                    int first_step, int64_t row_base,
                                                    const OpParams &p) {
    const uint32_t mask = static_cast<uint32_t>((row_base + first_step) & 254);
    const uint32_t lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int j = 0; j < kHalfSteps; j += 2) {
        const int step = first_step + j;
        const int s0 = slice_step + j;
        float b0, b1;
        pair_unpack16(lp, bw[j / 2], b0, b1);
        const uint32_t a0 = join_entry(f[j], side_byte(slice, s0));
        const uint32_t a1 = join_entry(f[j + 1], side_byte(slice, s0 + 1));
        const uint32_t r0 = apply_op_f(p, bf16_to_float(a0), b0);
        const uint32_t r1 = apply_op_f(p, bf16_to_float(a1), b1);
        if (kPolicy == LCT_DENSE_OUTPUT) {
            __builtin_amdgcn_raw_buffer_store_b32(pair_word16(lp, r0, r1), io.dense,
                                                  lp.offset2 ^ (mask * 2u) ^ static_cast<uint32_t>(2 * j),
                                                  step * kLanes * 2, kStreaming);
        } else {
            slice[s0 * kWave + lane] = static_cast<uint8_t>(side_byte_of(r0));
            slice[(s0 + 1) * kWave + lane] = static_cast<uint8_t>(side_byte_of(r1));
            const uint32_t e = pair_word8(lp, (r0 >> 7) & 0xFFu, (r1 >> 7) & 0xFFu);
            __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(e), io.exp_out,
                                                  lp.offset1 ^ mask ^ static_cast<uint32_t>(j),
                                                  step * kLanes, kStreaming);
        }
    }
}

// The same for the last (partial) block: per element, masked.
template <int kPolicy>
__device__ __forceinline__ void pointwise_half_partial(const uint32_t (&f)[kHalfSteps],
                                                       uint8_t *slice, int slice_step,
                                                       const PointwiseIo &io, int first_step,
                                                       int64_t row_base, uint32_t valid_in_block,
                                                       const OpParams &p) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int j = 0; j < kHalfSteps; ++j) {
        const int step = first_step + j;
        const uint32_t col = threadIdx.x ^ static_cast<uint32_t>((row_base + step) & 254);
        const uint32_t off = static_cast<uint32_t>(step) * kLanes + col;
        const bool valid = off < valid_in_block;
        const uint32_t b = valid ? __builtin_amdgcn_raw_buffer_load_b16(io.other, off * 2, 0, 0) : 0u;
        const uint32_t a = join_entry(f[j], side_byte(slice, slice_step + j));
        const uint32_t r = valid ? apply_op(p, a, b) : 0u;
        if (kPolicy == LCT_DENSE_OUTPUT) {
            if (valid)
                __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(r), io.dense, off * 2,
                                                      0, kStreaming);
        } else {
            slice[(slice_step + j) * kWave + lane] = static_cast<uint8_t>(side_byte_of(r));
            if (valid)
                __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>((r >> 7) & 0xFFu),
                                                     io.exp_out, off, 0, kStreaming);
        }
    }
}

// Chunks [c_begin, c_end) with one overlay variant; `side_next` holds A's
// side bytes of chunk c_begin on entry.
template <bool kFull, Overlay kOverlay, int S, int kPolicy>
__device__ __forceinline__ void pointwise_chunks(StreamCursor &cursor, const LaneOverlay &lane,
                                                 const uint8_t *tail_lds, uint8_t *slice,
                                                 SideChunk &side_next, const PointwiseIo &io,
                                                 const LanePair &lp, int64_t row_base,
                                                 uint32_t valid_in_block, int c_begin, int c_end,
                                                 const OpParams &p) {
    const uint32_t voffset = side_fetch_offset();
#pragma unroll 1
    for (int c = c_begin; c < c_end; c += kChunkSteps) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int first = c + half * kHalfSteps;
            uint32_t bw[kHalfSteps / 2];
            if (kFull) {
                // B words of this half, in flight while the entries decode.
                const uint32_t mask2 = static_cast<uint32_t>((row_base + first) & 254) * 2u;
#pragma unroll
                for (int j = 0; j < kHalfSteps; j += 2)
                    bw[j / 2] = __builtin_amdgcn_raw_buffer_load_b32(
                        io.other, lp.offset2 ^ mask2 ^ static_cast<uint32_t>(2 * j),
                        (first + j) * kLanes * 2, 0);
            }
            uint32_t f[kHalfSteps];
            decode_fields<kFull, kOverlay>(cursor, lane, tail_lds, first, row_base,
                                           valid_in_block, f);
            if (half == 0) {
                store_side_chunk(slice, side_next);
                if (c + kChunkSteps < S) side_next = fetch_side_chunk(io.side, voffset, c + kChunkSteps);
            }
            if (kFull)
                pointwise_half_full<kPolicy>(f, bw, slice, half * kHalfSteps, io, lp, first,
                                             row_base, p);
            else
                pointwise_half_partial<kPolicy>(f, slice, half * kHalfSteps, io, first, row_base,
                                                valid_in_block, p);
        }
        if (kPolicy == LCT_COMPRESSED_OUTPUT) {
            // The slice now holds the chunk's result side bytes.
            const uint4 q = reinterpret_cast<const uint4 *>(slice)[threadIdx.x & (kWave - 1)];
            store_b128<kStreaming>(q, io.side_out, voffset + static_cast<uint32_t>(c) * kLanes);
        }
    }
}

template <bool kFull, int S, int kPolicy>
__device__ __forceinline__ void pointwise_rows(StreamCursor cursor, const LaneOverlay &lane,
                                               const uint8_t *tail_lds, uint8_t *slice,
                                               SideChunk side_next, const PointwiseIo &io,
                                               int64_t row_base, uint32_t valid_in_block,
                                               const OpParams &p) {
    const LanePair lp;
    const int split = min(S, lane.wave_start & ~(kChunkSteps - 1));
    pointwise_chunks<kFull, kNoOverlay, S, kPolicy>(cursor, lane, tail_lds, slice, side_next, io,
                                                    lp, row_base, valid_in_block, 0, split, p);
    if (split == S) return;
    if (lane.lds)
        pointwise_chunks<kFull, kLdsOverlay, S, kPolicy>(cursor, lane, tail_lds, slice, side_next,
                                                         io, lp, row_base, valid_in_block, split,
                                                         S, p);
    else
        pointwise_chunks<kFull, kHbmOverlay, S, kPolicy>(cursor, lane, tail_lds, slice, side_next,
                                                         io, lp, row_base, valid_in_block, split,
                                                         S, p);
}

__global__ __launch_bounds__(kLanes) void pointwise_kernel(
    const int32_t *__restrict__ encoded, const uint8_t *__restrict__ side,
    const uint16_t *__restrict__ other, void *output, uint8_t *auxiliary,
    const int32_t *__restrict__ shifted_decode, const int32_t *__restrict__ center_ptr,
    const float *__restrict__ alpha, const float *__restrict__ beta, int64_t n_blocks,
    int64_t logical_numel, int S, int W, int rare, int op, int alpha_is_one, int beta_is_one,
    int policy, lct_overflow ov, int has_overlay) {
    extern __shared__ uint32_t stage[];   // stage_bytes(W)
    __shared__ DecodeTables tb;
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ uint8_t tail_lds[kTailLds];
    __shared__ __attribute__((aligned(16))) uint8_t side_slices[kWavesPerBlock][kChunkSteps * kWave];
    int32_t *map_start = reinterpret_cast<int32_t *>(&side_slices[0][0]);
    int32_t *map_offset = map_start + kLanes;
    const int64_t block = blockIdx.x;
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    const uint32_t block_elems = static_cast<uint32_t>(S) * kLanes;
    const int64_t remaining = logical_numel - logical_base;
    const uint32_t valid = remaining < block_elems ? static_cast<uint32_t>(remaining) : block_elems;
    PointwiseIo io;
    io.side = make_rsrc(side + logical_base, block_elems);
    io.other = make_rsrc(other + logical_base, 2u * valid);
    io.dense = make_rsrc(static_cast<uint16_t *>(output) + logical_base, 2u * valid);
    io.side_out = make_rsrc(static_cast<uint8_t *>(output) + logical_base, block_elems);
    io.exp_out = make_rsrc(auxiliary != nullptr ? auxiliary + logical_base : nullptr,
                           auxiliary != nullptr ? valid : 0u);
    const SideChunk first = fetch_side_chunk(io.side, side_fetch_offset(), 0);

    build_decode_tables(tb, shifted_decode, center_ptr[0]);
    stage_payload(stage, encoded, n_blocks * kLanes, block, W);
    const LaneOverlay lane = build_overlay(ov, has_overlay != 0, block, n_blocks, S, map_start,
                                           map_offset, scratch, tail_lds, kTailLds);
    const OpParams p = load_op_params(op, alpha_is_one, beta_is_one, alpha, beta);
    wait_memory();
    __syncthreads();   // payload and tails visible; overflow maps no longer read

    StreamCursor cursor;
    cursor.init(stage + threadIdx.x, &tb, static_cast<uint32_t>(W), rare);
    uint8_t *slice = side_slices[threadIdx.x / kWave];
#define LCT_POINTWISE_CASE(FULL, POLICY)                                                       \
    if (S == 128)                                                                              \
        pointwise_rows<FULL, 128, POLICY>(cursor, lane, tail_lds, slice, first, io, row_base,   \
                                          valid, p);                                           \
    else                                                                                       \
        pointwise_rows<FULL, 256, POLICY>(cursor, lane, tail_lds, slice, first, io, row_base,   \
                                          valid, p);
    const bool full = valid == block_elems;
    if (policy == LCT_DENSE_OUTPUT) {
        if (full) { LCT_POINTWISE_CASE(true, LCT_DENSE_OUTPUT) }
        else { LCT_POINTWISE_CASE(false, LCT_DENSE_OUTPUT) }
    } else {
        if (full) { LCT_POINTWISE_CASE(true, LCT_COMPRESSED_OUTPUT) }
        else { LCT_POINTWISE_CASE(false, LCT_COMPRESSED_OUTPUT) }
    }
#undef LCT_POINTWISE_CASE
}

template <bool kFull, int S, int kPolicy>
__device__ __forceinline__ void dual_rows(const StreamCursor &a_in, const LaneOverlay &a_lane,
                                          const uint8_t *__restrict__ a_side,
                                          const StreamCursor &b_in, const LaneOverlay &b_lane,
                                          const uint8_t *__restrict__ b_side, uint16_t *dense_block,
                                          uint8_t *side_out_block, uint8_t *exp_out_block,
                                          int64_t row_base, int64_t valid_in_block, float alpha) {
    StreamCursor a = a_in, b = b_in;
    const uint32_t t = threadIdx.x;
#pragma unroll 2
    for (int step = 0; step < S; step += 2) {
        uint32_t af0, af1, bf0, bf1;
        a.next_fields(af0, af1);
        b.next_fields(bf0, bf1);
        const uint32_t slot = static_cast<uint32_t>(step) * kLanes + t;
        const uint32_t asm0 = a_side[slot], asm1 = a_side[slot + kLanes];
        const uint32_t bsm0 = b_side[slot], bsm1 = b_side[slot + kLanes];
        overlay_pair<false, DecodeTables>(a_lane, nullptr, step, af0, af1);
        overlay_pair<false, DecodeTables>(b_lane, nullptr, step, bf0, bf1);
        uint32_t alen0 = af0 & 31u, alen1 = af1 & 31u, blen0 = bf0 & 31u, blen1 = bf1 & 31u;
        const uint32_t col = t ^ static_cast<uint32_t>((row_base + step) & 254);
        const uint32_t off0 = static_cast<uint32_t>(step) * kLanes + col;
        const uint32_t off1 = off0 + kLanes;
        bool v0 = true, v1 = true;
        if (!kFull) {
            v0 = off0 < valid_in_block;
            v1 = off1 < valid_in_block;
            alen0 = v0 ? alen0 : 0u;
            alen1 = v1 ? alen1 : 0u;
            blen0 = v0 ? blen0 : 0u;
            blen1 = v1 ? blen1 : 0u;
        }
        a.advance(alen0 + alen1);
        b.advance(blen0 + blen1);
        const uint32_t r0 = float_to_bf16(__builtin_fmaf(bf16_to_float(join_bf16(af0, asm0)), alpha,
                                                         bf16_to_float(join_bf16(bf0, bsm0))));
        const uint32_t r1 = float_to_bf16(__builtin_fmaf(bf16_to_float(join_bf16(af1, asm1)), alpha,
                                                         bf16_to_float(join_bf16(bf1, bsm1))));
        store_result<kPolicy>(r0, v0, slot, off0, dense_block, side_out_block, exp_out_block);
        store_result<kPolicy>(r1, v1, slot + kLanes, off1, dense_block, side_out_block,
                              exp_out_block);
    }
}

struct DualOperand {
    const int32_t *encoded;
    const uint8_t *side;
    const int32_t *shifted_decode;
    const int32_t *center;
    lct_overflow ov;
    int32_t has_overlay;
    // Per-stream maps from dual_tables_and_maps_kernel (start step, tail byte
    // offset from the tail base), or NULL: the overlay is built from the
    // compact list in the prologue.
    const int32_t *map_start;
    const int32_t *map_offset;
};

// Tail bytes of a tensor's overflow storage start here (the arena region
// after the entries when buffered); NULL when the tensor has no tails (no
// overlay, or a buffered reservation that failed).
__device__ __forceinline__ const uint8_t *tail_base_of(const lct_overflow &ov, bool present) {
    if (!present) return nullptr;
    if (ov.descriptor == nullptr) return ov.tail + ov.base;
    if (ov.descriptor[2] != 0) return nullptr;
    return ov.tail + ov.descriptor[0] + 2 * static_cast<int64_t>(ov.count[0]);
}

// This lane's overlay from the per-stream maps
// (LCT/kernels/generic/pointwise_scalar_dual.py:33-113 writes them).
__device__ __forceinline__ LaneOverlay overlay_from_maps(const DualOperand &x, int64_t block,
                                                         int S) {
    LaneOverlay lane{nullptr, S, 0, S, 0};
    const uint8_t *tails = tail_base_of(x.ov, x.has_overlay != 0);
    if (tails == nullptr) return lane;   // uniform
    const int64_t stream = block * kLanes + threadIdx.x;
    lane.tail = tails;
    lane.start = x.map_start[stream];
    lane.offset = x.map_offset[stream];
    lane.wave_start = __builtin_amdgcn_readfirstlane(wave_min(lane.start));
    return lane;
}

__global__ __launch_bounds__(kLanes) void dual_kernel(DualOperand a, DualOperand b,
                                                      const float *__restrict__ alpha,
                                                      void *output, uint8_t *auxiliary,
                                                      int64_t n_blocks, int64_t logical_numel,
                                                      int S, int W, int rare, int policy) {
    extern __shared__ uint32_t stage[];   // two stages of stage_bytes(W)
    __shared__ DecodeTables tb_a, tb_b;
    __shared__ int32_t map_start[kLanes], map_offset[kLanes], scratch[kWavesPerBlock];
    const int64_t block = blockIdx.x;
    uint32_t *stage_a = stage;
    uint32_t *stage_b = stage + stage_bytes(W) / 4;
    build_decode_tables(tb_a, a.shifted_decode, a.center[0]);
    build_decode_tables(tb_b, b.shifted_decode, b.center[0]);
    stage_payload(stage_a, a.encoded, n_blocks * kLanes, block, W);
    stage_payload(stage_b, b.encoded, n_blocks * kLanes, block, W);
    // build_overlay returns the tail pointer relative to the tail base of the
    // compact list's byte offsets; the maps carry the same offsets.
    const LaneOverlay a_lane = a.map_start != nullptr
        ? overlay_from_maps(a, block, S)
        : build_overlay(a.ov, a.has_overlay != 0, block, n_blocks, S, map_start, map_offset,
                        scratch, nullptr, 0);
    __syncthreads();
    const LaneOverlay b_lane = b.map_start != nullptr
        ? overlay_from_maps(b, block, S)
        : build_overlay(b.ov, b.has_overlay != 0, block, n_blocks, S, map_start, map_offset,
                        scratch, nullptr, 0);
    wait_memory();
    __syncthreads();

    const float alpha_value = alpha[0];
    StreamCursor ca, cb;
    ca.init(stage_a + threadIdx.x, &tb_a, static_cast<uint32_t>(W), rare);
    cb.init(stage_b + threadIdx.x, &tb_b, static_cast<uint32_t>(W), rare);
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    uint16_t *dense_block = static_cast<uint16_t *>(output) + logical_base;
    uint8_t *side_out_block = static_cast<uint8_t *>(output) + logical_base;
    uint8_t *exp_out_block = auxiliary + logical_base;
    const uint8_t *a_side = a.side + logical_base;
    const uint8_t *b_side = b.side + logical_base;
    const int64_t valid = logical_numel - logical_base;
    const bool full = valid >= static_cast<int64_t>(S) * kLanes;
#define LCT_DUAL_CASE(FULL, POLICY)                                                             \
    if (S == 128)                                                                               \
        dual_rows<FULL, 128, POLICY>(ca, a_lane, a_side, cb, b_lane, b_side, dense_block,      \
                                     side_out_block, exp_out_block, row_base, valid,           \
                                     alpha_value);                                             \
    else                                                                                        \
        dual_rows<FULL, 256, POLICY>(ca, a_lane, a_side, cb, b_lane, b_side, dense_block,      \
                                     side_out_block, exp_out_block, row_base, valid,           \
                                     alpha_value);
    if (policy == LCT_DENSE_OUTPUT) {
        if (full) { LCT_DUAL_CASE(true, LCT_DENSE_OUTPUT) }
        else { LCT_DUAL_CASE(false, LCT_DENSE_OUTPUT) }
    } else {
        if (full) { LCT_DUAL_CASE(true, LCT_COMPRESSED_OUTPUT) }
        else { LCT_DUAL_CASE(false, LCT_COMPRESSED_OUTPUT) }
    }
#undef LCT_DUAL_CASE
}

// Overflow rows of a pointwise result computed without the overlay
// (LCT/kernels/generic/pointwise.py:265-340): every tail byte of A is rebuilt
// into BF16 with its side byte, combined with B at its logical position and
// stored as pointwise_kernel stores results (_store_result, pointwise.py:44-65:
// dense BF16 at logical positions, or the side byte at the storage position
// and the exponent byte at the logical position, padding positions giving 0).
__global__ __launch_bounds__(kLanes) void pointwise_fallback_kernel(
    lct_overflow ov, const uint8_t *__restrict__ side, const uint16_t *__restrict__ other,
    void *__restrict__ output, uint8_t *__restrict__ auxiliary, const float *__restrict__ alpha,
    const float *__restrict__ beta, int64_t n_blocks, int64_t logical_numel, int S, int32_t op,
    int32_t alpha_is_one, int32_t beta_is_one, int32_t policy) {
    __shared__ TailEntries entries;
    const OpParams p = load_op_params(op, alpha_is_one, beta_is_one, alpha, beta);
    for (int64_t block = blockIdx.x; block < n_blocks; block += gridDim.x) {
        const TailWalk w = stage_block_entries(ov, block, n_blocks, S, entries);
        if (w.count == 0) continue;   // uniform
        for (int32_t i = threadIdx.x; i < w.bytes; i += kLanes) {
            int32_t step, lane;
            tail_position(w, entries, i, step, lane);
            const int64_t row = block * S + step;
            const int64_t storage = row * kLanes + lane;
            const int64_t logical = row * kLanes + (lane ^ static_cast<int32_t>(row & 254));
            const bool valid = logical < logical_numel;
            const uint32_t a = pack_tail(w.tail[i], side[storage]);
            const uint32_t r = valid ? apply_op(p, a, other[logical]) : 0u;
            if (policy == LCT_DENSE_OUTPUT) {
                if (valid) static_cast<uint16_t *>(output)[logical] = static_cast<uint16_t>(r);
            } else {
                static_cast<uint8_t *>(output)[storage] =
                    static_cast<uint8_t>((r & 0x7Fu) | ((r >> 8) & 0x80u));
                if (valid) auxiliary[logical] = static_cast<uint8_t>((r >> 7) & 0xFFu);
            }
        }
        __syncthreads();   // the entries are restaged for the next block
    }
}

// Both operands' per-stream maps set to "no overflow": start S, offset 0
// (pointwise_scalar_dual.py:17-30).
__global__ __launch_bounds__(kLanes) void dual_maps_init_kernel(int32_t *__restrict__ a_start,
                                                                int32_t *__restrict__ a_offset,
                                                                int32_t *__restrict__ b_start,
                                                                int32_t *__restrict__ b_offset,
                                                                int64_t n_streams, int S) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kLanes + threadIdx.x; i < n_streams;
         i += static_cast<int64_t>(gridDim.x) * kLanes) {
        a_start[i] = S;
        b_start[i] = S;
        a_offset[i] = 0;
        b_offset[i] = 0;
    }
}

// One operand's entries of one block into its per-stream maps: start step
// and tail byte offset (from the tail base) of every overflowing stream.
__device__ __forceinline__ void scatter_block_maps(const lct_overflow &ov, bool present,
                                                   int64_t block, int64_t n_blocks, int S,
                                                   int32_t *map_start, int32_t *map_offset,
                                                   int32_t *scratch) {
    if (tail_base_of(ov, present) == nullptr) return;   // uniform
    const int32_t count = ov.blocks[block];
    if (count <= 0) return;
    int64_t lane_off = 0, start_off = 0;
    if (ov.descriptor != nullptr) {
        lane_off = ov.descriptor[0];
        start_off = lane_off + ov.count[0];
    }
    const int32_t first = ov.blocks[n_blocks + block];
    const int32_t byte_base = ov.blocks[2 * n_blocks + block];
    const int t = threadIdx.x;
    const bool valid = t < count;
    const int32_t start = valid ? static_cast<int32_t>(ov.starts[start_off + first + t]) : S;
    const int32_t lane = valid ? static_cast<int32_t>(ov.lanes[lane_off + first + t]) : 0;
    int32_t total;
    const int32_t local = block_exclusive_scan(valid ? S - start : 0, scratch, &total);
    if (valid) {
        map_start[block * kLanes + lane] = start;
        map_offset[block * kLanes + lane] = byte_base + local;
    }
}

// pointwise_scalar_dual.py:33-113: workgroups 0 and 1 shift A's and B's
// decode tables by their centers; workgroup 2 + k expands block k's compact
// overflow lists of both operands into the per-stream maps.
__global__ __launch_bounds__(kLanes) void dual_tables_and_maps_kernel(
    const int32_t *__restrict__ a_base_decode, const int32_t *__restrict__ a_center,
    int32_t *__restrict__ a_shifted, const int32_t *__restrict__ b_base_decode,
    const int32_t *__restrict__ b_center, int32_t *__restrict__ b_shifted, lct_overflow a_ov,
    int32_t a_present, lct_overflow b_ov, int32_t b_present, int32_t *__restrict__ a_start,
    int32_t *__restrict__ a_offset, int32_t *__restrict__ b_start, int32_t *__restrict__ b_offset,
    int64_t n_blocks, int S) {
    __shared__ int32_t scratch[kWavesPerBlock];
    if (blockIdx.x < 2) {
        const int32_t *base = blockIdx.x == 0 ? a_base_decode : b_base_decode;
        const int32_t center = blockIdx.x == 0 ? a_center[0] : b_center[0];
        int32_t *out = blockIdx.x == 0 ? a_shifted : b_shifted;
        for (int i = threadIdx.x; i < 1024; i += kLanes) out[i] = shifted_decode_entry(base[i], center);
        return;
    }
    const int64_t block = blockIdx.x - 2;
    scatter_block_maps(a_ov, a_present != 0, block, n_blocks, S, a_start, a_offset, scratch);
    scatter_block_maps(b_ov, b_present != 0, block, n_blocks, S, b_start, b_offset, scratch);
}

int32_t check_overflow(const lct_overflow *o) {
    if (o == nullptr) return LCT_OK;
    if (!o->lanes || !o->starts || !o->tail || !o->blocks) return LCT_E_NULL;
    if (o->descriptor != nullptr && o->count == nullptr) return LCT_E_NULL;
    return LCT_OK;
}

int32_t check_sizes(int64_t size, int64_t logical_numel, const lct_geometry &g) {
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (logical_numel <= 0 || size <= 0 || size % g.block_symbols != 0 || logical_numel > size
        || logical_numel <= size - g.block_symbols || size / g.block_symbols > 0x7FFFFFFF)
        return LCT_E_SIZE;
    return LCT_OK;
}

}  // namespace
}  // namespace lct

using namespace lct;

extern "C" int32_t lct_pointwise_dense(const int32_t *encoded, const uint8_t *side,
                                       const void *other, void *output, uint8_t *auxiliary,
                                       const int32_t *shifted_decode, const int32_t *center,
                                       const float *alpha, const float *beta, int64_t size,
                                       int64_t logical_numel, lct_geometry g,
                                       int32_t rare_length, int32_t op, int32_t alpha_is_one,
                                       int32_t beta_is_one, int32_t output_policy,
                                       const lct_overflow *overflow, hipStream_t stream) {
    if (!encoded || !side || !other || !output || !shifted_decode || !center) return LCT_E_NULL;
    if (output_policy == LCT_COMPRESSED_OUTPUT && !auxiliary) return LCT_E_NULL;
    if (op == LCT_OP_SCALAR_MUL_ADD && ((!alpha_is_one && !alpha) || (!beta_is_one && !beta)))
        return LCT_E_NULL;
    if (int32_t e = check_sizes(size, logical_numel, g)) return e;
    if (int32_t e = check_overflow(overflow)) return e;
    if (op < LCT_OP_ADD || op > LCT_OP_SCALAR_MUL_ADD) return LCT_E_ARG;
    if (output_policy != LCT_DENSE_OUTPUT && output_policy != LCT_COMPRESSED_OUTPUT) return LCT_E_ARG;
    if (rare_length < 0 || rare_length > 8) return LCT_E_ARG;
    if ((reinterpret_cast<uintptr_t>(encoded) & 15) != 0) return LCT_E_ARG;
    const lct_overflow ov = overflow ? *overflow : lct_overflow{};
    const int64_t n_blocks = size / g.block_symbols;
    const size_t lds = static_cast<size_t>(stage_bytes(g.fixed_words));
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(&pointwise_kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(pointwise_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes), lds,
                       stream, encoded, side, static_cast<const uint16_t *>(other), output,
                       auxiliary, shifted_decode, center, alpha, beta, n_blocks, logical_numel,
                       g.steps, g.fixed_words, rare_length, op, alpha_is_one, beta_is_one,
                       output_policy, ov, overflow != nullptr ? 1 : 0);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_dual(const int32_t *a_encoded, const uint8_t *a_side,
                            const int32_t *a_shifted_decode, const int32_t *a_center,
                            const lct_overflow *a_overflow, const int32_t *b_encoded,
                            const uint8_t *b_side, const int32_t *b_shifted_decode,
                            const int32_t *b_center, const lct_overflow *b_overflow,
                            const float *alpha, void *output, uint8_t *auxiliary, int64_t size,
                            int64_t logical_numel, lct_geometry g, int32_t rare_length,
                            int32_t output_policy, hipStream_t stream) {
    if (!a_encoded || !a_side || !a_shifted_decode || !a_center || !b_encoded || !b_side
        || !b_shifted_decode || !b_center || !alpha || !output)
        return LCT_E_NULL;
    if (output_policy == LCT_COMPRESSED_OUTPUT && !auxiliary) return LCT_E_NULL;
    if (int32_t e = check_sizes(size, logical_numel, g)) return e;
    if (int32_t e = check_overflow(a_overflow)) return e;
    if (int32_t e = check_overflow(b_overflow)) return e;
    if (output_policy != LCT_DENSE_OUTPUT && output_policy != LCT_COMPRESSED_OUTPUT) return LCT_E_ARG;
    if (rare_length < 0 || rare_length > 8) return LCT_E_ARG;
    if (((reinterpret_cast<uintptr_t>(a_encoded) | reinterpret_cast<uintptr_t>(b_encoded)) & 15) != 0)
        return LCT_E_ARG;
    const DualOperand a{a_encoded, a_side, a_shifted_decode, a_center,
                        a_overflow ? *a_overflow : lct_overflow{}, a_overflow != nullptr,
                        nullptr, nullptr};
    const DualOperand b{b_encoded, b_side, b_shifted_decode, b_center,
                        b_overflow ? *b_overflow : lct_overflow{}, b_overflow != nullptr,
                        nullptr, nullptr};
    const int64_t n_blocks = size / g.block_symbols;
    const size_t lds = 2 * static_cast<size_t>(stage_bytes(g.fixed_words));
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(&dual_kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(dual_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes), lds,
                       stream, a, b, alpha, output, auxiliary, n_blocks, logical_numel, g.steps,
                       g.fixed_words, rare_length, output_policy);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_pointwise_fallback(const lct_overflow *overflow, const uint8_t *side,
                                          const void *other, void *output, uint8_t *auxiliary,
                                          const float *alpha, const float *beta, int64_t size,
                                          int64_t logical_numel, lct_geometry g, int32_t op,
                                          int32_t alpha_is_one, int32_t beta_is_one,
                                          int32_t output_policy, hipStream_t stream) {
    if (!overflow || !side || !other || !output) return LCT_E_NULL;
    if (output_policy == LCT_COMPRESSED_OUTPUT && !auxiliary) return LCT_E_NULL;
    if (op == LCT_OP_SCALAR_MUL_ADD && ((!alpha_is_one && !alpha) || (!beta_is_one && !beta)))
        return LCT_E_NULL;
    if (int32_t e = check_overflow(overflow)) return e;
    if (int32_t e = check_sizes(size, logical_numel, g)) return e;
    if (op < LCT_OP_ADD || op > LCT_OP_SCALAR_MUL_ADD) return LCT_E_ARG;
    if (output_policy != LCT_DENSE_OUTPUT && output_policy != LCT_COMPRESSED_OUTPUT) return LCT_E_ARG;
    const int64_t n_blocks = size / g.block_symbols;
    const uint32_t grid = static_cast<uint32_t>(n_blocks < 2048 ? n_blocks : 2048);
    hipLaunchKernelGGL(pointwise_fallback_kernel, dim3(grid), dim3(kLanes), 0, stream, *overflow,
                       side, static_cast<const uint16_t *>(other), output, auxiliary, alpha, beta,
                       n_blocks, logical_numel, g.steps, op, alpha_is_one, beta_is_one,
                       output_policy);
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_dual_maps_init(int32_t *a_stream_starts, int32_t *a_stream_offsets,
                                      int32_t *b_stream_starts, int32_t *b_stream_offsets,
                                      int64_t n_streams, int32_t steps, hipStream_t stream) {
    if (!a_stream_starts || !a_stream_offsets || !b_stream_starts || !b_stream_offsets)
        return LCT_E_NULL;
    if (n_streams <= 0 || n_streams > kMaxBlocks * kLanes) return LCT_E_SIZE;
    if (steps != 128 && steps != 256) return LCT_E_GEOMETRY;
    const int64_t groups = (n_streams + kLanes - 1) / kLanes;
    const uint32_t grid = static_cast<uint32_t>(groups < 4096 ? groups : 4096);
    hipLaunchKernelGGL(dual_maps_init_kernel, dim3(grid), dim3(kLanes), 0, stream,
                       a_stream_starts, a_stream_offsets, b_stream_starts, b_stream_offsets,
                       n_streams, static_cast<int>(steps));
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_dual_tables_and_maps(
    const int32_t *a_base_decode, const int32_t *a_center, int32_t *a_shifted_decode,
    const int32_t *b_base_decode, const int32_t *b_center, int32_t *b_shifted_decode,
    const lct_overflow *a_overflow, const lct_overflow *b_overflow, int32_t *a_stream_starts,
    int32_t *a_stream_offsets, int32_t *b_stream_starts, int32_t *b_stream_offsets,
    int64_t n_blocks, int32_t steps, hipStream_t stream) {
    if (!a_base_decode || !a_center || !a_shifted_decode || !b_base_decode || !b_center
        || !b_shifted_decode || !a_stream_starts || !a_stream_offsets || !b_stream_starts
        || !b_stream_offsets)
        return LCT_E_NULL;
    if (int32_t e = check_overflow(a_overflow)) return e;
    if (int32_t e = check_overflow(b_overflow)) return e;
    if (n_blocks <= 0 || n_blocks > kMaxBlocks) return LCT_E_SIZE;
    if (steps != 128 && steps != 256) return LCT_E_GEOMETRY;
    hipLaunchKernelGGL(dual_tables_and_maps_kernel, dim3(static_cast<uint32_t>(n_blocks + 2)),
                       dim3(kLanes), 0, stream, a_base_decode, a_center, a_shifted_decode,
                       b_base_decode, b_center, b_shifted_decode,
                       a_overflow ? *a_overflow : lct_overflow{}, a_overflow != nullptr ? 1 : 0,
                       b_overflow ? *b_overflow : lct_overflow{}, b_overflow != nullptr ? 1 : 0,
                       a_stream_starts, a_stream_offsets, b_stream_starts, b_stream_offsets,
                       n_blocks, static_cast<int>(steps));
    return static_cast<int32_t>(hipGetLastError());
}

extern "C" int32_t lct_dual_mapped(
    const int32_t *a_encoded, const uint8_t *a_side, const int32_t *a_shifted_decode,
    const int32_t *a_center, const int32_t *a_stream_starts, const int32_t *a_stream_offsets,
    const lct_overflow *a_overflow, const int32_t *b_encoded, const uint8_t *b_side,
    const int32_t *b_shifted_decode, const int32_t *b_center, const int32_t *b_stream_starts,
    const int32_t *b_stream_offsets, const lct_overflow *b_overflow, const float *alpha,
    void *output, uint8_t *auxiliary, int64_t size, int64_t logical_numel, lct_geometry g,
    int32_t rare_length, int32_t output_policy, hipStream_t stream) {
    if (!a_encoded || !a_side || !a_shifted_decode || !a_center || !b_encoded || !b_side
        || !b_shifted_decode || !b_center || !alpha || !output)
        return LCT_E_NULL;
    if ((a_overflow && (!a_stream_starts || !a_stream_offsets))
        || (b_overflow && (!b_stream_starts || !b_stream_offsets)))
        return LCT_E_NULL;
    if (output_policy == LCT_COMPRESSED_OUTPUT && !auxiliary) return LCT_E_NULL;
    if (int32_t e = check_sizes(size, logical_numel, g)) return e;
    if (int32_t e = check_overflow(a_overflow)) return e;
    if (int32_t e = check_overflow(b_overflow)) return e;
    if (output_policy != LCT_DENSE_OUTPUT && output_policy != LCT_COMPRESSED_OUTPUT) return LCT_E_ARG;
    if (rare_length < 0 || rare_length > 8) return LCT_E_ARG;
    if (((reinterpret_cast<uintptr_t>(a_encoded) | reinterpret_cast<uintptr_t>(b_encoded)) & 15) != 0)
        return LCT_E_ARG;
    // An operand without overflow storage reads no maps (its overlay is off).
    const DualOperand a{a_encoded, a_side, a_shifted_decode, a_center,
                        a_overflow ? *a_overflow : lct_overflow{}, a_overflow != nullptr,
                        a_overflow ? a_stream_starts : nullptr,
                        a_overflow ? a_stream_offsets : nullptr};
    const DualOperand b{b_encoded, b_side, b_shifted_decode, b_center,
                        b_overflow ? *b_overflow : lct_overflow{}, b_overflow != nullptr,
                        b_overflow ? b_stream_starts : nullptr,
                        b_overflow ? b_stream_offsets : nullptr};
    const int64_t n_blocks = size / g.block_symbols;
    const size_t lds = 2 * static_cast<size_t>(stage_bytes(g.fixed_words));
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(&dual_kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(dual_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes), lds,
                       stream, a, b, alpha, output, auxiliary, n_blocks, logical_numel, g.steps,
                       g.fixed_words, rare_length, output_policy);
    return static_cast<int32_t>(hipGetLastError());
}
