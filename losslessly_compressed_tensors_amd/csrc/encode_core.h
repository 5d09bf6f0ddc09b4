// Field split + fixed-payload Huffman encoder for gfx950: the device code of
// one codec block, shared by the encoder launches (encode.hip) and the fused
// compress (compress.hip).
//
// One workgroup per codec block, one thread per lane (= one Huffman stream),
// as the format requires (LCT/kernels/generic/encode.py:10-169).  Per step
// pair a lane takes two BF16 values at the swizzled logical offsets (one
// column for both rows), emits their side bytes in storage order, looks the
// exponent bytes up in an LDS copy of the shifted encode table and appends the
// concatenated pair code at its bit position `pos`.
//
// Memory traffic is organised per wave and per 16-step chunk:
//  * input: a wave's lanes read one aligned 64-column group (128 bytes of
//    BF16, or 64 exponent bytes) per row, so a chunk is 2 KiB (1 KiB) per
//    wave; it is fetched with 16-byte non-temporal buffer loads two chunks
//    ahead of use and staged in a wave-private LDS slice;
//  * side bytes: one 16-byte store per lane per chunk, with the cache policy
//    the launch picks (kSidePolicy).  Non-temporal stores go out as whole
//    128-byte lines: the waves of a pair hold the two 64-byte halves of each
//    row's line, so after a barrier each wave stores 8 of the chunk's 16 rows
//    (half-line stores wrote 208 MB against 186 MB of side bytes at 4096
//    blocks of 128 steps, and the public compress took 94 us against 89).
//    The default policy (its L2 merges the halves) stores each wave's own
//    half lines: at 1024 blocks of 256 steps (every block resident at once)
//    55 us against 57 us with the joined non-temporal lines.  Measured with
//    each call's outputs in fresh memory.  The input loads are non-temporal
//    (default-policy loads: 91 us against 88 in the encoder alone at 4096
//    blocks);
//  * payload: built in a zeroed LDS stage -- each pair ORs its code, placed at
//    the lane's bit position, into stage rows pos/32 and pos/32 + 1 (two
//    ds_or_b32, conflict-free: row stride 256 words), so no partial word is
//    carried in registers; after the loop the block copies rows 0..W-1 to
//    `encoded` with 16-byte stores of the default cache policy (each block's
//    rows are 1 KiB pieces 4 MiB apart; non-temporal stores of them took the
//    kernel from 82 to 88 us at 4096 blocks).  Rows W and W+1 are pad rows
//    that take the pairs that do not fit;
//  * side bytes: once a pair's two input rows are read, their side bytes take
//    the first 64 bytes of those rows in the input slice.
//
// Overflow rule (encode.py:73-90): a pair overflows when pos + len > 32W; the
// first overflowing pair's even step is the stream's extra_start and word W-1
// keeps only the bits before that pair (the overflowing pairs go to the pad
// rows).  A stream's position only grows, so the first overflowing pair is the
// one after the pairs that fit: extra_start = 2 * (pairs that fit).
#pragma once

#include "decode_core.h"

namespace lct {

constexpr int kEncChunk = 16;   // steps per staged input chunk
constexpr uint32_t kSliceBytes = 2 * kEncChunk * kWave;   // one wave's input chunk

using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

// Encode-table entry as the kernel keeps it in LDS: {reversed code (<= 16
// bits), code length}, 8 bytes, so one 8-byte read gives both without masks.
__device__ __forceinline__ uint2 repack_encode_entry(uint32_t packed) {
    return make_uint2(packed & 0xFFFFu, packed >> 20);
}

// Input of one 16-step chunk for this lane: BF16 chunks are two 16-byte
// pieces (8 rows x 128 bytes per piece and wave), exponent-byte chunks one
// (16 rows x 64 bytes).
struct InputChunk {
    u32x4 q0, q1;
};

// Byte offset (within the block's logical data) of this lane's 16-byte piece
// `piece` of the chunk starting at `first_step`.
template <bool kPrecomputed>
__device__ __forceinline__ uint32_t input_offset(int64_t row_base, int first_step, int piece) {
    const uint32_t j = threadIdx.x & (kWave - 1);
    const uint32_t wave = threadIdx.x / kWave;
    if (kPrecomputed) {
        const uint32_t step = static_cast<uint32_t>(first_step) + (j >> 2);
        const uint32_t group = wave ^ static_cast<uint32_t>(((row_base + step) & 0xC0) >> 6);
        return step * kLanes + group * kWave + (j & 3) * 16;
    }
    const uint32_t step = static_cast<uint32_t>(first_step + piece * 8) + (j >> 3);
    const uint32_t group = wave ^ static_cast<uint32_t>(((row_base + step) & 0xC0) >> 6);
    return (step * kLanes + group * kWave) * 2 + (j & 7) * 16;
}

// 16 bytes at `offset`; in the block holding the logical end, bytes at or past
// `valid_bytes` read as 0 and are fetched one by one when a piece straddles it.
template <bool kFull>
__device__ __forceinline__ u32x4 fetch_piece(__amdgpu_buffer_rsrc_t src, uint32_t offset,
                                             uint32_t valid_bytes) {
    if (kFull || offset + 16 <= valid_bytes)
        return __builtin_amdgcn_raw_buffer_load_b128(src, offset, 0, kStreaming);
    u32x4 out = {0u, 0u, 0u, 0u};
    if (offset < valid_bytes) {
        for (uint32_t k = 0; k < 16; ++k) {
            if (offset + k < valid_bytes) {
                const uint32_t b = __builtin_amdgcn_raw_buffer_load_b8(src, offset + k, 0, 0);
                out[k >> 2] |= b << ((k & 3) * 8);
            }
        }
    }
    return out;
}

template <bool kFull, bool kPrecomputed>
__device__ __forceinline__ InputChunk fetch_input(__amdgpu_buffer_rsrc_t src, int64_t row_base,
                                                  int first_step, uint32_t valid_bytes) {
    InputChunk c;
    c.q0 = fetch_piece<kFull>(src, input_offset<kPrecomputed>(row_base, first_step, 0),
                              valid_bytes);
    if (!kPrecomputed)
        c.q1 = fetch_piece<kFull>(src, input_offset<false>(row_base, first_step, 1), valid_bytes);
    return c;
}

// Slice layout: row r of the chunk at r * 128 (BF16) or r * 64 (bytes); a
// lane's piece lands at j * 16 (+ 1024 for the second BF16 piece).
template <bool kPrecomputed>
__device__ __forceinline__ void store_input(uint8_t *slice, const InputChunk &c) {
    const uint32_t j = threadIdx.x & (kWave - 1);
    reinterpret_cast<u32x4 *>(slice)[j] = c.q0;
    if (!kPrecomputed) reinterpret_cast<u32x4 *>(slice + 1024)[j] = c.q1;
}

// OR `value` into the stage word at `word` (ds_or_b32).  The pointer keeps
// its provenance (the dynamic stage, not the static input slices), so the
// compiler may move later pairs' slice and table reads above these writes.
__device__ __forceinline__ void lds_or(uint32_t *word, uint32_t value) {
    __hip_atomic_fetch_or(word, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Side byte of BF16 bits v in bits 0..7 (higher bits are not meaningful):
// mantissa bits 0..6 and the sign, one bit-field insert.
__device__ __forceinline__ uint32_t side_bits_low(uint32_t v) {
    uint32_t out;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(out) : "s"(0x7Fu), "v"(v), "v"(v >> 8));
    return out;
}

// Row r of a BF16 chunk occupies bytes r*128 .. r*128+127 of the slice; once
// the wave has read rows p and p+1 (both at once, LDS operations of a wave
// complete in order), their side bytes take the first 64 bytes of those rows.
constexpr uint32_t kInRowBytes = 2 * kWave;

template <bool kFull, bool kPrecomputed, int S, int kSidePolicy>
__device__ __forceinline__ void encode_block(
    __amdgpu_buffer_rsrc_t src, __amdgpu_buffer_rsrc_t side, const uint2 *__restrict__ table,
    uint32_t *__restrict__ stage, uint8_t *in_slice, int64_t row_base,
    uint32_t valid_in_block, int W, InputChunk next, bool &overflow_out, int &extra_out) {
    const uint32_t lane = threadIdx.x;
    const uint32_t j = lane & (kWave - 1);
    const uint32_t limit = static_cast<uint32_t>(W) * 32u;
    // Stage rows are 1 KiB apart; rows W and W+1 are pad rows that take the
    // words of pairs that do not fit.
    uint32_t *const lane_word = stage + lane;
    uint32_t *const pad_word = lane_word + W * kLanes;
    const uint32_t valid_bytes = valid_in_block * (kPrecomputed ? 1u : 2u);
    // Side bytes of a chunk leave as one 16-byte store per lane: row j/4 of
    // the chunk, bytes (j%4)*16.. of the wave's 64-byte segment.
    const uint32_t side_store_offset = side_fetch_offset();
    const uint32_t side_read = (j >> 2) * kInRowBytes + (j & 3) * 16;
    // Non-temporal side stores go out as whole 128-byte lines: the waves of a
    // pair (2p, 2p+1) hold the two halves of each row's line, so after a
    // barrier wave 2p stores rows 0..7 of the chunk and wave 2p+1 rows 8..15,
    // each lane 16 bytes read from the slice of the wave that encoded them.
    constexpr bool kJoinLines = kSidePolicy == kStreaming;
    const uint32_t wave = lane / kWave;
    const uint32_t join_row = (wave & 1u) * 8u + (j >> 3);
    const uint8_t *const join_read = in_slice - (wave & 1u) * kSliceBytes
                                     + ((j >> 2) & 1u) * kSliceBytes + join_row * kInRowBytes
                                     + (j & 3u) * 16u;
    const uint32_t join_store_offset = join_row * kLanes + (wave >> 1) * 128u + (j & 7u) * 16u;

    uint32_t pos = 0;
    // Pairs that fit.  pos only grows, so they are exactly the pairs before the
    // first one that does not, and that pair's even step is 2 * fits.
    uint32_t fits = 0;
    // Input chunks are fetched two ahead, alternating between `next` and
    // `later` (no copy of a register that a load is still filling); a fetch
    // past the block reads zeros from the range check, without memory traffic.
    InputChunk later = fetch_input<kFull, kPrecomputed>(src, row_base, kEncChunk, valid_bytes);
    auto chunk = [&](int c, InputChunk &held) {
        store_input<kPrecomputed>(in_slice, held);
        held = fetch_input<kFull, kPrecomputed>(src, row_base, c + 2 * kEncChunk, valid_bytes);
        // Column of this lane inside its wave's 64-column group: the row mask's
        // low six bits.  The chunk's first row is a multiple of 16, so row c+p
        // has mask ^ p (rows p and p+1 share it).
        const uint32_t colbase = j ^ static_cast<uint32_t>((row_base + c) & 62);
#pragma unroll
        for (int p = 0; p < kEncChunk; p += 2) {
            const int step = c + p;
            const uint32_t colg = colbase ^ static_cast<uint32_t>(p);
            // Byte offsets of the two exponents' table entries: exponent * 8.
            uint32_t t0, t1;
            if (kPrecomputed) {
                t0 = static_cast<uint32_t>(in_slice[p * kWave + colg]) * 8u;
                t1 = static_cast<uint32_t>(in_slice[(p + 1) * kWave + colg]) * 8u;
            } else {
                const uint32_t v0 = *reinterpret_cast<const uint16_t *>(in_slice + p * kInRowBytes + colg * 2);
                const uint32_t v1 = *reinterpret_cast<const uint16_t *>(in_slice + (p + 1) * kInRowBytes + colg * 2);
                t0 = (v0 >> 4) & 0x7F8u;
                t1 = (v1 >> 4) & 0x7F8u;
                in_slice[p * kInRowBytes + j] = static_cast<uint8_t>(side_bits_low(v0));
                in_slice[(p + 1) * kInRowBytes + j] = static_cast<uint8_t>(side_bits_low(v1));
            }
            const uint8_t *table_bytes = reinterpret_cast<const uint8_t *>(table);
            uint2 p0 = *reinterpret_cast<const uint2 *>(table_bytes + t0);
            uint2 p1 = *reinterpret_cast<const uint2 *>(table_bytes + t1);
            if (!kFull) {
                // Positions past the logical end carry no code (encode.py:255-256).
                const uint32_t off0 = static_cast<uint32_t>(step) * kLanes
                    + (lane ^ static_cast<uint32_t>((row_base + step) & 254));
                if (off0 >= valid_in_block) p0 = make_uint2(0u, 0u);
                if (off0 + kLanes >= valid_in_block) p1 = make_uint2(0u, 0u);
            }
            const uint32_t code = p0.x | (p1.x << p0.y);
            const uint32_t after = pos + p0.y + p1.y;
            // The pair's bits are ORed into the zeroed stage: rows pos/32 and
            // pos/32 + 1 (the second is the pad row W when the pair ends the
            // stream).  A pair that does not fit goes to the pad rows, so a
            // stream's word W-1 keeps exactly the bits before its first
            // overflowing pair (encode.py:73-90).
            const uint64_t placed = static_cast<uint64_t>(code) << (pos & 31u);
            const bool over = after > limit;
            uint32_t *const word = over ? pad_word : lane_word + (pos >> 5) * kLanes;
            lds_or(word, static_cast<uint32_t>(placed));
            lds_or(word + kLanes, static_cast<uint32_t>(placed >> 32));
            fits += over ? 0u : 1u;
            pos = after;
        }
        if (!kPrecomputed && kJoinLines) {
            __syncthreads();   // the pair's side bytes of this chunk are in its slices
            const u32x4 sides = *reinterpret_cast<const u32x4 *>(join_read);
            __builtin_amdgcn_raw_buffer_store_b128(sides, side, join_store_offset + c * kLanes, 0,
                                                   kSidePolicy);
            __syncthreads();   // read before the partner's next chunk overwrites its slice
        } else if (!kPrecomputed) {
            const u32x4 sides = *reinterpret_cast<const u32x4 *>(in_slice + side_read);
            __builtin_amdgcn_raw_buffer_store_b128(sides, side, side_store_offset + c * kLanes, 0,
                                                   kSidePolicy);
        }
    };
#pragma unroll 1
    for (int c = 0; c < S; c += 2 * kEncChunk) {
        chunk(c, next);
        chunk(c + kEncChunk, later);
    }
    overflow_out = pos > limit;
    extra_out = static_cast<int>(2 * fits);
}

// Where the encoder's table comes from: the center-shifted encode table; or
// the sampler's partial sums (int32 pairs written by an earlier launch, or
// epoch-tagged control words written by sampling workgroups of the same
// launch) plus the distribution's base tables: the center and shifted tables
// are then derived in every workgroup, and workgroup 0 also stores the center
// and the shifted decode table.
struct TableSource {
    const int32_t *shifted_encode;
    const int32_t *partials;
    int32_t n_groups;
    const int32_t *base_encode;
    const int32_t *base_decode;
    int32_t *center_out;
    int32_t *shifted_decode_out;
    const uint64_t *control;   // tagged partial sums, polled (fused compress)
    uint32_t epoch;
    int32_t polls;
};

// The workgroup's LDS encode table.  With sampler partials, wave 0 reduces
// them to the center while the raw base table waits in `raw` (LDS the first
// input chunk overwrites only later); workgroup 0 stores the center and the
// shifted decode table.  Contains a barrier when sampled.  Returns (uniform)
// whether polled partials failed to arrive within the poll limit (the block
// is then encoded under center 0 and reported as failed).
__device__ __forceinline__ bool setup_table(const TableSource &tables, uint2 *table,
                                            int32_t *raw, int32_t *shared, int64_t block) {
    const int t = threadIdx.x;
    if (tables.partials == nullptr && tables.control == nullptr) {
        table[t] = repack_encode_entry(static_cast<uint32_t>(tables.shifted_encode[t]));
        return false;
    }
    raw[t] = tables.base_encode[t];
    // Workgroup 0 also writes the shifted decode table: its base entries are
    // loaded with the rest, before the center is known.
    int32_t base[1024 / kLanes] = {};
    if (block == 0) {
#pragma unroll
        for (int k = 0; k < 1024 / kLanes; ++k) base[k] = tables.base_decode[t + k * kLanes];
    }
    if (tables.control != nullptr) {
        center_from_control(tables.control, tables.n_groups, tables.epoch, tables.polls, shared);
    } else {
        center_from_partials(tables.partials, tables.n_groups, shared);
        if (t == 0) shared[1] = 0;
    }
    __syncthreads();
    const int32_t center = shared[0];
    const bool failed = shared[1] != 0;
    table[t] = repack_encode_entry(static_cast<uint32_t>(raw[byte_to_index(t, center)]));
    if (block == 0) {
        if (t == 0) tables.center_out[0] = center;
#pragma unroll
        for (int k = 0; k < 1024 / kLanes; ++k)
            tables.shifted_decode_out[t + k * kLanes] = shifted_decode_entry(base[k], center);
    }
    return failed;
}

template <bool kFull, bool kPrecomputed, int kSidePolicy>
__device__ __forceinline__ bool encode_dispatch(int S, const void *source, int64_t logical_base,
                                                __amdgpu_buffer_rsrc_t side,
                                                const TableSource &tables, uint2 *table,
                                                int32_t *raw, int32_t *shared,
                                                int64_t block, uint32_t *stage,
                                                uint8_t *in_slice, int64_t row_base,
                                                uint32_t valid, int W, bool &overflow,
                                                int &extra) {
    // The element size is a compile-time constant here, so the source
    // resource stays in SGPRs.
    constexpr uint32_t kElemBytes = kPrecomputed ? 1u : 2u;
    const __amdgpu_buffer_rsrc_t src = make_rsrc(
        static_cast<const uint8_t *>(source) + logical_base * kElemBytes, valid * kElemBytes);
    // The first chunk is in flight while the table is set up.
    const InputChunk first = fetch_input<kFull, kPrecomputed>(src, row_base, 0,
                                                              valid * kElemBytes);
    const bool failed = setup_table(tables, table, raw, shared, block);
    __syncthreads();   // encode table and zeroed stage are visible
    if (S == 128)
        encode_block<kFull, kPrecomputed, 128, kSidePolicy>(src, side, table, stage, in_slice, row_base,
                                               valid, W, first, overflow, extra);
    else
        encode_block<kFull, kPrecomputed, 256, kSidePolicy>(src, side, table, stage, in_slice, row_base,
                                               valid, W, first, overflow, extra);
    return failed;
}

// LDS of one encoding workgroup: the payload stage is dynamic ((W + 2) rows
// of 256 words); the table, the input slices and the small scratch arrays are
// static in the kernel, so their addresses fold into LDS instruction offsets.
struct EncodeLds {
    uint32_t *stage;
    uint2 *table;       // 256 entries
    uint8_t *slices;    // kWavesPerBlock * kSliceBytes, 16-byte aligned
    int32_t *scratch;   // kWavesPerBlock ints
    int32_t *shared;    // 2 ints: center, polled-partials failure
};

// A block's overflow summary (uniform): overflowing streams, their tail bytes,
// and whether the block's center could not be read (fused compress only).
struct BlockSummary {
    int32_t count;
    int32_t bytes;
    bool failed;
};

// One codec block (the body of every encoder launch): field split, payload,
// per-stream extra starts, and -- when `summarize` -- the block's overflow
// count and tail bytes.  Contains barriers.
template <int kSidePolicy = kStreaming>
__device__ __forceinline__ BlockSummary encode_codec_block(
    const void *__restrict__ source, uint8_t *__restrict__ side, int32_t *__restrict__ encoded,
    const TableSource &tables, uint8_t *__restrict__ extra_starts, int64_t block,
    int64_t n_blocks, int64_t logical_numel, int S, int W, int precomputed, bool summarize,
    const EncodeLds &lds) {
    const int t = threadIdx.x;
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    const uint32_t block_elems = static_cast<uint32_t>(S) * kLanes;
    const int64_t remaining = logical_numel - logical_base;
    const uint32_t valid = remaining < block_elems ? static_cast<uint32_t>(remaining) : block_elems;
    const bool full = valid == block_elems;
    const __amdgpu_buffer_rsrc_t side_rsrc = make_rsrc(side + logical_base, block_elems);
    uint32_t *const stage = lds.stage;

    for (int i = t; i < (W + 2) * kLanes; i += kLanes) stage[i] = 0u;
    int32_t *raw = reinterpret_cast<int32_t *>(lds.slices);

    uint8_t *in_slice = lds.slices + (t / kWave) * kSliceBytes;
    bool overflow;
    int extra;
    bool failed;
    if (precomputed) {
        if (full) failed = encode_dispatch<true, true, kSidePolicy>(S, source, logical_base, side_rsrc, tables,
                                                       lds.table, raw, lds.shared, block, stage,
                                                       in_slice, row_base, valid, W, overflow,
                                                       extra);
        else failed = encode_dispatch<false, true, kSidePolicy>(S, source, logical_base, side_rsrc, tables,
                                                   lds.table, raw, lds.shared, block, stage,
                                                   in_slice, row_base, valid, W, overflow, extra);
    } else {
        if (full) failed = encode_dispatch<true, false, kSidePolicy>(S, source, logical_base, side_rsrc, tables,
                                                        lds.table, raw, lds.shared, block, stage,
                                                        in_slice, row_base, valid, W, overflow,
                                                        extra);
        else failed = encode_dispatch<false, false, kSidePolicy>(S, source, logical_base, side_rsrc, tables,
                                                    lds.table, raw, lds.shared, block, stage,
                                                    in_slice, row_base, valid, W, overflow,
                                                    extra);
    }

    const int64_t n_streams = n_blocks * kLanes;
    extra_starts[block * kLanes + t] = static_cast<uint8_t>(overflow ? extra : 255);
    __syncthreads();

    // Copy the W payload rows out, 16 bytes per thread per store.
    const int chunks = W * (kLanes / 4);
    for (int c = t; c < chunks; c += kLanes) {
        const int row = c / (kLanes / 4);
        const int quad = c % (kLanes / 4);
        const auto value = reinterpret_cast<const u32x4 *>(stage + row * kLanes)[quad];
        reinterpret_cast<u32x4 *>(encoded + row * n_streams + block * kLanes)[quad] = value;
    }

    BlockSummary summary{0, 0, failed};
    if (summarize) {
        // Both sums in one: tail bytes in bits 0..19 (at most 256 x 256),
        // streams from bit 20 (at most 256).
        const int32_t both = block_sum(overflow ? (S - extra) | (1 << 20) : 0, lds.scratch);
        summary.count = both >> 20;
        summary.bytes = both & 0xFFFFF;
    }
    return summary;
}

}  // namespace lct
