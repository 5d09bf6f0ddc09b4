// Field split + fixed-payload Huffman encoder for gfx950.
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
//    wave; it is fetched with 16-byte buffer loads one chunk ahead of use and
//    staged in a wave-private LDS slice;
//  * side bytes: collected in a wave-private LDS slice and written as one
//    16-byte store per lane per chunk (16 rows x the wave's 64 bytes);
//  * payload: built in LDS -- every pair writes the lane's current partial
//    word to stage row pos/32 (conflict-free: row stride 256 words), so each
//    row ends up holding the completed words; after the loop the block copies
//    rows 0..W-1 to `encoded` with 16-byte stores.  Row W is a pad row that
//    absorbs writes of overflowed lanes.
//
// Overflow rule (encode.py:73-90): a pair overflows when pos + len > 32W; the
// first overflowing pair's even step is the stream's extra_start and word W-1
// keeps only the bits before that pair.  The first-overflow bookkeeping runs in
// a wave-uniform branch that is skipped unless some lane of the wave overflows.
#include "decode_core.h"

namespace lct {
namespace {

constexpr int kEncChunk = 16;   // steps per staged input chunk

using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

// Encode-table entry repacked for the kernel: reversed code (<= 16 bits) in
// bits 0..15, code length in bits 16..20.
__device__ __forceinline__ uint32_t repack_encode_entry(uint32_t packed) {
    return (packed & 0xFFFFu) | ((packed >> 20) << 16);
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
        return __builtin_amdgcn_raw_buffer_load_b128(src, offset, 0, 0);
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

template <bool kFull, bool kPrecomputed, int S>
__device__ __forceinline__ void encode_block(
    __amdgpu_buffer_rsrc_t src, __amdgpu_buffer_rsrc_t side, const uint32_t *__restrict__ table,
    uint32_t *__restrict__ stage, uint8_t *in_slice, uint8_t *side_slice, int64_t row_base,
    uint32_t valid_in_block, int W, InputChunk next, bool &overflow_out, int &extra_out) {
    const uint32_t lane = threadIdx.x;
    const uint32_t j = lane & (kWave - 1);
    const uint32_t limit = static_cast<uint32_t>(W) * 32u;
    const uint32_t pad_slot = static_cast<uint32_t>(W) * kLanes + lane;
    const uint32_t valid_bytes = valid_in_block * (kPrecomputed ? 1u : 2u);
    // Side bytes of a chunk leave as one 16-byte store per lane: row j/4 of
    // the chunk, bytes (j%4)*16.. of the wave's 64-byte segment.
    const uint32_t side_store_offset = side_fetch_offset();

    uint32_t pos = 0, word_value = 0;
    bool overflow = false;
    int extra = S;
#pragma unroll 1
    for (int c = 0; c < S; c += kEncChunk) {
        store_input<kPrecomputed>(in_slice, next);
        if (c + kEncChunk < S)
            next = fetch_input<kFull, kPrecomputed>(src, row_base, c + kEncChunk, valid_bytes);
#pragma unroll
        for (int p = 0; p < kEncChunk; p += 2) {
            const int step = c + p;
            // Column of this lane inside its wave's 64-column group: the row
            // mask's low six bits (rows step, step+1 share the mask).
            const uint32_t colg = j ^ static_cast<uint32_t>((row_base + step) & 62);
            uint32_t e0, e1;
            if (kPrecomputed) {
                e0 = in_slice[p * kWave + colg];
                e1 = in_slice[(p + 1) * kWave + colg];
            } else {
                const uint16_t *rows = reinterpret_cast<const uint16_t *>(in_slice);
                const uint32_t v0 = rows[p * kWave + colg];
                const uint32_t v1 = rows[(p + 1) * kWave + colg];
                e0 = (v0 >> 7) & 0xFFu;
                e1 = (v1 >> 7) & 0xFFu;
                side_slice[p * kWave + j] = static_cast<uint8_t>(side_byte_of(v0));
                side_slice[(p + 1) * kWave + j] = static_cast<uint8_t>(side_byte_of(v1));
            }
            uint32_t p0 = table[e0], p1 = table[e1];
            if (!kFull) {
                // Positions past the logical end carry no code (encode.py:255-256).
                const uint32_t off0 = static_cast<uint32_t>(step) * kLanes
                    + (lane ^ static_cast<uint32_t>((row_base + step) & 254));
                p0 = off0 < valid_in_block ? p0 : 0u;
                p1 = off0 + kLanes < valid_in_block ? p1 : 0u;
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
            word_value = shift + len >= 32u ? carry : new_word;
            pos = pos_after;
        }
        if (!kPrecomputed) {
            const u32x4 sides = reinterpret_cast<const u32x4 *>(side_slice)[j];
            __builtin_amdgcn_raw_buffer_store_b128(sides, side, side_store_offset + c * kLanes, 0, 0);
        }
    }
    if (!overflow) stage[(pos >> 5) * kLanes + lane] = word_value;
    overflow_out = overflow;
    extra_out = extra;
}

// Where the encoder's table comes from: the center-shifted encode table, or
// the sampler's partial sums plus the distribution's base tables (the center
// and shifted tables are then derived in every workgroup; workgroup 0 also
// stores the center and the shifted decode table).
struct TableSource {
    const int32_t *shifted_encode;
    const int32_t *partials;
    int32_t n_groups;
    const int32_t *base_encode;
    const int32_t *base_decode;
    int32_t *center_out;
    int32_t *shifted_decode_out;
};

// The workgroup's LDS encode table.  With sampler partials, wave 0 reduces
// them to the center while the raw base table waits in `raw` (LDS the first
// input chunk overwrites only later); workgroup 0 stores the center and the
// shifted decode table.  Contains a barrier when sampled.
__device__ __forceinline__ void setup_table(const TableSource &tables, uint32_t *table,
                                            int32_t *raw, int32_t *shared_center,
                                            int64_t block) {
    const int t = threadIdx.x;
    if (tables.partials == nullptr) {
        table[t] = repack_encode_entry(static_cast<uint32_t>(tables.shifted_encode[t]));
        return;
    }
    raw[t] = tables.base_encode[t];
    center_from_partials(tables.partials, tables.n_groups, shared_center);
    __syncthreads();
    const int32_t center = *shared_center;
    table[t] = repack_encode_entry(static_cast<uint32_t>(raw[byte_to_index(t, center)]));
    if (block == 0) {
        if (t == 0) tables.center_out[0] = center;
        for (int i = t; i < 1024; i += kLanes)
            tables.shifted_decode_out[i] = shifted_decode_entry(tables.base_decode[i], center);
    }
}

template <bool kFull, bool kPrecomputed>
__device__ __forceinline__ void encode_dispatch(int S, __amdgpu_buffer_rsrc_t src,
                                                __amdgpu_buffer_rsrc_t side,
                                                const TableSource &tables, uint32_t *table,
                                                int32_t *raw, int32_t *shared_center,
                                                int64_t block, uint32_t *stage,
                                                uint8_t *in_slice, uint8_t *side_slice,
                                                int64_t row_base, uint32_t valid, int W,
                                                bool &overflow, int &extra) {
    // The first chunk is in flight while the table is set up.
    const InputChunk first = fetch_input<kFull, kPrecomputed>(
        src, row_base, 0, valid * (kPrecomputed ? 1u : 2u));
    setup_table(tables, table, raw, shared_center, block);
    __syncthreads();   // encode table and zeroed stage are visible
    if (S == 128)
        encode_block<kFull, kPrecomputed, 128>(src, side, table, stage, in_slice, side_slice,
                                               row_base, valid, W, first, overflow, extra);
    else
        encode_block<kFull, kPrecomputed, 256>(src, side, table, stage, in_slice, side_slice,
                                               row_base, valid, W, first, overflow, extra);
}

__global__ __launch_bounds__(kLanes) void encode_kernel(
    const void *__restrict__ source, uint8_t *__restrict__ side,
    int32_t *__restrict__ encoded, TableSource tables,
    uint8_t *__restrict__ extra_starts, int32_t *__restrict__ summaries,
    int64_t n_blocks, int64_t logical_numel, int S, int W, int precomputed,
    int write_summary) {
    extern __shared__ uint32_t stage[];   // (W + 1) rows x 256 lanes
    __shared__ uint32_t table[256];
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t shared_center;
    __shared__ __attribute__((aligned(16))) uint8_t in_slices[kWavesPerBlock][2 * kEncChunk * kWave];
    __shared__ __attribute__((aligned(16))) uint8_t side_slices[kWavesPerBlock][kEncChunk * kWave];
    const int t = threadIdx.x;
    const int64_t block = blockIdx.x;
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    const uint32_t block_elems = static_cast<uint32_t>(S) * kLanes;
    const int64_t remaining = logical_numel - logical_base;
    const uint32_t valid = remaining < block_elems ? static_cast<uint32_t>(remaining) : block_elems;
    const bool full = valid == block_elems;
    const uint32_t elem_bytes = precomputed ? 1u : 2u;
    const __amdgpu_buffer_rsrc_t src_rsrc = make_rsrc(
        static_cast<const uint8_t *>(source) + logical_base * elem_bytes, valid * elem_bytes);
    const __amdgpu_buffer_rsrc_t side_rsrc = make_rsrc(side + logical_base, block_elems);

    for (int i = t; i < (W + 1) * kLanes; i += kLanes) stage[i] = 0u;
    int32_t *raw = reinterpret_cast<int32_t *>(&in_slices[0][0]);

    uint8_t *in_slice = in_slices[t / kWave];
    uint8_t *side_slice = side_slices[t / kWave];
    bool overflow;
    int extra;
    if (precomputed) {
        if (full) encode_dispatch<true, true>(S, src_rsrc, side_rsrc, tables, table, raw,
                                              &shared_center, block, stage, in_slice, side_slice,
                                              row_base, valid, W, overflow, extra);
        else encode_dispatch<false, true>(S, src_rsrc, side_rsrc, tables, table, raw,
                                          &shared_center, block, stage, in_slice, side_slice,
                                          row_base, valid, W, overflow, extra);
    } else {
        if (full) encode_dispatch<true, false>(S, src_rsrc, side_rsrc, tables, table, raw,
                                               &shared_center, block, stage, in_slice,
                                               side_slice, row_base, valid, W, overflow, extra);
        else encode_dispatch<false, false>(S, src_rsrc, side_rsrc, tables, table, raw,
                                           &shared_center, block, stage, in_slice, side_slice,
                                           row_base, valid, W, overflow, extra);
    }

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
    const size_t lds = static_cast<size_t>(g.fixed_words + 1) * kLanes * sizeof(uint32_t);
    hipLaunchKernelGGL(encode_kernel, dim3(static_cast<uint32_t>(n_blocks)), dim3(kLanes),
                       lds, stream, source, side, encoded, tables,
                       extra_starts, summaries, n_blocks, logical_numel, g.steps,
                       g.fixed_words, precomputed, write_summary);
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
