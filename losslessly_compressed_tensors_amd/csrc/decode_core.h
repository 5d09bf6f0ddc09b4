// Stream decoder shared by the decode, pointwise and dual kernels (gfx950).
//
// Semantics: LCT/kernels/generic/decode.py:12-256 and
// LCT/kernels/primitives.py:7-36.  Each thread owns one stream of its block
// and decodes it two symbols at a time.
//
// MI355X mapping:
//  * the block's W payload rows (1 KiB each) are staged in LDS with 16-byte
//    loads; a lane's 32-bit window at bit position `pos` is
//    alignbit(row[pos/32 + 1], row[pos/32], pos) -- one ds_read2st64 and one
//    v_alignbit per pair, no 64-bit shifts and no per-lane global gathers;
//  * the lookup table has 256 16-bit entries (direct codes are at most 8 bits,
//    LCT/compression/huffman_tables.py:106-107) holding the exponent already
//    in BF16 position: entry = len | e_raw << 7, so a decoded value is one
//    bit-field insert away from its BF16 bits.  16-bit entries keep the table
//    in 128 dwords, which bounds LDS bank conflicts of the data-dependent
//    lookups.  An ESC prefix (or any code longer than 8 bits) is marked by
//    len = 31, which makes len0 + len1 >= 32; those pairs take a wave-uniform
//    branch that reads the 8-bit literal;
//  * a second 256-entry table maps an escaped table index to its exponent
//    field under the tensor's center;
//  * side bytes are fetched with 16-byte buffer loads one 16-step chunk ahead
//    of use and handed to the lanes through a wave-private LDS slice, so HBM
//    latency overlaps a whole chunk of decoding; outputs go out through raw
//    buffer stores (SGPR base, 32-bit lane offset).
#pragma once

#include "lct_device.h"

namespace lct {

// Cache policy of data touched once: non-temporal.  The decoder uses it for
// its payload staging and output stores; its side-byte loads keep the default
// policy (non-temporal there measures slower in combination on gfx950).
constexpr int kStreaming = 2;
constexpr int kChunkSteps = 16;   // steps per prefetched side-byte chunk

struct DecodeTables {
    uint16_t entry[256];
    uint16_t escape[256];

    // Entry of an escaped symbol's 8-bit literal (a table index).
    __device__ __forceinline__ uint32_t escaped(uint32_t literal, int32_t) const {
        return escape[literal];
    }
    // Entry of an overflow tail byte int8(e - 127) (length 0).
    static __device__ __forceinline__ uint32_t tail(uint32_t byte) {
        return ((byte + 127u) & 255u) << 7;
    }
};

// Tables of the fused update kernels: the same entries with the exponent in
// FP32 position (len | e_raw << 23), one dword each, so a decoded value is one
// bit-field insert away from its FP32 bits (join_float) and the entry needs no
// masking before that.  Lengths stay in bits 0..4, so (t0 + t1) & 127 still
// adds two lengths.  An escaped literal's exponent is computed from the
// center (index_to_exponent) instead of read from a second table: escapes are
// rare, and the 1 KiB this saves keeps the two-operand kernel's LDS at three
// workgroups per CU.
struct FloatDecodeTables {
    uint32_t entry[256];

    __device__ __forceinline__ uint32_t escaped(uint32_t literal, int32_t center) const {
        return static_cast<uint32_t>(
                   (index_to_exponent(static_cast<int32_t>(literal), center) + 127) & 255)
            << 23;
    }
    static __device__ __forceinline__ uint32_t tail(uint32_t byte) {
        return ((byte + 127u) & 255u) << 23;
    }
};

// FloatDecodeTables from the 1024-entry shifted decode table, one entry per
// thread of a 256-thread block.
__device__ __forceinline__ void build_float_decode_tables(
    FloatDecodeTables &tb, const int32_t *__restrict__ shifted_decode) {
    const int32_t packed = shifted_decode[threadIdx.x];
    const int32_t length = packed & 255;
    const uint32_t field = static_cast<uint32_t>(((packed >> 8) + 127) & 255) << 23;
    tb.entry[threadIdx.x] = (length >= 1 && length <= 8)
                                ? (static_cast<uint32_t>(length) | field)
                                : static_cast<uint32_t>(kEscapeLength);
}

// Entry `t` of both tables from entry t of the 1024-entry shifted decode
// table (len | exp << 8).
__device__ __forceinline__ void build_decode_entry(DecodeTables &tb, int t, int32_t packed,
                                                   int32_t center) {
    const int32_t length = packed & 255;
    const uint32_t field = static_cast<uint32_t>(((packed >> 8) + 127) & 255) << 7;
    tb.entry[t] = static_cast<uint16_t>((length >= 1 && length <= 8)
                                            ? (static_cast<uint32_t>(length) | field)
                                            : static_cast<uint32_t>(kEscapeLength));
    tb.escape[t] = static_cast<uint16_t>(((index_to_exponent(t, center) + 127) & 255) << 7);
}

// Both tables, one entry per thread of a 256-thread block.
__device__ __forceinline__ void build_decode_tables(DecodeTables &tb,
                                                    const int32_t *__restrict__ shifted_decode,
                                                    int32_t center) {
    build_decode_entry(tb, threadIdx.x, shifted_decode[threadIdx.x], center);
}

// Copy the W payload rows of `block` into stage rows 0..W-1 and zero the pad
// row W that a window starting in row W-1 reads as its high word.  A payload
// row of a block is 1 KiB contiguous in HBM; each row moves with one direct
// global-to-LDS load per wave (64 lanes x 16 bytes), so staging takes no
// registers.  The loads are non-temporal (each payload word is read once):
// on gfx950 that takes the decoder from 88.5 to 81.8 us at 4096 blocks.  The
// caller waits (vmcnt(0)) and synchronises before reading.
__device__ __forceinline__ void stage_payload(uint32_t *stage, const int32_t *__restrict__ encoded,
                                              int64_t n_streams, int64_t block, int W) {
    const int t = threadIdx.x;
    const int wave = t / kWave;
    const int j = t % kWave;
    for (int row = wave; row < W; row += kWavesPerBlock) {
        const int32_t *src = encoded + row * n_streams + block * kLanes + j * 4;
        __builtin_amdgcn_global_load_lds(
            src, (__attribute__((address_space(3))) void *)(stage + row * kLanes),
            16, 0, kStreaming);
    }
    stage[W * kLanes + t] = 0u;
}

// LDS bytes of the payload stage for W words per stream (W rows + 1 pad row).
__host__ __device__ constexpr int32_t stage_bytes(int W) { return (W + 1) * kLanes * 4; }

// Stages without the first three rows: each stream's words 0..2 start in
// registers (StreamCursorT::init_registers) and only rows 3..W-1 are staged,
// with no pad row.  Saves four rows (4 KiB) of LDS per workgroup.
constexpr int kRegisterRows = 3;

__host__ __device__ constexpr int32_t register_stage_bytes(int W) {
    return (W - kRegisterRows) * kLanes * 4;
}

// Rows first..W-1 of the block's payload into stage rows 0.. (16 bytes per lane
// per row, non-temporal, as stage_payload).
__device__ __forceinline__ void stage_payload_rows(uint32_t *stage,
                                                   const int32_t *__restrict__ encoded,
                                                   int64_t n_streams, int64_t block, int first,
                                                   int W) {
    const int wave = threadIdx.x / kWave;
    const int j = threadIdx.x % kWave;
    for (int row = first + wave; row < W; row += kWavesPerBlock) {
        const int32_t *src = encoded + row * n_streams + block * kLanes + j * 4;
        __builtin_amdgcn_global_load_lds(
            src, (__attribute__((address_space(3))) void *)(stage + (row - first) * kLanes), 16,
            0, kStreaming);
    }
}

// Words 0..2 of this lane's stream of `block` (non-temporal loads).
__device__ __forceinline__ void load_register_rows(const int32_t *__restrict__ encoded,
                                                   int64_t n_streams, int64_t block,
                                                   uint32_t (&w)[kRegisterRows]) {
    const int32_t *col = encoded + block * kLanes + threadIdx.x;
#pragma unroll
    for (int r = 0; r < kRegisterRows; ++r)
        w[r] = static_cast<uint32_t>(__builtin_nontemporal_load(col + r * n_streams));
}

// Wait for this thread's outstanding memory operations (including direct
// global-to-LDS loads) before a barrier publishes the staged data.
__device__ __forceinline__ void wait_memory() { __builtin_amdgcn_s_waitcnt(0); }

// Per-lane view of the overflow tails of one block.
struct LaneOverlay {
    const uint8_t *tail;   // global tail bytes of this lane start at tail[offset]
    int32_t start;         // first overflow step, S if none
    int32_t offset;        // byte offset of this lane's tail (LDS-relative if lds)
    int32_t wave_start;    // minimum `start` over the wave (wave-uniform)
    int32_t lds;           // block-uniform: the block's tails were staged in LDS
};

// The block's overflow-list header: its entry count (0 also when a buffered
// tensor's reservation failed), first entry and tail byte base, and where the
// entries, starts and tails begin.  All independent loads: a prologue that
// issues them first shares their round trip with its other loads.
struct OverlayHead {
    int32_t count;
    int32_t status;      // the buffered tensor's descriptor status (0: ok)
    int32_t first;
    int32_t byte_base;
    int64_t lane_off, start_off, tail_base;
};

__device__ __forceinline__ OverlayHead load_overlay_head(const lct_overflow &ov, bool present,
                                                         int64_t block, int64_t n_blocks) {
    OverlayHead h{0, 0, 0, 0, 0, 0, ov.base};
    if (!present) return h;
    h.count = ov.blocks[block];
    h.first = ov.blocks[n_blocks + block];
    h.byte_base = ov.blocks[2 * n_blocks + block];
    if (ov.descriptor != nullptr) {
        h.status = ov.descriptor[2];
        const int64_t arena = ov.descriptor[0];
        const int64_t total = ov.count[0];
        h.lane_off = arena;
        h.start_off = arena + total;
        h.tail_base = arena + 2 * total;
    }
    return h;
}

// Expand the block's compact overflow list into per-lane (start, offset), as
// decode.py:195-240 does.  When `tail_lds` is given and the block's tail bytes
// fit in `tail_cap`, they are copied into tail_lds so the step loop reads its
// overlay from LDS instead of issuing global loads.  Contains barriers; every
// thread of the block must call it, and the caller synchronises once more
// before reading tail_lds.  A buffered tensor whose allocation failed
// (descriptor status != 0) has no tails and is decoded without overlay.
// expand_overlay is the part after the block's header: count > 0 entries
// from `first`, tails from byte_base.
__device__ __forceinline__ LaneOverlay expand_overlay(const lct_overflow &ov, int32_t count,
                                                      int32_t first, int32_t byte_base,
                                                      int64_t lane_off, int64_t start_off,
                                                      int64_t tail_base, int S,
                                                      int32_t *map_start, int32_t *map_offset,
                                                      int32_t *scratch, uint8_t *tail_lds,
                                                      int32_t tail_cap) {
    const int t = threadIdx.x;
    LaneOverlay lane{nullptr, S, 0, S, 0};
    map_start[t] = S;
    map_offset[t] = 0;
    const bool valid = t < count;
    int32_t entry_lane = 0, entry_start = S;
    if (valid) {
        entry_lane = ov.lanes[lane_off + first + t];
        entry_start = ov.starts[start_off + first + t];
    }
    int32_t block_bytes;
    const int32_t local = block_exclusive_scan(valid ? S - entry_start : 0, scratch, &block_bytes);
    block_bytes = __builtin_amdgcn_readfirstlane(block_bytes);
    const bool staged = tail_lds != nullptr && block_bytes <= tail_cap;
    if (valid) {
        map_start[entry_lane] = entry_start;
        map_offset[entry_lane] = staged ? local : byte_base + local;
    }
    lane.tail = ov.tail + tail_base;
    if (staged) {
        const uint8_t *src = lane.tail + byte_base;
        for (int i = t; i < block_bytes; i += kLanes) tail_lds[i] = src[i];
    }
    __syncthreads();
    lane.start = map_start[t];
    lane.offset = map_offset[t];
    lane.wave_start = __builtin_amdgcn_readfirstlane(wave_min(lane.start));
    lane.lds = staged ? 1 : 0;
    return lane;
}

// With the header loaded up front (load_overlay_head).
__device__ __forceinline__ LaneOverlay build_overlay(const lct_overflow &ov, const OverlayHead &h,
                                                     int S, int32_t *map_start,
                                                     int32_t *map_offset, int32_t *scratch,
                                                     uint8_t *tail_lds, int32_t tail_cap) {
    const int32_t count = h.status != 0 ? 0 : h.count;
    if (count <= 0) return LaneOverlay{nullptr, S, 0, S, 0};   // uniform across the block
    return expand_overlay(ov, count, h.first, h.byte_base, h.lane_off, h.start_off, h.tail_base,
                          S, map_start, map_offset, scratch, tail_lds, tail_cap);
}

// Loading the header itself: the entry count first, the rest only for a block
// with entries (the decoders, whose blocks mostly have none).
__device__ __forceinline__ LaneOverlay build_overlay(const lct_overflow &ov, bool present,
                                                     int64_t block, int64_t n_blocks, int S,
                                                     int32_t *map_start, int32_t *map_offset,
                                                     int32_t *scratch, uint8_t *tail_lds,
                                                     int32_t tail_cap) {
    int32_t count = 0;
    if (present) {
        count = ov.blocks[block];
        if (ov.descriptor != nullptr && ov.descriptor[2] != 0) count = 0;
    }
    if (count <= 0) return LaneOverlay{nullptr, S, 0, S, 0};   // uniform across the block
    int64_t lane_off = 0, start_off = 0, tail_base = ov.base;
    if (ov.descriptor != nullptr) {
        const int64_t arena = ov.descriptor[0];
        const int64_t total = ov.count[0];
        lane_off = arena;
        start_off = arena + total;
        tail_base = arena + 2 * total;
    }
    return expand_overlay(ov, count, ov.blocks[n_blocks + block], ov.blocks[2 * n_blocks + block],
                          lane_off, start_off, tail_base, S, map_start, map_offset, scratch,
                          tail_lds, tail_cap);
}

// One lane's stream cursor over payload rows kStride words apart in LDS.
//
// The 64-bit window lives in registers: lo/hi are words w and w+1 of the
// lane's stream, nx is word w+2, and pos (0..31) is the bit offset in lo.  A
// pair consumes at most 32 bits, so it crosses at most one word boundary;
// on a crossing the registers shift down by one word and take the word that
// was read from LDS at the start of the same pair.  The only LDS accesses on
// the dependency chain are therefore the two table lookups.
//
// A decoded symbol is carried as its table entry: bits 0..4 hold the code
// length and bits 7..14 the BF16 exponent field, so two entries' lengths add
// without masking first: (t0 + t1) & 127 = len0 + len1, since each length is at
// most 31 and the exponent fields start at bit 7.  Direct codes are 1..8 bits,
// so the sum reaches 32 only when an entry holds the escape marker.
template <int kStride, class Tables = DecodeTables>
struct StreamCursorT {
    using TablesT = Tables;
    const uint32_t *stage;    // stage + lane; row r at stage[r * kStride]
    const Tables *tb;
    uint32_t pos;             // bit offset within lo
    uint32_t lo, hi, nx;      // stream words w, w+1, w+2
    uint32_t next_row;        // row of word w+3 (clamped to the pad row)
    uint32_t pad_row;         // W: the zero row after the payload
    uint32_t pending;         // word next_row, read at the start of a pair
    int32_t rare;
    int32_t center;           // the tensor's center (escaped literals of FloatDecodeTables)

    __device__ __forceinline__ void init(const uint32_t *stage_lane, const Tables *tables,
                                         uint32_t words, int32_t rare_length,
                                         int32_t center_value = 0) {
        stage = stage_lane;
        tb = tables;
        pos = 0;
        pad_row = words;
        lo = stage[0];
        hi = stage[kStride];
        nx = stage[min(2u, words) * kStride];
        next_row = min(3u, words);
        pending = 0;
        rare = rare_length;
        center = center_value;
    }

    // Start with the stream's words 0..2 in registers and rows 3..W-1 staged
    // (row r at stage_rows[(r - 3) * kStride]).  Past the stream's last word
    // the window re-reads word W-1 instead of a zero pad row: bits beyond a
    // stream's end never reach a decoded value (a code's table entries do not
    // depend on the bits after it).  Needs W >= 4.
    __device__ __forceinline__ void init_registers(const uint32_t *stage_rows,
                                                   const Tables *tables, uint32_t words,
                                                   int32_t rare_length, uint32_t w0, uint32_t w1,
                                                   uint32_t w2, int32_t center_value = 0) {
        stage = stage_rows - 3 * kStride;
        tb = tables;
        pos = 0;
        pad_row = words - 1;
        lo = w0;
        hi = w1;
        nx = w2;
        next_row = 3;
        pending = 0;
        rare = rare_length;
        center = center_value;
    }

    // Decode the next two symbols into entries f0/f1 (length | field << 7) and
    // return len0 + len1.  Also starts the read of the word a crossing needs.
    __device__ __forceinline__ uint32_t next_fields(uint32_t &f0, uint32_t &f1) {
        uint32_t bits, t0;
        first_lookup(bits, t0);
        uint32_t t1 = second_lookup(bits, t0);
        const uint32_t sum = resolve(bits, t0, t1);
        f0 = t0;
        f1 = t1;
        return sum;
    }

    // next_fields in three stages, for callers that interleave other work
    // between them: the word a crossing needs and the first symbol's entry ...
    __device__ __forceinline__ void first_lookup(uint32_t &bits, uint32_t &t0) {
        pending = stage[next_row * kStride];
        // Keep the read ahead of the lookups, so its latency overlaps theirs.
        __builtin_amdgcn_sched_barrier(0);
        bits = __builtin_amdgcn_alignbit(hi, lo, pos);
        t0 = tb->entry[bits & 255u];
    }

    // ... the second symbol's entry (ubfe reads its offset from t0[4:0], the
    // first code's length) ...
    __device__ __forceinline__ uint32_t second_lookup(uint32_t bits, uint32_t t0) const {
        return tb->entry[__builtin_amdgcn_ubfe(bits, t0, 8)];
    }

    // ... and escaped symbols; returns len0 + len1.
    __device__ __forceinline__ uint32_t resolve(uint32_t bits, uint32_t &t0, uint32_t &t1) const {
        uint32_t sum = (t0 + t1) & 127u;
        if (__builtin_expect(__any(sum >= 32u), 0)) {
            // ESC + 8-bit literal table index (primitives.py:29-35).
            const uint32_t escaped = static_cast<uint32_t>(rare) + 8u;
            uint32_t l0 = t0 & 31u;
            if (l0 == kEscapeLength) {
                l0 = escaped;
                t0 = tb->escaped((bits >> rare) & 255u, center) | escaped;
                t1 = tb->entry[(bits >> l0) & 255u];
            }
            if ((t1 & 31u) == kEscapeLength)
                t1 = tb->escaped((bits >> (l0 + static_cast<uint32_t>(rare))) & 255u, center)
                    | escaped;
            sum = (t0 + t1) & 127u;
        }
        return sum;
    }

    // Consume `bits` (at most 32) after next_fields.
    __device__ __forceinline__ void advance(uint32_t bits) {
        const uint32_t p = pos + bits;
        const bool cross = p >= 32u;
        pos = p & 31u;
        lo = cross ? hi : lo;
        hi = cross ? nx : hi;
        nx = cross ? pending : nx;
        next_row = cross ? min(next_row + 1u, pad_row) : next_row;
    }
};

// The codec kernels' cursor: one lane per stream of a block, rows of 256 words.
using StreamCursor = StreamCursorT<kLanes>;

// A cursor that keeps no window in registers: each pair reads the two words at
// its bit position (rows pos/32 and pos/32 + 1, 1 KiB apart: one
// ds_read2st64) and extracts 32 bits with alignbit.  Fewer instructions per
// pair than StreamCursorT (no window shifting) at the cost of one more LDS
// round trip on the pair's dependency chain; for kernels bounded by
// instruction issue rather than by that chain.  Needs the block's W rows and
// two zero pad rows staged (window_stage_bytes); the row is clamped to W, so
// no read leaves the stage whatever the payload holds.
__host__ __device__ constexpr int32_t window_stage_bytes(int W) { return (W + 2) * kLanes * 4; }

template <class Tables = DecodeTables>
struct WindowCursorT {
    using TablesT = Tables;
    const uint32_t *stage;   // stage + lane; row r at stage[r * kLanes]
    const Tables *tb;
    uint32_t pos;            // bits consumed
    uint32_t last_row;       // W: the first pad row
    int32_t rare;
    int32_t center;

    __device__ __forceinline__ void init(const uint32_t *stage_lane, const Tables *tables,
                                         uint32_t words, int32_t rare_length,
                                         int32_t center_value = 0) {
        stage = stage_lane;
        tb = tables;
        pos = 0;
        last_row = words;
        rare = rare_length;
        center = center_value;
    }

    __device__ __forceinline__ void first_lookup(uint32_t &bits, uint32_t &t0) {
        const uint32_t row = min(pos >> 5, last_row);
        const uint32_t *at = stage + row * kLanes;
        bits = __builtin_amdgcn_alignbit(at[kLanes], at[0], pos);
        t0 = tb->entry[bits & 255u];
    }

    __device__ __forceinline__ uint32_t second_lookup(uint32_t bits, uint32_t t0) const {
        return tb->entry[__builtin_amdgcn_ubfe(bits, t0, 8)];
    }

    // Escaped symbols (as StreamCursorT::resolve); returns len0 + len1.
    __device__ __forceinline__ uint32_t resolve(uint32_t bits, uint32_t &t0, uint32_t &t1) const {
        uint32_t sum = (t0 + t1) & 127u;
        if (__builtin_expect(__any(sum >= 32u), 0)) {
            const uint32_t escaped = static_cast<uint32_t>(rare) + 8u;
            uint32_t l0 = t0 & 31u;
            if (l0 == kEscapeLength) {
                l0 = escaped;
                t0 = tb->escaped((bits >> rare) & 255u, center) | escaped;
                t1 = tb->entry[(bits >> l0) & 255u];
            }
            if ((t1 & 31u) == kEscapeLength)
                t1 = tb->escaped((bits >> (l0 + static_cast<uint32_t>(rare))) & 255u, center)
                    | escaped;
            sum = (t0 + t1) & 127u;
        }
        return sum;
    }

    __device__ __forceinline__ uint32_t next_fields(uint32_t &f0, uint32_t &f1) {
        uint32_t bits, t0;
        first_lookup(bits, t0);
        uint32_t t1 = second_lookup(bits, t0);
        const uint32_t sum = resolve(bits, t0, t1);
        f0 = t0;
        f1 = t1;
        return sum;
    }

    __device__ __forceinline__ void advance(uint32_t bits) { pos += bits; }
};

using WindowCursor = WindowCursorT<>;

// BF16 bits of a decoded entry (exponent field at bits 7..14, nothing at bit 15
// or above) and its side byte: one multiply and one bit-field insert
// (v_bfi_b32 takes bits 0..6 and 15 from the spread side byte and the rest
// from the entry; the compiler otherwise narrows the masks and emits three
// instructions).
__device__ __forceinline__ uint32_t join_entry(uint32_t entry, uint32_t sm) {
    const uint32_t spread = sm * 257u;   // sign at bit 15, mantissa at bits 0..6
    uint32_t out;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(out) : "s"(0x807Fu), "v"(spread), "v"(entry));
    return out;
}

// FP32 bits of a decoded FloatDecodeTables entry and its side byte: v_perm
// copies the side byte into bytes 2 and 3 (mantissa at bits 16..22, sign at
// bit 31, zeros below bit 16), and one bit-field insert (mask 0x807FFFFF)
// takes those bits and the entry's exponent, dropping its length bits.
__device__ __forceinline__ uint32_t join_float(uint32_t entry, uint32_t sm) {
    const uint32_t spread = __builtin_amdgcn_perm(sm, sm, 0x00000C0Cu);
    uint32_t out;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(out) : "s"(0x807FFFFFu), "v"(spread), "v"(entry));
    return out;
}

// Exponent field of an overflow tail byte int8(e - 127).
__device__ __forceinline__ uint32_t tail_field(uint32_t byte) { return DecodeTables::tail(byte); }

// Overlay one lane's pair if it is at/after its overflow start: the entries
// become the tail bytes' exponent fields with length 0, so the pair consumes
// no payload bits.  kLdsTails picks the block's LDS copy (build_overlay staged
// it) or the tails in HBM; the two are separate instantiations so LDS reads
// stay ds_read instructions.  Tables is the cursor's table type, which fixes
// where an entry holds the exponent.
template <bool kLdsTails, class Tables>
__device__ __forceinline__ void overlay_pair(const LaneOverlay &lane, const uint8_t *tail_lds,
                                             int step, uint32_t &f0, uint32_t &f1) {
    if (step >= lane.start) {
        const int32_t i = lane.offset + (step - lane.start);
        const uint8_t *src = kLdsTails ? tail_lds : lane.tail;
        f0 = Tables::tail(src[i]);
        f1 = Tables::tail(src[i + 1]);
    }
}

// Side bytes reach the lanes through a wave-private LDS slice: each lane
// fetches 16 contiguous bytes of its wave's 64-byte row segments (one
// 16-byte buffer load covers 16 steps x 64 lanes per wave instruction), the
// wave stores them to its slice and each lane then reads its own byte per step
// (64 consecutive bytes per step: conflict-free).  A chunk is 16 steps: 1 KiB
// per wave, one 16-byte load per lane.
struct SideChunk {
    uint4 q0;
};

// Buffer offset of this lane's 16 bytes within a 16-step group.
__device__ __forceinline__ uint32_t side_fetch_offset() {
    const uint32_t j = threadIdx.x & (kWave - 1);
    const uint32_t wave = threadIdx.x / kWave;
    return (j >> 2) * kLanes + wave * kWave + (j & 3) * 16;
}

__device__ __forceinline__ SideChunk fetch_side_chunk(__amdgpu_buffer_rsrc_t side,
                                                      uint32_t voffset, int first_step) {
    SideChunk c;
    c.q0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                         side, voffset, first_step * kLanes, 0));
    return c;
}

// slice: this wave's 1 KiB; byte s*64 + lane holds step s of the chunk.
__device__ __forceinline__ void store_side_chunk(uint8_t *slice, const SideChunk &c) {
    const uint32_t j = threadIdx.x & (kWave - 1);
    reinterpret_cast<uint4 *>(slice)[j] = c.q0;
}

__device__ __forceinline__ uint32_t side_byte(const uint8_t *slice, int step_in_chunk) {
    return slice[step_in_chunk * kWave + (threadIdx.x & (kWave - 1))];
}

// ---- chunked stream walking shared by the decoder and the pointwise kernels

// Tail bytes per block that are staged in LDS (larger blocks read HBM).
constexpr int32_t kTailLds = 1024;

// Byte offset of this lane's logical column within row `step` of the block;
// rows step and step+1 share the swizzle mask.
__device__ __forceinline__ uint32_t logical_col2(int64_t row_base, int step) {
    return (threadIdx.x * 2u) ^ (static_cast<uint32_t>((row_base + step) & 254) * 2u);
}

// Overlay variants of a chunk: no lane of the wave overflows in it, or the
// block's tails are read from LDS, or from HBM.
enum Overlay { kNoOverlay, kLdsOverlay, kHbmOverlay };

// Steps decoded before each store phase: half a side chunk keeps the entries
// in 8 registers.
constexpr int kHalfSteps = kChunkSteps / 2;

// The entries of steps `step` and `step + 1` of this lane's stream.
template <bool kFull, Overlay kOverlay, class Cursor>
__device__ __forceinline__ void decode_pair(Cursor &cursor, const LaneOverlay &lane,
                                            const uint8_t *tail_lds, int step, int64_t row_base,
                                            uint32_t valid_in_block, uint32_t &f0,
                                            uint32_t &f1) {
    constexpr bool kRecount = !kFull || kOverlay != kNoOverlay;
    uint32_t sum = cursor.next_fields(f0, f1);
    if (kOverlay != kNoOverlay)
        overlay_pair<kOverlay == kLdsOverlay, typename Cursor::TablesT>(lane, tail_lds, step, f0,
                                                                         f1);
    if (!kFull) {
        // Padding positions of the last block consume no payload bits.
        const uint32_t off0 = static_cast<uint32_t>(step) * kLanes
            + (logical_col2(row_base, step) >> 1);
        if (off0 >= valid_in_block) f0 &= ~31u;
        if (off0 + kLanes >= valid_in_block) f1 &= ~31u;
    }
    if (kRecount) sum = (f0 + f1) & 127u;
    cursor.advance(sum);
}

template <bool kFull, Overlay kOverlay, class Cursor>
__device__ __forceinline__ void decode_fields(Cursor &cursor, const LaneOverlay &lane,
                                              const uint8_t *tail_lds, int first_step,
                                              int64_t row_base, uint32_t valid_in_block,
                                              uint32_t (&f)[kHalfSteps]) {
#pragma unroll
    for (int j = 0; j < kHalfSteps; j += 2)
        decode_pair<kFull, kOverlay>(cursor, lane, tail_lds, first_step + j, row_base,
                                     valid_in_block, f[j], f[j + 1]);
}

// ---- lane pairs
//
// Lanes j and j^1 hold adjacent columns (c, c+1), c even, of the same two rows
// (step, step+1): the swizzle mask is even, so it never changes bit 0 of a
// column.  Exchanging one value over DPP (quad_perm [1, 0, 3, 2]) lets the
// even lane handle both columns of row `step` and the odd lane both columns of
// row `step + 1` with one 4-byte access (2 bytes for byte data).
struct LanePair {
    bool odd;
    uint32_t pack16;      // v_perm selector: two 16-bit values, own column's in place
    uint32_t pack8;       // v_perm selector: two bytes, own column's in place
    uint32_t low16;       // v_perm selector: row `step` value of own column into bits 16..31
    uint32_t high16;      // v_perm selector: row `step+1` value of own column into bits 16..31
    uint32_t offset2;     // byte offset of the pair's word (16-bit data), before the swizzle
    uint32_t offset1;     // byte offset of the pair's 2 bytes (byte data), before the swizzle

    __device__ __forceinline__ LanePair() {
        const uint32_t t = threadIdx.x;
        odd = (t & 1u) != 0;
        pack16 = odd ? 0x01000504u : 0x05040100u;
        pack8 = odd ? 0x0C0C0004u : 0x0C0C0400u;
        // v_perm_b32(recv, own, sel): bytes 0..3 select own, 4..7 recv, 12 = 0.
        low16 = odd ? 0x07060C0Cu : 0x01000C0Cu;
        high16 = odd ? 0x03020C0Cu : 0x05040C0Cu;
        offset2 = ((t * 2u) & ~3u) | (odd ? kLanes * 2u : 0u);
        offset1 = (t & ~1u) | (odd ? static_cast<uint32_t>(kLanes) : 0u);
    }
};

__device__ __forceinline__ uint32_t swap_pair(uint32_t value) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_mov_dpp(static_cast<int>(value), 0xB1, 0xF, 0xF, false));
}

// The word to store for 16-bit results v0 (row step) and v1 (row step+1) of
// this lane's column.
__device__ __forceinline__ uint32_t pair_word16(const LanePair &lp, uint32_t v0, uint32_t v1) {
    const uint32_t recv = swap_pair(lp.odd ? v0 : v1);
    return __builtin_amdgcn_perm(recv, lp.odd ? v1 : v0, lp.pack16);
}

// The 2 bytes to store for byte results v0 (row step) and v1 (row step+1).
__device__ __forceinline__ uint32_t pair_word8(const LanePair &lp, uint32_t v0, uint32_t v1) {
    const uint32_t recv = swap_pair(lp.odd ? v0 : v1);
    return __builtin_amdgcn_perm(recv, lp.odd ? v1 : v0, lp.pack8);
}

// From the pair's loaded words (own: this lane's load, row step + odd) give
// this lane's column of rows step and step+1 as FP32 bit patterns (BF16 in
// the high half).
__device__ __forceinline__ void pair_unpack16(const LanePair &lp, uint32_t own, float &v0,
                                              float &v1) {
    const uint32_t recv = swap_pair(own);
    v0 = __builtin_bit_cast(float, __builtin_amdgcn_perm(recv, own, lp.low16));
    v1 = __builtin_bit_cast(float, __builtin_amdgcn_perm(recv, own, lp.high16));
}

}  // namespace lct
