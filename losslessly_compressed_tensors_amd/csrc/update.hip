// Single-pass pointwise update with compressed output (gfx950).
//
// The reference's compressed-output path (LCT/codec/pointwise.py:262-278)
// runs the fused pointwise kernel with COMPRESSED_OUTPUT, which writes the
// result's side bytes and exponent bytes to HBM
// (LCT/kernels/generic/pointwise.py:43-65), and then re-encodes them through
// encode_components(precomputed=True) (LCT/codec/encode.py:22-186): a center
// estimated from up to 4096 sampled exponent bytes of the result
// (LCT/kernels/common/tables.py:9-49), the encoder kernel
// (LCT/kernels/generic/encode.py:10-169), the block scan and the compaction.
// The result's exponent and side bytes make a round trip through HBM between
// the two passes.  Here they never leave the chip:
//
//  * pointwise_sample_kernel computes the operation's result only at the
//    sampled positions, decoding each sampled stream's prefix from its payload
//    words, and writes the exponent sum and count of each group of 64 samples;
//  * pointwise_encode_kernel reduces those sums to the result's center in
//    every workgroup, shifts the result distribution's encode table by it, and
//    then, per codec block, decodes A, applies the operation with the dense
//    operand B and encodes the result in the same pass.  Its outputs are the
//    encoder's: side bytes, every payload word, extra starts and the block
//    summaries.  Rows that an overflowing stream cannot hold also get the
//    result's exponent bytes written (logical order, those rows only), which
//    is where the compaction reads their tails, as in the precomputed path.
//
// The encoder side writes each payload word straight to HBM when the word
// completes (one 4-byte store by the lanes whose word completed in a pair,
// merged in L2), so the workgroup's LDS holds only A's payload: at W = 25,
// four blocks fit per CU.  The result's side bytes leave with the default
// cache policy: a wave writes 64 bytes of each 128-byte row line, and
// non-temporal stores of half lines wrote 16% more than the side bytes (C4:
// 73.6 MB against 62.9 MB per launch; with the default policy 63.3 MB, at
// equal kernel time).
#include <algorithm>

#include "batch.h"
#include "pointwise_ops.h"
#include "reserve.h"

namespace lct {
namespace {

// Cache policy of the result's side-byte stores: the default (see above).
constexpr int kSideStore = 0;

struct OperandA {
    const int32_t *encoded;
    const uint8_t *side;
    const int32_t *shifted_decode;
    const int32_t *center;
    lct_overflow ov;
    int32_t has_overlay;
};

struct OpArgs {
    const float *alpha;
    const float *beta;
    int32_t op;
    int32_t alpha_is_one;
    int32_t beta_is_one;
};

// The in-launch overflow bookkeeping of the *_encode_fused launches (control
// == nullptr: the block summaries go to `summaries` for a later launch).
struct KernelBookkeeping {
    uint64_t *control;
    uint32_t epoch;
    int32_t *counts;
    int32_t *blocks;
    int32_t *descriptor;
    int32_t *buffer_meta;
    int32_t max_free_regions;
    lct_pending_frees frees;
    int32_t lock_spins;
    int32_t polls;
    uint64_t *gate;      // batched launches: GatedReserve's word (nullptr: none)
    int32_t post_gate;   // this job applies the frees and posts the gate
    // In-launch center sampling of the two-operand launch (sample_groups > 0):
    // workgroups g < sample_groups publish sample group g's partial sums in
    // control[g] (tagged), and every block reads the center from there
    // instead of from `partials`.
    const uint16_t *a_samples;
    const uint16_t *b_samples;
    uint16_t *result_samples;
    int64_t sample_size;
    int32_t sample_groups;
};

// Publish sample group `group`'s kept-exponent sum and count (one wave,
// compress.hip's layout: sum as int16 in bits 16..31, count in bits 0..15).
__device__ __forceinline__ void publish_sample_group(const KernelBookkeeping &bk, int64_t group,
                                                     int32_t sum, int32_t kept) {
    if (threadIdx.x == 0) {
        const uint32_t value = (static_cast<uint32_t>(static_cast<uint16_t>(sum)) << 16)
                               | static_cast<uint32_t>(kept);
        control_store(bk.control + group, tagged_word(bk.epoch, value));
    }
}

// Workgroup 0's share of the result's shifted decode table: the base
// table's 1024 entries, 4 per thread, loaded at the start of its prologue
// (with the other loads) and shifted once the center is known, so that the
// workgroup that also writes the table has no extra memory round trip.
struct BaseDecodeShare {
    int32_t v[1024 / kLanes];
};

__device__ __forceinline__ BaseDecodeShare load_base_decode(const int32_t *__restrict__ base_decode,
                                                            bool needed) {
    BaseDecodeShare b{};
    if (needed) {
#pragma unroll
        for (int k = 0; k < 1024 / kLanes; ++k) b.v[k] = base_decode[threadIdx.x + k * kLanes];
    }
    return b;
}

__device__ __forceinline__ void store_shifted_decode(int32_t *__restrict__ out,
                                                     const BaseDecodeShare &b, int32_t center) {
#pragma unroll
    for (int k = 0; k < 1024 / kLanes; ++k)
        out[threadIdx.x + k * kLanes] = shifted_decode_entry(b.v[k], center);
}

// After a block (every thread, past the summary's barriers): its overflow
// count and tail bytes go to `summaries`, or -- in a fused launch (kBooked:
// its own kernel instantiation, so the separate launch's kernel holds none of
// the bookkeeping's arguments in registers) -- to the control array as a
// tagged word, and workgroup 0 then does the bookkeeping
// of the one-launch compress: with a buffer the lock, the deferred frees and
// the free list in `lds_free_list` (the payload stage, free by now), the
// polled scan into the block metadata and the overflow-block list, and the
// reservation (lct_prefix_allocate / lct_allocate_compact's results).
template <bool kBooked>
__device__ __forceinline__ void publish_block(const KernelBookkeeping &bk,
                                              int32_t *__restrict__ summaries, int64_t block,
                                              int64_t n_blocks, int32_t count, int32_t bytes,
                                              int32_t *lds_free_list, bool failed = false) {
    if (!kBooked) {
        if (threadIdx.x == 0) {
            summaries[block] = count;
            summaries[n_blocks + block] = bytes;
        }
        return;
    }
    if (threadIdx.x == 0) {
        // count <= 256 and bytes <= 256 * 256 fit 9 and 17 bits; a block
        // whose center did not arrive is marked failed.
        const uint32_t value = failed ? (kFailedBlock << 17)
                                      : (static_cast<uint32_t>(count) << 17)
                                            | static_cast<uint32_t>(bytes);
        control_store(bk.control + kControlPartials + block, tagged_word(bk.epoch, value));
    }
    if (block != 0) return;
    PolledSummaries polled{bk.control, bk.epoch, static_cast<int32_t>(n_blocks), bk.polls, false};
    if (bk.buffer_meta != nullptr) {
        GatedReserve reserve{
            LdsReserve<false>{AllocatorMeta(bk.buffer_meta, bk.max_free_regions, bk.lock_spins),
                              bk.descriptor, bk.frees, lds_free_list, {}, -1, kStatusOk},
            bk.gate, bk.post_gate != 0, bk.epoch, bk.polls, false};
        scan_allocate<false>(polled, summaries, bk.counts, bk.blocks,
                             static_cast<int32_t>(n_blocks), reserve);
    } else {
        NoReserve reserve;
        scan_allocate<false>(polled, summaries, bk.counts, bk.blocks,
                             static_cast<int32_t>(n_blocks), reserve);
    }
}

// Cursors of the fused encode kernels, over FloatDecodeTables: decoded
// entries become FP32 operands with one v_perm and one v_bfi (join_float).
using UpdateCursor = StreamCursorT<kLanes, FloatDecodeTables>;
using UpdateWindow = WindowCursorT<FloatDecodeTables>;

// Overflow start and tail byte index of one stream (block, lane) of A, from
// the block's entry list (ascending lanes, tails concatenated in entry order:
// LCT/kernels/generic/compaction.py:137-228, decode.py:195-240).  `start` is S
// when the stream does not overflow.
__device__ __forceinline__ void stream_overlay(const lct_overflow &ov, bool present, int64_t block,
                                               int64_t n_blocks, int32_t lane, int S,
                                               int32_t &start, int64_t &tail_index) {
    start = S;
    tail_index = 0;
    if (!present) return;
    int32_t count = ov.blocks[block];
    if (ov.descriptor != nullptr && ov.descriptor[2] != 0) count = 0;
    if (count <= 0) return;
    int64_t lane_off = 0, start_off = 0, tail_base = ov.base;
    if (ov.descriptor != nullptr) {
        const int64_t arena = ov.descriptor[0];
        const int64_t total = ov.count[0];
        lane_off = arena;
        start_off = arena + total;
        tail_base = arena + 2 * total;
    }
    const int32_t first = ov.blocks[n_blocks + block];
    int64_t offset = tail_base + ov.blocks[2 * n_blocks + block];
    for (int32_t e = 0; e < count; ++e) {
        const int32_t entry_lane = ov.lanes[lane_off + first + e];
        const int32_t entry_start = ov.starts[start_off + first + e];
        if (entry_lane == lane) {
            start = entry_start;
            tail_index = offset;
            return;
        }
        offset += S - entry_start;
    }
}

// One sample per thread: the result's exponent at sample position i.  A's
// value there comes from a_samples (A's values at the same positions, recorded
// when A was made) or, without it, from A's streams: the sampled stream's W
// words are staged in this thread's LDS column and its pairs decoded up to the
// sample's step.  The result's values go to result_samples when given.
// Sample group `group` (the single launch's blockIdx.x); `words`: the dynamic
// LDS, (W + 1) rows x kSampleGroup.
__device__ __forceinline__ void pointwise_sample_group(
    const OperandA &a, const uint16_t *__restrict__ a_samples, const uint16_t *__restrict__ other,
    const OpArgs &args, int64_t n_blocks, int64_t logical_numel, int64_t sample_size, int S,
    int W, int rare, int32_t *__restrict__ partials, uint16_t *__restrict__ result_samples,
    int64_t group, uint32_t *words) {
    __shared__ DecodeTables tb;
    const int t = threadIdx.x;
    if (a_samples != nullptr) {
        const int64_t i = group * kSampleGroup + t;
        const bool active = i < sample_size;
        const int shift = __builtin_ctzll(static_cast<uint64_t>(sample_size));
        uint32_t result = 0;
        if (active) {
            const int64_t pos = sample_position(i, logical_numel, sample_size, shift);
            const OpParams p = load_op_params(args.op, args.alpha_is_one, args.beta_is_one,
                                              args.alpha, args.beta);
            result = apply_op(p, a_samples[i], other[pos]);
            if (result_samples != nullptr) result_samples[i] = static_cast<uint16_t>(result);
        }
        const int32_t exp = static_cast<int32_t>((result >> 7) & 255u) - 127;
        const bool keep = active && exp >= -120;
        const int32_t sum = wave_sum(keep ? exp : 0);
        const int32_t kept = wave_sum(keep ? 1 : 0);
        if (t == 0) {
            partials[2 * group] = sum;
            partials[2 * group + 1] = kept;
        }
        return;
    }
    int32_t packed[256 / kSampleGroup];
#pragma unroll
    for (int k = 0; k < 256 / kSampleGroup; ++k) packed[k] = a.shifted_decode[t + k * kSampleGroup];
    const int32_t center = a.center[0];
    const OpParams p = load_op_params(args.op, args.alpha_is_one, args.beta_is_one, args.alpha,
                                      args.beta);

    const int64_t i = group * kSampleGroup + t;
    const bool active = i < sample_size;
    const int shift = __builtin_ctzll(static_cast<uint64_t>(sample_size));
    const int64_t pos = active ? sample_position(i, logical_numel, sample_size, shift) : 0;
    const int64_t row = pos / kLanes;                 // storage row of the sample
    const int32_t lane = static_cast<int32_t>((pos % kLanes) ^ (row & 254));
    const int64_t block = row >> (S == 128 ? 7 : 8);   // S is 128 or 256
    const int32_t step = static_cast<int32_t>(row & (S - 1));
    const int64_t n_streams = n_blocks * kLanes;
    // The stream's words go straight to this thread's LDS column (row w at
    // words[w * 64 + t]); all W loads are in flight at once.  Inactive lanes
    // read stream 0.
    const int32_t *column = a.encoded + (active ? block * kLanes + lane : 0);
    for (int w = 0; w < W; ++w)
        __builtin_amdgcn_global_load_lds(
            column + w * n_streams,
            (__attribute__((address_space(3))) void *)(words + w * kSampleGroup), 4, 0, 0);
    words[W * kSampleGroup + t] = 0u;
    const uint32_t sm = active ? a.side[row * kLanes + lane] : 0u;
    const uint32_t b = active ? other[pos] : 0u;
#pragma unroll
    for (int k = 0; k < 256 / kSampleGroup; ++k)
        build_decode_entry(tb, t + k * kSampleGroup, packed[k], center);
    int32_t start;
    int64_t tail_index;
    stream_overlay(a.ov, active && a.has_overlay != 0, block, n_blocks, lane, S, start, tail_index);
    wait_memory();
    __syncthreads();   // decode tables and staged words

    uint32_t field = 0;
    if (step >= start) {
        field = tail_field(a.ov.tail[tail_index + (step - start)]);
    } else if (active) {
        // Steps before `start` hold payload codes; so do all earlier steps of
        // the stream, none of which is padding (their logical offsets are
        // below this sample's).
        StreamCursorT<kSampleGroup> cursor;
        cursor.init(words + t, &tb, static_cast<uint32_t>(W), rare);
        for (int pair = 0; pair < step / 2; ++pair) {
            uint32_t f0, f1;
            cursor.advance(cursor.next_fields(f0, f1));
        }
        uint32_t f0, f1;
        cursor.next_fields(f0, f1);
        field = (step & 1) ? f1 : f0;
    }
    const uint32_t result = apply_op(p, join_entry(field, sm), b);
    if (active && result_samples != nullptr) result_samples[i] = static_cast<uint16_t>(result);
    const int32_t exp = static_cast<int32_t>((result >> 7) & 255u) - 127;
    const bool keep = active && exp >= -120;
    const int32_t sum = wave_sum(keep ? exp : 0);
    const int32_t kept = wave_sum(keep ? 1 : 0);
    if (t == 0) {
        partials[2 * group] = sum;
        partials[2 * group + 1] = kept;
    }
}

__global__ __launch_bounds__(kSampleGroup) void pointwise_sample_kernel(
    OperandA a, const uint16_t *__restrict__ a_samples, const uint16_t *__restrict__ other,
    OpArgs args, int64_t n_blocks, int64_t logical_numel, int64_t sample_size, int S, int W,
    int rare, int32_t *__restrict__ partials, uint16_t *__restrict__ result_samples) {
    extern __shared__ uint32_t words[];   // (W + 1) rows x kSampleGroup
    pointwise_sample_group(a, a_samples, other, args, n_blocks, logical_numel, sample_size, S, W,
                           rare, partials, result_samples, blockIdx.x, words);
}

// ---- the fused decode -> operation -> encode kernel
//
// Memory operations are arranged for gfx9's single load/store counter
// (vmcnt): a chunk's A side bytes and B words are fetched one chunk ahead,
// before the previous chunk's stores are issued, and every store is
// unconditional -- lanes that must not write get an out-of-range buffer offset,
// which the hardware drops.  The compiler can then wait for exactly the loads
// it needs without also waiting for recent stores.

// Buffer offset rejected by the range check of every resource used here
// (num_records < 2^31): loads return 0, stores are dropped.
constexpr uint32_t kOutOfRange = 0x80000000u;

// Encoder state of one lane's output stream.  Word r of the stream is at byte
// r * row_bytes + 4 * lane of the block's payload resource.  pos counts the
// bits of every pair so far, so once a pair does not fit, pos stays above the
// limit and every later pair overflows too (encode.py:73-90: only the first
// overflowing pair matters); word and row_off then keep the bits before that
// pair, which finish() stores.
struct StreamWriter {
    __amdgpu_buffer_rsrc_t out;
    uint32_t row_bytes;   // 4 * n_streams
    uint32_t row_off;     // byte offset of the word being filled
    uint32_t end_off;     // row_off of row W
    uint32_t limit;       // 32 W
    uint32_t pos;         // bits of all pairs so far
    uint32_t word;        // bits of the word being filled
    uint32_t fits;        // pairs that fit

    __device__ __forceinline__ bool overflowed() const { return pos > limit; }

    // Hold row_bytes in a VGPR from here on: a row advance is then one
    // v_cndmask and one v_add per pair (with row_bytes in an SGPR beside the
    // SGPR condition, gfx9's one-scalar-operand limit costs a copy per pair).
    __device__ __forceinline__ void keep_row_bytes_in_vgpr() { asm volatile("" : "+v"(row_bytes)); }

    // The first pair that did not fit is the one after the pairs that fit, so
    // its (even) step is twice their count.
    __device__ __forceinline__ int32_t extra_start() const { return static_cast<int32_t>(2 * fits); }

    // Append the pair code of encode entries e0/e1 ({reversed code, length};
    // {0, 0} = no code), following encode.py:66-90.  Returns whether the pair
    // (and so every later one) overflows.  A pair that completes a word
    // stores it.
    __device__ __forceinline__ bool put(uint2 e0, uint2 e1) {
        const uint32_t code = e0.x | (e1.x << e0.y);
        const uint32_t len = e0.y + e1.y;
        const uint32_t shift = pos & 31u;
        const uint64_t placed = static_cast<uint64_t>(code) << shift;
        const uint32_t new_word = word | static_cast<uint32_t>(placed);
        const uint32_t after = pos + len;
        const bool ok = after <= limit;
        const bool completes = ok && shift + len >= 32u;
        __builtin_amdgcn_raw_buffer_store_b32(new_word, out, completes ? row_off : kOutOfRange,
                                              0, 0);
        row_off += completes ? row_bytes : 0u;
        word = ok ? (completes ? static_cast<uint32_t>(placed >> 32) : new_word) : word;
        fits += ok ? 1u : 0u;
        pos = after;
        return !ok;
    }

    // Append a pair that is known to fit (its chunk passed fits_chunk): the
    // same bits and stores as put() without the overflow bookkeeping; the
    // chunk's caller adds its pairs to `fits` at the end.
    __device__ __forceinline__ void put_fast(uint2 e0, uint2 e1) {
        const uint32_t code = e0.x | (e1.x << e0.y);
        const uint32_t len = e0.y + e1.y;
        const uint32_t shift = pos & 31u;
        const uint64_t placed = static_cast<uint64_t>(code) << shift;
        const uint32_t new_word = word | static_cast<uint32_t>(placed);
        const bool completes = shift + len >= 32u;
        __builtin_amdgcn_raw_buffer_store_b32(new_word, out, completes ? row_off : kOutOfRange,
                                              0, 0);
        row_off += completes ? row_bytes : 0u;
        word = completes ? static_cast<uint32_t>(placed >> 32) : new_word;
        pos += len;
    }

    // Whether every pair of the next `steps` steps fits for every lane of the
    // wave (a symbol's code is at most 16 bits: ESC of at most 8 bits and an
    // 8-bit literal).  Wave-uniform.
    __device__ __forceinline__ bool fits_chunk(int steps) const {
        return __all(pos + 16u * static_cast<uint32_t>(steps) <= limit);
    }

    // After the last pair: the word being filled (the bits before the first
    // pair that did not fit, for an overflowing stream), then zero words up to
    // row W-1.
    __device__ __forceinline__ void finish() {
        for (; row_off < end_off; row_off += row_bytes) {
            __builtin_amdgcn_raw_buffer_store_b32(word, out, row_off, 0, 0);
            word = 0u;
        }
    }
};

// Encode-table entry as the kernel keeps it in LDS: {reversed code (<= 16
// bits), code length}, 8 bytes, so one 8-byte read gives both without masks
// (shifted tables: tables.py:53-67).
__device__ __forceinline__ uint2 repack_encode_entry(uint32_t packed) {
    return make_uint2(packed & 0xFFFFu, packed >> 20);
}

// Exponent bytes of a pair of BF16 results r (step s0 in bits 0..15, s0 + 1 in
// bits 16..31): bytes 0 and 2 of r >> 7.  The shift is kept opaque so that
// each encode-table address is one byte-selecting shift (SDWA) of it, where
// the compiler would otherwise fold shift and mask into two ops per index.
__device__ __forceinline__ uint32_t exponent_bytes(uint32_t r) {
    uint32_t x = r >> 7;
    asm("" : "+v"(x));
    return x;
}

// The side byte of a high-half BF16 result in bits 16..23: the mantissa stays
// in bits 16..22 and the sign comes down from bit 31 (one v_bfi_b32 after a
// shift; the compiler otherwise builds it from three instructions).
__device__ __forceinline__ uint32_t side_byte_at_16(uint32_t h) {
    uint32_t out;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(out) : "s"(0x007F0000u), "v"(h), "v"(h >> 8));
    return out;
}

struct UpdateIo {
    __amdgpu_buffer_rsrc_t side;       // A's side bytes (storage order)
    __amdgpu_buffer_rsrc_t other;      // B, BF16 in logical order
    __amdgpu_buffer_rsrc_t side_out;   // result side bytes (storage order)
    __amdgpu_buffer_rsrc_t exponents;  // result exponent bytes of overflow rows (logical order)
};

// B words of the 16-step chunk at `first` (one 4-byte word per lane per step
// pair, lane-pair layout), or zeros without memory traffic when !fetch.
__device__ __forceinline__ void fetch_b_chunk(uint32_t (&bw)[kChunkSteps / 2],
                                              const UpdateIo &io, const LanePair &lp,
                                              int64_t row_base, int first, bool fetch) {
    const uint32_t mask2 = static_cast<uint32_t>((row_base + first) & 254) * 2u;
#pragma unroll
    for (int j = 0; j < kChunkSteps; j += 2)
        bw[j / 2] = __builtin_amdgcn_raw_buffer_load_b32(
            io.other, fetch ? (lp.offset2 ^ mask2 ^ static_cast<uint32_t>(2 * j)) : kOutOfRange,
            (first + j) * kLanes * 2, 0);
}

// Results r0/r1 (BF16 in the high halves) of this lane's pair at `step`: side
// bytes replace A's in the wave's slice, the exponent bytes are encoded, and
// an overflowing pair's exponent bytes go to the exponent array (positions
// past the tensor's end are outside its resource and are dropped).
__device__ __forceinline__ void emit_pair(StreamWriter &writer, const uint2 *enc,
                                          uint8_t *slice, int s0, uint32_t h0, uint32_t h1,
                                          bool v0, bool v1, uint32_t off0, const UpdateIo &io) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    slice[s0 * kWave + lane] = static_cast<uint8_t>(side_byte_at_16(h0) >> 16);
    slice[(s0 + 1) * kWave + lane] = static_cast<uint8_t>(side_byte_at_16(h1) >> 16);
    const uint32_t x0 = high_exponent_byte(h0);
    const uint32_t x1 = high_exponent_byte(h1);
    // Positions past the logical end carry no code (encode.py:255-256).
    const uint2 e0 = v0 ? enc[x0] : make_uint2(0u, 0u);
    const uint2 e1 = v1 ? enc[x1] : make_uint2(0u, 0u);
    const bool over = writer.put(e0, e1);
    const uint32_t exp_off = over ? off0 : kOutOfRange;
    __builtin_amdgcn_raw_buffer_store_b8(x0, io.exponents, exp_off, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b8(x1, io.exponents, exp_off + kLanes, 0, 0);
}

// Chunks [c_begin, c_end) with one overlay variant of A.  On entry side_next
// and b_next hold chunk c_begin's A side bytes and B words (B only for full
// blocks); on exit those of chunk c_end.  kForm < 0: the operation is chosen at
// run time (the last, partial block).
template <bool kFull, Overlay kOverlay, int S, int kForm>
__device__ __forceinline__ void update_chunks(UpdateCursor &cursor, const LaneOverlay &lane,
                                              const uint8_t *tail_lds, uint8_t *slice,
                                              SideChunk &side_next,
                                              uint32_t (&b_next)[kChunkSteps / 2],
                                              StreamWriter &writer, const uint2 *enc,
                                              const UpdateIo &io, const LanePair &lp,
                                              int64_t row_base, uint32_t valid_in_block,
                                              int c_begin, int c_end, const OpParams &p) {
    const uint32_t voffset = side_fetch_offset();
#pragma unroll 1
    for (int c = c_begin; c < c_end; c += kChunkSteps) {
        store_side_chunk(slice, side_next);
        uint32_t b_cur[kChunkSteps / 2];
#pragma unroll
        for (int k = 0; k < kChunkSteps / 2; ++k) b_cur[k] = b_next[k];
        const bool more = c + kChunkSteps < S;
        side_next = fetch_side_chunk(io.side, more ? voffset : kOutOfRange, c + kChunkSteps);
        if (kFull) fetch_b_chunk(b_next, io, lp, row_base, c + kChunkSteps, more);
        const uint32_t mask = static_cast<uint32_t>((row_base + c) & 254);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int first = c + half * kHalfSteps;
            uint32_t f[kHalfSteps];
            decode_fields<kFull, kOverlay>(cursor, lane, tail_lds, first, row_base,
                                           valid_in_block, f);
#pragma unroll
            for (int j = 0; j < kHalfSteps; j += 2) {
                const int s0 = half * kHalfSteps + j;   // step within the chunk
                const int step = c + s0;
                // Logical offset (in the block) of this lane's element of row
                // `step`; row step+1 shares the swizzle mask, and the chunk's
                // first row is a multiple of 16, so the mask of row c+s0 is
                // mask ^ s0.
                const uint32_t off0 = static_cast<uint32_t>(step) * kLanes
                    + (threadIdx.x ^ mask ^ static_cast<uint32_t>(s0));
                const float a0 = __uint_as_float(join_float(f[j], side_byte(slice, s0)));
                const float a1 = __uint_as_float(join_float(f[j + 1], side_byte(slice, s0 + 1)));
                uint32_t h0, h1;
                bool v0 = true, v1 = true;
                if (kFull) {
                    float b0, b1;
                    pair_unpack16(lp, b_cur[s0 / 2], b0, b1);
                    h0 = round_bf16_high(apply_form<kForm>(p, a0, b0));
                    h1 = round_bf16_high(apply_form<kForm>(p, a1, b1));
                } else {
                    v0 = off0 < valid_in_block;
                    v1 = off0 + kLanes < valid_in_block;
                    // Outside the tensor the resource returns 0.
                    const uint32_t b0 = __builtin_amdgcn_raw_buffer_load_b16(io.other, off0 * 2, 0, 0);
                    const uint32_t b1 = __builtin_amdgcn_raw_buffer_load_b16(
                        io.other, (off0 + kLanes) * 2, 0, 0);
                    // Padding positions hold 0 (side byte 0, no code).
                    h0 = v0 ? apply_op_f(p, a0, bf16_to_float(b0)) << 16 : 0u;
                    h1 = v1 ? apply_op_f(p, a1, bf16_to_float(b1)) << 16 : 0u;
                }
                emit_pair(writer, enc, slice, s0, h0, h1, v0, v1, off0, io);
            }
        }
        // The slice now holds the chunk's result side bytes.
        const uint4 q = reinterpret_cast<const uint4 *>(slice)[threadIdx.x & (kWave - 1)];
        store_b128<kSideStore>(q, io.side_out, voffset + static_cast<uint32_t>(c) * kLanes);
    }
}

// ---- the pipelined full-block path
//
// Each stream's decode is a chain of dependent LDS lookups, and only about 2.7
// waves per SIMD exist at C4's 688 blocks, so the chains' latency used to go
// unhidden.  Here the wave interleaves, pair by pair, the arithmetic and
// encoding of one 8-step half with the decoding of the next half: the two are
// independent, so the compiler fills each lookup's wait with the other half's
// work.  A chunk in which no lane of the wave can overflow (fits_chunk) also
// skips the overflow bookkeeping and the exponent stores, which only overflow
// rows need.

// The arithmetic and encoding of this lane's pair at chunk step s0 (absolute
// step c + s0), in stages that the caller interleaves with a decode's lookups:
// A's entries f0/f1 joined with A's side bytes from the slice and B from the
// pair's word (emit_operands), the operation, BF16 rounding, the result's side
// bytes into the slice and the encode-table reads (emit_result), and the
// exponent codes into the stream (emit_codes).
struct EmitState {
    uint32_t sa0, sa1;   // A's side bytes
    float b0, b1;        // B
    uint32_t r;          // the results' BF16 bits (step s0 low, s0 + 1 high)
    uint2 e0, e1;        // their encode entries
};

__device__ __forceinline__ void emit_operands(EmitState &st, const uint8_t *slice, int s0,
                                              uint32_t b_word, const LanePair &lp) {
    st.sa0 = side_byte(slice, s0);
    st.sa1 = side_byte(slice, s0 + 1);
    pair_unpack16(lp, b_word, st.b0, st.b1);
}

template <int kForm>
__device__ __forceinline__ void emit_result(EmitState &st, const uint2 *enc, uint8_t *slice,
                                            int s0, uint32_t f0, uint32_t f1,
                                            const OpParams &p) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const float a0 = __uint_as_float(join_float(f0, st.sa0));
    const float a1 = __uint_as_float(join_float(f1, st.sa1));
    const uint32_t r = round_pair_bf16(apply_form<kForm>(p, a0, st.b0),
                                       apply_form<kForm>(p, a1, st.b1));
    // Side bytes: the mantissa and, from r >> 8, the sign of each half.
    const uint32_t sign_down = r >> 8;
    uint32_t side0, side1;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(side0) : "s"(0x7Fu), "v"(r), "v"(sign_down));
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(side1) : "s"(0x007F0000u), "v"(r), "v"(sign_down));
    slice[s0 * kWave + lane] = static_cast<uint8_t>(side0);
    slice[(s0 + 1) * kWave + lane] = static_cast<uint8_t>(side1 >> 16);
    const uint32_t x = exponent_bytes(r);
    st.e0 = enc[x & 255u];
    st.e1 = enc[(x >> 16) & 255u];
    st.r = r;
}

template <bool kFast>
__device__ __forceinline__ void emit_codes(const EmitState &st, StreamWriter &writer,
                                           uint32_t off0, const UpdateIo &io) {
    if (kFast) {
        writer.put_fast(st.e0, st.e1);
    } else {
        const bool over = writer.put(st.e0, st.e1);
        const uint32_t exp_off = over ? off0 : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b8(st.r >> 7, io.exponents, exp_off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b8(st.r >> 23, io.exponents, exp_off + kLanes, 0, 0);
    }
}

// One half (8 steps from chunk step `half` * 8) of emitting f, interleaved pair
// by pair with decoding the 8 steps from `next_step` into g (kDecode).  The
// order within a pair is pinned with scheduling barriers: each of the
// decode's two dependent lookups is followed by independent emit work that
// fills its latency.
template <Overlay kOverlay, int kForm, bool kFast, bool kDecode, class Cursor>
__device__ __forceinline__ void pipelined_half(Cursor &cursor, const LaneOverlay &lane,
                                               const uint8_t *tail_lds, uint8_t *slice,
                                               StreamWriter &writer, const uint2 *enc,
                                               const UpdateIo &io, const LanePair &lp,
                                               const OpParams &p, int64_t row_base, int c,
                                               int half, uint32_t mask,
                                               const uint32_t (&b_cur)[kChunkSteps / 2],
                                               const uint32_t (&f)[kHalfSteps],
                                               uint32_t (&g)[kHalfSteps], int next_step) {
#pragma unroll
    for (int j = 0; j < kHalfSteps; j += 2) {
        const int s0 = half * kHalfSteps + j;
        const uint32_t off0 = static_cast<uint32_t>(c + s0) * kLanes
            + (threadIdx.x ^ mask ^ static_cast<uint32_t>(s0));
        EmitState st;
        uint32_t bits = 0, t0 = 0, t1 = 0;
        if (kDecode) cursor.first_lookup(bits, t0);
        __builtin_amdgcn_sched_barrier(0);
        emit_operands(st, slice, s0, b_cur[s0 / 2], lp);
        __builtin_amdgcn_sched_barrier(0);
        if (kDecode) t1 = cursor.second_lookup(bits, t0);
        __builtin_amdgcn_sched_barrier(0);
        emit_result<kForm>(st, enc, slice, s0, f[j], f[j + 1], p);
        __builtin_amdgcn_sched_barrier(0);
        if (kDecode) {
            uint32_t sum = cursor.resolve(bits, t0, t1);
            if (kOverlay != kNoOverlay) {
                overlay_pair<kOverlay == kLdsOverlay, typename Cursor::TablesT>(lane, tail_lds,
                                                                                next_step + j,
                                                                                t0, t1);
                sum = (t0 + t1) & 127u;
            }
            cursor.advance(sum);
            g[j] = t0;
            g[j + 1] = t1;
        }
        __builtin_amdgcn_sched_barrier(0);
        emit_codes<kFast>(st, writer, off0, io);
    }
}

// Both halves of the chunk at c; f holds the first half's entries on entry and
// the next chunk's first half's on exit (when kDecodeNext).
template <Overlay kOverlay, int kForm, bool kFast, bool kDecodeNext, class Cursor>
__device__ __forceinline__ void pipelined_chunk(Cursor &cursor, const LaneOverlay &lane,
                                                const uint8_t *tail_lds, uint8_t *slice,
                                                StreamWriter &writer, const uint2 *enc,
                                                const UpdateIo &io, const LanePair &lp,
                                                const OpParams &p, int64_t row_base, int c,
                                                uint32_t mask,
                                                const uint32_t (&b_cur)[kChunkSteps / 2],
                                                uint32_t (&f)[kHalfSteps]) {
    uint32_t g[kHalfSteps];
    pipelined_half<kOverlay, kForm, kFast, true>(cursor, lane, tail_lds, slice, writer, enc, io,
                                                 lp, p, row_base, c, 0, mask, b_cur, f, g,
                                                 c + kHalfSteps);
    pipelined_half<kOverlay, kForm, kFast, kDecodeNext>(cursor, lane, tail_lds, slice, writer,
                                                        enc, io, lp, p, row_base, c, 1, mask,
                                                        b_cur, g, f, c + kChunkSteps);
    if (kFast) writer.fits += kChunkSteps / 2;
}

// Chunks [c_begin, c_end) of a full block with one overlay variant of A; as
// update_chunks<true, ...>.  The segment's first half is decoded before the
// loop and its last chunk decodes nothing further, so no step outside the
// segment is decoded with this variant.
// A's side bytes and B's words of the next two chunks (fetched two chunks
// ahead: one chunk of work is shorter than HBM's latency under load).
struct Prefetch {
    SideChunk side1, side2;
    uint32_t b1[kChunkSteps / 2], b2[kChunkSteps / 2];
};

// One chunk at c using the side bytes and B words in (side, b) -- the copy of
// the two that holds chunk c -- and refilling them with chunk c + 32.  The two
// copies alternate, so a chunk's loads are issued two chunks before use and no
// register copy of an in-flight load (which would wait for it) is made.
template <Overlay kOverlay, int S, int kForm, class Cursor>
__device__ __forceinline__ void pipelined_step(Cursor &cursor, const LaneOverlay &lane,
                                               const uint8_t *tail_lds, uint8_t *slice,
                                               SideChunk &side, uint32_t (&b)[kChunkSteps / 2],
                                               StreamWriter &writer, const uint2 *enc,
                                               const UpdateIo &io, const LanePair &lp,
                                               int64_t row_base, int c, int c_end,
                                               const OpParams &p, uint32_t (&f)[kHalfSteps]) {
    const uint32_t voffset = side_fetch_offset();
    store_side_chunk(slice, side);
    uint32_t b_cur[kChunkSteps / 2];
#pragma unroll
    for (int k = 0; k < kChunkSteps / 2; ++k) b_cur[k] = b[k];
    const bool more = c + 2 * kChunkSteps < S;
    side = fetch_side_chunk(io.side, more ? voffset : kOutOfRange, c + 2 * kChunkSteps);
    fetch_b_chunk(b, io, lp, row_base, c + 2 * kChunkSteps, more);
    const uint32_t mask = static_cast<uint32_t>((row_base + c) & 254);
    const bool fast = writer.fits_chunk(kChunkSteps);
    const bool next = c + kChunkSteps < c_end;
#define LCT_CHUNK(FAST, NEXT)                                                                 \
    pipelined_chunk<kOverlay, kForm, FAST, NEXT>(cursor, lane, tail_lds, slice, writer, enc, \
                                                 io, lp, p, row_base, c, mask, b_cur, f)
    if (fast) {
        if (next) LCT_CHUNK(true, true);
        else LCT_CHUNK(true, false);
    } else {
        if (next) LCT_CHUNK(false, true);
        else LCT_CHUNK(false, false);
    }
#undef LCT_CHUNK
    // The slice now holds the chunk's result side bytes.
    const uint4 q = reinterpret_cast<const uint4 *>(slice)[threadIdx.x & (kWave - 1)];
    store_b128<kSideStore>(q, io.side_out, voffset + static_cast<uint32_t>(c) * kLanes);
}

// Chunks [c_begin, c_end); pf.side1/b1 hold chunk c_begin's data and
// side2/b2 chunk c_begin + 16's.  On exit the same holds for c_end.
template <Overlay kOverlay, int S, int kForm, class Cursor>
__device__ __forceinline__ void update_chunks_pipelined(
    Cursor &cursor, const LaneOverlay &lane, const uint8_t *tail_lds, uint8_t *slice,
    Prefetch &pf, StreamWriter &writer, const uint2 *enc, const UpdateIo &io,
    const LanePair &lp, int64_t row_base, int c_begin, int c_end, const OpParams &p) {
    if (c_begin >= c_end) return;
    uint32_t f[kHalfSteps];
    decode_fields<true, kOverlay>(cursor, lane, tail_lds, c_begin, row_base, 0u, f);
    int c = c_begin;
#pragma unroll 1
    for (; c + kChunkSteps < c_end; c += 2 * kChunkSteps) {
        pipelined_step<kOverlay, S, kForm>(cursor, lane, tail_lds, slice, pf.side1, pf.b1,
                                           writer, enc, io, lp, row_base, c, c_end, p, f);
        pipelined_step<kOverlay, S, kForm>(cursor, lane, tail_lds, slice, pf.side2, pf.b2,
                                           writer, enc, io, lp, row_base, c + kChunkSteps, c_end,
                                           p, f);
    }
    if (c < c_end) {
        pipelined_step<kOverlay, S, kForm>(cursor, lane, tail_lds, slice, pf.side1, pf.b1,
                                           writer, enc, io, lp, row_base, c, c_end, p, f);
        // An odd number of chunks: the next chunk's data is in the second copy.
        // Swapping waits for its loads, once per block at most.
        const SideChunk side = pf.side1;
        pf.side1 = pf.side2;
        pf.side2 = side;
#pragma unroll
        for (int k = 0; k < kChunkSteps / 2; ++k) {
            const uint32_t b = pf.b1[k];
            pf.b1[k] = pf.b2[k];
            pf.b2[k] = b;
        }
    }
}

template <bool kFull, int S, int kForm>
__device__ __forceinline__ void update_rows(UpdateCursor cursor, const LaneOverlay &lane,
                                            const uint8_t *tail_lds, uint8_t *slice,
                                            SideChunk side_next, StreamWriter &writer,
                                            const uint2 *enc, const UpdateIo &io,
                                            int64_t row_base, uint32_t valid_in_block,
                                            const OpParams &p) {
    const LanePair lp;
    const int split = min(S, lane.wave_start & ~(kChunkSteps - 1));
    if (kFull) {
        // Full blocks decode with the LDS-window cursor (the stage has two pad
        // rows); the partial block keeps the register window.
        UpdateWindow wc;
        wc.init(cursor.stage, cursor.tb, cursor.pad_row, cursor.rare, cursor.center);
        Prefetch pf;
        pf.side1 = side_next;
        pf.side2 = fetch_side_chunk(io.side, side_fetch_offset(), kChunkSteps);
        fetch_b_chunk(pf.b1, io, lp, row_base, 0, true);
        fetch_b_chunk(pf.b2, io, lp, row_base, kChunkSteps, true);
        update_chunks_pipelined<kNoOverlay, S, kForm>(wc, lane, tail_lds, slice, pf, writer,
                                                      enc, io, lp, row_base, 0, split, p);
        if (split == S) return;
        if (lane.lds)
            update_chunks_pipelined<kLdsOverlay, S, kForm>(wc, lane, tail_lds, slice, pf,
                                                           writer, enc, io, lp, row_base, split,
                                                           S, p);
        else
            update_chunks_pipelined<kHbmOverlay, S, kForm>(wc, lane, tail_lds, slice, pf,
                                                           writer, enc, io, lp, row_base, split,
                                                           S, p);
        return;
    }
    uint32_t b_next[kChunkSteps / 2];
    update_chunks<kFull, kNoOverlay, S, kForm>(cursor, lane, tail_lds, slice, side_next, b_next,
                                               writer, enc, io, lp, row_base, valid_in_block, 0,
                                               split, p);
    if (split == S) return;
    if (lane.lds)
        update_chunks<kFull, kLdsOverlay, S, kForm>(cursor, lane, tail_lds, slice, side_next,
                                                    b_next, writer, enc, io, lp, row_base,
                                                    valid_in_block, split, S, p);
    else
        update_chunks<kFull, kHbmOverlay, S, kForm>(cursor, lane, tail_lds, slice, side_next,
                                                    b_next, writer, enc, io, lp, row_base,
                                                    valid_in_block, split, S, p);
}

// Full blocks take the operation's form as a template parameter; the last,
// partial block decides at run time.
template <int S>
__device__ __forceinline__ void update_block(int32_t form, bool full, const UpdateCursor &cursor,
                                             const LaneOverlay &lane, const uint8_t *tail_lds,
                                             uint8_t *slice, const SideChunk &side_next,
                                             StreamWriter &writer, const uint2 *enc,
                                             const UpdateIo &io, int64_t row_base,
                                             uint32_t valid_in_block, const OpParams &p) {
    if (!full) {
        update_rows<false, S, -1>(cursor, lane, tail_lds, slice, side_next, writer, enc, io,
                                  row_base, valid_in_block, p);
        return;
    }
    switch (form) {
    case kFormAxpy:
        update_rows<true, S, kFormAxpy>(cursor, lane, tail_lds, slice, side_next, writer, enc, io,
                                        row_base, valid_in_block, p);
        break;
    case kFormAxpby:
        update_rows<true, S, kFormAxpby>(cursor, lane, tail_lds, slice, side_next, writer, enc,
                                         io, row_base, valid_in_block, p);
        break;
    case kFormBxpa:
        update_rows<true, S, kFormBxpa>(cursor, lane, tail_lds, slice, side_next, writer, enc, io,
                                        row_base, valid_in_block, p);
        break;
    default:
        update_rows<true, S, kFormMul>(cursor, lane, tail_lds, slice, side_next, writer, enc, io,
                                       row_base, valid_in_block, p);
        break;
    }
}

// Codec block `block` of one fused update (the single launch's blockIdx.x);
// `stage`: the dynamic LDS, window_stage_bytes(W) (A's payload).
template <bool kBooked>
__device__ __forceinline__ void pointwise_encode_block(
    const OperandA &a, const uint16_t *__restrict__ other, const OpArgs &args,
    const int32_t *__restrict__ partials, int32_t n_groups,
    const int32_t *__restrict__ base_encode, const int32_t *__restrict__ base_decode,
    int32_t *__restrict__ center_out, int32_t *__restrict__ shifted_decode_out,
    uint8_t *__restrict__ side_out, int32_t *__restrict__ encoded_out,
    uint8_t *__restrict__ extra_starts, int32_t *__restrict__ summaries,
    uint8_t *__restrict__ exponents, int64_t n_blocks, int64_t logical_numel, int S, int W,
    int rare, const KernelBookkeeping &bk, int64_t block, uint32_t *stage) {
    __shared__ FloatDecodeTables tb;
    __shared__ uint2 enc[256];
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t shared_center;
    __shared__ uint8_t tail_lds[kTailLds];
    // The overflow maps (2 KiB) and the raw encode table (1 KiB) are only used
    // before the first side chunk is stored, so they share the side slices.
    __shared__ __attribute__((aligned(16))) uint8_t side_slices[kWavesPerBlock][kChunkSteps * kWave];
    int32_t *map_start = reinterpret_cast<int32_t *>(&side_slices[0][0]);
    int32_t *map_offset = map_start + kLanes;
    int32_t *raw_encode = map_offset + kLanes;
    const int t = threadIdx.x;
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    const uint32_t block_elems = static_cast<uint32_t>(S) * kLanes;
    const int64_t remaining = logical_numel - logical_base;
    const uint32_t valid = remaining < block_elems ? static_cast<uint32_t>(remaining) : block_elems;
    UpdateIo io;
    io.side = make_rsrc(a.side + logical_base, block_elems);
    io.other = make_rsrc(other + logical_base, 2u * valid);
    io.side_out = make_rsrc(side_out + logical_base, block_elems);
    io.exponents = make_rsrc(exponents + logical_base, valid);
    const SideChunk first = fetch_side_chunk(io.side, side_fetch_offset(), 0);

    // The result's center from the sampler's partial sums.
    raw_encode[t] = base_encode[t];
    center_from_partials(partials, n_groups, &shared_center);
    build_float_decode_tables(tb, a.shifted_decode);
    const int32_t a_center = a.center[0];
    stage_payload(stage, a.encoded, n_blocks * kLanes, block, W);
    stage[(W + 1) * kLanes + t] = 0u;   // the window cursor's second pad row
    __syncthreads();   // center and raw encode table
    const int32_t center = shared_center;
    enc[t] = repack_encode_entry(static_cast<uint32_t>(raw_encode[byte_to_index(t, center)]));
    if (block == 0) {
        if (t == 0) center_out[0] = center;
        for (int i = t; i < 1024; i += kLanes)
            shifted_decode_out[i] = shifted_decode_entry(base_decode[i], center);
    }
    __syncthreads();   // raw_encode is no longer read (it shares the maps' LDS)
    const LaneOverlay lane = build_overlay(a.ov, a.has_overlay != 0, block, n_blocks, S, map_start,
                                           map_offset, scratch, tail_lds, kTailLds);
    // (Issued here rather than with the prologue's first loads: hoisted, the
    // measured kernel was 0.8 us slower.)
    const OpParams p = load_op_params(args.op, args.alpha_is_one, args.beta_is_one, args.alpha,
                                      args.beta);
    wait_memory();
    __syncthreads();   // payload, tails and encode table visible; maps no longer read

    UpdateCursor cursor;
    cursor.init(stage + t, &tb, static_cast<uint32_t>(W), rare, a_center);
    const uint32_t row_bytes = static_cast<uint32_t>(n_blocks * kLanes * 4);
    StreamWriter writer{make_rsrc(encoded_out + block * kLanes,
                                  static_cast<uint32_t>(W - 1) * row_bytes + kLanes * 4),
                        row_bytes, static_cast<uint32_t>(t) * 4u,
                        static_cast<uint32_t>(W) * row_bytes + static_cast<uint32_t>(t) * 4u,
                        static_cast<uint32_t>(W) * 32u, 0u, 0u, 0u};
    writer.keep_row_bytes_in_vgpr();
    uint8_t *slice = side_slices[t / kWave];
    const bool full = valid == block_elems;
    const int32_t form = form_of(args.op, args.alpha_is_one, args.beta_is_one);
    if (S == 128)
        update_block<128>(form, full, cursor, lane, tail_lds, slice, first, writer, enc, io,
                          row_base, valid, p);
    else
        update_block<256>(form, full, cursor, lane, tail_lds, slice, first, writer, enc, io,
                          row_base, valid, p);
    writer.finish();
    const bool overflow = writer.overflowed();
    const int32_t extra = writer.extra_start();
    extra_starts[block * kLanes + t] = static_cast<uint8_t>(overflow ? extra : 255);
    // Streams from bit 20 (at most 256), tail bytes in bits 0..19 (at most
    // 256 x 256): one block scan.
    const int32_t both = block_sum(overflow ? (S - extra) | (1 << 20) : 0, scratch);
    publish_block<kBooked>(bk, summaries, block, n_blocks, both >> 20, both & 0xFFFFF,
                           reinterpret_cast<int32_t *>(stage));
}

template <bool kBooked>
__global__ __launch_bounds__(kLanes) void pointwise_encode_kernel(
    OperandA a, const uint16_t *__restrict__ other, OpArgs args,
    const int32_t *__restrict__ partials, int32_t n_groups,
    const int32_t *__restrict__ base_encode, const int32_t *__restrict__ base_decode,
    int32_t *__restrict__ center_out, int32_t *__restrict__ shifted_decode_out,
    uint8_t *__restrict__ side_out, int32_t *__restrict__ encoded_out,
    uint8_t *__restrict__ extra_starts, int32_t *__restrict__ summaries,
    uint8_t *__restrict__ exponents, int64_t n_blocks, int64_t logical_numel, int S, int W,
    int rare, KernelBookkeeping bk) {
    extern __shared__ uint32_t stage[];   // A's payload: window_stage_bytes(W)
    pointwise_encode_block<kBooked>(a, other, args, partials, n_groups, base_encode, base_decode,
                                    center_out, shifted_decode_out, side_out, encoded_out,
                                    extra_starts, summaries, exponents, n_blocks, logical_numel,
                                    S, W, rare, bk, blockIdx.x, stage);
}

// ---- several fused updates of one operation in three launches
//
// A layer's weights are a few codec blocks each, so one update's sampler,
// encoder and compaction are each bound by one block's latency; the batched
// form runs up to LCT_MAX_UPDATE_BATCH tensors' samplers in one launch, their
// encoders (with the in-launch bookkeeping, buffered) in a second and their
// compactions in a third.  Workgroup w of a launch works for the last job
// whose first workgroup is at most w.  The job tables travel in the kernel
// arguments.

struct UpdateSampleJob {
    OperandA a;
    const uint16_t *a_samples;
    const uint16_t *other;
    int32_t *partials;
    uint16_t *result_samples;
    int64_t n_blocks;
    int64_t logical_numel;
    int64_t sample_size;
    int32_t steps;
    int32_t fixed_words;
    int32_t rare;
};

struct UpdateSampleBatch {
    int32_t n_jobs;
    int32_t first_group[LCT_MAX_UPDATE_BATCH + 1];
    UpdateSampleJob jobs[LCT_MAX_UPDATE_BATCH];
    OpArgs args;
};

__global__ __launch_bounds__(kSampleGroup) void pointwise_sample_batch_kernel(
    UpdateSampleBatch batch) {
    extern __shared__ uint32_t words[];   // (max W + 1) rows x kSampleGroup
    const int32_t w = static_cast<int32_t>(blockIdx.x);
    int j = 0;
    for (int k = 1; k < batch.n_jobs; ++k)
        if (w >= batch.first_group[k]) j = k;
    const UpdateSampleJob &job = batch.jobs[j];
    pointwise_sample_group(job.a, job.a_samples, job.other, batch.args, job.n_blocks,
                           job.logical_numel, job.sample_size, job.steps, job.fixed_words,
                           job.rare, job.partials, job.result_samples,
                           w - batch.first_group[j], words);
}

struct UpdateEncodeJob {
    OperandA a;
    const uint16_t *other;
    const int32_t *partials;
    const int32_t *base_encode;
    const int32_t *base_decode;
    int32_t *center_out;
    int32_t *shifted_decode_out;
    uint8_t *side_out;
    int32_t *encoded_out;
    uint8_t *extra_starts;
    int32_t *summaries;
    uint8_t *exponents;
    uint64_t *control;
    int32_t *counts;
    int32_t *blocks;
    int32_t *descriptor;
    int64_t n_blocks;
    int64_t logical_numel;
    int32_t n_groups;
    int32_t steps;
    int32_t fixed_words;
    int32_t rare;
};

struct UpdateEncodeBatch {
    int32_t n_jobs;
    int32_t first_block[LCT_MAX_UPDATE_BATCH + 1];
    UpdateEncodeJob jobs[LCT_MAX_UPDATE_BATCH];
    OpArgs args;
    int32_t *buffer_meta;
    int32_t max_free_regions;
    lct_pending_frees frees;   // job 0 applies them
    uint64_t *gate;            // nullptr without frees
    uint32_t epoch;
    int32_t lock_spins;
    int32_t polls;
};

__global__ __launch_bounds__(kLanes) void pointwise_encode_batch_kernel(UpdateEncodeBatch batch) {
    extern __shared__ uint32_t stage[];   // window_stage_bytes(max W), or the free list
    const int32_t w = static_cast<int32_t>(blockIdx.x);
    int j = 0;
    for (int k = 1; k < batch.n_jobs; ++k)
        if (w >= batch.first_block[k]) j = k;
    const UpdateEncodeJob &job = batch.jobs[j];
    KernelBookkeeping bk{job.control, batch.epoch, job.counts, job.blocks, job.descriptor,
                         batch.buffer_meta, batch.max_free_regions, batch.frees,
                         batch.lock_spins, batch.polls, batch.gate, j == 0 ? 1 : 0};
    if (j != 0) bk.frees.count = 0;
    pointwise_encode_block<true>(job.a, job.other, batch.args, job.partials, job.n_groups,
                                 job.base_encode, job.base_decode, job.center_out,
                                 job.shifted_decode_out, job.side_out, job.encoded_out,
                                 job.extra_starts, job.summaries, job.exponents, job.n_blocks,
                                 job.logical_numel, job.steps, job.fixed_words, job.rare, bk,
                                 w - batch.first_block[j], stage);
}

// ---- the two-compressed form: alpha * A + B with compressed output
//
// The reference's weight update (LCT/LCTensor.py:91-99 -> codec/pointwise.py:
// 159-210 with dense_output=False) runs the dual kernel with
// COMPRESSED_OUTPUT (LCT/kernels/generic/pointwise_scalar_dual.py:17-346) and
// re-encodes its components.  As for one compressed operand, the sampler
// computes the result at the sample positions and the encode kernel decodes
// both operands, applies fma(a, alpha, b) (pointwise_scalar_dual.py:226) and
// encodes the result in one pass.

// One compressed operand of the sampler whose value at the sample has to be
// decoded from its stream: the state between issuing its loads and walking.
struct SampleWalk {
    int32_t start;        // first overflow step of the sampled stream, S if none
    int64_t tail_index;   // its tail's first byte
    uint32_t sm;          // side byte at the sample
};

// Stage the sampled stream's W words into this thread's LDS column of
// `words`, read the side byte and the stream's overflow entry.
__device__ __forceinline__ void sample_issue(const OperandA &x, bool active, int64_t row,
                                             int32_t lane, int64_t block, int64_t n_blocks,
                                             int S, int W, uint32_t *words, SampleWalk &w) {
    const int t = threadIdx.x;
    const int64_t n_streams = n_blocks * kLanes;
    const int32_t *column = x.encoded + (active ? block * kLanes + lane : 0);
    for (int r = 0; r < W; ++r)
        __builtin_amdgcn_global_load_lds(
            column + r * n_streams,
            (__attribute__((address_space(3))) void *)(words + r * kSampleGroup), 4, 0, 0);
    words[W * kSampleGroup + t] = 0u;
    w.sm = active ? x.side[row * kLanes + lane] : 0u;
    stream_overlay(x.ov, active && x.has_overlay != 0, block, n_blocks, lane, S, w.start,
                   w.tail_index);
}

// The operand's BF16 bits at the sample (after the staged words and tables
// are visible): the tail byte at or after the stream's overflow start, else
// the decoded prefix's last symbol.
__device__ __forceinline__ uint32_t sample_walk(const OperandA &x, const SampleWalk &w,
                                                bool active, int32_t step, uint32_t *words,
                                                const DecodeTables *tb, int W, int rare) {
    uint32_t field = 0;
    if (step >= w.start) {
        field = tail_field(x.ov.tail[w.tail_index + (step - w.start)]);
    } else if (active) {
        StreamCursorT<kSampleGroup> cursor;
        cursor.init(words + threadIdx.x, tb, static_cast<uint32_t>(W), rare);
        for (int pair = 0; pair < step / 2; ++pair) {
            uint32_t f0, f1;
            cursor.advance(cursor.next_fields(f0, f1));
        }
        uint32_t f0, f1;
        cursor.next_fields(f0, f1);
        field = (step & 1) ? f1 : f0;
    }
    return join_entry(field, w.sm);
}

__global__ __launch_bounds__(kSampleGroup) void dual_sample_kernel(
    OperandA a, const uint16_t *__restrict__ a_samples, OperandA b,
    const uint16_t *__restrict__ b_samples, const float *__restrict__ alpha, int64_t n_blocks,
    int64_t logical_numel, int64_t sample_size, int S, int W, int rare,
    int32_t *__restrict__ partials, uint16_t *__restrict__ result_samples) {
    extern __shared__ uint32_t words[];   // A's then B's: 2 x (W + 1) rows x kSampleGroup
    __shared__ DecodeTables tba, tbb;
    const int t = threadIdx.x;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kSampleGroup + t;
    const bool active = i < sample_size;
    const int shift = __builtin_ctzll(static_cast<uint64_t>(sample_size));
    const int64_t pos = active ? sample_position(i, logical_numel, sample_size, shift) : 0;
    const int64_t row = pos / kLanes;
    const int32_t lane = static_cast<int32_t>((pos % kLanes) ^ (row & 254));
    const int64_t block = row >> (S == 128 ? 7 : 8);   // S is 128 or 256
    const int32_t step = static_cast<int32_t>(row & (S - 1));
    const bool walk_a = a_samples == nullptr, walk_b = b_samples == nullptr;
    uint32_t *words_a = words, *words_b = words + (W + 1) * kSampleGroup;
    SampleWalk wa{}, wb{};
    if (walk_a) {
        int32_t packed[256 / kSampleGroup];
#pragma unroll
        for (int k = 0; k < 256 / kSampleGroup; ++k)
            packed[k] = a.shifted_decode[t + k * kSampleGroup];
        sample_issue(a, active, row, lane, block, n_blocks, S, W, words_a, wa);
        const int32_t center = a.center[0];
#pragma unroll
        for (int k = 0; k < 256 / kSampleGroup; ++k)
            build_decode_entry(tba, t + k * kSampleGroup, packed[k], center);
    }
    if (walk_b) {
        int32_t packed[256 / kSampleGroup];
#pragma unroll
        for (int k = 0; k < 256 / kSampleGroup; ++k)
            packed[k] = b.shifted_decode[t + k * kSampleGroup];
        sample_issue(b, active, row, lane, block, n_blocks, S, W, words_b, wb);
        const int32_t center = b.center[0];
#pragma unroll
        for (int k = 0; k < 256 / kSampleGroup; ++k)
            build_decode_entry(tbb, t + k * kSampleGroup, packed[k], center);
    }
    wait_memory();
    __syncthreads();   // decode tables and staged words
    const uint32_t av = walk_a ? sample_walk(a, wa, active, step, words_a, &tba, W, rare)
                               : (active ? a_samples[i] : 0u);
    const uint32_t bv = walk_b ? sample_walk(b, wb, active, step, words_b, &tbb, W, rare)
                               : (active ? b_samples[i] : 0u);
    const uint32_t result =
        float_to_bf16(__builtin_fmaf(bf16_to_float(av), alpha[0], bf16_to_float(bv)));
    if (active && result_samples != nullptr) result_samples[i] = static_cast<uint16_t>(result);
    const int32_t exp = static_cast<int32_t>((result >> 7) & 255u) - 127;
    const bool keep = active && exp >= -120;
    const int32_t sum = wave_sum(keep ? exp : 0);
    const int32_t kept = wave_sum(keep ? 1 : 0);
    if (t == 0) {
        partials[2 * blockIdx.x] = sum;
        partials[2 * blockIdx.x + 1] = kept;
    }
}

// The two-operand kernel keeps its LDS to about 52 KiB at W = 25, so that
// three workgroups fit per CU and the C4-sized grid (688 codec blocks) runs
// in one round on 256 CUs:
//  * payload rows 0..2 of each stream live in registers (the cursor's initial
//    window) and only rows 3..W-1 are staged; past a stream's last word the
//    cursor re-reads word W-1 instead of a zero pad row (bits beyond a
//    stream's end never reach a decoded value);
//  * side bytes move in 8-step halves: each wave's 1 KiB slice holds A's half
//    (which the result's side bytes then overwrite) and B's half.
constexpr int kHalfSlice = kHalfSteps * kWave;   // one operand's 8-step half, one wave

using u32x2 = __attribute__((ext_vector_type(2))) uint32_t;

// This lane's 8 bytes of a wave's 8-step half: step j >> 3, lanes (j & 7) * 8..
// of the wave's 64 columns, so lane j's bytes land at j * 8 of the half.
__device__ __forceinline__ uint32_t half_side_offset() {
    const uint32_t j = threadIdx.x & (kWave - 1);
    const uint32_t wave = threadIdx.x / kWave;
    return (j >> 3) * kLanes + wave * kWave + (j & 7) * 8;
}

__device__ __forceinline__ u32x2 fetch_half_side(__amdgpu_buffer_rsrc_t side, uint32_t voffset,
                                                 int first_step) {
    return __builtin_amdgcn_raw_buffer_load_b64(side, voffset, first_step * kLanes, 0);
}

__device__ __forceinline__ void store_half_side(uint8_t *half, u32x2 q) {
    reinterpret_cast<u32x2 *>(half)[threadIdx.x & (kWave - 1)] = q;
}

// Halves [c_begin, c_end) (steps, multiples of 8) with one overlay variant for
// both operands (tails read from HBM).  On entry side_a/side_b hold half
// c_begin's side bytes of A and B.
template <bool kFull, Overlay kOverlay, int S>
__device__ __forceinline__ void dual_halves(UpdateCursor &ca, const LaneOverlay &lane_a,
                                            UpdateCursor &cb, const LaneOverlay &lane_b,
                                            uint8_t *slice, u32x2 &side_a, u32x2 &side_b,
                                            __amdgpu_buffer_rsrc_t b_side, StreamWriter &writer,
                                            const uint2 *enc, const UpdateIo &io,
                                            int64_t row_base, uint32_t valid_in_block,
                                            int c_begin, int c_end, float alpha) {
    const uint32_t voffset = half_side_offset();
    uint8_t *half_a = slice;
    uint8_t *half_b = slice + kHalfSlice;
#pragma unroll 1
    for (int c = c_begin; c < c_end; c += kHalfSteps) {
        store_half_side(half_a, side_a);
        store_half_side(half_b, side_b);
        const bool more = c + kHalfSteps < S;
        side_a = fetch_half_side(io.side, more ? voffset : kOutOfRange, c + kHalfSteps);
        side_b = fetch_half_side(b_side, more ? voffset : kOutOfRange, c + kHalfSteps);
        // c is a multiple of 8 and the block's first row one of S, so the
        // swizzle mask of row c + j (j < 8 even) is mask ^ j.
        const uint32_t mask = static_cast<uint32_t>((row_base + c) & 254);
        uint32_t fa[kHalfSteps], fb[kHalfSteps];
        decode_fields<kFull, kOverlay>(ca, lane_a, nullptr, c, row_base, valid_in_block, fa);
        decode_fields<kFull, kOverlay>(cb, lane_b, nullptr, c, row_base, valid_in_block, fb);
#pragma unroll
        for (int j = 0; j < kHalfSteps; j += 2) {
            const int step = c + j;
            const uint32_t off0 = static_cast<uint32_t>(step) * kLanes
                + (threadIdx.x ^ mask ^ static_cast<uint32_t>(j));
            const bool v0 = kFull || off0 < valid_in_block;
            const bool v1 = kFull || off0 + kLanes < valid_in_block;
            const float a0 = __uint_as_float(join_float(fa[j], side_byte(half_a, j)));
            const float a1 = __uint_as_float(join_float(fa[j + 1], side_byte(half_a, j + 1)));
            const float b0 = __uint_as_float(join_float(fb[j], side_byte(half_b, j)));
            const float b1 = __uint_as_float(join_float(fb[j + 1], side_byte(half_b, j + 1)));
            // Padding positions hold 0 (side byte 0, no code).
            const uint32_t h0 = v0 ? round_bf16_high(__builtin_fmaf(a0, alpha, b0)) : 0u;
            const uint32_t h1 = v1 ? round_bf16_high(__builtin_fmaf(a1, alpha, b1)) : 0u;
            emit_pair(writer, enc, half_a, j, h0, h1, v0, v1, off0, io);
        }
        // A's half now holds the result's side bytes.
        const u32x2 q = reinterpret_cast<const u32x2 *>(half_a)[threadIdx.x & (kWave - 1)];
        __builtin_amdgcn_raw_buffer_store_b64(q, io.side_out, voffset, c * kLanes, kSideStore);
    }
}

// ---- the pipelined full-block path of the two-operand kernel: as for one
// operand, the arithmetic and encoding of one 8-step half are interleaved pair
// by pair with decoding the next half, here of both operands (two independent
// lookup chains), and chunks that cannot overflow use the lean writer.

struct DualEmit {
    uint32_t sa0, sa1, sb0, sb1;   // A's and B's side bytes
    uint32_t r;                    // the results' BF16 bits (step s0 low, s0 + 1 high)
    uint2 e0, e1;                  // their encode entries
};

__device__ __forceinline__ void dual_emit_operands(DualEmit &st, const uint8_t *half_a,
                                                   const uint8_t *half_b, int j) {
    st.sa0 = side_byte(half_a, j);
    st.sa1 = side_byte(half_a, j + 1);
    st.sb0 = side_byte(half_b, j);
    st.sb1 = side_byte(half_b, j + 1);
}

// fma(a, alpha, b) (pointwise_scalar_dual.py:226) rounded to BF16, the result's
// side bytes over A's in the half slice and the encode-table reads.
__device__ __forceinline__ void dual_emit_result(DualEmit &st, const uint2 *enc, uint8_t *half_a,
                                                 int j, uint32_t fa0, uint32_t fa1, uint32_t fb0,
                                                 uint32_t fb1, float alpha) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const float a0 = __uint_as_float(join_float(fa0, st.sa0));
    const float a1 = __uint_as_float(join_float(fa1, st.sa1));
    const float b0 = __uint_as_float(join_float(fb0, st.sb0));
    const float b1 = __uint_as_float(join_float(fb1, st.sb1));
    const uint32_t r = round_pair_bf16(__builtin_fmaf(a0, alpha, b0), __builtin_fmaf(a1, alpha, b1));
    const uint32_t sign_down = r >> 8;
    uint32_t side0, side1;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(side0) : "s"(0x7Fu), "v"(r), "v"(sign_down));
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(side1) : "s"(0x007F0000u), "v"(r), "v"(sign_down));
    half_a[j * kWave + lane] = static_cast<uint8_t>(side0);
    half_a[(j + 1) * kWave + lane] = static_cast<uint8_t>(side1 >> 16);
    const uint32_t x = exponent_bytes(r);
    st.e0 = enc[x & 255u];
    st.e1 = enc[(x >> 16) & 255u];
    st.r = r;
}

// One operand's staged lookups for the pair at `step` (kOverlay: tails from HBM).
template <Overlay kOverlay>
__device__ __forceinline__ void finish_pair(UpdateCursor &cursor, const LaneOverlay &lane,
                                            int step, uint32_t bits, uint32_t &t0,
                                            uint32_t &t1) {
    uint32_t sum = cursor.resolve(bits, t0, t1);
    if (kOverlay != kNoOverlay) {
        overlay_pair<false, FloatDecodeTables>(lane, nullptr, step, t0, t1);
        sum = (t0 + t1) & 127u;
    }
    cursor.advance(sum);
}

// The half at c: emit from fa/fb while decoding the half at c + 8 into them
// (kDecode).  Within a pair, each lookup's latency is filled with emit work
// that does not depend on it: the first lookups with the operation on the
// pair being emitted, the second lookups with its codes.  The side bytes of
// the next pair are read a pair ahead.
template <Overlay kOverlay, bool kFast, bool kDecode>
__device__ __forceinline__ void dual_pipelined_half(UpdateCursor &ca, const LaneOverlay &lane_a,
                                                    UpdateCursor &cb, const LaneOverlay &lane_b,
                                                    uint8_t *half_a, const uint8_t *half_b,
                                                    StreamWriter &writer, const uint2 *enc,
                                                    const UpdateIo &io, int c, uint32_t mask,
                                                    float alpha, uint32_t (&fa)[kHalfSteps],
                                                    uint32_t (&fb)[kHalfSteps]) {
    uint32_t ga[kHalfSteps], gb[kHalfSteps];
    DualEmit st;
    dual_emit_operands(st, half_a, half_b, 0);
#pragma unroll
    for (int j = 0; j < kHalfSteps; j += 2) {
        const uint32_t off0 = static_cast<uint32_t>(c + j) * kLanes
            + (threadIdx.x ^ mask ^ static_cast<uint32_t>(j));
        uint32_t bits_a = 0, ta0 = 0, ta1 = 0, bits_b = 0, tb0 = 0, tb1 = 0;
        if (kDecode) {
            ca.first_lookup(bits_a, ta0);
            cb.first_lookup(bits_b, tb0);
        }
        __builtin_amdgcn_sched_barrier(0);
        dual_emit_result(st, enc, half_a, j, fa[j], fa[j + 1], fb[j], fb[j + 1], alpha);
        DualEmit next = st;
        if (j + 2 < kHalfSteps) dual_emit_operands(next, half_a, half_b, j + 2);
        __builtin_amdgcn_sched_barrier(0);
        if (kDecode) {
            ta1 = ca.second_lookup(bits_a, ta0);
            tb1 = cb.second_lookup(bits_b, tb0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kFast) {
            writer.put_fast(st.e0, st.e1);
        } else {
            const bool over = writer.put(st.e0, st.e1);
            const uint32_t exp_off = over ? off0 : kOutOfRange;
            __builtin_amdgcn_raw_buffer_store_b8(st.r >> 7, io.exponents, exp_off, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b8(st.r >> 23, io.exponents, exp_off + kLanes, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kDecode) {
            finish_pair<kOverlay>(ca, lane_a, c + kHalfSteps + j, bits_a, ta0, ta1);
            finish_pair<kOverlay>(cb, lane_b, c + kHalfSteps + j, bits_b, tb0, tb1);
            ga[j] = ta0;
            ga[j + 1] = ta1;
            gb[j] = tb0;
            gb[j + 1] = tb1;
        }
        __builtin_amdgcn_sched_barrier(0);
        st = next;
    }
    if (kDecode) {
#pragma unroll
        for (int k = 0; k < kHalfSteps; ++k) {
            fa[k] = ga[k];
            fb[k] = gb[k];
        }
    }
    if (kFast) writer.fits += kHalfSteps / 2;
}

// A's and B's side bytes of the next kDualDepth halves: fetched that many
// halves ahead (one half of work is far shorter than HBM's latency under
// load), in copies that rotate, so no register copy of an in-flight load
// (which would wait for it) is made.  Copy 0 holds the half being started.
constexpr int kDualDepth = 2;

struct DualPrefetch {
    u32x2 a[kDualDepth], b[kDualDepth];

    // After k halves: copy k becomes copy 0 (waits for those loads; once per
    // overlay segment at most).
    __device__ __forceinline__ void rotate(int k) {
        u32x2 ta[kDualDepth], tb[kDualDepth];
#pragma unroll
        for (int i = 0; i < kDualDepth; ++i) {
            ta[i] = a[(i + k) % kDualDepth];
            tb[i] = b[(i + k) % kDualDepth];
        }
#pragma unroll
        for (int i = 0; i < kDualDepth; ++i) {
            a[i] = ta[i];
            b[i] = tb[i];
        }
    }
};

// The half at c using the side bytes in (side_a, side_b) -- the copy holding
// half c -- and refilling them with half c + 8 * kDualDepth.
template <Overlay kOverlay, int S>
__device__ __forceinline__ void dual_half_step(
    UpdateCursor &ca, const LaneOverlay &lane_a, UpdateCursor &cb, const LaneOverlay &lane_b,
    uint8_t *slice, u32x2 &side_a, u32x2 &side_b, __amdgpu_buffer_rsrc_t b_side,
    StreamWriter &writer, const uint2 *enc, const UpdateIo &io, int64_t row_base, int c,
    int c_end, float alpha, uint32_t (&fa)[kHalfSteps], uint32_t (&fb)[kHalfSteps]) {
    const uint32_t voffset = half_side_offset();
    uint8_t *half_a = slice;
    uint8_t *half_b = slice + kHalfSlice;
    store_half_side(half_a, side_a);
    store_half_side(half_b, side_b);
    const int ahead = c + kDualDepth * kHalfSteps;
    const bool more = ahead < S;
    side_a = fetch_half_side(io.side, more ? voffset : kOutOfRange, ahead);
    side_b = fetch_half_side(b_side, more ? voffset : kOutOfRange, ahead);
    const uint32_t mask = static_cast<uint32_t>((row_base + c) & 254);
    const bool fast = writer.fits_chunk(kHalfSteps);
    const bool next = c + kHalfSteps < c_end;
#define LCT_HALF(FAST, NEXT)                                                                   \
    dual_pipelined_half<kOverlay, FAST, NEXT>(ca, lane_a, cb, lane_b, half_a, half_b, writer, \
                                              enc, io, c, mask, alpha, fa, fb)
    if (fast) {
        if (next) LCT_HALF(true, true);
        else LCT_HALF(true, false);
    } else {
        if (next) LCT_HALF(false, true);
        else LCT_HALF(false, false);
    }
#undef LCT_HALF
    // A's half now holds the result's side bytes.
    const u32x2 q = reinterpret_cast<const u32x2 *>(half_a)[threadIdx.x & (kWave - 1)];
    __builtin_amdgcn_raw_buffer_store_b64(q, io.side_out, voffset, c * kLanes, kSideStore);
}

// Halves [c_begin, c_end) of a full block with one overlay variant of both
// operands (tails from HBM); as dual_halves<true, ...>.  On entry pf's copy i
// holds half c_begin + 8i; on exit the same holds for c_end.
template <Overlay kOverlay, int S>
__device__ __forceinline__ void dual_halves_pipelined(
    UpdateCursor &ca, const LaneOverlay &lane_a, UpdateCursor &cb, const LaneOverlay &lane_b,
    uint8_t *slice, DualPrefetch &pf, __amdgpu_buffer_rsrc_t b_side, StreamWriter &writer,
    const uint2 *enc, const UpdateIo &io, int64_t row_base, int c_begin, int c_end,
    float alpha) {
    if (c_begin >= c_end) return;
    uint32_t fa[kHalfSteps], fb[kHalfSteps];
    decode_fields<true, kOverlay>(ca, lane_a, nullptr, c_begin, row_base, 0u, fa);
    decode_fields<true, kOverlay>(cb, lane_b, nullptr, c_begin, row_base, 0u, fb);
    int c = c_begin;
#pragma unroll 1
    for (; c + (kDualDepth - 1) * kHalfSteps < c_end; c += kDualDepth * kHalfSteps) {
#pragma unroll
        for (int k = 0; k < kDualDepth; ++k)
            dual_half_step<kOverlay, S>(ca, lane_a, cb, lane_b, slice, pf.a[k], pf.b[k], b_side,
                                        writer, enc, io, row_base, c + k * kHalfSteps, c_end,
                                        alpha, fa, fb);
    }
    // Fewer than kDualDepth halves left.
    const int left = (c_end - c) / kHalfSteps;
#pragma unroll
    for (int k = 0; k < kDualDepth - 1; ++k)
        if (k < left)
            dual_half_step<kOverlay, S>(ca, lane_a, cb, lane_b, slice, pf.a[k], pf.b[k], b_side,
                                        writer, enc, io, row_base, c + k * kHalfSteps, c_end,
                                        alpha, fa, fb);
    if (left == 1) pf.rotate(1);
    else if (left == 2) pf.rotate(2);
    else if (left == 3) pf.rotate(3);
}

template <bool kFull, int S>
__device__ __forceinline__ void dual_rows(UpdateCursor ca, const LaneOverlay &lane_a,
                                          UpdateCursor cb, const LaneOverlay &lane_b,
                                          uint8_t *slice, u32x2 side_a, u32x2 side_b,
                                          __amdgpu_buffer_rsrc_t b_side, StreamWriter &writer,
                                          const uint2 *enc, const UpdateIo &io,
                                          int64_t row_base, uint32_t valid_in_block, float alpha) {
    const int split = min(S, min(lane_a.wave_start, lane_b.wave_start) & ~(kHalfSteps - 1));
    if (kFull) {
        DualPrefetch pf;
        pf.a[0] = side_a;
        pf.b[0] = side_b;
#pragma unroll
        for (int k = 1; k < kDualDepth; ++k) {
            pf.a[k] = fetch_half_side(io.side, half_side_offset(), k * kHalfSteps);
            pf.b[k] = fetch_half_side(b_side, half_side_offset(), k * kHalfSteps);
        }
        dual_halves_pipelined<kNoOverlay, S>(ca, lane_a, cb, lane_b, slice, pf, b_side, writer,
                                             enc, io, row_base, 0, split, alpha);
        dual_halves_pipelined<kHbmOverlay, S>(ca, lane_a, cb, lane_b, slice, pf, b_side, writer,
                                              enc, io, row_base, split, S, alpha);
        return;
    }
    dual_halves<kFull, kNoOverlay, S>(ca, lane_a, cb, lane_b, slice, side_a, side_b, b_side,
                                      writer, enc, io, row_base, valid_in_block, 0, split, alpha);
    if (split < S)
        dual_halves<kFull, kHbmOverlay, S>(ca, lane_a, cb, lane_b, slice, side_a, side_b, b_side,
                                           writer, enc, io, row_base, valid_in_block, split, S,
                                           alpha);
}

template <bool kBooked>
__global__ __launch_bounds__(kLanes) void dual_encode_kernel(
    OperandA a, OperandA b, const float *__restrict__ alpha,
    const int32_t *__restrict__ partials, int32_t n_groups,
    const int32_t *__restrict__ base_encode, const int32_t *__restrict__ base_decode,
    int32_t *__restrict__ center_out, int32_t *__restrict__ shifted_decode_out,
    uint8_t *__restrict__ side_out, int32_t *__restrict__ encoded_out,
    uint8_t *__restrict__ extra_starts, int32_t *__restrict__ summaries,
    uint8_t *__restrict__ exponents, int64_t n_blocks, int64_t logical_numel, int S, int W,
    int rare, KernelBookkeeping bk) {
    extern __shared__ uint32_t stages[];   // A's rows 3..W-1, then B's
    __shared__ FloatDecodeTables tba, tbb;
    __shared__ uint2 enc[256];
    __shared__ int32_t scratch[kWavesPerBlock];
    __shared__ int32_t shared_center[2];   // center, and whether its samples failed to arrive
    // The overflow maps (2 KiB) and the raw encode table (1 KiB) are only used
    // before the first side halves are stored, so they share the slices.
    __shared__ __attribute__((aligned(16))) uint8_t slices[kWavesPerBlock][2 * kHalfSlice];
    int32_t *map_start = reinterpret_cast<int32_t *>(&slices[0][0]);
    int32_t *map_offset = map_start + kLanes;
    int32_t *raw_encode = map_offset + kLanes;
    uint32_t *stage_a = stages;
    uint32_t *stage_b = stages + register_stage_bytes(W) / 4;
    const int t = threadIdx.x;
    const int64_t block = blockIdx.x;
    const bool sampled_here = kBooked && bk.sample_groups > 0;
    if (sampled_here && block < bk.sample_groups && t < kWave) {
        // fma(a, alpha, b) (pointwise_scalar_dual.py:226) at sample group
        // `block`'s positions from both operands' recorded values.
        const int64_t i = block * kSampleGroup + t;
        const bool active = i < bk.sample_size;
        uint32_t result = 0;
        if (active) {
            result = float_to_bf16(__builtin_fmaf(bf16_to_float(bk.a_samples[i]), alpha[0],
                                                  bf16_to_float(bk.b_samples[i])));
            if (bk.result_samples != nullptr)
                bk.result_samples[i] = static_cast<uint16_t>(result);
        }
        const int32_t exp = static_cast<int32_t>((result >> 7) & 255u) - 127;
        const bool keep = active && exp >= -120;
        const int32_t sum = wave_sum(keep ? exp : 0);
        const int32_t kept = wave_sum(keep ? 1 : 0);
        publish_sample_group(bk, block, sum, kept);
    }
    if (block >= n_blocks) return;   // a sample group past the last block
    const int64_t n_streams = n_blocks * kLanes;
    const int64_t row_base = block * S;
    const int64_t logical_base = row_base * kLanes;
    const uint32_t block_elems = static_cast<uint32_t>(S) * kLanes;
    const int64_t remaining = logical_numel - logical_base;
    const uint32_t valid = remaining < block_elems ? static_cast<uint32_t>(remaining) : block_elems;
    UpdateIo io;
    io.side = make_rsrc(a.side + logical_base, block_elems);
    io.other = make_rsrc(nullptr, 0u);
    io.side_out = make_rsrc(side_out + logical_base, block_elems);
    io.exponents = make_rsrc(exponents + logical_base, valid);
    const __amdgpu_buffer_rsrc_t b_side = make_rsrc(b.side + logical_base, block_elems);
    const u32x2 first_a = fetch_half_side(io.side, half_side_offset(), 0);
    const u32x2 first_b = fetch_half_side(b_side, half_side_offset(), 0);
    // Loads the prologue needs later, issued now so that they share one round
    // trip with the tables' loads instead of following its barriers.
    const OverlayHead head_a = load_overlay_head(a.ov, a.has_overlay != 0, block, n_blocks);
    const OverlayHead head_b = load_overlay_head(b.ov, b.has_overlay != 0, block, n_blocks);
    const BaseDecodeShare base0 = load_base_decode(base_decode, block == 0);
    const float alpha_value = alpha[0];
    // Each stream's first three words: the cursors' initial windows.
    uint32_t wa[kRegisterRows], wb[kRegisterRows];
    load_register_rows(a.encoded, n_streams, block, wa);
    load_register_rows(b.encoded, n_streams, block, wb);

    raw_encode[t] = base_encode[t];
    if (sampled_here) {
        center_from_control(bk.control, bk.sample_groups, bk.epoch, bk.polls, shared_center);
    } else {
        center_from_partials(partials, n_groups, shared_center);
        if (t == 0) shared_center[1] = 0;
    }
    build_float_decode_tables(tba, a.shifted_decode);
    build_float_decode_tables(tbb, b.shifted_decode);
    const int32_t a_center = a.center[0], b_center = b.center[0];
    stage_payload_rows(stage_a, a.encoded, n_streams, block, kRegisterRows, W);
    stage_payload_rows(stage_b, b.encoded, n_streams, block, kRegisterRows, W);
    __syncthreads();   // center and raw encode table
    const int32_t center = shared_center[0];
    const bool center_failed = shared_center[1] != 0;
    enc[t] = repack_encode_entry(static_cast<uint32_t>(raw_encode[byte_to_index(t, center)]));
    if (block == 0) {
        if (t == 0) center_out[0] = center;
        store_shifted_decode(shifted_decode_out, base0, center);
    }
    __syncthreads();   // raw_encode is no longer read (it shares the maps' LDS)
    const LaneOverlay lane_a = build_overlay(a.ov, head_a, S, map_start, map_offset, scratch,
                                             nullptr, 0);
    __syncthreads();   // B's overlay reuses the maps
    const LaneOverlay lane_b = build_overlay(b.ov, head_b, S, map_start, map_offset, scratch,
                                             nullptr, 0);
    wait_memory();
    __syncthreads();   // payloads and encode table visible; maps no longer read

    UpdateCursor ca, cb;
    ca.init_registers(stage_a + t, &tba, static_cast<uint32_t>(W), rare, wa[0], wa[1], wa[2],
                      a_center);
    cb.init_registers(stage_b + t, &tbb, static_cast<uint32_t>(W), rare, wb[0], wb[1], wb[2],
                      b_center);
    const uint32_t row_bytes = static_cast<uint32_t>(n_streams * 4);
    StreamWriter writer{make_rsrc(encoded_out + block * kLanes,
                                  static_cast<uint32_t>(W - 1) * row_bytes + kLanes * 4),
                        row_bytes, static_cast<uint32_t>(t) * 4u,
                        static_cast<uint32_t>(W) * row_bytes + static_cast<uint32_t>(t) * 4u,
                        static_cast<uint32_t>(W) * 32u, 0u, 0u, 0u};
    writer.keep_row_bytes_in_vgpr();
    uint8_t *slice = slices[t / kWave];
    const bool full = valid == block_elems;
#define LCT_DUAL_ROWS(FULL, SS)                                                                \
    dual_rows<FULL, SS>(ca, lane_a, cb, lane_b, slice, first_a, first_b, b_side, writer, enc,  \
                        io, row_base, valid, alpha_value)
    if (S == 128) {
        if (full) LCT_DUAL_ROWS(true, 128);
        else LCT_DUAL_ROWS(false, 128);
    } else {
        if (full) LCT_DUAL_ROWS(true, 256);
        else LCT_DUAL_ROWS(false, 256);
    }
#undef LCT_DUAL_ROWS
    writer.finish();
    const bool overflow = writer.overflowed();
    const int32_t extra = writer.extra_start();
    extra_starts[block * kLanes + t] = static_cast<uint8_t>(overflow ? extra : 255);
    // Streams from bit 20 (at most 256), tail bytes in bits 0..19 (at most
    // 256 x 256): one block scan.
    const int32_t both = block_sum(overflow ? (S - extra) | (1 << 20) : 0, scratch);
    publish_block<kBooked>(bk, summaries, block, n_blocks, both >> 20, both & 0xFFFFF,
                           reinterpret_cast<int32_t *>(stages), center_failed);
}

int32_t check_operand(const int32_t *encoded, const uint8_t *side, const int32_t *shifted_decode,
                      const int32_t *center, const lct_overflow *overflow) {
    if (!encoded || !side || !shifted_decode || !center) return LCT_E_NULL;
    if (overflow != nullptr) {
        if (!overflow->lanes || !overflow->starts || !overflow->tail || !overflow->blocks)
            return LCT_E_NULL;
        if (overflow->descriptor != nullptr && overflow->count == nullptr) return LCT_E_NULL;
    }
    return LCT_OK;
}

int32_t check_op(int32_t op, int32_t alpha_is_one, int32_t beta_is_one, const float *alpha,
                 const float *beta) {
    if (op < LCT_OP_ADD || op > LCT_OP_SCALAR_MUL_ADD) return LCT_E_ARG;
    if (op == LCT_OP_SCALAR_MUL_ADD && ((!alpha_is_one && !alpha) || (!beta_is_one && !beta)))
        return LCT_E_NULL;
    return LCT_OK;
}

int32_t check_shape(int64_t size, int64_t logical_numel, const lct_geometry &g,
                    int32_t rare_length) {
    if (!geometry_ok(g)) return LCT_E_GEOMETRY;
    if (logical_numel <= 0 || size <= 0 || size % g.block_symbols != 0 || logical_numel > size
        || logical_numel <= size - g.block_symbols || size / g.block_symbols > kMaxBlocks)
        return LCT_E_SIZE;
    if (rare_length < 0 || rare_length > 8) return LCT_E_ARG;
    return LCT_OK;
}

int32_t check_samples(int64_t sample_size, int64_t logical_numel) {
    if (sample_size <= 0 || sample_size > kMaxSamples || sample_size > logical_numel)
        return LCT_E_SIZE;
    if (sample_size != logical_numel && (sample_size & (sample_size - 1)) != 0) return LCT_E_ARG;
    return LCT_OK;
}

}  // namespace
}  // namespace lct

using namespace lct;

extern "C" int32_t lct_pointwise_sample(const int32_t *encoded, const uint8_t *side,
                                        const int32_t *shifted_decode, const int32_t *center,
                                        const lct_overflow *overflow, const void *a_samples,
                                        const void *other, const float *alpha,
                                        const float *beta, int64_t size,
                                        int64_t logical_numel, lct_geometry g,
                                        int32_t rare_length, int32_t op, int32_t alpha_is_one,
                                        int32_t beta_is_one, int64_t sample_size,
                                        int32_t *partials, void *result_samples,
                                        hipStream_t stream) {
    if (int32_t e = check_operand(encoded, side, shifted_decode, center, overflow)) return e;
    if (!other || !partials) return LCT_E_NULL;
    if (int32_t e = check_op(op, alpha_is_one, beta_is_one, alpha, beta)) return e;
    if (int32_t e = check_shape(size, logical_numel, g, rare_length)) return e;
    if (int32_t e = check_samples(sample_size, logical_numel)) return e;
    const OperandA a{encoded, side, shifted_decode, center,
                     overflow ? *overflow : lct_overflow{}, overflow != nullptr};
    const OpArgs args{alpha, beta, op, alpha_is_one, beta_is_one};
    const int64_t n_blocks = size / g.block_symbols;
    const size_t lds = static_cast<size_t>(g.fixed_words + 1) * kSampleGroup * sizeof(uint32_t);
    hipLaunchKernelGGL(pointwise_sample_kernel, dim3(sample_groups(sample_size)),
                       dim3(kSampleGroup), lds, stream, a,
                       static_cast<const uint16_t *>(a_samples),
                       static_cast<const uint16_t *>(other), args, n_blocks, logical_numel,
                       sample_size, g.steps, g.fixed_words, rare_length, partials,
                       static_cast<uint16_t *>(result_samples));
    return static_cast<int32_t>(hipGetLastError());
}

namespace {

// The host side of lct_bookkeeping: validated against the launch's block
// count, in the kernel's form (bk.control == nullptr without one).  Also
// raises `lds` to the free list's LDS copy when buffered.
int32_t prepare_bookkeeping(const lct_bookkeeping *in, int64_t n_blocks, KernelBookkeeping &bk,
                            size_t &lds) {
    bk = KernelBookkeeping{};
    if (in == nullptr) return LCT_OK;
    if (!in->control || !in->counts || !in->blocks) return LCT_E_NULL;
    if (n_blocks > kMaxBlocks) return LCT_E_SIZE;
    if (in->control_words < kControlPartials + n_blocks) return LCT_E_SIZE;
    // Epoch 0 would match a control array's initial zeros.
    if (in->epoch == 0) return LCT_E_ARG;
    if ((reinterpret_cast<uintptr_t>(in->control) & 7) != 0) return LCT_E_ARG;
    if (in->buffer_meta != nullptr) {
        if (!in->descriptor) return LCT_E_NULL;
        if (in->max_free_regions <= 0 || in->max_free_regions > 4096
            || (in->max_free_regions & (in->max_free_regions - 1)) != 0)
            return LCT_E_ARG;
        if (in->frees.count < 0 || in->frees.count > LCT_MAX_PENDING_FREES) return LCT_E_ARG;
        for (int i = 0; i < in->frees.count; ++i)
            if (in->frees.descriptor[i] == nullptr) return LCT_E_NULL;
        const size_t list = static_cast<size_t>(in->max_free_regions) * 8;
        if (list > lds) lds = list;
    }
    bk.control = in->control;
    bk.epoch = in->epoch;
    bk.counts = in->counts;
    bk.blocks = in->blocks;
    bk.descriptor = in->buffer_meta != nullptr ? in->descriptor : nullptr;
    bk.buffer_meta = in->buffer_meta;
    bk.max_free_regions = in->max_free_regions;
    if (in->buffer_meta != nullptr) bk.frees = in->frees;
    bk.lock_spins = lock_spins();
    bk.polls = ready_polls();
    return LCT_OK;
}

int32_t launch_pointwise_encode(
    const int32_t *encoded, const uint8_t *side, const int32_t *shifted_decode,
    const int32_t *center, const lct_overflow *overflow, const void *other, const float *alpha,
    const float *beta, const int32_t *partials, int64_t sample_size, const int32_t *base_encode,
    const int32_t *base_decode, int32_t *center_out, int32_t *shifted_decode_out,
    uint8_t *side_out, int32_t *encoded_out, uint8_t *extra_starts, int32_t *summaries,
    uint8_t *exponents, int64_t size, int64_t logical_numel, lct_geometry g, int32_t rare_length,
    int32_t op, int32_t alpha_is_one, int32_t beta_is_one, const lct_bookkeeping *bookkeeping,
    hipStream_t stream) {
    if (int32_t e = check_operand(encoded, side, shifted_decode, center, overflow)) return e;
    if (!other || !partials || !base_encode || !base_decode || !center_out || !shifted_decode_out
        || !side_out || !encoded_out || !extra_starts || !summaries || !exponents)
        return LCT_E_NULL;
    if (int32_t e = check_op(op, alpha_is_one, beta_is_one, alpha, beta)) return e;
    if (int32_t e = check_shape(size, logical_numel, g, rare_length)) return e;
    if (int32_t e = check_samples(sample_size, logical_numel)) return e;
    // 16-byte accesses: A's payload staging, A's and the result's side bytes.
    if (((reinterpret_cast<uintptr_t>(encoded) | reinterpret_cast<uintptr_t>(side)
          | reinterpret_cast<uintptr_t>(side_out)) & 15) != 0)
        return LCT_E_ARG;
    const int64_t n_blocks = size / g.block_symbols;
    // The result's payload words are addressed with 32-bit buffer offsets.
    if (static_cast<int64_t>(g.fixed_words) * n_blocks * kLanes * 4 >= (int64_t{1} << 31))
        return LCT_E_SIZE;
    const OperandA a{encoded, side, shifted_decode, center,
                     overflow ? *overflow : lct_overflow{}, overflow != nullptr};
    const OpArgs args{alpha, beta, op, alpha_is_one, beta_is_one};
    const int32_t groups = sample_groups(sample_size);
    size_t lds = static_cast<size_t>(window_stage_bytes(g.fixed_words));
    KernelBookkeeping bk;
    if (int32_t e = prepare_bookkeeping(bookkeeping, n_blocks, bk, lds)) return e;
    const auto kernel = bk.control != nullptr ? pointwise_encode_kernel<true>
                                              : pointwise_encode_kernel<false>;
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(n_blocks)),
                       dim3(kLanes), lds, stream, a, static_cast<const uint16_t *>(other), args,
                       partials, groups, base_encode, base_decode, center_out,
                       shifted_decode_out, side_out, encoded_out, extra_starts, summaries,
                       exponents, n_blocks, logical_numel, g.steps, g.fixed_words, rare_length,
                       bk);
    return static_cast<int32_t>(hipGetLastError());
}

}  // namespace

extern "C" int32_t lct_pointwise_encode(
    const int32_t *encoded, const uint8_t *side, const int32_t *shifted_decode,
    const int32_t *center, const lct_overflow *overflow, const void *other, const float *alpha,
    const float *beta, const int32_t *partials, int64_t sample_size, const int32_t *base_encode,
    const int32_t *base_decode, int32_t *center_out, int32_t *shifted_decode_out,
    uint8_t *side_out, int32_t *encoded_out, uint8_t *extra_starts, int32_t *summaries,
    uint8_t *exponents, int64_t size, int64_t logical_numel, lct_geometry g, int32_t rare_length,
    int32_t op, int32_t alpha_is_one, int32_t beta_is_one, hipStream_t stream) {
    return launch_pointwise_encode(encoded, side, shifted_decode, center, overflow, other, alpha,
                                   beta, partials, sample_size, base_encode, base_decode,
                                   center_out, shifted_decode_out, side_out, encoded_out,
                                   extra_starts, summaries, exponents, size, logical_numel, g,
                                   rare_length, op, alpha_is_one, beta_is_one, nullptr, stream);
}

extern "C" int32_t lct_pointwise_encode_fused(
    const int32_t *encoded, const uint8_t *side, const int32_t *shifted_decode,
    const int32_t *center, const lct_overflow *overflow, const void *other, const float *alpha,
    const float *beta, const int32_t *partials, int64_t sample_size, const int32_t *base_encode,
    const int32_t *base_decode, int32_t *center_out, int32_t *shifted_decode_out,
    uint8_t *side_out, int32_t *encoded_out, uint8_t *extra_starts, int32_t *summaries,
    uint8_t *exponents, int64_t size, int64_t logical_numel, lct_geometry g, int32_t rare_length,
    int32_t op, int32_t alpha_is_one, int32_t beta_is_one, const lct_bookkeeping *bookkeeping,
    hipStream_t stream) {
    if (!bookkeeping) return LCT_E_NULL;
    return launch_pointwise_encode(encoded, side, shifted_decode, center, overflow, other, alpha,
                                   beta, partials, sample_size, base_encode, base_decode,
                                   center_out, shifted_decode_out, side_out, encoded_out,
                                   extra_starts, summaries, exponents, size, logical_numel, g,
                                   rare_length, op, alpha_is_one, beta_is_one, bookkeeping,
                                   stream);
}

extern "C" int32_t lct_dual_sample(const int32_t *a_encoded, const uint8_t *a_side,
                                   const int32_t *a_shifted_decode, const int32_t *a_center,
                                   const lct_overflow *a_overflow, const void *a_samples,
                                   const int32_t *b_encoded, const uint8_t *b_side,
                                   const int32_t *b_shifted_decode, const int32_t *b_center,
                                   const lct_overflow *b_overflow, const void *b_samples,
                                   const float *alpha, int64_t size, int64_t logical_numel,
                                   lct_geometry g, int32_t rare_length, int64_t sample_size,
                                   int32_t *partials, void *result_samples,
                                   hipStream_t stream) {
    if (int32_t e = check_operand(a_encoded, a_side, a_shifted_decode, a_center, a_overflow))
        return e;
    if (int32_t e = check_operand(b_encoded, b_side, b_shifted_decode, b_center, b_overflow))
        return e;
    if (!alpha || !partials) return LCT_E_NULL;
    if (int32_t e = check_shape(size, logical_numel, g, rare_length)) return e;
    if (int32_t e = check_samples(sample_size, logical_numel)) return e;
    const OperandA a{a_encoded, a_side, a_shifted_decode, a_center,
                     a_overflow ? *a_overflow : lct_overflow{}, a_overflow != nullptr};
    const OperandA b{b_encoded, b_side, b_shifted_decode, b_center,
                     b_overflow ? *b_overflow : lct_overflow{}, b_overflow != nullptr};
    const int64_t n_blocks = size / g.block_symbols;
    const size_t lds = 2 * static_cast<size_t>(g.fixed_words + 1) * kSampleGroup * sizeof(uint32_t);
    hipLaunchKernelGGL(dual_sample_kernel, dim3(sample_groups(sample_size)), dim3(kSampleGroup),
                       lds, stream, a, static_cast<const uint16_t *>(a_samples), b,
                       static_cast<const uint16_t *>(b_samples), alpha, n_blocks, logical_numel,
                       sample_size, g.steps, g.fixed_words, rare_length, partials,
                       static_cast<uint16_t *>(result_samples));
    return static_cast<int32_t>(hipGetLastError());
}

namespace {

int32_t launch_dual_encode(
    const int32_t *a_encoded, const uint8_t *a_side, const int32_t *a_shifted_decode,
    const int32_t *a_center, const lct_overflow *a_overflow, const int32_t *b_encoded,
    const uint8_t *b_side, const int32_t *b_shifted_decode, const int32_t *b_center,
    const lct_overflow *b_overflow, const float *alpha, const int32_t *partials,
    int64_t sample_size, const int32_t *base_encode, const int32_t *base_decode,
    int32_t *center_out, int32_t *shifted_decode_out, uint8_t *side_out, int32_t *encoded_out,
    uint8_t *extra_starts, int32_t *summaries, uint8_t *exponents, int64_t size,
    int64_t logical_numel, lct_geometry g, int32_t rare_length,
    const lct_bookkeeping *bookkeeping, hipStream_t stream) {
    if (int32_t e = check_operand(a_encoded, a_side, a_shifted_decode, a_center, a_overflow))
        return e;
    if (int32_t e = check_operand(b_encoded, b_side, b_shifted_decode, b_center, b_overflow))
        return e;
    // With both operands' recorded sample values the launch samples the center.
    const bool sample_here = bookkeeping != nullptr && bookkeeping->a_samples != nullptr
        && bookkeeping->b_samples != nullptr;
    if (!alpha || (!partials && !sample_here) || !base_encode || !base_decode || !center_out
        || !shifted_decode_out || !side_out || !encoded_out || !extra_starts || !summaries
        || !exponents)
        return LCT_E_NULL;
    if (int32_t e = check_shape(size, logical_numel, g, rare_length)) return e;
    if (int32_t e = check_samples(sample_size, logical_numel)) return e;
    // 16-byte accesses: payload staging, A's, B's and the result's side bytes.
    if (((reinterpret_cast<uintptr_t>(a_encoded) | reinterpret_cast<uintptr_t>(b_encoded)
          | reinterpret_cast<uintptr_t>(a_side) | reinterpret_cast<uintptr_t>(b_side)
          | reinterpret_cast<uintptr_t>(side_out)) & 15) != 0)
        return LCT_E_ARG;
    const int64_t n_blocks = size / g.block_symbols;
    // The result's payload words are addressed with 32-bit buffer offsets.
    if (static_cast<int64_t>(g.fixed_words) * n_blocks * kLanes * 4 >= (int64_t{1} << 31))
        return LCT_E_SIZE;
    const OperandA a{a_encoded, a_side, a_shifted_decode, a_center,
                     a_overflow ? *a_overflow : lct_overflow{}, a_overflow != nullptr};
    const OperandA b{b_encoded, b_side, b_shifted_decode, b_center,
                     b_overflow ? *b_overflow : lct_overflow{}, b_overflow != nullptr};
    // Rows 0..2 of every stream start in registers (W = 2 or 3 never occurs in
    // a reference geometry).
    if (g.fixed_words <= kRegisterRows) return LCT_E_GEOMETRY;
    size_t lds = 2 * static_cast<size_t>(register_stage_bytes(g.fixed_words));
    KernelBookkeeping bk;
    if (int32_t e = prepare_bookkeeping(bookkeeping, n_blocks, bk, lds)) return e;
    int64_t grid = n_blocks;
    if (sample_here) {
        bk.a_samples = bookkeeping->a_samples;
        bk.b_samples = bookkeeping->b_samples;
        bk.result_samples = bookkeeping->result_samples;
        bk.sample_size = sample_size;
        bk.sample_groups = sample_groups(sample_size);
        grid = std::max<int64_t>(n_blocks, bk.sample_groups);
    }
    const auto kernel = bk.control != nullptr ? dual_encode_kernel<true>
                                              : dual_encode_kernel<false>;
    if (hipError_t e = reserve_dynamic_lds(reinterpret_cast<const void *>(kernel), lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(grid)), dim3(kLanes),
                       lds, stream, a, b, alpha, partials, sample_groups(sample_size),
                       base_encode, base_decode, center_out, shifted_decode_out, side_out,
                       encoded_out, extra_starts, summaries, exponents, n_blocks, logical_numel,
                       g.steps, g.fixed_words, rare_length, bk);
    return static_cast<int32_t>(hipGetLastError());
}

}  // namespace

extern "C" int32_t lct_dual_encode(
    const int32_t *a_encoded, const uint8_t *a_side, const int32_t *a_shifted_decode,
    const int32_t *a_center, const lct_overflow *a_overflow, const int32_t *b_encoded,
    const uint8_t *b_side, const int32_t *b_shifted_decode, const int32_t *b_center,
    const lct_overflow *b_overflow, const float *alpha, const int32_t *partials,
    int64_t sample_size, const int32_t *base_encode, const int32_t *base_decode,
    int32_t *center_out, int32_t *shifted_decode_out, uint8_t *side_out, int32_t *encoded_out,
    uint8_t *extra_starts, int32_t *summaries, uint8_t *exponents, int64_t size,
    int64_t logical_numel, lct_geometry g, int32_t rare_length, hipStream_t stream) {
    return launch_dual_encode(a_encoded, a_side, a_shifted_decode, a_center, a_overflow,
                              b_encoded, b_side, b_shifted_decode, b_center, b_overflow, alpha,
                              partials, sample_size, base_encode, base_decode, center_out,
                              shifted_decode_out, side_out, encoded_out, extra_starts, summaries,
                              exponents, size, logical_numel, g, rare_length, nullptr, stream);
}

extern "C" int32_t lct_dual_encode_fused(
    const int32_t *a_encoded, const uint8_t *a_side, const int32_t *a_shifted_decode,
    const int32_t *a_center, const lct_overflow *a_overflow, const int32_t *b_encoded,
    const uint8_t *b_side, const int32_t *b_shifted_decode, const int32_t *b_center,
    const lct_overflow *b_overflow, const float *alpha, const int32_t *partials,
    int64_t sample_size, const int32_t *base_encode, const int32_t *base_decode,
    int32_t *center_out, int32_t *shifted_decode_out, uint8_t *side_out, int32_t *encoded_out,
    uint8_t *extra_starts, int32_t *summaries, uint8_t *exponents, int64_t size,
    int64_t logical_numel, lct_geometry g, int32_t rare_length,
    const lct_bookkeeping *bookkeeping, hipStream_t stream) {
    if (!bookkeeping) return LCT_E_NULL;
    return launch_dual_encode(a_encoded, a_side, a_shifted_decode, a_center, a_overflow,
                              b_encoded, b_side, b_shifted_decode, b_center, b_overflow, alpha,
                              partials, sample_size, base_encode, base_decode, center_out,
                              shifted_decode_out, side_out, encoded_out, extra_starts, summaries,
                              exponents, size, logical_numel, g, rare_length, bookkeeping,
                              stream);
}

extern "C" int32_t lct_pointwise_update_batch(
    const lct_update_job *jobs, int32_t n_jobs, int32_t op, int32_t alpha_is_one,
    int32_t beta_is_one, const float *alpha, const float *beta, int32_t *partials,
    int64_t partial_words, uint8_t *extra_starts, int64_t extra_bytes, int32_t *summaries,
    int64_t summary_words, uint64_t *control, int64_t control_words, uint32_t epoch,
    int32_t *buffer_meta, int32_t max_free_regions, uint8_t *arena,
    const lct_pending_frees *frees, hipStream_t stream) {
    if (!jobs || !partials || !extra_starts || !summaries || !control || !buffer_meta || !arena)
        return LCT_E_NULL;
    if (n_jobs <= 0 || n_jobs > LCT_MAX_UPDATE_BATCH) return LCT_E_ARG;
    if (int32_t e = check_op(op, alpha_is_one, beta_is_one, alpha, beta)) return e;
    if (epoch == 0 || (reinterpret_cast<uintptr_t>(control) & 7) != 0) return LCT_E_ARG;
    if (max_free_regions <= 0 || max_free_regions > 4096
        || (max_free_regions & (max_free_regions - 1)) != 0)
        return LCT_E_ARG;
    UpdateSampleBatch sample{};
    UpdateEncodeBatch encode{};
    CompactBatch compact{};
    sample.n_jobs = encode.n_jobs = compact.n_jobs = n_jobs;
    sample.args = encode.args = OpArgs{alpha, beta, op, alpha_is_one, beta_is_one};
    encode.buffer_meta = buffer_meta;
    encode.max_free_regions = max_free_regions;
    if (frees != nullptr) {
        if (frees->count < 0 || frees->count > LCT_MAX_PENDING_FREES) return LCT_E_ARG;
        for (int i = 0; i < frees->count; ++i)
            if (frees->descriptor[i] == nullptr) return LCT_E_NULL;
        encode.frees = *frees;
    }
    encode.epoch = epoch;
    encode.lock_spins = lock_spins();
    encode.polls = ready_polls();
    // Word 0 of the control array is the frees' gate; job j's words follow.
    encode.gate = encode.frees.count > 0 ? control : nullptr;
    compact.arena = arena;
    compact.steps = 0;
    compact.precomputed = 1;
    int64_t groups = 0, blocks_total = 0, partial_used = 0, extra_used = 0, summary_used = 0,
            control_used = 1;
    int max_words = 0;
    for (int j = 0; j < n_jobs; ++j) {
        const lct_update_job &in = jobs[j];
        const lct_geometry &g = in.geometry;
        const lct_overflow *ov = in.has_overflow ? &in.overflow : nullptr;
        if (int32_t e = check_operand(in.encoded, in.side, in.shifted_decode, in.center, ov))
            return e;
        if (!in.other || !in.base_encode || !in.base_decode || !in.center_out
            || !in.shifted_decode_out || !in.side_out || !in.encoded_out || !in.exponents
            || !in.counts || !in.blocks || !in.descriptor)
            return LCT_E_NULL;
        if (int32_t e = check_shape(in.size, in.logical_numel, g, in.rare_length)) return e;
        if (int32_t e = check_samples(in.sample_size, in.logical_numel)) return e;
        if (((reinterpret_cast<uintptr_t>(in.encoded) | reinterpret_cast<uintptr_t>(in.side)
              | reinterpret_cast<uintptr_t>(in.side_out)) & 15) != 0)
            return LCT_E_ARG;
        const int64_t nb = in.size / g.block_symbols;
        if (static_cast<int64_t>(g.fixed_words) * nb * kLanes * 4 >= (int64_t{1} << 31))
            return LCT_E_SIZE;
        // The compaction launch takes one step count for all its jobs.
        if (compact.steps != 0 && compact.steps != g.steps) return LCT_E_ARG;
        compact.steps = g.steps;
        const int32_t n_groups = sample_groups(in.sample_size);
        const OperandA a{in.encoded, in.side, in.shifted_decode, in.center,
                         ov ? *ov : lct_overflow{}, ov != nullptr};
        UpdateSampleJob &sj = sample.jobs[j];
        sj.a = a;
        sj.a_samples = static_cast<const uint16_t *>(in.a_samples);
        sj.other = static_cast<const uint16_t *>(in.other);
        sj.partials = partials + partial_used;
        sj.result_samples = static_cast<uint16_t *>(in.result_samples);
        sj.n_blocks = nb;
        sj.logical_numel = in.logical_numel;
        sj.sample_size = in.sample_size;
        sj.steps = g.steps;
        sj.fixed_words = g.fixed_words;
        sj.rare = in.rare_length;
        UpdateEncodeJob &ej = encode.jobs[j];
        ej.a = a;
        ej.other = sj.other;
        ej.partials = sj.partials;
        ej.base_encode = in.base_encode;
        ej.base_decode = in.base_decode;
        ej.center_out = in.center_out;
        ej.shifted_decode_out = in.shifted_decode_out;
        ej.side_out = in.side_out;
        ej.encoded_out = in.encoded_out;
        ej.extra_starts = extra_starts + extra_used;
        ej.summaries = summaries + summary_used;
        ej.exponents = in.exponents;
        ej.control = control + control_used;
        ej.counts = in.counts;
        ej.blocks = in.blocks;
        ej.descriptor = in.descriptor;
        ej.n_blocks = nb;
        ej.logical_numel = in.logical_numel;
        ej.n_groups = n_groups;
        ej.steps = g.steps;
        ej.fixed_words = g.fixed_words;
        ej.rare = in.rare_length;
        CompactBatchJob &cj = compact.jobs[j];
        cj.source = in.exponents;
        cj.blocks = in.blocks;
        cj.counts = in.counts;
        cj.descriptor = in.descriptor;
        cj.extra_starts = ej.extra_starts;
        cj.n_blocks = nb;
        cj.logical_numel = in.logical_numel;
        sample.first_group[j] = static_cast<int32_t>(groups);
        encode.first_block[j] = compact.first_block[j] = static_cast<int32_t>(blocks_total);
        groups += n_groups;
        blocks_total += nb;
        partial_used += 2 * n_groups;
        extra_used += nb * kLanes;
        summary_used += 5 * nb + 1;
        control_used += kControlPartials + nb;
        if (g.fixed_words > max_words) max_words = g.fixed_words;
    }
    if (partial_used > partial_words || extra_used > extra_bytes
        || summary_used > summary_words || control_used > control_words)
        return LCT_E_SIZE;
    if (blocks_total > 0x7FFFFFFF) return LCT_E_SIZE;
    sample.first_group[n_jobs] = static_cast<int32_t>(groups);
    encode.first_block[n_jobs] = compact.first_block[n_jobs] = static_cast<int32_t>(blocks_total);

    const size_t sample_lds = static_cast<size_t>(max_words + 1) * kSampleGroup * 4;
    hipLaunchKernelGGL(pointwise_sample_batch_kernel, dim3(static_cast<uint32_t>(groups)),
                       dim3(kSampleGroup), sample_lds, stream, sample);
    if (hipError_t e = hipGetLastError()) return static_cast<int32_t>(e);
    const size_t encode_lds = std::max(static_cast<size_t>(window_stage_bytes(max_words)),
                                       static_cast<size_t>(max_free_regions) * 8);
    if (hipError_t e = reserve_dynamic_lds(
            reinterpret_cast<const void *>(&pointwise_encode_batch_kernel), encode_lds))
        return static_cast<int32_t>(e);
    hipLaunchKernelGGL(pointwise_encode_batch_kernel, dim3(static_cast<uint32_t>(blocks_total)),
                       dim3(kLanes), encode_lds, stream, encode);
    if (hipError_t e = hipGetLastError()) return static_cast<int32_t>(e);
    return static_cast<int32_t>(
        launch_compact_batch(compact, static_cast<uint32_t>(blocks_total), stream));
}
