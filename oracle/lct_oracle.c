/* CPU oracle for the LCT BF16 exponent-Huffman codec -- TEST INFRASTRUCTURE.
 *
 * Serial per-lane restatement of the reference's Triton codec kernels.  It is
 * the parity checker for the HIP kernels and the host-core baseline; the
 * product library never links or calls it.  Citations are file:line in the
 * reference repository.  Blocks are independent, so the block loops run under
 * OpenMP when built with -fopenmp (the host-core baseline); every result is
 * independent of the thread count.
 *
 * Parity pinning (which check fixes each function) is listed in the test
 * files under tests/; functions here carry no self-checks.
 */
#include "lct_oracle.h"

#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int32_t lcto_num_threads(void) {
#ifdef _OPENMP
    return (int32_t)omp_get_max_threads();
#else
    return 1;
#endif
}

/* Thread count of later parallel regions (the CPU baseline's 1-thread
 * figure); no effect without OpenMP. */
void lcto_set_num_threads(int32_t n) {
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}

/* Storage row r, lane l -> logical column l ^ (r & 254)
 * (LCT/kernels/generic/layout.py:15-18). */
static inline int64_t logical_offset(int64_t row, int32_t lane, int32_t lanes) {
    return row * lanes + (int64_t)(lane ^ (int32_t)(row & 254));
}

/* Source element as the kernels read it: int16 sign-extended, or uint8. */
static inline int32_t load_source(const void *source, int precomputed,
                                  int64_t index) {
    if (precomputed) return (int32_t)((const uint8_t *)source)[index];
    return (int32_t)((const int16_t *)source)[index];
}

static inline int32_t exponent_byte(int32_t value, int precomputed) {
    return precomputed ? (value & 255) : ((value >> 7) & 0xFF);
}

/* ---- center and shifted tables (LCT/kernels/common/tables.py) ---------- */

/* tables.py:24-31: sample i lies in region [i*n/M, (i+1)*n/M) at a hashed
 * offset. */
static int64_t sample_position(int64_t i, int64_t logical_numel, int64_t sample_size) {
    uint32_t hashed = (uint32_t)i * 0x9E3779B9u;
    int64_t start = i * logical_numel / sample_size;
    int64_t end = (i + 1) * logical_numel / sample_size;
    uint64_t jitter = ((uint64_t)hashed * (uint64_t)(end - start)) >> 32;
    return start + (int64_t)jitter;
}

void lcto_sample_positions(int64_t logical_numel, int64_t sample_size, int64_t *out) {
    for (int64_t i = 0; i < sample_size; ++i)
        out[i] = sample_position(i, logical_numel, sample_size);
}

int32_t lcto_estimate_center(const void *source, int64_t logical_numel,
                             int64_t sample_size, int precomputed) {
    /* tables.py:15-49: one jittered sample per region, exponent >= -120. */
    int64_t total = 0, kept = 0;
    for (int64_t i = 0; i < sample_size; ++i) {
        int32_t value = load_source(source, precomputed,
                                    sample_position(i, logical_numel, sample_size));
        int32_t exp = exponent_byte(value, precomputed) - 127;
        if (exp >= -120) {
            total += exp;
            kept += 1;
        }
    }
    if (kept == 0) return 0;
    int64_t center = total >= 0 ? (total + kept / 2) / kept
                                : -((-total + kept / 2) / kept);
    if (center < -128) center = -128;
    if (center > 127) center = 127;
    return (int32_t)center;
}

/* Table index of a centred delta; index 0 is exact zero (tables.py:53-67). */
static inline int32_t inverse_index_exponent(int32_t symbol, int32_t center) {
    /* tables.py:109-116 / primitives.py:29-35: index -> unbiased exponent. */
    int32_t zero_delta = (-127 - center) & 255;
    if (symbol == 0) return -127;
    int32_t delta = symbol - (symbol <= zero_delta ? 1 : 0);
    if (delta >= 128) delta -= 256;
    return delta + center;
}

void lcto_shift_tables(const int32_t *base_encode, const int32_t *base_decode,
                       int32_t center, int32_t *shifted_encode,
                       int32_t *shifted_decode) {
    int32_t zero_delta = (-127 - center) & 255;
    for (int32_t raw = 0; raw < 256; ++raw) {
        int32_t exp = raw - 127;
        int32_t delta = (exp - center) & 255;
        int32_t index = exp == -127 ? 0 : delta + (delta < zero_delta ? 1 : 0);
        shifted_encode[raw] = base_encode[index];
    }
    for (int32_t i = 0; i < 1024; ++i) {
        int32_t packed = base_decode[i];
        int32_t length = packed & 255;
        int32_t symbol = (packed >> 8) & 255;
        int32_t exponent = inverse_index_exponent(symbol, center);
        shifted_decode[i] = length == 0
            ? 0 : (int32_t)((uint32_t)length | ((uint32_t)exponent << 8));
    }
}

/* ---- encoder (LCT/kernels/generic/encode.py:10-169) -------------------- */

void lcto_encode(const void *source, int precomputed, uint8_t *side,
                 int32_t *encoded, const int32_t *shifted_encode,
                 uint8_t *extra_starts, int32_t *summaries, int64_t size,
                 int64_t logical_numel, lcto_geometry g) {
    const int32_t B = g.block_symbols, L = g.lanes, S = g.steps, W = g.fixed_words;
    const int64_t n_blocks = (size + B - 1) / B;
    const int64_t n_streams = n_blocks * L;
#pragma omp parallel for schedule(static)
    for (int64_t block = 0; block < n_blocks; ++block) {
        int32_t bad_count = 0, bad_bytes = 0;
        const int full_block = (block + 1) * B <= logical_numel;
        for (int32_t lane = 0; lane < L; ++lane) {
            const int64_t stream = block * L + lane;
            int32_t word = 0, shift = 0, overflow = 0, extra_start = S;
            uint32_t word_value = 0;
            const int has_data = block * B + lane < size;
            for (int32_t step = 0; step < S; step += 2) {
                const int64_t storage = block * B + (int64_t)step * L + lane;
                const int64_t row0 = block * S + step;
                const int64_t in0 = logical_offset(row0, lane, L);
                const int64_t in1 = logical_offset(row0 + 1, lane, L);
                const int valid0 = storage < size;
                const int valid1 = storage + L < size;
                const int iv0 = full_block || in0 < logical_numel;
                const int iv1 = full_block || in1 < logical_numel;
                int32_t v0 = iv0 ? load_source(source, precomputed, in0) : 0;
                int32_t v1 = iv1 ? load_source(source, precomputed, in1) : 0;
                int32_t byte0 = exponent_byte(v0, precomputed);
                int32_t byte1 = exponent_byte(v1, precomputed);
                if (!precomputed) {
                    /* encode.py:57-65: side byte = sign | 7 mantissa bits.
                     * Padding past the logical end is written as 0 here; the
                     * reference leaves it unwritten (torch.empty). */
                    if (valid0)
                        side[storage] = iv0 ? (uint8_t)((v0 & 0x7F) | ((v0 >> 8) & 0x80)) : 0;
                    if (valid1)
                        side[storage + L] = iv1 ? (uint8_t)((v1 & 0x7F) | ((v1 >> 8) & 0x80)) : 0;
                }
                uint32_t packed0 = iv0 ? (uint32_t)shifted_encode[byte0] : 0u;
                uint32_t packed1 = iv1 ? (uint32_t)shifted_encode[byte1] : 0u;
                int32_t len0 = (int32_t)(packed0 >> 20);
                int32_t len1 = (int32_t)(packed1 >> 20);
                int32_t length = len0 + len1;
                uint32_t code = (packed0 & 0xFFFFFu) | ((packed1 & 0xFFFFFu) << len0);

                uint32_t new_word = word_value | (code << shift);
                int crosses = shift + length >= 32;
                int pair_overflow = (int64_t)word * 32 + shift + length > (int64_t)W * 32;
                if (!full_block) pair_overflow = pair_overflow && valid0;
                int first_overflow = !overflow && pair_overflow;
                if (first_overflow) extra_start = step;
                uint32_t store_value = first_overflow ? word_value : new_word;
                if (crosses && word < W) {
                    int32_t safe_word = word < W - 1 ? word : W - 1;
                    encoded[(int64_t)safe_word * n_streams + stream] = (int32_t)store_value;
                }
                /* A 32-bit shift must yield 0 (encode.py:87 relies on it). */
                uint32_t carry = shift == 0 ? 0u : code >> (32 - shift);
                word_value = crosses ? carry : new_word;
                word += crosses ? 1 : 0;
                shift = crosses ? shift + length - 32 : shift + length;
                overflow = overflow || pair_overflow;
            }
            if (has_data && word < W && shift != 0)
                encoded[(int64_t)word * n_streams + stream] = (int32_t)word_value;
            const int bad = has_data && overflow;
            extra_starts[stream] = (uint8_t)(bad ? extra_start : 255);
            if (bad) {
                bad_count += 1;
                bad_bytes += S - extra_start;
            }
        }
        if (summaries) {
            summaries[block] = bad_count;
            summaries[n_blocks + block] = bad_bytes;
        }
    }
}

/* ---- block scans (LCT/kernels/generic/metadata.py:13-31) --------------- */

void lcto_prefix(int32_t *summaries, int64_t n_blocks, int32_t *counts) {
    int32_t count_run = 0, byte_run = 0;
    for (int64_t b = 0; b < n_blocks; ++b) {
        int32_t c = summaries[b], bytes = summaries[n_blocks + b];
        summaries[2 * n_blocks + b] = count_run;
        summaries[3 * n_blocks + b] = byte_run;
        count_run += c;
        byte_run += bytes;
    }
    counts[0] = count_run;
    counts[1] = byte_run;
    counts[2] = 0;
    counts[3] = 0;
}

/* ---- overflow compaction (LCT/kernels/generic/compaction.py:137-228) --- */

void lcto_compact_extra(const void *source, int precomputed,
                        const uint8_t *extra_starts, const int32_t *summaries,
                        int64_t n_blocks, int64_t size, int64_t logical_numel,
                        lcto_geometry g, uint8_t *lanes, uint8_t *starts,
                        uint8_t *tail, int64_t lane_off, int64_t start_off,
                        int64_t tail_off, int32_t *blocks_out) {
    const int32_t B = g.block_symbols, L = g.lanes, S = g.steps;
    const int64_t n_streams = n_blocks * L;
#pragma omp parallel for schedule(static)
    for (int64_t block = 0; block < n_blocks; ++block) {
        const int32_t count = summaries[block];
        const int32_t first = summaries[2 * n_blocks + block];
        const int32_t byte_base = summaries[3 * n_blocks + block];
        if (count > 0) {
            int32_t rank = 0, local = 0;
            for (int32_t lane = 0; lane < L; ++lane) {
                const int64_t stream = block * L + lane;
                const int32_t start = extra_starts[stream];
                if (stream >= n_streams || start == 255) continue;
                for (int32_t row = start; row < S; ++row) {
                    const int64_t storage = block * B + (int64_t)row * L + lane;
                    if (storage >= size) continue;
                    const int64_t in = logical_offset(block * S + row, lane, L);
                    int32_t value = in < logical_numel
                        ? load_source(source, precomputed, in) : 0;
                    int32_t e = precomputed ? value - 127
                                            : ((value >> 7) & 255) - 127;
                    tail[tail_off + byte_base + local + (row - start)] = (uint8_t)(int8_t)e;
                }
                local += S - start;
                lanes[lane_off + first + rank] = (uint8_t)lane;
                starts[start_off + first + rank] = (uint8_t)start;
                rank += 1;
            }
        }
        blocks_out[block] = count;
        blocks_out[n_blocks + block] = first;
        blocks_out[2 * n_blocks + block] = byte_base;
    }
}

/* ---- decoder (LCT/kernels/generic/decode.py, primitives.py) ------------ */

/* primitives.py:17-36 */
static inline void decode_symbol(uint64_t current, const int32_t *decode_table,
                                 int32_t center, int32_t rare_length,
                                 int32_t *value, int32_t *length) {
    int32_t first = decode_table[current & 1023u];
    int32_t first_length = first & 255;
    if (first_length == 0) {
        int32_t symbol = (int32_t)((current >> rare_length) & 255u);
        *value = inverse_index_exponent(symbol, center);
        *length = rare_length + 8;
    } else {
        *value = first >> 8;
        *length = first_length;
    }
}

/* primitives.py:7-14 */
static inline int16_t pack_bf16(int32_t value, int32_t sign_mantissa) {
    return (int16_t)((((value + 127) & 255) << 7) | (sign_mantissa & 0x7F)
                     | ((sign_mantissa & 0x80) << 8));
}

/* Per-lane overflow start/offset of one block (decode.py:195-240). */
static void block_overflow_map(const lcto_overflow *o, int64_t block,
                               int64_t n_blocks, int32_t L, int32_t S,
                               int32_t *stream_start, int64_t *stream_offset) {
    for (int32_t l = 0; l < L; ++l) {
        stream_start[l] = S;
        stream_offset[l] = 0;
    }
    if (!o || !o->blocks) return;
    const int32_t count = o->blocks[block];
    if (count <= 0) return;
    const int32_t first = o->blocks[n_blocks + block];
    int64_t running = o->blocks[2 * n_blocks + block];
    for (int32_t e = 0; e < count; ++e) {
        int32_t lane = o->lanes[o->lane_off + first + e];
        int32_t start = o->starts[o->start_off + first + e];
        stream_start[lane] = start;
        stream_offset[lane] = running;
        running += S - start;
    }
}

/* Decode block `block` into logical BF16 bits; positions past logical_numel
 * are skipped.  Mirrors _decode_rows_impl's pair loop (decode.py:36-171). */
static void decode_block(const int32_t *encoded, const uint8_t *side,
                         const int32_t *decode_table, int32_t center,
                         int32_t rare_length, int64_t size,
                         int64_t logical_numel, lcto_geometry g,
                         const lcto_overflow *overflow, int64_t block,
                         int16_t *out, int64_t out_base) {
    const int32_t B = g.block_symbols, L = g.lanes, S = g.steps, W = g.fixed_words;
    const int64_t n_blocks = (size + B - 1) / B;
    const int64_t n_streams = n_blocks * L;
    int32_t stream_start[256];
    int64_t stream_offset[256];
    block_overflow_map(overflow, block, n_blocks, L, S, stream_start, stream_offset);
    for (int32_t lane = 0; lane < L; ++lane) {
        const int64_t stream = block * L + lane;
        int32_t word = 0, shift = 0;
        uint64_t window = (uint64_t)(uint32_t)encoded[stream]
            | ((uint64_t)(uint32_t)encoded[n_streams + stream] << 32);
        for (int32_t step = 0; step < S; step += 2) {
            int32_t next = word + 2 < W - 1 ? word + 2 : W - 1;
            uint64_t prefetch = (uint64_t)(uint32_t)encoded[(int64_t)next * n_streams + stream];
            int32_t shift_now = shift;
            for (int32_t half = 0; half < 2; ++half) {
                const int32_t s = step + half;
                const int64_t storage = block * B + (int64_t)s * L + lane;
                int32_t value, length;
                decode_symbol(window >> shift_now, decode_table, center,
                              rare_length, &value, &length);
                if (s >= stream_start[lane]) {
                    const uint8_t *t = overflow->tail + overflow->tail_off;
                    value = (int32_t)t[stream_offset[lane] + s - stream_start[lane]];
                }
                if (storage < size) {
                    const int64_t offset = logical_offset(block * S + s, lane, L);
                    if (offset < logical_numel)
                        out[offset - out_base] = pack_bf16(value, side[storage]);
                    shift_now += length;
                }
            }
            if (shift_now >= 32) {
                window = (window >> 32) | (prefetch << 32);
                word += 1;
                shift = shift_now - 32;
            } else {
                shift = shift_now;
            }
        }
    }
}

void lcto_decode(const int32_t *encoded, const uint8_t *side, int16_t *output,
                 const int32_t *shifted_decode, int32_t center,
                 int32_t rare_length, int64_t size, int64_t logical_numel,
                 lcto_geometry g, const lcto_overflow *overflow) {
    const int64_t n_blocks = (size + g.block_symbols - 1) / g.block_symbols;
#pragma omp parallel for schedule(static)
    for (int64_t block = 0; block < n_blocks; ++block)
        decode_block(encoded, side, shifted_decode, center, rare_length, size,
                     logical_numel, g, overflow, block, output, 0);
}

/* ---- pointwise arithmetic (LCT/kernels/generic/pointwise.py) ----------- */

static inline float bf16_to_f32(uint16_t bits) {
    uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* Round to nearest even; NaN becomes the canonical 0x7FFF. */
uint16_t lcto_f32_to_bf16(float value) {
    uint32_t u;
    memcpy(&u, &value, sizeof u);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return 0x7FFF;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* pointwise.py:340-363: add/multiply of BF16 operands round once from FP32;
 * scalar_mul_add keeps FP32 scaling and a fused multiply-add. */
uint16_t lcto_apply(int op, uint16_t left, uint16_t right, float alpha,
                    float beta, int alpha_is_one, int beta_is_one) {
    float a = bf16_to_f32(left), b = bf16_to_f32(right), r;
    if (op == LCTO_ADD) {
        r = a + b;
    } else if (op == LCTO_MULTIPLY) {
        r = a * b;
    } else if (alpha_is_one) {
        r = beta_is_one ? a + b : __builtin_fmaf(b, beta, a);
    } else {
        if (!beta_is_one) b = b * beta;
        r = __builtin_fmaf(a, alpha, b);
    }
    return lcto_f32_to_bf16(r);
}

/* lcto_apply over n element pairs (dense operands of an optimizer step). */
void lcto_apply_n(int op, const uint16_t *left, const uint16_t *right, int64_t n,
                  float alpha, float beta, int alpha_is_one, int beta_is_one,
                  uint16_t *out) {
    for (int64_t i = 0; i < n; ++i)
        out[i] = lcto_apply(op, left[i], right[i], alpha, beta, alpha_is_one, beta_is_one);
}

/* _store_result (pointwise.py:43-65) for one storage position. */
static inline void store_result(uint16_t bits, int policy, int logical_valid,
                                int64_t storage, int64_t logical, void *output,
                                uint8_t *auxiliary) {
    if (policy == 0) {
        if (logical_valid) ((uint16_t *)output)[logical] = bits;
        return;
    }
    if (!logical_valid) bits = 0;
    ((uint8_t *)output)[storage] = (uint8_t)((bits & 0x7F) | ((bits >> 8) & 0x80));
    if (logical_valid) auxiliary[logical] = (uint8_t)((bits >> 7) & 0xFF);
}

void lcto_pointwise(const int32_t *encoded, const uint8_t *side,
                    const int32_t *shifted_decode, int32_t center,
                    int32_t rare_length, int64_t size, int64_t logical_numel,
                    lcto_geometry g, const lcto_overflow *overflow,
                    const uint16_t *other, int op, float alpha, float beta,
                    int alpha_is_one, int beta_is_one, int policy,
                    void *output, uint8_t *auxiliary) {
    const int32_t B = g.block_symbols, L = g.lanes, S = g.steps;
    const int64_t n_blocks = (size + B - 1) / B;
#pragma omp parallel for schedule(static)
    for (int64_t block = 0; block < n_blocks; ++block) {
        /* Decode into a block-local logical buffer, then apply the op. */
        int16_t *local = (int16_t *)malloc((size_t)B * sizeof(int16_t));
        const int64_t row_base = block * S;
        const int64_t logical_base = row_base * L;
        decode_block(encoded, side, shifted_decode, center, rare_length, size,
                     logical_numel, g, overflow, block, local, logical_base);
        for (int32_t step = 0; step < S; ++step) {
            for (int32_t lane = 0; lane < L; ++lane) {
                const int64_t storage = block * B + (int64_t)step * L + lane;
                if (storage >= size) continue;
                const int64_t logical = logical_offset(row_base + step, lane, L);
                const int valid = logical < logical_numel;
                uint16_t bits = 0;
                if (valid)
                    bits = lcto_apply(op, (uint16_t)local[logical - logical_base],
                                      other[logical], alpha, beta,
                                      alpha_is_one, beta_is_one);
                store_result(bits, policy, valid, storage, logical, output,
                             auxiliary);
            }
        }
        free(local);
    }
}

void lcto_dual(const int32_t *a_encoded, const uint8_t *a_side,
               const int32_t *a_shifted_decode, int32_t a_center,
               const lcto_overflow *a_overflow,
               const int32_t *b_encoded, const uint8_t *b_side,
               const int32_t *b_shifted_decode, int32_t b_center,
               const lcto_overflow *b_overflow, int32_t rare_length,
               int64_t size, int64_t logical_numel, lcto_geometry g,
               float alpha, int policy, void *output, uint8_t *auxiliary) {
    const int32_t B = g.block_symbols, L = g.lanes, S = g.steps;
    const int64_t n_blocks = (size + B - 1) / B;
#pragma omp parallel for schedule(static)
    for (int64_t block = 0; block < n_blocks; ++block) {
        int16_t *a_local = (int16_t *)malloc(2 * (size_t)B * sizeof(int16_t));
        int16_t *b_local = a_local + B;
        const int64_t row_base = block * S;
        const int64_t logical_base = row_base * L;
        decode_block(a_encoded, a_side, a_shifted_decode, a_center, rare_length,
                     size, logical_numel, g, a_overflow, block, a_local,
                     logical_base);
        decode_block(b_encoded, b_side, b_shifted_decode, b_center, rare_length,
                     size, logical_numel, g, b_overflow, block, b_local,
                     logical_base);
        for (int32_t step = 0; step < S; ++step) {
            for (int32_t lane = 0; lane < L; ++lane) {
                const int64_t storage = block * B + (int64_t)step * L + lane;
                if (storage >= size) continue;
                const int64_t logical = logical_offset(row_base + step, lane, L);
                const int valid = logical < logical_numel;
                uint16_t bits = 0;
                if (valid) {
                    /* pointwise_scalar_dual.py:226: fma(a, alpha, b) in FP32. */
                    float a = bf16_to_f32((uint16_t)a_local[logical - logical_base]);
                    float b = bf16_to_f32((uint16_t)b_local[logical - logical_base]);
                    bits = lcto_f32_to_bf16(__builtin_fmaf(a, alpha, b));
                }
                store_result(bits, policy, valid, storage, logical, output,
                             auxiliary);
            }
        }
        free(a_local);
    }
}

/* ---- allocator (LCT/kernels/tensor_buffer.py) -------------------------- */

void lcto_buffer_reset(int32_t *meta, int32_t R, int32_t capacity_bytes) {
    /* tensor_buffer.py:18-34 */
    for (int32_t i = 0; i < 2 * R; ++i) meta[i] = 0;
    meta[R] = capacity_bytes;
    meta[2 * R] = 1;
    meta[2 * R + 1] = 0;
    meta[2 * R + 2] += 1;
}

void lcto_buffer_allocate(int32_t *meta, int32_t R, int32_t requested_bytes,
                          int32_t item_count, int32_t item_bytes,
                          int32_t *descriptor) {
    /* tensor_buffer.py:37-91 */
    int32_t *starts = meta, *sizes = meta + R;
    int32_t count = meta[2 * R];
    int32_t request = requested_bytes + (item_bytes ? item_count * item_bytes : 0);
    int32_t generation = meta[2 * R + 2];
    int32_t size = ((request + 15) / 16) * 16;
    int32_t slot = R;
    for (int32_t i = 0; i < count && i < R; ++i)
        if (sizes[i] >= size) { slot = i; break; }
    int success = request > 0 && slot < count;
    int32_t start = 0, region = 0;
    if (success) {
        start = starts[slot];
        region = sizes[slot];
        if (region == size) {
            for (int32_t i = slot; i + 1 < count; ++i) {
                starts[i] = starts[i + 1];
                sizes[i] = sizes[i + 1];
            }
            meta[2 * R] = count - 1;
        } else {
            starts[slot] = start + size;
            sizes[slot] = region - size;
        }
    }
    descriptor[0] = success ? start : -1;
    descriptor[1] = success ? size : 0;
    descriptor[2] = request <= 0 ? 2 : (success ? 0 : 1);
    descriptor[3] = generation;
}

int32_t lcto_buffer_free(int32_t *meta, int32_t R, int32_t *descriptor) {
    /* tensor_buffer.py:94-179 */
    int32_t *starts = meta, *sizes = meta + R;
    int32_t offset = descriptor[0], size = descriptor[1];
    int32_t count = meta[2 * R];
    int valid = descriptor[2] == 0 && descriptor[3] == meta[2 * R + 2]
        && offset >= 0 && size > 0;
    if (!valid) return 4;
    int32_t insert = 0;
    for (int32_t i = 0; i < count; ++i)
        if (starts[i] < offset) insert += 1;
    int has_prev = insert > 0, has_next = insert < count;
    int32_t prev_start = has_prev ? starts[insert - 1] : 0;
    int32_t prev_size = has_prev ? sizes[insert - 1] : 0;
    int32_t next_start = has_next ? starts[insert] : 0;
    int32_t next_size = has_next ? sizes[insert] : 0;
    int merge_prev = has_prev && prev_start + prev_size == offset;
    int merge_next = has_next && offset + size == next_start;
    if (merge_prev && merge_next) {
        sizes[insert - 1] = prev_size + size + next_size;
        for (int32_t i = insert; i + 1 < count; ++i) {
            starts[i] = starts[i + 1];
            sizes[i] = sizes[i + 1];
        }
        meta[2 * R] = count - 1;
    } else if (merge_prev) {
        sizes[insert - 1] = prev_size + size;
    } else if (merge_next) {
        starts[insert] = offset;
        sizes[insert] = next_size + size;
    } else {
        if (count >= R) return 3;
        for (int32_t i = count - 1; i >= insert; --i) {
            starts[i + 1] = starts[i];
            sizes[i + 1] = sizes[i];
        }
        starts[insert] = offset;
        sizes[insert] = size;
        meta[2 * R] = count + 1;
    }
    descriptor[2] = 5;
    return 0;
}
