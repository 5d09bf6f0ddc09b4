/* CPU oracle for the LCT BF16 exponent-Huffman codec -- TEST INFRASTRUCTURE.
 *
 * A plain-C restatement of the reference's codec kernels, written as the
 * serial per-lane loops the Triton kernels express.  It is the parity checker
 * for the HIP kernels and the host-core baseline timed by bench.py.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product path (losslessly_compressed_tensors_amd) never does.
 *
 * Every function names the reference file:line it follows (paths relative to
 * the reference repository root).  All pointers are host pointers.
 */
#ifndef LCT_ORACLE_H
#define LCT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Stream geometry (B, L, S, W): block symbols, lanes, steps, fixed words. */
typedef struct {
    int32_t block_symbols;
    int32_t lanes;
    int32_t steps;
    int32_t fixed_words;
} lcto_geometry;

/* Center of the sampled unbiased exponents (LCT/kernels/common/tables.py:9-49,
 * sample size min(n, 4096) from LCT/codec/encode.py:19,64). */
/* Positions of the center's samples (tables.py:24-31), out[sample_size]. */
void lcto_sample_positions(int64_t logical_numel, int64_t sample_size, int64_t *out);

int32_t lcto_estimate_center(const void *source, int64_t logical_numel,
                             int64_t sample_size, int precomputed);

/* Raw-exponent-byte encode table and exponent-valued decode table for one
 * center (LCT/kernels/common/tables.py:52-67, 102-118). */
void lcto_shift_tables(const int32_t *base_encode, const int32_t *base_decode,
                       int32_t center, int32_t *shifted_encode,
                       int32_t *shifted_decode);

/* Field split + fixed-payload encoder (LCT/kernels/generic/encode.py:10-169).
 * source: int16 BF16 bits (precomputed=0) or uint8 exponent bytes
 * (precomputed=1), logical order.  side: uint8[size], written only when
 * precomputed=0.  encoded: int32[streams*W + 4].  summaries: int32[4*nb] or
 * NULL. */
void lcto_encode(const void *source, int precomputed, uint8_t *side,
                 int32_t *encoded, const int32_t *shifted_encode,
                 uint8_t *extra_starts, int32_t *summaries, int64_t size,
                 int64_t logical_numel, lcto_geometry g);

/* Exclusive block scans and totals (LCT/kernels/generic/metadata.py:13-31).
 * counts[4] = {total_count, total_bytes, 0, 0}. */
void lcto_prefix(int32_t *summaries, int64_t n_blocks, int32_t *counts);

/* Overflow compaction with block metadata (LCT/kernels/generic/
 * compaction.py:137-228, BUILD_META branch).  Entries go to lanes[lane_off+.],
 * starts[start_off+.]; tail bytes int8(e-127) to tail[tail_off+.]. */
void lcto_compact_extra(const void *source, int precomputed,
                        const uint8_t *extra_starts, const int32_t *summaries,
                        int64_t n_blocks, int64_t size, int64_t logical_numel,
                        lcto_geometry g, uint8_t *lanes, uint8_t *starts,
                        uint8_t *tail, int64_t lane_off, int64_t start_off,
                        int64_t tail_off, int32_t *blocks_out);

/* Overflow metadata of one compressed tensor, as the decoder reads it
 * (LCT/kernels/generic/decode.py:195-240).  blocks == NULL means none. */
typedef struct {
    const uint8_t *lanes;
    const uint8_t *starts;
    const uint8_t *tail;
    const int32_t *blocks;   /* int32[3*nb]: count, first, byte_base */
    int64_t lane_off, start_off, tail_off;
} lcto_overflow;

/* Decoder with fused overflow overlay (LCT/kernels/generic/decode.py:12-256,
 * primitives.py:7-36).  output: int16[logical_numel]. */
void lcto_decode(const int32_t *encoded, const uint8_t *side, int16_t *output,
                 const int32_t *shifted_decode, int32_t center,
                 int32_t rare_length, int64_t size, int64_t logical_numel,
                 lcto_geometry g, const lcto_overflow *overflow);

/* Pointwise arithmetic on BF16 bit patterns, one element
 * (LCT/kernels/generic/pointwise.py:340-363, _store_result :43-65). */
enum { LCTO_ADD = 0, LCTO_MULTIPLY = 1, LCTO_SCALAR_MUL_ADD = 2 };
uint16_t lcto_apply(int op, uint16_t left, uint16_t right, float alpha,
                    float beta, int alpha_is_one, int beta_is_one);
uint16_t lcto_f32_to_bf16(float value);
void lcto_apply_n(int op, const uint16_t *left, const uint16_t *right, int64_t n,
                  float alpha, float beta, int alpha_is_one, int beta_is_one,
                  uint16_t *out);

/* Fused decode + op on one compressed and one dense operand
 * (LCT/kernels/generic/pointwise.py:84-337).  policy 0: dense BF16 output
 * int16[logical_numel]; policy 1: side bytes uint8[size] in storage order into
 * `output` and exponent bytes in logical order into `auxiliary`. */
void lcto_pointwise(const int32_t *encoded, const uint8_t *side,
                    const int32_t *shifted_decode, int32_t center,
                    int32_t rare_length, int64_t size, int64_t logical_numel,
                    lcto_geometry g, const lcto_overflow *overflow,
                    const uint16_t *other, int op, float alpha, float beta,
                    int alpha_is_one, int beta_is_one, int policy,
                    void *output, uint8_t *auxiliary);

/* Fused alpha*A + B with both operands compressed
 * (LCT/kernels/generic/pointwise_scalar_dual.py:118-346). */
void lcto_dual(const int32_t *a_encoded, const uint8_t *a_side,
               const int32_t *a_shifted_decode, int32_t a_center,
               const lcto_overflow *a_overflow,
               const int32_t *b_encoded, const uint8_t *b_side,
               const int32_t *b_shifted_decode, int32_t b_center,
               const lcto_overflow *b_overflow, int32_t rare_length,
               int64_t size, int64_t logical_numel, lcto_geometry g,
               float alpha, int policy, void *output, uint8_t *auxiliary);

/* First-fit free-list allocator (LCT/kernels/tensor_buffer.py:18-192).
 * meta = int32[2R + 3]: free_starts[R] | free_sizes[R] | count | lock | gen. */
void lcto_buffer_reset(int32_t *meta, int32_t max_free_regions,
                       int32_t capacity_bytes);
void lcto_buffer_allocate(int32_t *meta, int32_t max_free_regions,
                          int32_t requested_bytes, int32_t item_count,
                          int32_t item_bytes, int32_t *descriptor);
int32_t lcto_buffer_free(int32_t *meta, int32_t max_free_regions,
                         int32_t *descriptor);

/* Number of OpenMP threads the oracle's parallel loops use (1 if built
 * without OpenMP). */
int32_t lcto_num_threads(void);
void lcto_set_num_threads(int32_t n);

#ifdef __cplusplus
}
#endif
#endif
