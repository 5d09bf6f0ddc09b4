// Elementwise arithmetic of the fused pointwise kernels (gfx950).
//
// LCT/kernels/generic/pointwise.py:340-363: operands are widened to FP32;
// add and multiply round once; scalar_mul_add is FP32 fma(a, alpha, b) (b
// pre-scaled by beta in FP32 when beta is given, fma(b, beta, a) when alpha
// is one, a + b when both are one); the result is rounded to BF16 to
// nearest-even, NaN giving 0x7FFF.
#pragma once

#include "decode_core.h"

namespace lct {

struct OpParams {
    int32_t op;
    int32_t alpha_is_one;
    int32_t beta_is_one;
    float alpha;
    float beta;
};

__device__ __forceinline__ uint32_t apply_op_f(const OpParams &p, float a, float b) {
    float r;
    if (p.op == LCT_OP_ADD) {
        r = a + b;
    } else if (p.op == LCT_OP_MULTIPLY) {
        r = a * b;
    } else if (p.alpha_is_one) {
        r = p.beta_is_one ? a + b : __builtin_fmaf(b, p.beta, a);
    } else {
        if (!p.beta_is_one) b = b * p.beta;
        r = __builtin_fmaf(a, p.alpha, b);
    }
    return float_to_bf16(r);
}

__device__ __forceinline__ uint32_t apply_op(const OpParams &p, uint32_t left, uint32_t right) {
    return apply_op_f(p, bf16_to_float(left), bf16_to_float(right));
}

// Branch-free arithmetic forms.  Every (op, alpha_is_one, beta_is_one)
// combination of the three operations is one of these, chosen once per launch
// by form_of(); each computes exactly what apply_op_f computes:
//  * kFormAxpy:  fma(a, alpha, b) -- add and the alpha*a + b forms (alpha is
//    1.0 where alpha_is_one or for add: fma(a, 1, b) rounds a + b once);
//  * kFormAxpby: fma(a, alpha, fl(b * beta));
//  * kFormBxpa:  fma(b, beta, a) -- alpha_is_one with beta;
//  * kFormMul:   a * b.
enum OpForm : int32_t { kFormAxpy = 0, kFormAxpby = 1, kFormBxpa = 2, kFormMul = 3 };

__host__ __device__ constexpr int32_t form_of(int32_t op, int32_t alpha_is_one,
                                              int32_t beta_is_one) {
    return op == LCT_OP_MULTIPLY ? kFormMul
         : op == LCT_OP_ADD ? kFormAxpy
         : alpha_is_one ? (beta_is_one ? kFormAxpy : kFormBxpa)
                        : (beta_is_one ? kFormAxpy : kFormAxpby);
}

template <int kForm>
__device__ __forceinline__ float apply_form(const OpParams &p, float a, float b) {
    if (kForm == kFormAxpy) return __builtin_fmaf(a, p.alpha, b);
    if (kForm == kFormAxpby) return __builtin_fmaf(a, p.alpha, b * p.beta);
    if (kForm == kFormBxpa) return __builtin_fmaf(b, p.beta, a);
    return a * b;
}

// The BF16 rounding of `value` (nearest-even, NaN -> 0x7FFF) in the high half
// of the result; the low half is not meaningful.  The exponent byte is then
// bits 23..30 and the side byte bits 16..22 plus bit 31.
__device__ __forceinline__ uint32_t round_bf16_high(float value) {
    const uint32_t u = __float_as_uint(value);
    const uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);
    return __builtin_isnan(value) ? 0x7FFF0000u : r;
}

__device__ __forceinline__ uint32_t high_exponent_byte(uint32_t h) { return (h >> 23) & 0xFFu; }

// Two results rounded to BF16 at once: x0's bits in the low half, x1's in the
// high half.  gfx950's v_cvt_pk_bf16_f32 rounds to nearest even exactly as
// float_to_bf16 does for every FP32 pattern that is not a NaN (checked over all
// 2^32 patterns on the device); a NaN becomes the canonical 0x7FFF, in a branch
// the whole wave skips unless one of its results is a NaN.
typedef float lct_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 lct_bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t round_pair_bf16(float x0, float x1) {
    const lct_f32x2 v = {x0, x1};
    uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, lct_bf16x2));
    const bool nan0 = __builtin_isnan(x0), nan1 = __builtin_isnan(x1);
    if (__builtin_expect(__any(nan0 || nan1), 0)) {
        r = nan0 ? ((r & 0xFFFF0000u) | 0x7FFFu) : r;
        r = nan1 ? ((r & 0x0000FFFFu) | 0x7FFF0000u) : r;
    }
    return r;
}

// Side byte of a high-half BF16 in bits 0..7 (higher bits are not meaningful).
__device__ __forceinline__ uint32_t high_side_byte(uint32_t h) {
    return __builtin_amdgcn_ubfe(h, 16, 7) | ((h >> 24) & 0x80u);
}

// Operation parameters of one launch; alpha/beta are device float32[1],
// read only where the flags say they are used.
__device__ __forceinline__ OpParams load_op_params(int32_t op, int32_t alpha_is_one,
                                                   int32_t beta_is_one, const float *alpha,
                                                   const float *beta) {
    OpParams p{op, alpha_is_one, beta_is_one, 1.0f, 1.0f};
    if (op == LCT_OP_SCALAR_MUL_ADD) {
        if (!alpha_is_one) p.alpha = alpha[0];
        if (!beta_is_one) p.beta = beta[0];
    }
    return p;
}

}  // namespace lct
