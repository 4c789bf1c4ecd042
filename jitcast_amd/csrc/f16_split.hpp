// Three-term fp16 products for the fp32 group kernel (group_attention_f32.hip): an fp32 value as an
// fp16 pair (hi, lo), so a product runs as three fp16 MFMA products accumulated in fp32, and the
// range check that sends values fp16 cannot hold to fp32 MFMA.
#pragma once

#include "jc_common.hpp"
#include "lp_common.hpp"

namespace jc {

constexpr float kF16Max = 65504.f;  // fp16's largest finite value

// v - h for the low (HI = false) or high half h of a packed fp16 pair, exact in fp32 (one
// v_fma_mix_f32: v * 1 - h, rounded once)
template <bool HI>
__device__ __forceinline__ float sub_half(float v, uint32_t h) {
    float r;
    if constexpr (HI) {
        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(r) : "v"(v), "v"(h));
    } else {
        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel_hi:[0,0,1]" : "=v"(r) : "v"(v), "v"(h));
    }
    return r;
}
// v = hi + lo with hi = fp16(v) and lo = fp16(v - hi), both rounded to nearest, for |v| <= 65504:
// hi + lo is within 2^-22 |v| + 2^-25 of v (lo's rounding; where lo is subnormal its step 2^-24
// sets the absolute term). A product a.b becomes a_hi.b_hi + a_hi.b_lo + a_lo.b_hi, accumulated in
// fp32: fp16 products are exact in fp32, so each is within about 2^-20 |a.b| + 2^-25 (|a| + |b|).
__device__ __forceinline__ void split_f16(floatx4 v, halfx4& hi, halfx4& lo) {
    hi = __builtin_convertvector(v, halfx4);
    const lp::u32x2 h = __builtin_bit_cast(lp::u32x2, hi);
    const floatx4 r{sub_half<false>(v[0], h[0]), sub_half<true>(v[1], h[0]), sub_half<false>(v[2], h[1]),
                    sub_half<true>(v[3], h[1])};
    lo = __builtin_convertvector(r, halfx4);
}
__device__ __forceinline__ floatx4 v4(const float (&v)[4]) { return floatx4{v[0], v[1], v[2], v[3]}; }
// max(acc, |a|, |b|) in one v_max3_f32 (a NaN operand is ignored, as by fmaxf)
__device__ __forceinline__ float abs_max3(float acc, float a, float b) {
    float r;
    asm("v_max3_f32 %0, |%1|, |%2|, %3" : "=v"(r) : "v"(a), "v"(b), "v"(acc));
    return r;
}
__device__ __forceinline__ float abs_max4(float acc, floatx4 v) { return abs_max3(abs_max3(acc, v[0], v[1]), v[2], v[3]); }

}  // namespace jc
