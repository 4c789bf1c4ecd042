// Shared device helpers for the gfx950 attention kernels: MFMA operand types, wave-64 lane
// exchanges, the XCD-aware workgroup remap and the launch-error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jc {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: 8 accelerator complex dies, each with its own L2
constexpr float kLog2e = 1.4426950408889634f;

// v_permlane32_swap_b32 with both operands = v swaps the upper half of one copy with the lower
// half of the other: every lane ends up holding {its own v, lane (l ^ 32)'s v} across the two
// results (in an order that depends on the half). Symmetric reductions over a lane pair (l, l^32)
// therefore need no select.
__device__ __forceinline__ float pair_max(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float pair_sum(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 2^x on the hardware transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum over the four lanes j, j+16, j+32, j+48 (v_permlane16_swap then v_permlane32_swap)
__device__ __forceinline__ float quad_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    return pair_max(v);
}

__device__ __forceinline__ float quad_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    return pair_sum(v);
}

// The three-term fp16 split of fp32 operands (dtype JC_F16X3): hi = fp16(v) and lo = fp16(v - hi),
// each saturated to +-65504 as the FP16 GEMM mode's operands are (NaN kept).
__device__ __forceinline__ _Float16 f16_sat(float v) { return (_Float16)(v != v ? v : fminf(fmaxf(v, -65504.f), 65504.f)); }

__device__ __forceinline__ void split_f16x4(floatx4 v, halfx4& hi, halfx4& lo) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
        hi[u] = f16_sat(v[u]);
        lo[u] = f16_sat(v[u] - (float)hi[u]);
    }
}

// Dims e..e+3 of a row of `inner` values, stored as a GEMM A-operand split row of 3 * inner fp16
// values: [hi | hi | lo].
__device__ __forceinline__ void store_split_row(_Float16* row, int inner, int e, floatx4 v) {
    halfx4 hi, lo;
    split_f16x4(v, hi, lo);
    *reinterpret_cast<halfx4*>(row + e) = hi;
    *reinterpret_cast<halfx4*>(row + inner + e) = hi;
    *reinterpret_cast<halfx4*>(row + 2 * inner + e) = lo;
}

// Dims e..e+7 (lo4: e..e+3, hi4: e+4..e+7) as split pieces, three 16-byte stores.
__device__ __forceinline__ void store_split_row8(_Float16* row, int inner, int e, floatx4 lo4, floatx4 hi4) {
    halfx4 h0, l0, h1, l1;
    split_f16x4(lo4, h0, l0);
    split_f16x4(hi4, h1, l1);
    const halfx8 hi = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
    const halfx8 lo = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
    *reinterpret_cast<halfx8*>(row + e) = hi;
    *reinterpret_cast<halfx8*>(row + inner + e) = hi;
    *reinterpret_cast<halfx8*>(row + 2 * inner + e) = lo;
}

__device__ __forceinline__ void store_split_one(_Float16* row, int inner, int e, float v) {
    const _Float16 hi = f16_sat(v), lo = f16_sat(v - (float)hi);
    row[e] = hi;
    row[inner + e] = hi;
    row[2 * inner + e] = lo;
}

// Workgroups are dispatched round-robin over the XCDs (workgroup i runs on XCD i % 8). This remap
// gives each XCD one contiguous range of logical workgroup ids, so neighbouring logical ids (which
// the kernels arrange to share K/V tiles) meet in the same L2.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t total) {
    uint32_t per = total / kXcds, rem = total % kXcds;
    uint32_t xcd = bid % kXcds, slot = bid / kXcds;
    return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

}  // namespace jc
