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

// Workgroups are dispatched round-robin over the XCDs (workgroup i runs on XCD i % 8). This remap
// gives each XCD one contiguous range of logical workgroup ids, so neighbouring logical ids (which
// the kernels arrange to share K/V tiles) meet in the same L2.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t total) {
    uint32_t per = total / kXcds, rem = total % kXcds;
    uint32_t xcd = bid % kXcds, slot = bid / kXcds;
    return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

}  // namespace jc
