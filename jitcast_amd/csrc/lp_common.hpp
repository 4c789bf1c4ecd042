// Shared pieces of the bf16 / fp16 attention kernels (time_attention_lp.hip,
// time_attention_lpw.hip): storage-type traits and conversions, the MFMA wrappers, the buffer
// resource, the V^T key permutation, and the encodings of the extra QK^T step that carries the key
// mask and the running max.
#pragma once

#include "jc_common.hpp"

namespace jc {
namespace lp {

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format (gfx9 family)

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Lp;
template <>
struct Lp<__bf16> {
    typedef bf16x8 x8;
    static __device__ __forceinline__ floatx16 mfma(x8 a, x8 b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Lp<_Float16> {
    typedef halfx8 x8;
    static __device__ __forceinline__ floatx16 mfma(x8 a, x8 b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

// 8 storage values <-> 8 floats (16 bytes <-> 2 float4); conversions round to nearest even
template <typename T>
__device__ __forceinline__ void widen8(u32x4 raw, floatx4& lo, floatx4& hi) {
    typedef T t8 __attribute__((ext_vector_type(8)));
    t8 v = __builtin_bit_cast(t8, raw);
#pragma unroll
    for (int u = 0; u < 4; u++) {
        lo[u] = (float)v[u];
        hi[u] = (float)v[4 + u];
    }
}

template <typename T>
__device__ __forceinline__ u32x4 narrow8(floatx4 lo, floatx4 hi) {
    typedef T t8 __attribute__((ext_vector_type(8)));
    t8 v;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        v[u] = (T)lo[u];
        v[4 + u] = (T)hi[u];
    }
    return __builtin_bit_cast(u32x4, v);
}

template <typename T>
__device__ __forceinline__ u32x2 narrow4(floatx4 x) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    t4 v;
#pragma unroll
    for (int u = 0; u < 4; u++) v[u] = (T)x[u];
    return __builtin_bit_cast(u32x2, v);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// Position of key `key` (a multiple of 4) of a block inside its V^T row: within each 16-key group,
// key 16c + 8a + 4g + u sits at 16c + 8g + 4a + u.
__device__ __forceinline__ int vt_pos(int key) { return (key & ~15) | ((key & 4) << 1) | ((key & 8) >> 1); }

// Encodings of the extra QK^T step (dims 0 and 1 of a 16-dim step, the rest zero):
//   K' = [bias_k, 1]     bias_k = 0 for a live key, kBigK for a dead one
//   Q' = [kBigQ, b_m]    b_m = -m: the query's reference max, rounded to T
// so the MFMA yields s - m for live keys and about -2^100 (bf16) or -2^25 (fp16) for dead ones.
template <typename T>
struct Enc;
template <>
struct Enc<__bf16> {
    static constexpr uint32_t kLive = 0x3F800000u;  // (0, 1.0)
    static constexpr uint32_t kDead = 0x3F80F180u;  // (-2^100, 1.0)
    static constexpr uint32_t kBigQ = 0x3F80u;      // 1.0
    static constexpr uint32_t kOnes = 0x3F803F80u;  // (1.0, 1.0)
    static constexpr float kMax = 3.0e38f;
    static __device__ __forceinline__ float dot2(uint32_t p, float acc) {
        typedef __bf16 t2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(t2, p), __builtin_bit_cast(t2, kOnes), acc, false);
    }
};
template <>
struct Enc<_Float16> {
    static constexpr uint32_t kLive = 0x3C000000u;  // (0, 1.0)
    static constexpr uint32_t kDead = 0x3C00F800u;  // (-32768, 1.0); times kBigQ = 1024: -2^25
    static constexpr uint32_t kBigQ = 0x6400u;      // 1024.0
    static constexpr uint32_t kOnes = 0x3C003C00u;
    static constexpr float kMax = 65504.f;
    static __device__ __forceinline__ float dot2(uint32_t p, float acc) {
        typedef _Float16 t2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(t2, p), __builtin_bit_cast(t2, kOnes), acc, false);
    }
};

template <typename T>
__device__ __forceinline__ uint32_t to_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (T)x);
}
template <typename T>
__device__ __forceinline__ float from_bits(uint32_t b) {
    return (float)__builtin_bit_cast(T, (uint16_t)b);
}

// Online softmax without a per-element max or subtraction on the common path: scores arrive
// already relative to the query's reference max m (the extra MFMA step), P = exp2(S) is rounded to
// T, and the block's row sum comes from v_dot2 over the packed P (the same rounded values the PV
// MFMA consumes). Only when some query's block sum leaves [2^-16, 2^16] (first block) or exceeds
// 2^16 (later blocks) does the wave take the slow path: the exact block max, a new reference
// rounded to T, P recomputed, and the O/l rescale. Bounding P by 2^16 keeps every sum finite.
constexpr float kSumHi = 65536.f;
constexpr float kSumLo = 1.0f / 65536.f;

// EXACT: the head is exactly DHP wide, so every head-width expression folds to a constant
}  // namespace lp
}  // namespace jc
