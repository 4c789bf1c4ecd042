// The Timestral block's elementwise stages, for gfx950:
//   - token assembly (TimestralKernels.assembleTokens, J/timestral/tornado/TimestralKernels.java,
//     queued in TimestralForward.java:329-331): each row's encoder tokens from the patch embedding,
//     then the horizon's decoder tokens, each the learned forecast query;
//   - SwiGLU (Kernels.swiGlu / swiGluHalf, J/tornado/Kernels.java:832-856; CPU CpuTimestral.java
//     165-172): act[t][j] = SiLU(up[t][j]) * up[t][f + j], in fp32, the storage-type variant
//     saturated to the type's finite range.
// Both are HBM-bound: the assembly copies 16 bytes per thread; SwiGLU reads 2 and writes 1 value per
// output in a grid-stride loop, 16 bytes of each per thread where the rows allow it.
#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "lp_common.hpp"

namespace jc {
namespace {

// x [(r*n + t)*d + j] = emb [(r*enc + t)*d + j] for t < enc, query[j] after
__global__ __launch_bounds__(256) void ts_assemble(const floatx4* __restrict__ emb, const floatx4* __restrict__ query,
                                                   floatx4* __restrict__ x, int rows, int enc, int n, int d4) {
    const uint64_t total = (uint64_t)rows * n * d4;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += stride) {
        const int j = (int)(id % d4);
        const uint64_t tok = id / d4;
        const int t = (int)(tok % n);
        const uint64_t r = tok / n;
        x[id] = t < enc ? emb[(r * enc + t) * d4 + j] : query[j];
    }
}

template <typename T>
__device__ __forceinline__ float ld(const T* p, uint64_t i) {
    return (float)p[i];
}

template <typename T>
__device__ __forceinline__ void st(T* p, uint64_t i, float v) {
    if constexpr (sizeof(T) == 4) {
        p[i] = v;
    } else {
        p[i] = (T)(v != v ? v : fminf(fmaxf(v, -lp::Enc<T>::kMax), lp::Enc<T>::kMax));
    }
}

// act [t*f + j] = g / (1 + exp(-g)) * u with g = up[t*2f + j], u = up[t*2f + f + j]
template <typename T>
__global__ __launch_bounds__(256) void swiglu(const T* __restrict__ up, T* __restrict__ act, uint64_t tokens, int f) {
    const uint64_t total = tokens * (uint64_t)f;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += stride) {
        const uint64_t t = id / (uint64_t)f;
        const uint64_t j = id - t * (uint64_t)f;
        const float g = ld(up, t * 2 * f + j), u = ld(up, t * 2 * f + f + j);
        st(act, id, g / (1.f + expf(-g)) * u);
    }
}

// the same per element, 16 bytes of each operand per thread (f a multiple of 16 / sizeof(T), both
// buffers 16-byte aligned): one 64-bit division per 4 or 8 outputs and 16-byte loads and stores
template <typename T>
__global__ __launch_bounds__(256) void swiglu_vec(const T* __restrict__ up, T* __restrict__ act, uint64_t tokens,
                                                  int f) {
    constexpr int V = 16 / sizeof(T);
    struct alignas(16) Vec {
        T x[V];
    };
    const uint64_t fv = (uint64_t)(f / V);
    const uint64_t total = tokens * fv;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += stride) {
        const uint64_t t = id / fv;
        const T* gp = up + t * 2 * (uint64_t)f + (id - t * fv) * V;
        const Vec gv = *reinterpret_cast<const Vec*>(gp);
        const Vec uv = *reinterpret_cast<const Vec*>(gp + f);
        Vec o;
#pragma unroll
        for (int k = 0; k < V; k++) {
            const float g = ld(gv.x, k), u = ld(uv.x, k);
            st(o.x, k, g / (1.f + expf(-g)) * u);
        }
        *reinterpret_cast<Vec*>(act + id * V) = o;
    }
}

// JC_F16X3: SwiGLU's fp32 result (swiglu_vec<float>'s expression) written as the A-operand split
// [hi | hi | lo] of the next GEMM, rows of 3f fp16, so no split pass follows. f a multiple of 4.
__global__ __launch_bounds__(256) void swiglu_x3(const float* __restrict__ up, _Float16* __restrict__ act3,
                                                 uint64_t tokens, int f) {
    const uint64_t fv = (uint64_t)(f / 4);
    const uint64_t total = tokens * fv;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += stride) {
        const uint64_t t = id / fv, j = (id - t * fv) * 4;
        const float* gp = up + t * 2 * (uint64_t)f + j;
        const floatx4 gv = *reinterpret_cast<const floatx4*>(gp);
        const floatx4 uv = *reinterpret_cast<const floatx4*>(gp + f);
        floatx4 o;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float g = gv[k], u = uv[k];
            o[k] = g / (1.f + expf(-g)) * u;
        }
        halfx4 hi, lo;
        split_f16x4(o, hi, lo);
        _Float16* row = act3 + t * 3 * (uint64_t)f;
        *reinterpret_cast<halfx4*>(row + j) = hi;
        *reinterpret_cast<halfx4*>(row + f + j) = hi;
        *reinterpret_cast<halfx4*>(row + 2 * (uint64_t)f + j) = lo;
    }
}

dim3 grid_for(uint64_t items) {
    const uint64_t blocks = (items + 255) / 256;
    return dim3((uint32_t)(blocks < 16384 ? (blocks ? blocks : 1) : 16384));
}

}  // namespace

hipError_t ts_assemble_launch(const float* emb, const float* query, float* x, int rows, int enc, int n, int d,
                              hipStream_t stream) {
    hipLaunchKernelGGL(ts_assemble, grid_for((uint64_t)rows * n * (d / 4)), dim3(256), 0, stream,
                       (const floatx4*)emb, (const floatx4*)query, (floatx4*)x, rows, enc, n, d / 4);
    return hipGetLastError();
}

hipError_t swiglu_launch(const void* up, void* act, uint64_t tokens, int f, int dtype_code, hipStream_t stream) {
    if (dtype_code == 3) {  // JC_F16X3: the caller checked f % 4 == 0 and the alignment
        hipLaunchKernelGGL(swiglu_x3, grid_for(tokens * (uint64_t)(f / 4)), dim3(256), 0, stream, (const float*)up,
                           (_Float16*)act, tokens, f);
        return hipGetLastError();
    }
    const int v = dtype_code == 0 ? 4 : 8;
    if (f % v == 0 && ((uintptr_t)up & 15u) == 0 && ((uintptr_t)act & 15u) == 0) {
        const dim3 g = grid_for(tokens * (uint64_t)(f / v));
        if (dtype_code == 0) {
            hipLaunchKernelGGL(swiglu_vec<float>, g, dim3(256), 0, stream, (const float*)up, (float*)act, tokens, f);
        } else if (dtype_code == 1) {
            hipLaunchKernelGGL(swiglu_vec<__bf16>, g, dim3(256), 0, stream, (const __bf16*)up, (__bf16*)act, tokens, f);
        } else {
            hipLaunchKernelGGL(swiglu_vec<_Float16>, g, dim3(256), 0, stream, (const _Float16*)up, (_Float16*)act,
                               tokens, f);
        }
        return hipGetLastError();
    }
    const dim3 grid = grid_for(tokens * (uint64_t)f);
    if (dtype_code == 0) {
        hipLaunchKernelGGL(swiglu<float>, grid, dim3(256), 0, stream, (const float*)up, (float*)act, tokens, f);
    } else if (dtype_code == 1) {
        hipLaunchKernelGGL(swiglu<__bf16>, grid, dim3(256), 0, stream, (const __bf16*)up, (__bf16*)act, tokens, f);
    } else {
        hipLaunchKernelGGL(swiglu<_Float16>, grid, dim3(256), 0, stream, (const _Float16*)up, (_Float16*)act, tokens, f);
    }
    return hipGetLastError();
}

}  // namespace jc
