// The attention output gate as a standalone pass: att[i] *= sigmoid(g[i]) (TimestralKernels.gate,
// TimestralKernels.java:572-578; oracle CpuTimestral.java:156-161). The time-attention kernels fuse
// the same gate into their epilogue; this entry point serves callers that gate another producer.
// Memory-bound: 8 bytes (fp32) or 4 bytes (bf16/fp16) read and 4 or 2 written per element; each
// thread handles 4 consecutive elements per grid-stride step.
#include "jc_common.hpp"
#include "jc_kernels.hpp"

namespace jc {
namespace {

__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + fast_exp2(-x * kLog2e)); }

template <typename T>
__global__ void gate_kernel(T* __restrict__ att, const T* __restrict__ g, uint64_t count) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * 4;
    for (uint64_t i = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < count; i += stride) {
        if (i + 4 <= count) {
            typedef T t4 __attribute__((ext_vector_type(4)));
            t4 a = *reinterpret_cast<const t4*>(att + i);
            const t4 b = *reinterpret_cast<const t4*>(g + i);
#pragma unroll
            for (int u = 0; u < 4; u++) a[u] = (T)((float)a[u] * sigmoid((float)b[u]));
            *reinterpret_cast<t4*>(att + i) = a;
        } else {
            for (uint64_t k = i; k < count; k++) att[k] = (T)((float)att[k] * sigmoid((float)g[k]));
        }
    }
}

template <typename T>
hipError_t launch(void* att, const void* g, uint64_t count, hipStream_t stream) {
    uint64_t blocks = (count / 4 + 255) / 256 + 1;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(gate_kernel<T>, dim3((uint32_t)blocks), dim3(256), 0, stream, (T*)att, (const T*)g, count);
    return hipGetLastError();
}

}  // namespace

hipError_t gate_launch(void* att, const void* g, uint64_t count, int dtype, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    switch (dtype) {
        case 0: return launch<float>(att, g, count, stream);
        case 1: return launch<__bf16>(att, g, count, stream);
        default: return launch<_Float16>(att, g, count, stream);
    }
}

}  // namespace jc
