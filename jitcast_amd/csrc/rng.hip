// The portable seeded RNG on the device (the numpy twin is jitcast_amd/rng.py): SplitMix64
// (Steele, Lea and Flood, OOPSLA 2014) output i >= 1 of stream s is mix(s + i*0x9E3779B97F4A7C15);
// a uniform is the top 24 bits * 2^-24; normals are Box-Muller pairs in double, rounded to float.
// Used to synthesise benchmark inputs in HBM without a host round trip.
#include "jc_common.hpp"
#include "jc_kernels.hpp"

namespace jc {
namespace {

__device__ __forceinline__ uint64_t splitmix(uint64_t s, uint64_t i) {
    uint64_t z = s + i * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ double unit(uint64_t s, uint64_t i) {
    return (double)(splitmix(s, i) >> 40) * (1.0 / 16777216.0);
}

__global__ void fill_normal(float* __restrict__ out, uint64_t count, uint64_t stream, double mean, double stdv) {
    uint64_t pairs = (count + 1) / 2;
    for (uint64_t p = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; p < pairs;
         p += (uint64_t)gridDim.x * blockDim.x) {
        double u1 = unit(stream, 2 * p + 1), u2 = unit(stream, 2 * p + 2);
        double rad = sqrt(-2.0 * log(1.0 - u1));
        double a = 2.0 * 3.141592653589793 * u2;
        out[2 * p] = (float)(mean + stdv * (rad * cos(a)));
        if (2 * p + 1 < count) out[2 * p + 1] = (float)(mean + stdv * (rad * sin(a)));
    }
}

__global__ void fill_uniform(float* __restrict__ out, uint64_t count, uint64_t stream, double lo, double hi) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < count;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = (float)(lo + (hi - lo) * unit(stream, i + 1));
}

}  // namespace

hipError_t fill_normal_launch(float* out, uint64_t count, uint64_t stream_seed, double mean, double stdv,
                              hipStream_t stream) {
    uint64_t pairs = (count + 1) / 2;
    uint64_t blocks = (pairs + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_normal, dim3((uint32_t)blocks), dim3(256), 0, stream, out, count, stream_seed, mean, stdv);
    return hipGetLastError();
}

hipError_t fill_uniform_launch(float* out, uint64_t count, uint64_t stream_seed, double lo, double hi,
                               hipStream_t stream) {
    uint64_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_uniform, dim3((uint32_t)blocks), dim3(256), 0, stream, out, count, stream_seed, lo, hi);
    return hipGetLastError();
}

}  // namespace jc
