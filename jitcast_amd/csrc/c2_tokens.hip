// The token moves around the Chronos-2 encoder, for gfx950: assembling the context, [REG] and future
// tokens into the encoder input (Chronos2Kernels.assembleTokens, Chronos2Kernels.java:66-85) and
// gathering the future tokens for the output patch embedding (Chronos2Kernels.gatherFuture,
// Chronos2Kernels.java:684-694). Both are HBM-bound copies of d floats per token: one thread per
// 16 bytes, rows of d a multiple of 4.
#include "jc_common.hpp"
#include "jc_kernels.hpp"

namespace jc {
namespace {

// x [(r*n + t)*d + j]: emb [(r*ne + t)*d + j] for t < nc, reg[j] for nc <= t < nc + nreg, emb
// [(r*ne + t - nreg)*d + j] after, with ne = n - nreg
__global__ __launch_bounds__(256) void assemble_tokens(const floatx4* __restrict__ emb, const floatx4* __restrict__ reg,
                                                       floatx4* __restrict__ x, int rows, int nc, int nreg, int n, int d4) {
    const uint64_t total = (uint64_t)rows * n * d4;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const int ne = n - nreg;
    for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += stride) {
        const int j = (int)(id % d4);
        const uint64_t tok = id / d4;
        const int t = (int)(tok % n);
        const uint64_t r = tok / n;
        floatx4 v;
        if (t < nc) v = emb[(r * ne + t) * d4 + j];
        else if (t < nc + nreg) v = reg[j];
        else v = emb[(r * ne + t - nreg) * d4 + j];
        x[id] = v;
    }
}

// dec [(r*h + i)*d + j] = y [(r*n + fs + i)*d + j]
__global__ __launch_bounds__(256) void gather_future(const floatx4* __restrict__ y, floatx4* __restrict__ dec, int rows,
                                                     int fs, int n, int h, int d4) {
    const uint64_t total = (uint64_t)rows * h * d4;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += stride) {
        const int j = (int)(id % d4);
        const uint64_t tok = id / d4;
        const int i = (int)(tok % h);
        const uint64_t r = tok / h;
        dec[id] = y[(r * n + fs + i) * d4 + j];
    }
}

dim3 copy_grid(uint64_t items) {
    const uint64_t blocks = (items + 255) / 256;
    return dim3((uint32_t)(blocks < 16384 ? (blocks ? blocks : 1) : 16384));
}

}  // namespace

hipError_t assemble_tokens_launch(const float* emb, const float* reg, float* x, int rows, int nc, int nreg, int n, int d,
                                  hipStream_t stream) {
    hipLaunchKernelGGL(assemble_tokens, copy_grid((uint64_t)rows * n * (d / 4)), dim3(256), 0, stream,
                       (const floatx4*)emb, (const floatx4*)reg, (floatx4*)x, rows, nc, nreg, n, d / 4);
    return hipGetLastError();
}

hipError_t gather_future_launch(const float* y, float* dec, int rows, int fs, int n, int h, int d, hipStream_t stream) {
    hipLaunchKernelGGL(gather_future, copy_grid((uint64_t)rows * h * (d / 4)), dim3(256), 0, stream, (const floatx4*)y,
                       (floatx4*)dec, rows, fs, n, h, d / 4);
    return hipGetLastError();
}

}  // namespace jc
