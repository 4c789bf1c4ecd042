// The plain GEMMs on hipBLASLt (jc_blas.cpp): one engine per context.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace jc {

struct Blas;

enum BlasStatus { kBlasDone, kBlasDecline, kBlasError };

// A handle on the current device; nullptr when hipBLASLt cannot start.
Blas* blas_create();
void blas_destroy(Blas* b);

// C[m, n] (+)= act(A[m, :k] . W[n, :k]^T + bias[n]) (row-major; flags as Kernels.gemm's) on `stream`.
// kBlasDecline: a combination this path does not take (an activation with ACCUMULATE, fp16 output,
// no reproducible algorithm for the shape); the caller runs its own kernel. Same operands, same bits:
// only algorithms that run without a workspace are used, and none is given.
BlasStatus blas_gemm(Blas* b, const void* a, int lda, const void* w, const float* bias, void* c, int ldc, int m, int n,
                     int k, int flags, int ab_dtype, int c_dtype, hipStream_t stream);

}  // namespace jc
