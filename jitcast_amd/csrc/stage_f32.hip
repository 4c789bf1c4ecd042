// The fp32 kernels around the attention cores in a Chronos-2 encoder layer, for gfx950: the GEMM
// with its epilogue flags and RMSNorm.
//
// GEMM: C[m, n] (+)= act(A[m, :] . W[n, :] + b[n]) with W in PyTorch's [out, in] layout, the
// contract of Kernels.gemm (Kernels.java:59-103): flags BIAS = 1, ACCUMULATE = 2, SILU = 4,
// RELU = 16 (Kernels.java:50-56), applied in the order bias, activation, accumulate. fp32 in and
// out with fp32 MFMA accumulation (v_mfma_f32_32x32x2_f32), so results stay within fp32 rounding
// of the oracle's double-accumulated Ops.Linear.apply (Ops.java:33-50).
//
// Tiling: a 256-thread workgroup owns a 128x128 tile of C; wave w owns the 64x64 quarter
// (w / 2, w % 2) as 2x2 MFMA tiles of 32x32 (64 accumulator VGPRs). K advances 16 at a time through
// a double-buffered LDS stage (A and W tiles, 128 rows x 16 floats each, rows padded to 20 floats
// so a wave's 16-byte reads of 16 consecutive rows hit 64 distinct banks); the next stage's global
// loads are in flight in registers while the current one is multiplied, with one barrier per stage.
// Within a stage, MFMA step s (0..7) contracts k = 8g + s in lane half g: the A and B operands of all
// 8 steps are then two 16-byte LDS reads per lane and tile (the contraction order is a permutation
// of k, the same for both operands).
//
// MFMA layouts (32x32x2 f32): A lane i+32g = A[i][g], B lane j+32g = B[g][j], D lane j+32g reg r =
// D[8(r/4) + 4g + r%4][j].
//
// Workgroups are ordered so that the ones sharing an A row block are adjacent and, through the XCD
// remap, run on the same XCD (the A block is read once per XCD L2; W is small and stays in the
// shared cache).
//
// RMSNorm: y = x * (1 / sqrt(mean(x^2) + eps)) * w per row of d (Kernels.rmsNorm,
// Kernels.java:800-829; oracle Ops.rmsNorm, Ops.java:53-68). One wave per row.
#include "jc_common.hpp"
#include "jc_kernels.hpp"

namespace jc {
namespace {

constexpr int kBM = 128, kBN = 128, kBK = 16;
constexpr int kPitch = kBK + 4;  // floats per staged row
constexpr int kThreads = 256;

struct GemmTile {
    float a[2][kBM * kPitch];
    float w[2][kBN * kPitch];
};

__device__ __forceinline__ float epilogue(float v, const GemmArgs& g, int row, int col) {
    if (g.flags & kGemmBias) v += g.bias[col];
    if (g.flags & kGemmSilu) v = v / (1.f + __expf(-v));
    // Math.max(v, 0f): NaN stays NaN
    if (g.flags & kGemmRelu) v = (v > 0.f || v != v) ? v : 0.f;
    const size_t ci = (size_t)row * g.ldc + col;
    if (g.flags & kGemmAccumulate) v += g.c[ci];
    return v;
}

__global__ __launch_bounds__(kThreads, 2) void gemm_f32(const GemmArgs g) {
    __shared__ GemmTile lds;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int j = lane % 32, hg = lane / 32;
    const uint32_t nbn = (g.n + kBN - 1) / kBN;
    const uint32_t total = nbn * ((g.m + kBM - 1) / kBM);
    const uint32_t logical = xcd_remap(blockIdx.x, total);
    const int m0 = (logical / nbn) * kBM, n0 = (logical % nbn) * kBN;
    const int wm = wave / 2, wn = wave % 2;

    // staging: 512 float4 pieces per operand tile (row p / 4, k 4(p % 4)), two per thread
    floatx4 ra[2], rw[2];
    auto load = [&](int k0) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int p = tid + u * kThreads, r = p / 4, kc = 4 * (p % 4);
            const int ar = m0 + r, wr = n0 + r;
            ra[u] = ar < g.m ? *reinterpret_cast<const floatx4*>(g.a + (size_t)ar * g.lda + k0 + kc) : floatx4{0.f, 0.f, 0.f, 0.f};
            rw[u] = wr < g.n ? *reinterpret_cast<const floatx4*>(g.w + (size_t)wr * g.k + k0 + kc) : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int p = tid + u * kThreads, r = p / 4, kc = 4 * (p % 4);
            *reinterpret_cast<floatx4*>(&lds.a[buf][r * kPitch + kc]) = ra[u];
            *reinterpret_cast<floatx4*>(&lds.w[buf][r * kPitch + kc]) = rw[u];
        }
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int ti = 0; ti < 2; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++) acc[ti][tj] = floatx16{0};

    const int stages = g.k / kBK;
    load(0);
    store(0);
    __syncthreads();
    for (int st = 0; st < stages; st++) {
        const int buf = st & 1;
        if (st + 1 < stages) load((st + 1) * kBK);
        // this stage's operands: 8 k values (8hg..8hg+7) of the lane's row in each tile
        floatx4 av[2][2], wv[2][2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float* ap = &lds.a[buf][(64 * wm + 32 * t + j) * kPitch + 8 * hg];
            const float* wp = &lds.w[buf][(64 * wn + 32 * t + j) * kPitch + 8 * hg];
            av[t][0] = *reinterpret_cast<const floatx4*>(ap);
            av[t][1] = *reinterpret_cast<const floatx4*>(ap + 4);
            wv[t][0] = *reinterpret_cast<const floatx4*>(wp);
            wv[t][1] = *reinterpret_cast<const floatx4*>(wp + 4);
        }
#pragma unroll
        for (int s = 0; s < 8; s++)
#pragma unroll
            for (int ti = 0; ti < 2; ti++)
#pragma unroll
                for (int tj = 0; tj < 2; tj++)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[ti][s / 4][s % 4], wv[tj][s / 4][s % 4],
                                                                       acc[ti][tj], 0, 0, 0);
        if (st + 1 < stages) store(buf ^ 1);
        __syncthreads();
    }

    // epilogue: reg r of lane (j, hg) in tile (ti, tj) is C[row 8(r/4) + 4hg + r%4][col j]
#pragma unroll
    for (int ti = 0; ti < 2; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            const int col = n0 + 64 * wn + 32 * tj + j;
            if (col >= g.n) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + 64 * wm + 32 * ti + 8 * (r / 4) + 4 * hg + r % 4;
                if (row < g.m) g.c[(size_t)row * g.ldc + col] = epilogue(acc[ti][tj][r], g, row, col);
            }
        }
}

// one wave per row; the sum of squares in fp32 lanes, combined across the wave
__global__ __launch_bounds__(256) void rms_norm_f32(const float* __restrict__ x, float* __restrict__ y,
                                                    const float* __restrict__ w, int rows, int d, float eps) {
    const int row = blockIdx.x * 4 + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (row >= rows) return;
    const floatx4* xr = reinterpret_cast<const floatx4*>(x + (size_t)row * d);
    float ss = 0.f;
    for (int i = lane; i < d / 4; i += kWave) {
        const floatx4 v = xr[i];
        ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float inv = 1.f / sqrtf(ss / d + eps);
    floatx4* yr = reinterpret_cast<floatx4*>(y + (size_t)row * d);
    const floatx4* wr = reinterpret_cast<const floatx4*>(w);
    for (int i = lane; i < d / 4; i += kWave) yr[i] = xr[i] * inv * (w ? wr[i] : floatx4{1.f, 1.f, 1.f, 1.f});
}

}  // namespace

hipError_t gemm_f32_launch(const GemmArgs& g, hipStream_t stream) {
    const uint64_t grid = (uint64_t)((g.m + kBM - 1) / kBM) * ((g.n + kBN - 1) / kBN);
    hipLaunchKernelGGL(gemm_f32, dim3((uint32_t)grid), dim3(kThreads), 0, stream, g);
    return hipGetLastError();
}

hipError_t rms_norm_f32_launch(const float* x, float* y, const float* w, int rows, int d, float eps, hipStream_t stream) {
    hipLaunchKernelGGL(rms_norm_f32, dim3((uint32_t)((rows + 3) / 4)), dim3(256), 0, stream, x, y, w, rows, d, eps);
    return hipGetLastError();
}

}  // namespace jc
