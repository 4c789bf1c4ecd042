// The bf16 / fp16 kernels of the Chronos-2 encoder layer for gfx950: the GEMM with fp32
// accumulation (the reference's FP16 GEMM modes: Kernels.gemmHalf and GemmEx FP16->FP32,
// Kernels.java:115-232, Chronos2Forward.java:377-409, with Kernels.gemm's epilogue flags,
// Kernels.java:50-103), RMSNorm writing the storage-type twin of its output (Kernels.rmsNorm's
// `twin`, Kernels.java:800-829), and the fp32 -> storage-type conversion (Kernels.toHalf).
//
// GEMM: C[m, n] (+)= act(A[m, :k] . W[n, :k] + b[n]) with A and W in bf16 (or fp16), fp32 MFMA
// accumulation (v_mfma_f32_32x32x16_{bf16,f16}) and C either fp32 (any flags, ACCUMULATE included:
// the residual stream stays fp32) or the storage type (the next GEMM's or the attention's input).
// Storage-type outputs saturate to the type's finite range, as the reference's FP16 twins do
// (Kernels.java:42-46).
//
// Tiling (measured best of 128/256 x 128/256 x 32/64 on the layer's shapes): a 1024-thread
// workgroup owns a 256x256 tile of C; wave w owns the 64x64 block (w / 4, w % 4) as 2x2 MFMA tiles
// of 32x32. K advances 64 at a time through double-buffered LDS (A and W tiles of 256 rows x 64
// elements, rows padded to 72 elements so that 16-byte reads of consecutive rows hit distinct
// banks); the next stage's loads are in flight in registers during the current stage's 32 MFMAs
// per wave. MFMA layouts (32x32x16): A lane i+32g = A[i][8g..8g+7], B lane j+32g = B[8g..8g+7][j],
// D lane j+32g reg r = D[8(r/4) + 4g + r%4][j].
#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "lp_common.hpp"

namespace jc {
namespace {

using namespace lp;

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kPitch = kBK + 8;  // elements per staged row
constexpr int kWM = 4, kWN = 4;  // waves along M and N
constexpr int kThreads = kWM * kWN * kWave;
constexpr int kPieces = kBM * kBK / 8 / kThreads;  // 16-byte pieces per thread and operand

template <typename T>
struct LpTile {
    uint16_t a[2][kBM * kPitch];
    uint16_t w[2][kBN * kPitch];
};

// clamp to the storage type's finite range, keeping NaN (TornadoMath.clamp propagates it)
__device__ __forceinline__ float clamp_finite(float v, float m) { return v != v ? v : fminf(fmaxf(v, -m), m); }

template <typename T>
__device__ __forceinline__ T saturate(float v) {
    return (T)clamp_finite(v, Enc<T>::kMax);
}

template <typename T, bool OUT_LP>
__global__ __launch_bounds__(kThreads, 1) void gemm_lp(const GemmLpArgs g) {
    typedef typename Lp<T>::x8 x8;
    __shared__ LpTile<T> lds;
    const T* __restrict__ A = static_cast<const T*>(g.a);
    const T* __restrict__ W = static_cast<const T*>(g.w);
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int j = lane % 32, hg = lane / 32;
    const uint32_t nbn = (g.n + kBN - 1) / kBN;
    const uint32_t total = nbn * ((g.m + kBM - 1) / kBM);
    const uint32_t logical = xcd_remap(blockIdx.x, total);
    const int m0 = (logical / nbn) * kBM, n0 = (logical % nbn) * kBN;
    const int wm = wave / kWN, wn = wave % kWN;

    // staging: 2048 pieces per operand tile (row p / 8, k 8(p % 8)); k past g.k reads as zero
    u32x4 ra[kPieces], rw[kPieces];
    auto load = [&](int k0) {
#pragma unroll
        for (int u = 0; u < kPieces; u++) {
            const int p = tid + u * kThreads, r = p / (kBK / 8), kc = k0 + 8 * (p % (kBK / 8));
            const int ar = m0 + r, wr = n0 + r;
            ra[u] = ar < g.m && kc < g.k ? *reinterpret_cast<const u32x4*>(A + (size_t)ar * g.lda + kc) : u32x4{0u, 0u, 0u, 0u};
            rw[u] = wr < g.n && kc < g.k ? *reinterpret_cast<const u32x4*>(W + (size_t)wr * g.k + kc) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int u = 0; u < kPieces; u++) {
            const int p = tid + u * kThreads, r = p / (kBK / 8), kc = 8 * (p % (kBK / 8));
            *reinterpret_cast<u32x4*>(&lds.a[buf][r * kPitch + kc]) = ra[u];
            *reinterpret_cast<u32x4*>(&lds.w[buf][r * kPitch + kc]) = rw[u];
        }
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int ti = 0; ti < 2; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++) acc[ti][tj] = floatx16{0};

    const int stages = (g.k + kBK - 1) / kBK;
    load(0);
    store(0);
    __syncthreads();
    for (int st = 0; st < stages; st++) {
        const int buf = st & 1;
        if (st + 1 < stages) load((st + 1) * kBK);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; kk++) {
            x8 av[2], wv[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                av[t] = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(&lds.a[buf][(64 * wm + 32 * t + j) * kPitch + 16 * kk + 8 * hg]));
                wv[t] = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(&lds.w[buf][(64 * wn + 32 * t + j) * kPitch + 16 * kk + 8 * hg]));
            }
#pragma unroll
            for (int ti = 0; ti < 2; ti++)
#pragma unroll
                for (int tj = 0; tj < 2; tj++) acc[ti][tj] = Lp<T>::mfma(av[ti], wv[tj], acc[ti][tj]);
        }
        if (st + 1 < stages) store(buf ^ 1);
        __syncthreads();
    }

    // epilogue: reg r of lane (j, hg) in tile (ti, tj) is C[row 8(r/4) + 4hg + r%4][col j]; bias,
    // activation, accumulate, in Kernels.gemm's order
#pragma unroll
    for (int ti = 0; ti < 2; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            const int col = n0 + 64 * wn + 32 * tj + j;
            if (col >= g.n) continue;
            const float b = (g.flags & kGemmBias) ? g.bias[col] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + 64 * wm + 32 * ti + 8 * (r / 4) + 4 * hg + r % 4;
                if (row >= g.m) continue;
                float v = acc[ti][tj][r] + b;
                if (g.flags & kGemmSilu) v = v / (1.f + __expf(-v));
                if (g.flags & kGemmRelu) v = (v > 0.f || v != v) ? v : 0.f;
                const size_t ci = (size_t)row * g.ldc + col;
                if (OUT_LP) {
                    static_cast<T*>(g.c)[ci] = saturate<T>(v);
                } else {
                    float* c = static_cast<float*>(g.c);
                    if (g.flags & kGemmAccumulate) v += c[ci];
                    c[ci] = v;
                }
            }
        }
}

// y = twin(x * (1 / sqrt(mean(x^2) + eps)) * w), one wave per row, x fp32, y in the storage type
template <typename T>
__global__ __launch_bounds__(256) void rms_norm_lp(const float* __restrict__ x, T* __restrict__ y,
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
    const floatx4* wr = reinterpret_cast<const floatx4*>(w);
    T* yr = y + (size_t)row * d;
    for (int i = lane; i < d / 4; i += kWave) {
        const floatx4 v = xr[i] * inv * (w ? wr[i] : floatx4{1.f, 1.f, 1.f, 1.f});
        floatx4 s;
#pragma unroll
        for (int u = 0; u < 4; u++) s[u] = clamp_finite(v[u], Enc<T>::kMax);
        *reinterpret_cast<u32x2*>(yr + 4 * i) = narrow4<T>(s);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void to_lp(const float* __restrict__ x, T* __restrict__ y, uint64_t count) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride)
        y[i] = saturate<T>(x[i]);
}

}  // namespace

hipError_t gemm_lp_launch(const GemmLpArgs& g, bool fp16, bool out_lp, hipStream_t stream) {
    const uint64_t grid = (uint64_t)((g.m + kBM - 1) / kBM) * ((g.n + kBN - 1) / kBN);
    if (fp16) {
        if (out_lp) hipLaunchKernelGGL((gemm_lp<_Float16, true>), dim3((uint32_t)grid), dim3(kThreads), 0, stream, g);
        else hipLaunchKernelGGL((gemm_lp<_Float16, false>), dim3((uint32_t)grid), dim3(kThreads), 0, stream, g);
    } else {
        if (out_lp) hipLaunchKernelGGL((gemm_lp<__bf16, true>), dim3((uint32_t)grid), dim3(kThreads), 0, stream, g);
        else hipLaunchKernelGGL((gemm_lp<__bf16, false>), dim3((uint32_t)grid), dim3(kThreads), 0, stream, g);
    }
    return hipGetLastError();
}

hipError_t rms_norm_lp_launch(const float* x, void* y, const float* w, int rows, int d, float eps, bool fp16,
                              hipStream_t stream) {
    const dim3 grid((uint32_t)((rows + 3) / 4));
    if (fp16) hipLaunchKernelGGL(rms_norm_lp<_Float16>, grid, dim3(256), 0, stream, x, (_Float16*)y, w, rows, d, eps);
    else hipLaunchKernelGGL(rms_norm_lp<__bf16>, grid, dim3(256), 0, stream, x, (__bf16*)y, w, rows, d, eps);
    return hipGetLastError();
}

hipError_t to_lp_launch(const float* x, void* y, uint64_t count, bool fp16, hipStream_t stream) {
    const uint64_t blocks = count / 256 + 1;
    const dim3 grid((uint32_t)(blocks < 8192 ? blocks : 8192));
    if (fp16) hipLaunchKernelGGL(to_lp<_Float16>, grid, dim3(256), 0, stream, x, (_Float16*)y, count);
    else hipLaunchKernelGGL(to_lp<__bf16>, grid, dim3(256), 0, stream, x, (__bf16*)y, count);
    return hipGetLastError();
}

}  // namespace jc
