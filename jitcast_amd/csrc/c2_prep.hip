// The host ends of the Chronos-2 forward, on gfx950, so a forecast moves only the raw series and
// the finished quantiles across PCIe:
//   ModelLayout.of (J/chronos2/ModelLayout.java:70-116): the most recent context_length steps of a
//     row, NaN-padded on the left to whole patches; the live mask (a context patch with at least
//     one observed value; [REG] and the future tokens always live);
//   ModelPrep.of and instanceNorm / scaled / asinh (J/chronos2/ModelPrep.java:38-115): per row the
//     mean and population std of the observed values in double, rounded to float (a zero std
//     floored at 1e-5, (0, 1) for a row with none), and the patch tokens (time encoding,
//     arcsinh((x - loc) / scale) or 0, observed flag);
//   ModelPrep.finish (J/chronos2/ModelPrep.java:117-143): sinh(raw) * scale + loc, quantiles
//     level-major per token -> [rows][Q][h*P].
// Each operation rounds as the reference's does: float arithmetic where it uses float, double
// where it uses double, and no contraction into fused multiply-adds (the pragma below), so only
// the order of the double sums (a tree here, sequential in the reference) and the last bit of the
// double log / sqrt / sinh can differ.
// An optional row order gathers the input rows into the encoder's order (prep) and scatters the
// forecasts back (finish); its entries are clamped into range, so no index reaches past a buffer.
#include "jc_common.hpp"
#include "jc_kernels.hpp"

#pragma clang fp contract(off)

namespace jc {
namespace {

constexpr int kPrepThreads = 256;

__device__ __forceinline__ float c2_scaled(float x, float loc, float scale, bool arcsinh) {
    const float v = (x - loc) / scale;
    if (!arcsinh) return v;
    const double a = fabs((double)v);
    const double r = log(a + sqrt(a * a + 1.0));
    return (float)(v < 0.f ? -r : r);
}

template <typename V>
__device__ __forceinline__ V block_sum(V v, V* red) {
    // wave sums through the lane shuffle, then the 4 wave partials through LDS
    for (int o = kWave / 2; o > 0; o /= 2) v += __shfl_xor(v, o);
    const int wv = threadIdx.x / kWave, ln = threadIdx.x % kWave;
    if (ln == 0) red[wv] = v;
    __syncthreads();
    V t = 0;
    for (int w = 0; w < kPrepThreads / kWave; w++) t += red[w];
    __syncthreads();
    return t;
}

// one workgroup per output row i (input row order[i])
__global__ __launch_bounds__(kPrepThreads) void c2_prep_kernel(const float* __restrict__ ctx, int64_t ld_ctx, int steps,
                                                               const float* __restrict__ fut, int64_t ld_fut,
                                                               int fut_steps, const int32_t* __restrict__ order,
                                                               int rows, int kept, int nc, int h, int patch, int nreg,
                                                               float time_scale, int arcsinh, float* __restrict__ tok,
                                                               float* __restrict__ loc_out, float* __restrict__ scale_out,
                                                               int32_t* __restrict__ live) {
    __shared__ double red_d[kPrepThreads / kWave];
    __shared__ int red_i[kPrepThreads / kWave];
    const int i = blockIdx.x;
    const int src = order ? min(max(order[i], 0), rows - 1) : i;
    const int padded = nc * patch, lead = padded - kept;  // window[u] = u < lead ? NaN : crow[u - lead]
    const float* crow = ctx + (int64_t)src * ld_ctx + (steps - kept);
    const int tid = threadIdx.x;

    // instanceNorm: the observed values' sum and count, then the squared deviations, in double
    double sum = 0.0;
    int cnt = 0;
    for (int u = tid; u < kept; u += kPrepThreads) {
        const float v = crow[u];
        if (!isnan(v)) {
            sum += (double)v;
            cnt++;
        }
    }
    sum = block_sum(sum, red_d);
    cnt = block_sum(cnt, red_i);
    const float loc = cnt ? (float)(sum / cnt) : 0.f;
    double ss = 0.0;
    for (int u = tid; u < kept; u += kPrepThreads) {
        const float v = crow[u];
        if (!isnan(v)) {
            const float d = v - loc;
            ss += (double)d * (double)d;
        }
    }
    ss = block_sum(ss, red_d);
    float scale = 1.f;
    if (cnt) {
        scale = (float)sqrt(ss / cnt);
        if (scale == 0.f) scale = 1e-5f;
    }
    if (tid == 0) {
        loc_out[i] = loc;
        scale_out[i] = scale;
    }

    // tokens [(i*(nc+h) + p)*3P + {s, P + s, 2P + s}]: time encoding, scaled value or 0, observed
    const int ne = nc + h, w3 = 3 * patch;
    for (int u = tid; u < padded; u += kPrepThreads) {
        const int p = u / patch, s = u % patch;
        const float v = u < lead ? __builtin_nanf("") : crow[u - lead];
        const bool obs = !isnan(v);
        float* o = tok + ((int64_t)i * ne + p) * w3;
        o[s] = (float)(u - padded) / time_scale;
        o[patch + s] = obs ? c2_scaled(v, loc, scale, arcsinh != 0) : 0.f;
        o[2 * patch + s] = obs ? 1.f : 0.f;
    }
    const float* frow = fut ? fut + (int64_t)src * ld_fut : nullptr;
    for (int u = tid; u < h * patch; u += kPrepThreads) {
        const int p = u / patch, s = u % patch;
        const float v = (frow && u < fut_steps) ? frow[u] : __builtin_nanf("");
        const bool obs = !isnan(v);
        float* o = tok + ((int64_t)i * ne + nc + p) * w3;
        o[s] = (float)u / time_scale;
        o[patch + s] = obs ? c2_scaled(v, loc, scale, arcsinh != 0) : 0.f;
        o[2 * patch + s] = obs ? 1.f : 0.f;
    }

    // live [i*n + t]: a context patch with an observed value; [REG] and the future tokens always
    const int n = nc + nreg + h;
    for (int p = tid; p < n; p += kPrepThreads) {
        int lv = 1;
        if (p < nc) {
            lv = 0;
            for (int s = 0; s < patch; s++) {
                const int u = p * patch + s;
                if (u >= lead && !isnan(crow[u - lead])) {
                    lv = 1;
                    break;
                }
            }
        }
        live[(int64_t)i * n + p] = lv;
    }
}

// out [dst][k][p*P + s] = sinh(raw[(i*h + p)*Q*P + k*P + s]) * scale[i] + loc[i], dst = order[i]
__global__ __launch_bounds__(256) void c2_finish_kernel(const float* __restrict__ raw, const float* __restrict__ loc,
                                                        const float* __restrict__ scale,
                                                        const int32_t* __restrict__ order, int rows, int h, int q,
                                                        int patch, int arcsinh, float* __restrict__ out) {
    const int64_t per_row = (int64_t)h * q * patch;
    const int64_t total = (int64_t)rows * per_row;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += stride) {
        const int i = (int)(id / per_row);
        const int64_t r = id % per_row;  // (p*Q + k)*P + s: raw's order within the row
        const int s = (int)(r % patch);
        const int k = (int)((r / patch) % q);
        const int p = (int)(r / ((int64_t)patch * q));
        float v = raw[id];
        if (arcsinh) v = (float)sinh((double)v);
        const int dst = order ? min(max(order[i], 0), rows - 1) : i;
        out[(int64_t)dst * per_row + (int64_t)k * h * patch + (int64_t)p * patch + s] = v * scale[i] + loc[i];
    }
}

}  // namespace

hipError_t c2_prep_launch(const float* ctx, int64_t ld_ctx, int steps, const float* fut, int64_t ld_fut, int fut_steps,
                          const int32_t* order, int rows, int kept, int nc, int h, int patch, int nreg, float time_scale,
                          int arcsinh, float* tok, float* loc, float* scale, int32_t* live, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(c2_prep_kernel, dim3((uint32_t)rows), dim3(kPrepThreads), 0, stream, ctx, ld_ctx, steps, fut,
                       ld_fut, fut_steps, order, rows, kept, nc, h, patch, nreg, time_scale, arcsinh, tok, loc, scale,
                       live);
    return hipGetLastError();
}

hipError_t c2_finish_launch(const float* raw, const float* loc, const float* scale, const int32_t* order, int rows,
                            int h, int q, int patch, int arcsinh, float* out, hipStream_t stream) {
    const int64_t total = (int64_t)rows * h * q * patch;
    if (total == 0) return hipSuccess;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(c2_finish_kernel, dim3((uint32_t)(blocks < 16384 ? blocks : 16384)), dim3(256), 0, stream, raw, loc,
                       scale, order, rows, h, q, patch, arcsinh, out);
    return hipGetLastError();
}

}  // namespace jc
