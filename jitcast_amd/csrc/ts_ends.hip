// The host ends of a Timestral block, on gfx950, so a block moves only its window and the finished
// quantiles across PCIe:
//   BlockPrep.of (J/timestral/BlockPrep.java:40-75): per row the causal patch scaler
//     (Scaler.causalPatchLocScale, J/timestral/Scaler.java:40-64) or, for a known covariate row, the
//     whole-row statistics (Scaler.instanceNorm, Scaler.java:87-110); the scaled window
//     (Scaler.affine / asinh, Scaler.java:88-101) and the embedding input of every encoder token
//     [values, missing flags];
//   BlockPrep.finish (BlockPrep.java:77-101): Quantiles.apply's monotone fan-out
//     (J/timestral/Quantiles.java:52-77), Scaler.invert with the frame of the last context patch,
//     and Scaler.clampNonFinite (Scaler.java:118-130) over each step's quantiles.
// Every running sum keeps the reference's order: one wave walks a row 64 steps at a time, and the
// double sums that the reference accumulates step by step (cumX, M2, the instance sums) are chained
// lane by lane in step order, so they round exactly as the sequential loops do. The divisions,
// square roots and the per-step work run on all lanes at once. Float arithmetic stays float, max and
// clamp propagate NaN as Java's Math.max / Math.min do, and nothing is contracted into fused
// multiply-adds (the pragma below). Only the last bit of the double log / sqrt / sinh / exp / log1p
// of the device's math library can differ from the JDK's, which the rounding to float almost always
// hides.
#include "jc_common.hpp"
#include "jc_kernels.hpp"

#pragma clang fp contract(off)

namespace jc {
namespace {

// Java's Math.max / Math.min: NaN if either operand is NaN, and +0 above -0
__device__ __forceinline__ double jmax(double a, double b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == 0.0 && b == 0.0) return signbit(a) ? b : a;
    return a >= b ? a : b;
}
__device__ __forceinline__ float jmaxf(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == 0.f && b == 0.f) return signbit(a) ? b : a;
    return a >= b ? a : b;
}
__device__ __forceinline__ float jminf(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == 0.f && b == 0.f) return signbit(a) ? a : b;
    return a <= b ? a : b;
}
__device__ __forceinline__ float jclampf(float v) {
    // Math.max(-Float.MAX_VALUE, Math.min(Float.MAX_VALUE, v))
    const float big = 3.40282347e38f;
    return v != v ? v : v > big ? big : v < -big ? -big : v;
}

__device__ __forceinline__ double lane_value(double v, int k) {
    const int64_t b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(uint32_t)b, k);
    const int hi = __builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), k);
    return __longlong_as_double(((int64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// The running total after each lane's step, with the steps taken in lane order: carry + v[0] + v[1]
// + ... one double add at a time, as the reference's loop adds them. Lanes whose `take` is false
// add nothing. carry becomes the total over the wave.
__device__ __forceinline__ double seq_prefix(double v, bool take, double& carry) {
    const uint64_t m = __ballot(take);
    const int lane = threadIdx.x % kWave;
    double acc = carry, mine = 0.0;
#pragma unroll
    for (int k = 0; k < kWave; k++) {
        const double s = lane_value(v, k);
        if ((m >> k) & 1) acc += s;
        if (lane == k) mine = acc;
    }
    carry = acc;
    return mine;
}

// Two independent running totals of seq_prefix in one pass over the lanes, so the two chains of
// dependent adds overlap; each keeps its own step order and rounding.
__device__ __forceinline__ void seq_prefix2(double va, bool ta, double& ca, double& pa, double vb, bool tb,
                                            double& cb, double& pb) {
    const uint64_t ma = __ballot(ta), mb = __ballot(tb);
    const int lane = threadIdx.x % kWave;
    double acc_a = ca, acc_b = cb;
    pa = 0.0;
    pb = 0.0;
#pragma unroll
    for (int k = 0; k < kWave; k++) {
        const double sa = lane_value(va, k), sb = lane_value(vb, k);
        if ((ma >> k) & 1) acc_a += sa;
        if ((mb >> k) & 1) acc_b += sb;
        if (lane == k) {
            pa = acc_a;
            pb = acc_b;
        }
    }
    ca = acc_a;
    cb = acc_b;
}

__device__ __forceinline__ float ts_asinh(float v) {
    const double a = fabs((double)v);
    const double r = log(a + sqrt(a * a + 1.0));
    return (float)(v < 0.f ? -r : r);
}

// Scaler.affine: asinh((x - loc) / max(scale, FLOAT32_EPS)) on an observed step, 0 elsewhere
__device__ __forceinline__ float affine(float x, float loc, float scale, bool obs, bool asinh) {
    if (!obs) return 0.f;
    const float v = (x - loc) / jmaxf(scale, 1.1920929e-7f);
    return asinh ? ts_asinh(v) : v;
}

struct PrepArgs {
    const float* window;
    const uint8_t* observed;
    const int32_t* known;
    float* tok;
    float* scaled;
    float* loc;
    float* scale;
    int w, patch, chunk, use_asinh;
    float minimum_scale;
};

__device__ __forceinline__ void store_step(const PrepArgs& a, int row, int i, float x, bool ob, float l, float s,
                                           bool asinh) {
    const int64_t o = (int64_t)row * a.w + i;
    const float v = affine(x, l, s, ob, asinh);
    a.loc[o] = l;
    a.scale[o] = s;
    if (a.scaled) a.scaled[o] = v;
    const int p = i / a.patch, st = i % a.patch;
    float* t = a.tok + ((int64_t)row * (a.w / a.patch) + p) * 2 * a.patch;
    t[st] = v;
    t[a.patch + st] = ob ? 0.f : 1.f;
}

// one wave per row; a chunk is the largest whole number of patches that fits 64 lanes, so a
// patch's loc and scale come from a lane of the same chunk
__global__ __launch_bounds__(kWave) void ts_prep_kernel(const PrepArgs a) {
    const int row = blockIdx.x, lane = threadIdx.x;
    const float* x = a.window + (int64_t)row * a.w;
    const uint8_t* obs = a.observed + (int64_t)row * a.w;
    const bool known = a.known && a.known[row] != 0;
    const uint64_t le = lane == kWave - 1 ? ~0ull : (2ull << lane) - 1;  // lanes 0..lane

    if (known) {
        // Scaler.instanceNorm: n, the sum of the observed values in step order, the 0/1 test
        double n = 0.0, sum = 0.0;
        bool zero_one = true, any = false;
        for (int base = 0; base < a.w; base += kWave) {
            const int i = base + lane;
            const bool act = i < a.w;
            const float xf = act ? x[i] : 0.f;
            const bool ob = act && obs[i] != 0;
            const uint64_t om = __ballot(ob);
            n += (double)__popcll(om);
            any |= om != 0;
            zero_one &= __ballot(act && !(xf == 0.f || xf == 1.f || !ob)) == 0;
            seq_prefix((double)xf, ob, sum);
        }
        n = jmax(n, 1.0);
        const float loc = (float)(sum / n);
        double ss = 0.0;
        for (int base = 0; base < a.w; base += kWave) {
            const int i = base + lane;
            const bool act = i < a.w;
            const float xf = act ? x[i] : 0.f;
            const float d = (act && obs[i] != 0) ? xf - loc : 0.f;
            seq_prefix((double)d * d, act, ss);
        }
        const float scale = jmaxf((float)sqrt((double)(float)(ss / n)), a.minimum_scale);
        const bool binary = zero_one && any;
        const float l = binary ? 0.f : loc, s = binary ? 1.f : scale;
        const bool asinh = a.use_asinh && !binary;
        for (int i = lane; i < a.w; i += kWave) store_step(a, row, i, x[i], obs[i] != 0, l, s, asinh);
        return;
    }

    // Scaler.causalPatchLocScale: running weighted mean and Welford M2 in double. Chunk c + 1's cumX
    // chain runs in the same pass as chunk c's M2 chain (it needs only chunk c's total).
    const double ms = (double)a.minimum_scale;
    double cw = 0.0, cx = 0.0, m2 = 0.0, prev = 0.0;
    struct Chunk {
        float xf;
        bool ob, act;
        double xi, wv, cum_w, cum_x;
    };
    auto load = [&](int base, Chunk& c) {
        const int i = base + lane;
        c.act = lane < a.chunk && i < a.w;
        c.xf = c.act ? x[i] : 0.f;
        c.ob = c.act && obs[i] != 0;
        c.xi = (double)c.xf;
        c.wv = c.ob ? 1.0 : 0.0;
        const uint64_t om = __ballot(c.ob);
        c.cum_w = cw + (double)__popcll(om & le);  // counts: exact in any order
        cw += (double)__popcll(om);
    };
    Chunk cur, nxt;
    load(0, cur);
    cur.cum_x = seq_prefix(cur.wv * cur.xi, cur.act, cx);
    for (int base = 0; base < a.w; base += a.chunk) {
        const bool more = base + a.chunk < a.w;  // uniform across the wave
        if (more) load(base + a.chunk, nxt);
        const double mean = cur.cum_x / jmax(cur.cum_w, 1.0);
        const double before = __shfl(mean, lane == 0 ? 0 : lane - 1);
        const double pm = lane == 0 ? prev : before;
        const double term = (cur.xi - pm) * (cur.xi - mean) * cur.wv;
        double m2_i;
        if (more) {
            seq_prefix2(nxt.wv * nxt.xi, nxt.act, cx, nxt.cum_x, term, cur.act, m2, m2_i);
        } else {
            m2_i = seq_prefix(term, cur.act, m2);
        }
        prev = __shfl(mean, a.chunk - 1);
        // at a patch's last step: loc = mean, scale = max(sqrt(M2 / max(max(cumW, 1) - 1, 1)), min)
        const double var = m2_i / jmax(jmax(cur.cum_w, 1.0) - 1.0, 1.0);
        const float pl = (float)mean, ps = (float)jmax(sqrt(var), ms);
        const int last = (lane / a.patch) * a.patch + a.patch - 1;
        const float l = __shfl(pl, last), sc = __shfl(ps, last);
        if (cur.act) store_step(a, row, base + lane, cur.xf, cur.ob, l, sc, a.use_asinh != 0);
        cur = nxt;
    }
}

struct FinishArgs {
    const float* raw;
    const float* loc;
    const float* scale;
    float* out;
    int rows, w, anchor, steps, q, median, use_asinh;
    float width[kTsMaxQuantiles];
};

__device__ __forceinline__ float softplus(float x) {
    // torch's softplus: x above 20, else log1p(exp(x)) (in double, rounded to float)
    return x > 20.f ? x : (float)log1p(exp((double)x));
}

// one thread per (row, forecast step): its q raw values in, its q quantiles out (in place allowed)
__global__ __launch_bounds__(256) void ts_finish_kernel(const FinishArgs a) {
    const int64_t total = (int64_t)a.rows * a.steps;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += stride) {
        const int row = (int)(id / a.steps);
        const float* r = a.raw + id * a.q;
        float* o = a.out + id * a.q;
        // Quantiles.apply: each level's increment is read before that level is written
        const float m = r[a.median];
        float up = 0.f;
        for (int i = a.median + 1; i < a.q; i++) {
            up += a.width[i] * softplus(r[i]);
            o[i] = jclampf(m + up);
        }
        float down = 0.f;
        for (int i = a.median - 1; i >= 0; i--) {
            down += a.width[i] * softplus(r[i]);
            o[i] = jclampf(m - down);
        }
        o[a.median] = jclampf(m);
        // Scaler.invert with the last context patch's frame, then clampNonFinite over the q values
        const int64_t an = (int64_t)row * a.w + a.anchor;
        const float l = a.loc[an], s = a.scale[an];
        float hi = -INFINITY, lo = INFINITY;
        for (int k = 0; k < a.q; k++) {
            const float v = a.use_asinh ? (float)sinh((double)o[k]) : o[k];
            const float y = v * s + l;
            o[k] = y;
            if (isfinite(y)) {
                hi = jmaxf(hi, y);
                lo = jminf(lo, y);
            }
        }
        for (int k = 0; k < a.q; k++) {
            const float y = o[k];
            const float z = y == INFINITY ? hi : y == -INFINITY ? lo : y;
            o[k] = isinf(z) ? 0.f : z;
        }
    }
}

}  // namespace

hipError_t ts_prep_launch(const float* window, const uint8_t* observed, int rows, int w, int patch,
                          const int32_t* known, float minimum_scale, int use_asinh, float* tok, float* scaled,
                          float* loc, float* scale, hipStream_t stream) {
    if (rows == 0 || w == 0) return hipSuccess;
    const PrepArgs a{window, observed, known, tok, scaled, loc, scale, w, patch, (kWave / patch) * patch,
                     use_asinh, minimum_scale};
    hipLaunchKernelGGL(ts_prep_kernel, dim3((uint32_t)rows), dim3(kWave), 0, stream, a);
    return hipGetLastError();
}

hipError_t ts_finish_launch(const float* raw, const float* loc, const float* scale, int rows, int w, int anchor,
                            int steps, int q, const float* width, int median, int use_asinh, float* out,
                            hipStream_t stream) {
    const int64_t total = (int64_t)rows * steps;
    if (total == 0) return hipSuccess;
    FinishArgs a{raw, loc, scale, out, rows, w, anchor, steps, q, median, use_asinh, {}};
    for (int k = 0; k < q; k++) a.width[k] = width[k];
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(ts_finish_kernel, dim3((uint32_t)(blocks < 16384 ? blocks : 16384)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace jc
