// Host-side statistics of Timestral's forecasting pipeline: the per-row scale of the observed
// context (Scaler.lastLocScale, J/timestral/Scaler.java:65-79) with the row's observed range for the
// cap bounds (TimestralPipeline._cap_quantiles, TimestralPipeline.java:378-395), and the advancing
// refine frames of a decoded block (Scaler.advancingFrames, Scaler.java:161-236). They run on every
// pass of the pipeline over the whole context, which for long contexts costs more host time than the
// rest of the pipeline; a sequential loop per row touches each value once.
//
// The arithmetic is the reference's double arithmetic in its order, with no contraction into FMAs
// (the pragma below), and max / min propagate NaN as the pipeline's array code does, so the results
// are bit-identical to it.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <thread>
#include <vector>

#include "../../include/jitcast_hip.h"

namespace jc {
int host_fail(int code, const char* fmt, ...);
}

namespace {

// max / min that return NaN when either operand is NaN
inline double nmax(double a, double b) { return (std::isnan(a) || a > b) ? a : b; }
inline double nmin(double a, double b) { return (std::isnan(a) || a < b) ? a : b; }
inline float nmaxf(float a, float b) { return (std::isnan(a) || a > b) ? a : b; }
inline float nminf(float a, float b) { return (std::isnan(a) || a < b) ? a : b; }

struct Welford {
    double w, mean, m2;
};

// welford_combine (Scaler.java:229-240): a then b; a state of weight 0 has mean and m2 0
inline Welford combine(const Welford& a, const Welford& b) {
#pragma clang fp contract(off)
    const double w = a.w + b.w;
    const double w_safe = nmax(w, std::numeric_limits<double>::min());
    const double delta = b.mean - a.mean;
    const double mean = a.mean + delta * b.w / w_safe;
    const double m2 = a.m2 + b.m2 + delta * delta * a.w * b.w / w_safe;
    if (w == 0) return {w, 0.0, 0.0};
    return {w, mean, m2};
}

// fn(r0, r1) over [0, rows) in contiguous ranges, on up to 16 host threads when there are at least
// 2^18 values to go through (rows are independent, so each row's arithmetic is unchanged)
template <class F>
void for_rows(int rows, int64_t per_row, F fn) {
    const int64_t total = (int64_t)rows * per_row;
    const int hw = (int)std::max(1u, std::thread::hardware_concurrency());
    const int nt = total < (1 << 18) ? 1 : std::min({rows, hw, 16});
    if (nt <= 1) {
        fn(0, rows);
        return;
    }
    std::vector<std::thread> pool;
    int started = 1;  // ranges 1..started-1 run on their own threads
    try {
        pool.reserve(nt - 1);
        for (; started < nt; started++)
            pool.emplace_back(fn, (int)((int64_t)rows * started / nt), (int)((int64_t)rows * (started + 1) / nt));
    } catch (...) {  // no more threads: the remaining ranges run on this one
    }
    fn(0, (int)((int64_t)rows / nt));
    for (int i = started; i < nt; i++) fn((int)((int64_t)rows * i / nt), (int)((int64_t)rows * (i + 1) / nt));
    for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

int jc_ts_context_stats(const float* x, const uint8_t* observed, int rows, int t, float minimum_scale, float* loc,
                        float* scale, float* lo, float* hi) {
#pragma clang fp contract(off)
    if (rows < 0 || t < 0 || (rows > 0 && t > 0 && (!x || !observed)))
        return jc::host_fail(JC_EINVAL, "jc_ts_context_stats: bad arguments (rows=%d t=%d)", rows, t);
    const double min_s = (double)minimum_scale;
    for_rows(rows, t, [&](int ra, int rb) {
#pragma clang fp contract(off)
    for (int r = ra; r < rb; r++) {
        const float* xr = x + (size_t)r * t;
        const uint8_t* mr = observed + (size_t)r * t;
        double cum_w = 0.0, cum_x = 0.0, m2 = 0.0, prev = 0.0, mean = 0.0;
        float mx = -std::numeric_limits<float>::infinity(), mn = std::numeric_limits<float>::infinity();
        for (int i = 0; i < t; i++) {
            const double w = mr[i] ? 1.0 : 0.0;
            const double xi = (double)xr[i];
            cum_w = cum_w + w;
            cum_x = cum_x + w * xi;
            mean = cum_x / (cum_w > 1.0 ? cum_w : 1.0);
            m2 = m2 + (xi - prev) * (xi - mean) * w;
            prev = mean;
            if (mr[i]) {
                mx = nmaxf(mx, xr[i]);
                mn = nminf(mn, xr[i]);
            }
        }
        const double cw = cum_w > 1.0 ? cum_w : 1.0;
        const double var = m2 / ((cw - 1.0) > 1.0 ? (cw - 1.0) : 1.0);
        if (loc) loc[r] = (float)mean;
        if (scale) scale[r] = (float)nmax(std::sqrt(var), min_s);
        if (hi) hi[r] = mx == -std::numeric_limits<float>::infinity() ? 0.0f : mx;
        if (lo) lo[r] = mn == std::numeric_limits<float>::infinity() ? 0.0f : mn;
    }
    });
    return JC_OK;
}

int jc_ts_advancing_frames(const float* context, const uint8_t* observed, const double* sinh_median, int rows, int t,
                           int patch, int n_pred, float minimum_scale, double* locs, double* scales) {
#pragma clang fp contract(off)
    if (rows < 0 || t < patch || patch < 1 || t % patch != 0 || n_pred < 0 ||
        (rows > 0 && n_pred > 0 && (!context || !observed || !sinh_median || !locs || !scales)))
        return jc::host_fail(JC_EINVAL, "jc_ts_advancing_frames: bad arguments (rows=%d t=%d patch=%d n_pred=%d)", rows,
                             t, patch, n_pred);
    const int n_ctx = t / patch;
    const int n = n_ctx + n_pred;
    const double clip = std::sqrt((double)std::numeric_limits<float>::max()) / 1e3;
    const double min_s = (double)minimum_scale;
    for_rows(rows, t, [&](int ra, int rb) {
#pragma clang fp contract(off)
    std::vector<Welford> st(n);
    std::vector<double> folded(patch);
    for (int r = ra; r < rb; r++) {
        const float* cr = context + (size_t)r * t;
        const uint8_t* mr = observed + (size_t)r * t;
        // each context patch's (count, mean, m2), summed in order within the patch
        for (int p = 0; p < n_ctx; p++) {
            double cnt = 0.0, s = 0.0;
            for (int i = 0; i < patch; i++) {
                const double w = mr[p * patch + i] ? 1.0 : 0.0;
                cnt = cnt + w;
                s = s + (double)cr[p * patch + i] * w;
            }
            const double mu = s / (cnt > 1.0 ? cnt : 1.0);
            double s2 = 0.0;
            for (int i = 0; i < patch; i++) {
                const double w = mr[p * patch + i] ? 1.0 : 0.0;
                const double dv = (double)cr[p * patch + i] - mu;
                s2 = s2 + w * (dv * dv);
            }
            st[p] = cnt == 0 ? Welford{cnt, 0.0, 0.0} : Welford{cnt, mu, s2};
        }
        for (int p = n_ctx; p < n; p++) st[p] = {0.0, 0.0, 0.0};
        // cumulative_welford: an inclusive Hillis-Steele scan; position k takes k - d's state of the
        // previous step (the zero state before the start), so k runs downwards in place
        for (int d = 1; d < n; d *= 2)
            for (int k = n - 1; k >= 0; k--) st[k] = combine(k >= d ? st[k - d] : Welford{0.0, 0.0, 0.0}, st[k]);
        Welford c = st[n_ctx - 1];
        const double offset = c.mean;
        const double* sm = sinh_median + (size_t)r * n_pred * patch;
        for (int h = 0; h < n_pred; h++) {
            const double var = nmax(c.m2 / nmax(c.w - 1.0, 1.0), 0.0);
            const double sc = nmax(std::sqrt(var), min_s);
            locs[(size_t)r * n_pred + h] = c.mean;
            scales[(size_t)r * n_pred + h] = sc;
            double tot = 0.0;
            for (int i = 0; i < patch; i++) {
                const double fv = nmax(-clip, nmin(clip, sm[h * patch + i] * sc + c.mean - offset));
                folded[i] = fv + offset;
                tot = tot + folded[i];
            }
            const double b_mean = tot / patch;
            double b_m2 = 0.0;
            for (int i = 0; i < patch; i++) {
                const double dv = folded[i] - b_mean;
                b_m2 = b_m2 + dv * dv;
            }
            c = combine(c, Welford{(double)patch, b_mean, b_m2});
        }
    }
    });
    return JC_OK;
}

}  // extern "C"
