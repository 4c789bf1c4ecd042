// The C++ caller of the ABI (include/jitcast_hip.h), beside the Java binding and the Python ctypes
// host: a program that links libjitcast_hip.so directly and checks, on the GPU, against the CPU
// oracle (oracle/jc_oracle.c, test infrastructure) on the same seeded inputs:
//   - the runtime: jc_init, jc_device_info, jc_alloc / jc_free, host and device copies, jc_sync;
//   - Chronos-2 time attention (fp32, RoPE table from jc_c2_rope_table; n = 129, so the row's last
//     query is the folded one) within 1e-4 (Chronos2Golden.java:218-234's metric);
//   - Chronos-2 group attention with groups of 3, 1 and 6 rows (jc_c2_group_bounds) within 1e-4;
//   - jc_linear with BIAS | RELU against the oracle's linear and relu within 1e-5;
//   - one plan: the time attention captured between jc_plan_begin and jc_plan_end, replayed, and
//     equal to the eager result bit for bit;
//   - error reporting: a bad head width returns JC_EINVAL with a message, jc_plan_end without a
//     capture returns JC_ESTATE.
// Prints one line per check and exits 0 only when all pass. Build: make -C tests/cxx.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "jc_oracle.h"
#include "jitcast_hip.h"

namespace {

int failures = 0;

void check(bool ok, const char* what, double err = 0.0) {
    std::printf("%-52s %s", what, ok ? "ok" : "FAILED");
    if (err > 0.0) std::printf("  (rel err %.3e)", err);
    std::printf("\n");
    if (!ok) failures++;
}

#define CALL(x)                                                                          \
    do {                                                                                 \
        int rc_ = (x);                                                                   \
        if (rc_ != JC_OK) {                                                              \
            std::printf("%s returned %d: %s\n", #x, rc_, jc_last_error());               \
            return 1;                                                                    \
        }                                                                                \
    } while (0)

// SplitMix64 (Steele, Lea, Flood 2014), 24-bit uniforms, Box-Muller normals: deterministic inputs
struct Rng {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return (double)(next() >> 40) / 16777216.0; }
    float normal() {
        const double u1 = uniform() + 1.0 / 33554432.0, u2 = uniform();
        return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
};

double rel_max_error(const float* got, const float* exp, size_t count) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < count; i++) {
        num = std::fmax(num, std::fabs((double)got[i] - (double)exp[i]));
        den = std::fmax(den, std::fabs((double)exp[i]));
    }
    return den > 0.0 ? num / den : num;
}

template <typename T>
T* upload(jc_ctx* ctx, const std::vector<T>& host) {
    void* d = nullptr;
    if (jc_alloc(ctx, host.size() * sizeof(T), &d) != JC_OK) return nullptr;
    if (jc_memcpy_h2d(ctx, d, host.data(), host.size() * sizeof(T)) != JC_OK) return nullptr;
    return static_cast<T*>(d);
}

}  // namespace

int main() {
    jc_ctx* ctx = nullptr;
    CALL(jc_init(0, &ctx));
    int cus = 0;
    char arch[64] = {0};
    CALL(jc_device_info(ctx, &cus, arch, sizeof arch));
    std::printf("device: %s, %d compute units, ABI %d\n", arch, cus, jc_version());

    // ---- Chronos-2 time attention, fp32 ---------------------------------------------------------
    const int rows = 3, n = 129, heads = 2, dh = 64, inner = 128;
    Rng rng{17};
    std::vector<float> qkv((size_t)rows * n * 3 * inner);
    for (float& x : qkv) x = rng.normal();
    std::vector<int32_t> live((size_t)rows * n, 1);
    for (int t = 0; t < 40; t++) live[(size_t)1 * n + t] = 0;                      // row 1: left padding
    for (int t = 0; t < n; t++) live[(size_t)2 * n + t] = rng.uniform() < 0.5 ? 1 : 0;  // row 2: random
    std::vector<float> table((size_t)n * dh);
    CALL(jc_c2_rope_table(n, dh, 10000.f, table.data()));
    float* d_qkv = upload(ctx, qkv);
    int32_t* d_live = upload(ctx, live);
    float* d_table = upload(ctx, table);
    void *d_out = nullptr, *d_out2 = nullptr;
    CALL(jc_alloc(ctx, (size_t)rows * n * inner * 4, &d_out));
    CALL(jc_alloc(ctx, (size_t)rows * n * inner * 4, &d_out2));
    if (!d_qkv || !d_live || !d_table) {
        std::printf("upload failed: %s\n", jc_last_error());
        return 1;
    }
    CALL(jc_c2_time_attention(ctx, d_qkv, d_out, d_live, d_table, rows, n, heads, dh, inner, JC_F32));
    std::vector<float> got((size_t)rows * n * inner), exp((size_t)rows * n * inner);
    CALL(jc_memcpy_d2h(ctx, got.data(), d_out, got.size() * 4));
    CALL(jc_sync(ctx));
    if (jco_c2_time_attention(qkv.data(), exp.data(), live.data(), rows, n, heads, dh, inner, 10000.f, 0) != 0) {
        std::printf("oracle failed\n");
        return 1;
    }
    const double e_time = rel_max_error(got.data(), exp.data(), got.size());
    check(e_time <= 1e-4, "c2 time attention fp32 (n = 129, RoPE)", e_time);

    // ---- the same launch as a plan --------------------------------------------------------------
    jc_plan* plan = nullptr;
    CALL(jc_plan_begin(ctx, 129));
    CALL(jc_c2_time_attention(ctx, d_qkv, d_out2, d_live, d_table, rows, n, heads, dh, inner, JC_F32));
    CALL(jc_plan_end(ctx, &plan));
    CALL(jc_plan_launch(plan));
    CALL(jc_sync(ctx));
    std::vector<float> replay(got.size());
    CALL(jc_memcpy_d2h(ctx, replay.data(), d_out2, replay.size() * 4));
    CALL(jc_sync(ctx));
    check(std::memcmp(replay.data(), got.data(), got.size() * 4) == 0 && jc_plan_key(plan) == 129,
          "plan replay equals the eager launch bit for bit");
    CALL(jc_plan_destroy(plan));

    // ---- Chronos-2 group attention, fp32 ---------------------------------------------------------
    const int grows = 10, gn = 5;
    std::vector<int32_t> group = {0, 0, 0, 1, 2, 2, 2, 2, 2, 2};
    std::vector<int32_t> gstart(grows), gend(grows);
    CALL(jc_c2_group_bounds(group.data(), grows, gstart.data(), gend.data()));
    std::vector<float> gqkv((size_t)grows * gn * 3 * inner);
    for (float& x : gqkv) x = rng.normal();
    std::vector<int32_t> glive((size_t)grows * gn, 1);
    glive[(size_t)4 * gn + 2] = 0;
    glive[(size_t)5 * gn + 2] = 0;
    float* d_gqkv = upload(ctx, gqkv);
    int32_t* d_glive = upload(ctx, glive);
    int32_t* d_gs = upload(ctx, gstart);
    int32_t* d_ge = upload(ctx, gend);
    void* d_gout = nullptr;
    CALL(jc_alloc(ctx, (size_t)grows * gn * inner * 4, &d_gout));
    CALL(jc_c2_group_attention(ctx, d_gqkv, d_gout, d_glive, d_gs, d_ge, grows, gn, heads, dh, inner, JC_F32));
    std::vector<float> ggot((size_t)grows * gn * inner), gexp(ggot.size());
    CALL(jc_memcpy_d2h(ctx, ggot.data(), d_gout, ggot.size() * 4));
    CALL(jc_sync(ctx));
    if (jco_c2_group_attention(gqkv.data(), gexp.data(), glive.data(), group.data(), grows, gn, heads, dh, inner, 0)) {
        std::printf("oracle failed\n");
        return 1;
    }
    const double e_group = rel_max_error(ggot.data(), gexp.data(), ggot.size());
    check(e_group <= 1e-4, "c2 group attention fp32 (groups of 3, 1, 6)", e_group);

    // ---- jc_linear: C = relu(A W^T + b) ----------------------------------------------------------
    const int m = 70, k = 64, nout = 48;
    std::vector<float> a((size_t)m * k), w((size_t)nout * k), b(nout), lexp((size_t)m * nout), lgot(lexp.size());
    for (float& x : a) x = rng.normal();
    for (float& x : w) x = 0.1f * rng.normal();
    for (float& x : b) x = rng.normal();
    float* d_a = upload(ctx, a);
    float* d_w = upload(ctx, w);
    float* d_b = upload(ctx, b);
    void* d_c = nullptr;
    CALL(jc_alloc(ctx, lexp.size() * 4, &d_c));
    CALL(jc_linear(ctx, d_a, k, d_w, d_b, static_cast<float*>(d_c), nout, m, nout, k, JC_GEMM_BIAS | JC_GEMM_RELU));
    CALL(jc_memcpy_d2h(ctx, lgot.data(), d_c, lgot.size() * 4));
    CALL(jc_sync(ctx));
    jco_linear(a.data(), m, w.data(), b.data(), k, nout, lexp.data(), 1);
    jco_relu(lexp.data(), (int64_t)lexp.size());
    const double e_lin = rel_max_error(lgot.data(), lexp.data(), lgot.size());
    check(e_lin <= 1e-5, "linear with bias and ReLU", e_lin);

    // ---- errors ----------------------------------------------------------------------------------
    const int bad = jc_c2_time_attention(ctx, d_qkv, d_out, d_live, d_table, rows, n, heads, 60, inner, JC_F32);
    check(bad == JC_EINVAL && std::strlen(jc_last_error()) > 0, "a head width of 60 is rejected with a message");
    jc_plan* none = nullptr;
    check(jc_plan_end(ctx, &none) == JC_ESTATE && none == nullptr, "plan_end without a capture is JC_ESTATE");

    for (void* p : {(void*)d_qkv, (void*)d_live, (void*)d_table, d_out, d_out2, (void*)d_gqkv, (void*)d_glive,
                    (void*)d_gs, (void*)d_ge, d_gout, (void*)d_a, (void*)d_w, (void*)d_b, d_c})
        CALL(jc_free(ctx, p));
    CALL(jc_destroy(ctx));
    std::printf("abi harness: %s\n", failures ? "FAILED" : "all checks passed");
    return failures ? 1 : 0;
}
