// The C ABI of libjitcast_hip (include/jitcast_hip.h): argument checks, error capture and the
// runtime helpers. Every entry point returns a jc_status and records a message; no exception or
// abort crosses the boundary.
#include "../../include/jitcast_hip.h"

#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <new>
#include <vector>

#include "jc_blas.hpp"
#include "jc_kernels.hpp"

struct jc_ctx {
    int device;
    hipStream_t own;     // created by jc_init
    hipStream_t stream;  // where launches go (own, or a caller's)
    int cus;
    char arch[64];
    bool capturing;          // between jc_plan_begin and jc_plan_end
    hipStream_t capture_on;  // the stream being captured
    uint64_t capture_key;
    jc::Blas* blas;          // hipBLASLt for the plain GEMMs (nullptr: the library's own kernels)
    std::vector<struct jc_prof_record>* prof;  // per-kernel timing (jc_profile), nullptr when off
    // the group kernel's tile order (kGroupOrderTiles entries): eager calls fill `order` behind the
    // last group kernel that read it (`order_read`, recorded on whichever stream that ran); a plan
    // being captured fills its own buffer, `capture_order`, which the plan keeps
    int32_t* order;
    hipEvent_t order_read;
    int32_t* capture_order;
};

// One timed launch: HIP events on the context's stream before and after it.
struct jc_prof_record {
    const char* name;
    hipEvent_t a, b;
};

struct jc_plan {
    jc_ctx* ctx;
    hipGraph_t graph;
    hipGraphExec_t exec;
    uint64_t key;
    std::vector<std::pair<void*, size_t>> owned;  // device buffers adopted by the plan
    hipEvent_t done = nullptr;                    // recorded behind every replay, on its stream
    int32_t* order = nullptr;                     // the group kernels' tile order (64 KB), the plan's own
};

namespace {

thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(const char* where, hipError_t e) {
    return fail(JC_EHIP, "%s: %s (%d)", where, hipGetErrorString(e), (int)e);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Makes the context's device current for this thread.
int use(jc_ctx* ctx, const char* where) {
    if (!ctx) return fail(JC_EINVAL, "%s: null context", where);
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail(where, e);
    return JC_OK;
}

size_t dtype_size(int dtype) { return dtype == JC_F32 ? 4 : 2; }

// Times the launches made in its scope when the context profiles (jc_profile) and its stream is not
// being captured: an event before, one after, kept until jc_profile_report reads them.
class ProfScope {
  public:
    ProfScope(jc_ctx* ctx, const char* name) {
        if (!ctx || !ctx->prof) return;
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(ctx->stream, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return;
        if (hipEventCreate(&rec_.a) != hipSuccess) return;
        if (hipEventCreate(&rec_.b) != hipSuccess || hipEventRecord(rec_.a, ctx->stream) != hipSuccess) {
            (void)hipEventDestroy(rec_.a);
            if (rec_.b) (void)hipEventDestroy(rec_.b);
            return;
        }
        rec_.name = name;
        ctx_ = ctx;
    }
    ~ProfScope() {
        if (!ctx_) return;
        bool kept = hipEventRecord(rec_.b, ctx_->stream) == hipSuccess;
        if (kept) {
            try {
                ctx_->prof->push_back(rec_);
            } catch (...) {
                kept = false;
            }
        }
        if (!kept) {
            (void)hipEventDestroy(rec_.a);
            (void)hipEventDestroy(rec_.b);
        }
    }
    ProfScope(const ProfScope&) = delete;
    ProfScope& operator=(const ProfScope&) = delete;

  private:
    jc_ctx* ctx_ = nullptr;
    jc_prof_record rec_{nullptr, nullptr, nullptr};
};

void prof_clear(jc_ctx* ctx) {
    if (!ctx->prof) return;
    for (auto& r : *ctx->prof) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    ctx->prof->clear();
}

// JITCAST_HIP_LP_KERNEL picks the bf16/fp16 time-attention kernel: "stream" (time_attention_lp,
// which takes every shape), "wide" (time_attention_lpw) or "persist" (time_attention_lpp), the
// last two for the shapes they take ("persist" covers time_attention_lpp, rows of 257..513 tokens,
// and time_attention_lps, rows of 65..160). Unset, Chronos-2 uses a persistent kernel where one
// fits, else the row-wide one, and Timestral the streaming one: its row-wide variant holds every token's
// table row in LDS and fits one workgroup per CU (measured on config 3: 6.30 ms against 6.04 ms
// per 12 layers). Read at every launch, so a host can switch at run time.
enum LpKernel { kLpStream, kLpWide, kLpPersist };
LpKernel lp_choice(bool ts) {
    const char* e = getenv("JITCAST_HIP_LP_KERNEL");
    if (e && !strcmp(e, "stream")) return kLpStream;
    if (e && !strcmp(e, "wide")) return kLpWide;
    if (e && !strcmp(e, "persist")) return kLpPersist;
    return ts ? kLpStream : kLpPersist;
}

// JITCAST_HIP_GEMM=own runs the plain GEMMs on the library's own MFMA kernels (gemm_f32, gemm_lp)
// instead of hipBLASLt. Read at every call.
bool use_blas(const jc_ctx* ctx) {
    if (!ctx->blas) return false;
    const char* e = getenv("JITCAST_HIP_GEMM");
    return !(e && !strcmp(e, "own"));
}

}  // namespace

namespace jc {
int host_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace jc

// The workspace of jc_c2_layer_static: device memory in the library's own code object, so that
// entry point allocates nothing. Each GPU holds its own copy, at its own address, until the process
// ends. In host code `scratch` names a host-side stand-in, never the device memory: kernels and
// copies take the address hipGetSymbolAddress returns for the current device (scratch_ptr).
static __device__ __align__(256) unsigned char scratch[JC_C2_LAYER_STATIC_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // per device; set once by jc_init with that device current

// Resolves this device's copy of `scratch` once; the device must be current.
int scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return JC_OK;  // jc_c2_layer_static then reports it
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return JC_OK;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail("jc_init: hipGetSymbolAddress(scratch)", e);
    if (!p) return fail(JC_EHIP, "jc_init: hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_ptr[device] = p;
    return JC_OK;
}

void* scratch_ptr(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_ptr[device];
}
}  // namespace

extern "C" {

const char* jc_last_error(void) { return g_err; }

int jc_version(void) { return 1; }

int jc_init(int device, jc_ctx** out) {
    g_err[0] = 0;
    if (!out) return fail(JC_EINVAL, "jc_init: null output pointer");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail("jc_init: hipGetDeviceCount", e);
    if (device < 0 || device >= count)
        return fail(JC_EINVAL, "jc_init: device %d out of range (%d devices)", device, count);
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail("jc_init: hipSetDevice", e);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail("jc_init: hipGetDeviceProperties", e);
    int src = scratch_setup(device);
    if (src) return src;
    jc_ctx* ctx = new (std::nothrow) jc_ctx();
    if (!ctx) return fail(JC_ENOMEM, "jc_init: out of host memory");
    ctx->device = device;
    ctx->cus = prop.multiProcessorCount;
    snprintf(ctx->arch, sizeof ctx->arch, "%s", prop.gcnArchName);
    e = hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return hip_fail("jc_init: hipStreamCreate", e);
    }
    ctx->stream = ctx->own;
    e = hipMalloc((void**)&ctx->order, sizeof(int32_t) * jc::kGroupOrderTiles);
    if (e == hipSuccess) {
        e = hipEventCreateWithFlags(&ctx->order_read, hipEventDisableTiming);
        if (e != hipSuccess) (void)hipFree(ctx->order);
    }
    if (e != hipSuccess) {
        (void)hipStreamDestroy(ctx->own);
        delete ctx;
        return hip_fail("jc_init: the group tile-order buffer", e);
    }
    ctx->capture_order = nullptr;
    ctx->capturing = false;
    ctx->capture_on = nullptr;
    ctx->capture_key = 0;
    ctx->blas = jc::blas_create();  // nullptr leaves the GEMMs on the library's own kernels
    ctx->prof = nullptr;
    *out = ctx;
    return JC_OK;
}

int jc_destroy(jc_ctx* ctx) {
    if (!ctx) return JC_OK;
    (void)hipSetDevice(ctx->device);
    if (ctx->capturing) {
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(ctx->capture_on, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        ctx->capturing = false;
        (void)hipFree(ctx->capture_order);
    }
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipEventSynchronize(ctx->order_read);  // the last group kernel that read it, on any stream
    (void)hipEventDestroy(ctx->order_read);
    (void)hipFree(ctx->order);
    if (ctx->prof) {
        prof_clear(ctx);
        delete ctx->prof;
    }
    jc::blas_destroy(ctx->blas);
    (void)hipStreamDestroy(ctx->own);
    delete ctx;
    return JC_OK;
}

int jc_set_stream(jc_ctx* ctx, void* stream) {
    if (!ctx) return fail(JC_EINVAL, "jc_set_stream: null context");
    if (ctx->capturing && (hipStream_t)stream != ctx->capture_on)
        return fail(JC_ESTATE, "jc_set_stream: the context is capturing a plan on another stream");
    ctx->stream = (hipStream_t)stream;  // NULL is the device's default (null) stream
    return JC_OK;
}

void* jc_stream(jc_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int jc_profile(jc_ctx* ctx, int on) {
    int rc = use(ctx, "jc_profile");
    if (rc) return rc;
    if (ctx->prof) {
        (void)hipStreamSynchronize(ctx->stream);
        prof_clear(ctx);
    }
    if (!on) {
        delete ctx->prof;
        ctx->prof = nullptr;
        return JC_OK;
    }
    if (!ctx->prof) {
        ctx->prof = new (std::nothrow) std::vector<jc_prof_record>();
        if (!ctx->prof) return fail(JC_ENOMEM, "jc_profile: out of host memory");
    }
    return JC_OK;
}

int jc_profile_report(jc_ctx* ctx, char* buf, size_t len) {
    const char* W = "jc_profile_report";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (!buf || len == 0) return fail(JC_EINVAL, "%s: null or empty buffer", W);
    buf[0] = 0;
    if (!ctx->prof) return fail(JC_ESTATE, "%s: profiling is off (jc_profile(ctx, 1) first)", W);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(W, e);
    struct Sum {
        int calls = 0;
        double total = 0, lo = 1e30, hi = 0;
    };
    std::map<std::string, Sum> by;
    double all = 0;
    int n = 0;
    try {
        for (const auto& r : *ctx->prof) {
            float ms = 0.f;
            if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) continue;
            Sum& s = by[r.name];
            s.calls++;
            s.total += ms;
            s.lo = std::min(s.lo, (double)ms);
            s.hi = std::max(s.hi, (double)ms);
            all += ms;
            n++;
        }
        std::vector<std::pair<std::string, Sum>> rows(by.begin(), by.end());
        std::sort(rows.begin(), rows.end(), [](const auto& x, const auto& y) { return x.second.total > y.second.total; });
        size_t at = (size_t)snprintf(buf, len, "%-34s %7s %11s %10s %10s %10s\n", "kernel", "calls", "total ms", "mean ms",
                                     "min ms", "max ms");
        for (const auto& row : rows) {
            if (at >= len) break;
            const Sum& s = row.second;
            at += (size_t)snprintf(buf + at, len - at, "%-34s %7d %11.4f %10.4f %10.4f %10.4f\n", row.first.c_str(),
                                   s.calls, s.total, s.total / s.calls, s.lo, s.hi);
        }
        if (at < len) snprintf(buf + at, len - at, "%-34s %7d %11.4f\n", "all timed launches", n, all);
    } catch (...) {
        prof_clear(ctx);
        return fail(JC_ENOMEM, "%s: out of host memory", W);
    }
    prof_clear(ctx);
    return JC_OK;
}

int jc_alloc(jc_ctx* ctx, size_t bytes, void** dptr) {
    int rc = use(ctx, "jc_alloc");
    if (rc) return rc;
    if (!dptr) return fail(JC_EINVAL, "jc_alloc: null output pointer");
    *dptr = nullptr;
    if (bytes == 0) return JC_OK;
    hipError_t e = hipMalloc(dptr, bytes);
    if (e != hipSuccess) {
        *dptr = nullptr;
        return e == hipErrorOutOfMemory ? fail(JC_ENOMEM, "jc_alloc: out of device memory for %zu bytes", bytes)
                                        : hip_fail("jc_alloc: hipMalloc", e);
    }
    return JC_OK;
}

int jc_free(jc_ctx* ctx, void* dptr) {
    int rc = use(ctx, "jc_free");
    if (rc) return rc;
    if (!dptr) return JC_OK;
    hipError_t e = hipFree(dptr);
    return e == hipSuccess ? JC_OK : hip_fail("jc_free: hipFree", e);
}

static int copy(jc_ctx* ctx, void* dst, const void* src, size_t bytes, hipMemcpyKind kind, const char* where) {
    int rc = use(ctx, where);
    if (rc) return rc;
    if (ctx->capturing && kind != hipMemcpyDeviceToDevice)
        return fail(JC_ESTATE, "%s: host copies cannot be captured into a plan (upload before jc_plan_begin)", where);
    if (bytes == 0) return JC_OK;
    if (!dst || !src) return fail(JC_EINVAL, "%s: null pointer", where);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, ctx->stream);
    if (e != hipSuccess) return hip_fail(where, e);
    if (kind != hipMemcpyDeviceToDevice) {
        // host buffers are pageable: wait so the caller may reuse or read them on return
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return hip_fail(where, e);
    }
    return JC_OK;
}

int jc_memcpy_h2d(jc_ctx* ctx, void* dst, const void* src, size_t bytes) {
    return copy(ctx, dst, src, bytes, hipMemcpyHostToDevice, "jc_memcpy_h2d");
}
int jc_memcpy_d2h(jc_ctx* ctx, void* dst, const void* src, size_t bytes) {
    return copy(ctx, dst, src, bytes, hipMemcpyDeviceToHost, "jc_memcpy_d2h");
}
int jc_memcpy_d2d(jc_ctx* ctx, void* dst, const void* src, size_t bytes) {
    return copy(ctx, dst, src, bytes, hipMemcpyDeviceToDevice, "jc_memcpy_d2d");
}

int jc_sync(jc_ctx* ctx) {
    int rc = use(ctx, "jc_sync");
    if (rc) return rc;
    if (ctx->capturing) return fail(JC_ESTATE, "jc_sync: the context is capturing a plan");
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail("jc_sync", e);
}

int jc_device_info(jc_ctx* ctx, int* cus, char* arch, size_t arch_len) {
    if (!ctx) return fail(JC_EINVAL, "jc_device_info: null context");
    if (cus) *cus = ctx->cus;
    if (arch && arch_len) snprintf(arch, arch_len, "%s", ctx->arch);
    return JC_OK;
}

// ---- the portable RNG --------------------------------------------------------------------

int jc_fill_normal(jc_ctx* ctx, float* dptr, uint64_t count, uint64_t stream_seed, float mean, float stdv) {
    int rc = use(ctx, "jc_fill_normal");
    if (rc) return rc;
    if (count && !dptr) return fail(JC_EINVAL, "jc_fill_normal: null device pointer");
    hipError_t e = jc::fill_normal_launch(dptr, count, stream_seed, mean, stdv, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail("jc_fill_normal", e);
}

int jc_fill_uniform(jc_ctx* ctx, float* dptr, uint64_t count, uint64_t stream_seed, float lo, float hi) {
    int rc = use(ctx, "jc_fill_uniform");
    if (rc) return rc;
    if (count && !dptr) return fail(JC_EINVAL, "jc_fill_uniform: null device pointer");
    hipError_t e = jc::fill_uniform_launch(dptr, count, stream_seed, lo, hi, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail("jc_fill_uniform", e);
}

// ---- Chronos-2 ------------------------------------------------------------------------------

int jc_c2_rope_table(int n, int dh, float theta, float* table) {
    if (n < 0 || dh < 2 || dh % 2 || !table || !(theta > 0.f))
        return fail(JC_EINVAL, "jc_c2_rope_table: bad arguments (n=%d dh=%d theta=%g)", n, dh, (double)theta);
    int half = dh / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; i++) {
        float ex = (float)(2 * i) / (float)dh;
        inv[i] = 1.0f / (float)std::pow((double)theta, (double)ex);
    }
    for (int p = 0; p < n; p++) {
        for (int e = 0; e < half; e++) {
            float a = (float)p * inv[e];
            table[(size_t)p * dh + e] = (float)std::cos((double)a);
            table[(size_t)p * dh + half + e] = (float)std::sin((double)a);
        }
    }
    return JC_OK;
}

// Checks shared by the time-attention entry points: a valid head width for the dtype, an inner
// width the rows can be read with, a row short enough for the kernels' per-row state, pointers
// aligned for 16-byte loads, and 32-bit byte offsets within one row of qkv.
static int check_time_common(const char* W, const void* qkv, const void* out, const void* table, const void* gate,
                             int rows, int n, int heads, int dh, int inner, int dtype, int max_dh) {
    if (rows < 0 || n < 0 || heads < 1) return fail(JC_EINVAL, "%s: bad shape rows=%d n=%d heads=%d", W, rows, n, heads);
    if (dtype != JC_F32 && dtype != JC_BF16 && dtype != JC_F16) return fail(JC_EINVAL, "%s: dtype %d", W, dtype);
    const int mult = dtype == JC_F32 ? 8 : 16;
    if (dh < mult || dh > max_dh || dh % mult)
        return fail(JC_EINVAL, "%s: head width %d (need a multiple of %d, <= %d)", W, dh, mult, max_dh);
    const int imult = dtype == JC_F32 ? 4 : 8;
    if (inner < heads * dh || inner % imult)
        return fail(JC_EINVAL, "%s: inner %d (need >= heads*dh = %d and a multiple of %d)", W, inner, heads * dh,
                    imult);
    if (n > jc::time_attention_max_tokens())
        return fail(JC_EINVAL, "%s: %d tokens per row (at most %d)", W, n, jc::time_attention_max_tokens());
    if ((size_t)rows * n == 0) return JC_OK;
    if (!qkv || !out) return fail(JC_EINVAL, "%s: null device pointer", W);
    if (!aligned16(qkv) || !aligned16(out) || (table && !aligned16(table)) || (gate && !aligned16(gate)))
        return fail(JC_EINVAL, "%s: qkv, out, rope_table and gate must be 16-byte aligned", W);
    if ((uint64_t)rows * heads * ((n + 31) / 32) > 0x7fffffffull) return fail(JC_EINVAL, "%s: grid too large", W);
    if ((uint64_t)n * 3 * inner * dtype_size(dtype) >= 0x80000000ull)
        return fail(JC_EINVAL, "%s: one row of qkv (n*3*inner) must stay under 2 GiB", W);
    return JC_OK;
}

// fp32 goes to the fp32 kernel; bf16/fp16 to the row-wide kernel when lp_use_wide() picks it and
// the shape fits it, else to the streaming kernel, which takes every shape. Both give the same
// results to within rounding.
static int launch_time(jc_ctx* ctx, const char* W, const jc::TimeArgs& a, int dh, bool ts, int dtype) {
    hipError_t e;
    const bool fp16 = dtype == JC_F16;
    if (dtype == JC_F32) {
        ProfScope ps(ctx, ts ? "ts time_attention_f32" : "c2 time_attention_f32");
        e = jc::time_attention_f32_launch(a, dh, ts, ctx->stream);
    } else if (lp_choice(ts) == kLpPersist && jc::time_attention_lpp_fits(a, dh, ts)) {
        ProfScope ps(ctx, ts ? "ts time_attention_lpp" : "c2 time_attention_lpp");
        e = jc::time_attention_lpp_launch(a, fp16, ctx->cus, ctx->stream);
    } else if (lp_choice(ts) == kLpPersist && jc::time_attention_lps_fits(a, dh, ts)) {
        ProfScope ps(ctx, ts ? "ts time_attention_lps" : "c2 time_attention_lps");
        e = jc::time_attention_lps_launch(a, fp16, ctx->cus, ctx->stream);
    } else if (lp_choice(ts) != kLpStream && jc::time_attention_lpw_fits(a, dh)) {
        ProfScope ps(ctx, ts ? "ts time_attention_lpw" : "c2 time_attention_lpw");
        e = jc::time_attention_lpw_launch(a, dh, ts, fp16, ctx->stream);
    } else {
        ProfScope ps(ctx, ts ? "ts time_attention_lp" : "c2 time_attention_lp");
        e = jc::time_attention_lp_launch(a, dh, ts, fp16, ctx->stream);
    }
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

// jc_c2_time_attention after use(). x3 (fp32, dh 64): out is the JC_F16X3 layer's split operand, fp16
// [rows*n, 3*inner] rows [hi | hi | lo] of each output value.
static int c2_time(jc_ctx* ctx, const char* W, const void* qkv, void* out, const int32_t* live, const float* table,
                   int rows, int n, int heads, int dh, int inner, int dtype, bool x3) {
    int rc = check_time_common(W, qkv, out, table, nullptr, rows, n, heads, dh, inner, dtype, 64);
    if (rc || (size_t)rows * n == 0) return rc;
    if (!live) return fail(JC_EINVAL, "%s: null live mask", W);
    jc::TimeArgs a{};
    a.qkv = qkv;
    a.out = out;
    a.valid = live;
    a.table = table;
    a.rows = rows;
    a.n = n;
    a.heads = heads;
    a.inner = inner;
    a.enc = n;
    a.ll = n;
    a.table_rows = n;
    a.qscale = 1.4426950408889634f;  // unscaled scores, exp via exp2
    if (x3) {
        if (dtype != JC_F32) return fail(JC_EINVAL, "%s: the split output needs fp32", W);
        ProfScope ps(ctx, "c2 time_attention_f32 (split out)");
        hipError_t e = jc::time_attention_f32_x3_launch(a, dh, ctx->stream);
        return e == hipSuccess ? JC_OK : hip_fail(W, e);
    }
    return launch_time(ctx, W, a, dh, false, dtype);
}

int jc_c2_time_attention(jc_ctx* ctx, const void* qkv, void* out, const int32_t* live, const float* table, int rows,
                         int n, int heads, int dh, int inner, int dtype) {
    const char* W = "jc_c2_time_attention";
    int rc = use(ctx, W);
    if (rc) return rc;
    return c2_time(ctx, W, qkv, out, live, table, rows, n, heads, dh, inner, dtype, false);
}

int jc_ts_rope_table(int enc, int n, int dh, int rope_dim, float theta, float* table) {
    if (enc < 0 || n < enc || dh < 2 || dh % 2 || rope_dim < 2 || rope_dim % 2 || rope_dim > dh || !table ||
        !(theta > 0.f))
        return fail(JC_EINVAL, "jc_ts_rope_table: bad arguments (enc=%d n=%d dh=%d rope_dim=%d theta=%g)", enc, n, dh,
                    rope_dim, (double)theta);
    const int half = dh / 2;
    std::vector<float> inv(half, 0.f);
    for (int i = 0; i < rope_dim / 2; i++) {
        float ex = (float)(2 * i) / (float)rope_dim;
        inv[i] = 1.0f / (float)std::pow((double)theta, (double)ex);
    }
    for (int p = 0; p < enc + n; p++) {
        const float position = (float)(p - enc);
        for (int e = 0; e < half; e++) {
            const float ang = position * inv[e];
            table[(size_t)p * dh + e] = (float)std::cos((double)ang);
            table[(size_t)p * dh + half + e] = (float)std::sin((double)ang);
        }
    }
    return JC_OK;
}

int jc_ts_time_attention(jc_ctx* ctx, const void* qkv, void* out, const int32_t* key_valid, const int32_t* known,
                         const int32_t* pos, const float* table, const void* gate, int rows, int enc, int ll, int n,
                         int heads, int dh, int d, int dtype) {
    const char* W = "jc_ts_time_attention";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (enc < 0 || ll < 0 || ll > enc || n < enc)
        return fail(JC_EINVAL, "%s: token counts (need 0 <= ll <= enc <= n; got ll=%d enc=%d n=%d)", W, ll, enc, n);
    rc = check_time_common(W, qkv, out, table, gate, rows, n, heads, dh, d, dtype, 128);
    if (rc || (size_t)rows * n == 0) return rc;
    if (enc > 0 && !key_valid) return fail(JC_EINVAL, "%s: null key_valid", W);
    jc::TimeArgs a{};
    a.qkv = qkv;
    a.out = out;
    a.valid = key_valid;
    a.known = known;
    a.pos = pos;
    a.table = table;
    a.gate = gate;
    a.rows = rows;
    a.n = n;
    a.heads = heads;
    a.inner = d;
    a.enc = enc;
    a.ll = ll;
    a.table_rows = enc + n;
    a.qscale = (float)(1.4426950408889634 / std::sqrt((double)dh));
    return launch_time(ctx, W, a, dh, true, dtype);
}

int jc_ts_gate(jc_ctx* ctx, void* att, const void* g, int64_t count, int dtype) {
    const char* W = "jc_ts_gate";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (count < 0) return fail(JC_EINVAL, "%s: count %lld", W, (long long)count);
    if (dtype != JC_F32 && dtype != JC_BF16 && dtype != JC_F16) return fail(JC_EINVAL, "%s: dtype %d", W, dtype);
    if (count == 0) return JC_OK;
    if (!att || !g) return fail(JC_EINVAL, "%s: null device pointer", W);
    const size_t align = dtype == JC_F32 ? 16 : 8;
    if (((uintptr_t)att % align) || ((uintptr_t)g % align))
        return fail(JC_EINVAL, "%s: att and g must be %zu-byte aligned", W, align);
    ProfScope ps(ctx, "ts gate");
    hipError_t e = jc::gate_launch(att, g, (uint64_t)count, dtype, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

static int check_group_common(const char* W, const void* qkv, const void* out, const void* gate, const int32_t* gs,
                              const int32_t* ge, int rows, int n, int heads, int dh, int inner, int dtype, int max_dh) {
    if (rows < 0 || n < 0 || heads < 1) return fail(JC_EINVAL, "%s: bad shape rows=%d n=%d heads=%d", W, rows, n, heads);
    if (dh < 8 || dh > max_dh || dh % 8)
        return fail(JC_EINVAL, "%s: head width %d (need a multiple of 8, <= %d)", W, dh, max_dh);
    if (inner < heads * dh || inner % 4)
        return fail(JC_EINVAL, "%s: inner %d (need >= heads*dh = %d and a multiple of 4)", W, inner, heads * dh);
    if (dtype != JC_F32 && dtype != JC_BF16 && dtype != JC_F16) return fail(JC_EINVAL, "%s: dtype %d", W, dtype);
    if ((size_t)rows * n == 0) return JC_OK;
    if (!qkv || !out || !gs || !ge) return fail(JC_EINVAL, "%s: null device pointer", W);
    if (!aligned16(qkv) || !aligned16(out) || (gate && !aligned16(gate)))
        return fail(JC_EINVAL, "%s: qkv, out and gate must be 16-byte aligned", W);
    if ((uint64_t)((rows + 15) / 16) * n > 0x7fffffffull) return fail(JC_EINVAL, "%s: grid too large", W);
    return JC_OK;
}

// The group kernel's tile order for a launch on ctx's stream (group_tile_order_launch): into the
// captured plan's buffer, or into the context's behind the last group kernel that read it. Null
// (the kernel's fixed order) without a buffer, past its capacity or with JITCAST_HIP_GROUP_ORDER=0
// (read at every call). Follow the group launch with group_order_done.
static hipError_t group_order(jc_ctx* ctx, const int32_t* gs, const int32_t* ge, int rows, const int32_t** order) {
    *order = nullptr;
    const char* env = getenv("JITCAST_HIP_GROUP_ORDER");
    if ((env && env[0] == '0') || (rows + 15) / 16 > jc::kGroupOrderTiles) return hipSuccess;
    int32_t* buf = ctx->capturing ? ctx->capture_order : ctx->order;
    if (!buf) return hipSuccess;
    if (!ctx->capturing) {
        // a capture the caller began on this stream: the context's buffer and its event are not
        // the graph's, so the kernel keeps its fixed order there
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(ctx->stream, &st);
        if (e != hipSuccess) return e;
        if (st != hipStreamCaptureStatusNone) return hipSuccess;
        e = hipStreamWaitEvent(ctx->stream, ctx->order_read, 0);
        if (e != hipSuccess) return e;
    }
    hipError_t e = jc::group_tile_order_launch(gs, ge, rows, buf, ctx->stream);
    if (e == hipSuccess) *order = buf;
    return e;
}

static hipError_t group_order_done(jc_ctx* ctx, const int32_t* order) {
    return order && !ctx->capturing ? hipEventRecord(ctx->order_read, ctx->stream) : hipSuccess;
}

// jc_c2_group_attention after use(); x3 as for c2_time.
static int c2_group(jc_ctx* ctx, const char* W, const void* qkv, void* out, const int32_t* live,
                    const int32_t* group_start, const int32_t* group_end, int rows, int n, int heads, int dh, int inner,
                    int dtype, bool x3) {
    int rc = check_group_common(W, qkv, out, nullptr, group_start, group_end, rows, n, heads, dh, inner, dtype, 64);
    if (rc || (size_t)rows * n == 0) return rc;
    if (!live) return fail(JC_EINVAL, "%s: null live mask", W);
    if (x3 && dtype != JC_F32) return fail(JC_EINVAL, "%s: the split output needs fp32", W);
    jc::GroupArgs a{};
    a.qkv = qkv;
    a.out = out;
    a.valid = live;
    a.gstart = group_start;
    a.gend = group_end;
    a.rows = rows;
    a.n = n;
    a.heads = heads;
    a.inner = inner;
    a.enc = n;
    a.qscale = 1.4426950408889634f;  // unscaled scores, exp via exp2
    ProfScope ps(ctx, x3 ? "c2 group_attention (split out)" : dtype == JC_F32 ? "c2 group_attention_f32" : "c2 group_attention_lp");
    hipError_t e = group_order(ctx, group_start, group_end, rows, &a.order);
    if (e == hipSuccess)
        e = x3 ? jc::group_attention_f32_x3_launch(a, dh, ctx->stream)
               : jc::group_attention_launch(a, dh, false, dtype, ctx->stream);
    if (e == hipSuccess) e = group_order_done(ctx, a.order);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_c2_group_attention(jc_ctx* ctx, const void* qkv, void* out, const int32_t* live, const int32_t* group_start,
                          const int32_t* group_end, int rows, int n, int heads, int dh, int inner, int dtype) {
    const char* W = "jc_c2_group_attention";
    int rc = use(ctx, W);
    if (rc) return rc;
    return c2_group(ctx, W, qkv, out, live, group_start, group_end, rows, n, heads, dh, inner, dtype, false);
}

int jc_ts_variate_attention(jc_ctx* ctx, const void* qkv, void* out, const int32_t* key_valid,
                            const int32_t* group_start, const int32_t* group_end, const int32_t* role, int covariates,
                            const void* gate, int rows, int enc, int n, int heads, int dh, int d, int dtype) {
    const char* W = "jc_ts_variate_attention";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (enc < 0 || n < enc) return fail(JC_EINVAL, "%s: token counts (need 0 <= enc <= n; got enc=%d n=%d)", W, enc, n);
    rc = check_group_common(W, qkv, out, gate, group_start, group_end, rows, n, heads, dh, d, dtype, 128);
    if (rc || (size_t)rows * n == 0) return rc;
    if (enc > 0 && !key_valid) return fail(JC_EINVAL, "%s: null key_valid", W);
    if (covariates && !role) return fail(JC_EINVAL, "%s: covariates without a role array", W);
    jc::GroupArgs a{};
    a.qkv = qkv;
    a.out = out;
    a.valid = key_valid;
    a.gstart = group_start;
    a.gend = group_end;
    a.role = role;
    a.gate = gate;
    a.rows = rows;
    a.n = n;
    a.heads = heads;
    a.inner = d;
    a.enc = enc;
    a.covariates = covariates;
    a.qscale = (float)(1.4426950408889634 / std::sqrt((double)dh));
    ProfScope ps(ctx, dtype == JC_F32 ? "ts variate_attention_f32" : "ts variate_attention_lp");
    hipError_t e = group_order(ctx, group_start, group_end, rows, &a.order);
    if (e == hipSuccess) e = jc::group_attention_launch(a, dh, true, dtype, ctx->stream);
    if (e == hipSuccess) e = group_order_done(ctx, a.order);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

// ---- plans: one captured hipGraph per batch shape ----------------------------------------------

int jc_plan_begin(jc_ctx* ctx, uint64_t shape_key) {
    const char* W = "jc_plan_begin";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (ctx->capturing) return fail(JC_ESTATE, "%s: a plan is already being captured", W);
    if (ctx->stream == nullptr)
        return fail(JC_ESTATE, "%s: the null stream cannot be captured (jc_set_stream a created stream)", W);
    int32_t* order = nullptr;  // the plan's own tile-order buffer, so replays on any stream share nothing
    hipError_t e = hipMalloc((void**)&order, sizeof(int32_t) * jc::kGroupOrderTiles);
    if (e != hipSuccess) return hip_fail("jc_plan_begin: the group tile-order buffer", e);
    e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        (void)hipFree(order);
        return hip_fail(W, e);
    }
    ctx->capture_order = order;
    ctx->capturing = true;
    ctx->capture_on = ctx->stream;
    ctx->capture_key = shape_key;
    return JC_OK;
}

int jc_plan_end(jc_ctx* ctx, jc_plan** out) {
    const char* W = "jc_plan_end";
    if (!out) return fail(JC_EINVAL, "%s: null output pointer", W);
    *out = nullptr;
    int rc = use(ctx, W);
    if (rc) return rc;
    if (!ctx->capturing) return fail(JC_ESTATE, "%s: no plan is being captured", W);
    ctx->capturing = false;
    int32_t* order = ctx->capture_order;
    ctx->capture_order = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->capture_on, &graph);
    if (e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        (void)hipFree(order);
        return hip_fail(W, e);
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        (void)hipFree(order);
        return hip_fail("jc_plan_end: hipGraphInstantiate", e);
    }
    jc_plan* plan = new (std::nothrow) jc_plan();
    if (!plan) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        (void)hipFree(order);
        return fail(JC_ENOMEM, "%s: out of host memory", W);
    }
    plan->order = order;
    plan->ctx = ctx;
    plan->graph = graph;
    plan->exec = exec;
    plan->key = ctx->capture_key;
    e = hipEventCreateWithFlags(&plan->done, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        (void)hipFree(order);
        delete plan;
        return hip_fail("jc_plan_end: hipEventCreateWithFlags", e);
    }
    *out = plan;
    return JC_OK;
}

static int plan_launch(jc_plan* plan, hipStream_t stream, const char* W) {
    if (!plan) return fail(JC_EINVAL, "%s: null plan", W);
    int rc = use(plan->ctx, W);
    if (rc) return rc;
    if (plan->ctx->capturing) return fail(JC_ESTATE, "%s: the context is capturing a plan", W);
    hipError_t e = hipGraphLaunch(plan->exec, stream);
    if (e != hipSuccess) return hip_fail(W, e);
    // jc_plan_destroy waits for this event, so a replay on any stream ends before the graph and
    // its buffers are released, whatever stream the context launches on by then
    e = hipEventRecord(plan->done, stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_plan_launch(jc_plan* plan) {
    return plan_launch(plan, plan ? plan->ctx->stream : nullptr, "jc_plan_launch");
}

int jc_plan_launch_on(jc_plan* plan, void* stream) {
    return plan_launch(plan, stream ? (hipStream_t)stream : (plan ? plan->ctx->stream : nullptr), "jc_plan_launch_on");
}

int jc_plan_adopt(jc_plan* plan, void* dptr, size_t bytes) {
    if (!plan) return fail(JC_EINVAL, "jc_plan_adopt: null plan");
    if (!dptr) return fail(JC_EINVAL, "jc_plan_adopt: null device pointer");
    try {
        plan->owned.emplace_back(dptr, bytes);
    } catch (...) {
        return fail(JC_ENOMEM, "jc_plan_adopt: out of host memory");
    }
    return JC_OK;
}

int64_t jc_plan_device_bytes(jc_plan* plan) {
    if (!plan) return 0;
    int64_t total = 0;
    for (const auto& b : plan->owned) total += (int64_t)b.second;
    return total;
}

uint64_t jc_plan_key(jc_plan* plan) { return plan ? plan->key : 0; }

int jc_plan_destroy(jc_plan* plan) {
    if (!plan) return JC_OK;
    (void)hipSetDevice(plan->ctx->device);
    int rc = JC_OK;
    hipError_t e = hipEventSynchronize(plan->done);  // the last replay, on whichever stream it ran
    if (e != hipSuccess) rc = hip_fail("jc_plan_destroy", e);
    (void)hipEventDestroy(plan->done);
    (void)hipGraphExecDestroy(plan->exec);
    (void)hipGraphDestroy(plan->graph);
    for (const auto& b : plan->owned) {
        e = hipFree(b.first);
        if (e != hipSuccess && rc == JC_OK) rc = hip_fail("jc_plan_destroy: hipFree", e);
    }
    e = hipFree(plan->order);
    if (e != hipSuccess && rc == JC_OK) rc = hip_fail("jc_plan_destroy: hipFree", e);
    delete plan;
    return rc;
}


// ---- The Chronos-2 encoder layer around the attention cores ----------------------------------

static int check_linear(const char* W, const float* a, int lda, const float* w, const float* bias, const float* c,
                        int ldc, int m, int n, int k, int flags) {
    if (m < 0 || n < 0 || k < 0) return fail(JC_EINVAL, "%s: negative size (m=%d n=%d k=%d)", W, m, n, k);
    if ((size_t)m * n == 0) return JC_OK;
    if (!a || !w || !c) return fail(JC_EINVAL, "%s: null a, w or c", W);
    if (k % 16) return fail(JC_EINVAL, "%s: k must be a multiple of 16 (got %d)", W, k);
    if (lda < k || lda % 4) return fail(JC_EINVAL, "%s: lda must be >= k and a multiple of 4 (got %d)", W, lda);
    if (ldc < n) return fail(JC_EINVAL, "%s: ldc must be >= n (got %d)", W, ldc);
    if (!aligned16(a) || !aligned16(w)) return fail(JC_EINVAL, "%s: a and w must be 16-byte aligned", W);
    if (flags & ~(JC_GEMM_BIAS | JC_GEMM_ACCUMULATE | JC_GEMM_SILU | JC_GEMM_RELU))
        return fail(JC_EINVAL, "%s: unknown flags 0x%x", W, flags);
    if ((flags & JC_GEMM_SILU) && (flags & JC_GEMM_RELU)) return fail(JC_EINVAL, "%s: SILU and RELU together", W);
    if ((flags & JC_GEMM_BIAS) && !bias) return fail(JC_EINVAL, "%s: JC_GEMM_BIAS without a bias", W);
    return JC_OK;
}

static int launch_linear(jc_ctx* ctx, const char* W, const float* a, int lda, const float* w, const float* bias,
                         float* c, int ldc, int m, int n, int k, int flags) {
    if (bias) flags |= JC_GEMM_BIAS;
    int rc = check_linear(W, a, lda, w, bias, c, ldc, m, n, k, flags);
    if (rc || (size_t)m * n == 0) return rc;
    if (use_blas(ctx)) {
        ProfScope ps(ctx, "gemm fp32 (hipBLASLt)");
        const jc::BlasStatus bs = jc::blas_gemm(ctx->blas, a, lda, w, bias, c, ldc, m, n, k, flags, JC_F32, JC_F32,
                                                ctx->stream);
        if (bs == jc::kBlasDone) return JC_OK;
        if (bs == jc::kBlasError) return fail(JC_EHIP, "%s: hipblasLtMatmul failed", W);
    }
    jc::GemmArgs g{a, w, bias, c, m, n, k, lda, ldc, flags};
    ProfScope ps(ctx, "gemm_f32");
    hipError_t e = jc::gemm_f32_launch(g, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_linear(jc_ctx* ctx, const float* a, int lda, const float* w, const float* bias, float* c, int ldc, int m, int n,
              int k, int flags) {
    const char* W = "jc_linear";
    int rc = use(ctx, W);
    if (rc) return rc;
    return launch_linear(ctx, W, a, lda, w, bias, c, ldc, m, n, k, flags);
}

static int launch_rms(jc_ctx* ctx, const char* W, const float* x, const float* w, float* y, int rows, int d, float eps) {
    if (rows < 0 || d < 0) return fail(JC_EINVAL, "%s: negative size", W);
    if ((size_t)rows * d == 0) return JC_OK;
    if (!x || !y) return fail(JC_EINVAL, "%s: null x or y", W);
    if (d % 4) return fail(JC_EINVAL, "%s: d must be a multiple of 4 (got %d)", W, d);
    if (!aligned16(x) || !aligned16(y) || (w && !aligned16(w))) return fail(JC_EINVAL, "%s: 16-byte alignment", W);
    ProfScope ps(ctx, "rms_norm_f32");
    hipError_t e = jc::rms_norm_f32_launch(x, y, w, rows, d, eps, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_rms_norm(jc_ctx* ctx, const float* x, const float* w, float* y, int rows, int d, float eps) {
    const char* W = "jc_rms_norm";
    int rc = use(ctx, W);
    if (rc) return rc;
    return launch_rms(ctx, W, x, w, y, rows, d, eps);
}

static size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

int64_t jc_c2_layer_workspace_bytes(int rows, int n, int d, int inner, int dff, int dtype) {
    if (rows < 0 || n < 0 || d < 0 || inner < 0 || dff < 0) return -1;
    const size_t t = (size_t)rows * n;
    if (dtype == JC_F32) {
        const size_t big = (size_t)(3 * inner > dff ? 3 * inner : dff);
        return (int64_t)(round256(t * d * 4) + round256(t * big * 4) + round256(t * (size_t)inner * 4));
    }
    if (dtype == JC_F16X3) {
        const size_t big = (size_t)(3 * inner > dff ? 3 * inner : dff);
        size_t wide = (size_t)(d > inner ? d : inner);
        if ((size_t)dff > wide) wide = (size_t)dff;
        return (int64_t)(round256(t * big * 4) + round256(t * (size_t)inner * 4) + round256(t * 3 * wide * 2));
    }
    if (dtype != JC_BF16 && dtype != JC_F16) return -1;
    const size_t big = (size_t)(12 * inner > 2 * dff ? 12 * inner : 2 * dff);  // bytes per token
    return (int64_t)(round256(t * d * 2) + round256(t * big) + round256(t * (size_t)inner * 4) +
                     round256(t * (size_t)inner * 2));
}

static int layer_lp(jc_ctx* ctx, const char* W, float* x, const jc_c2_layer_weights* w, const int32_t* live,
                    const float* table, const int32_t* group_start, const int32_t* group_end, void* workspace, int rows,
                    int n, int d, int heads, int dh, int dff, float eps, int dtype);
static int layer_x3(jc_ctx* ctx, const char* W, float* x, const jc_c2_layer_weights* w, const int32_t* live,
                    const float* table, const int32_t* group_start, const int32_t* group_end, void* workspace, int rows,
                    int n, int d, int heads, int dh, int dff, float eps);

static int c2_layer(jc_ctx* ctx, const char* W, float* x, const jc_c2_layer_weights* w, const int32_t* live,
                    const float* table, const int32_t* group_start, const int32_t* group_end, void* workspace, int rows,
                    int n, int d, int heads, int dh, int dff, float eps, int dtype) {
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || n < 0 || d <= 0 || heads <= 0 || dh <= 0 || dff <= 0)
        return fail(JC_EINVAL, "%s: sizes must be positive (rows=%d n=%d d=%d heads=%d dh=%d dff=%d)", W, rows, n, d,
                    heads, dh, dff);
    if ((size_t)rows * n == 0) return JC_OK;
    if (!x || !w || !workspace) return fail(JC_EINVAL, "%s: null x, weights or workspace", W);
    if (d % 16 || dff % 16 || dh % 16 || dh > 64)
        return fail(JC_EINVAL, "%s: d and dff must be multiples of 16, dh a multiple of 16 up to 64 (d=%d dff=%d dh=%d)",
                    W, d, dff, dh);
    if (((uintptr_t)workspace & 255u) != 0) return fail(JC_EINVAL, "%s: workspace must be 256-byte aligned", W);
    if (!w->time_norm || !w->time_qkv || !w->time_o || !w->group_norm || !w->group_qkv || !w->group_o ||
        !w->mlp_norm || !w->wi || !w->wo)
        return fail(JC_EINVAL, "%s: a null weight matrix or norm", W);
    if (dtype == JC_BF16 || dtype == JC_F16)
        return layer_lp(ctx, W, x, w, live, table, group_start, group_end, workspace, rows, n, d, heads, dh, dff, eps,
                        dtype);
    if (dtype == JC_F16X3)
        return layer_x3(ctx, W, x, w, live, table, group_start, group_end, workspace, rows, n, d, heads, dh, dff, eps);
    if (dtype != JC_F32)
        return fail(JC_EINVAL, "%s: dtype must be JC_F32, JC_BF16, JC_F16 or JC_F16X3 (got %d)", W, dtype);
    const int inner = heads * dh, T = rows * n;
    const size_t big_cols = (size_t)(3 * inner > dff ? 3 * inner : dff);
    char* ws = static_cast<char*>(workspace);
    float* hn = reinterpret_cast<float*>(ws);
    float* big = reinterpret_cast<float*>(ws + round256((size_t)T * d * 4));  // qkv [T, 3*inner] or act [T, dff]
    float* att = reinterpret_cast<float*>(ws + round256((size_t)T * d * 4) + round256((size_t)T * big_cols * 4));

    // time attention sub-layer (Chronos2Forward.java:260-271)
    if ((rc = launch_rms(ctx, W, x, w->time_norm, hn, T, d, eps))) return rc;
    if ((rc = launch_linear(ctx, W, hn, d, static_cast<const float*>(w->time_qkv), w->time_qkv_bias, big, 3 * inner, T, 3 * inner, d, 0))) return rc;
    if ((rc = jc_c2_time_attention(ctx, big, att, live, table, rows, n, heads, dh, inner, JC_F32))) return rc;
    if ((rc = launch_linear(ctx, W, att, inner, static_cast<const float*>(w->time_o), w->time_o_bias, x, d, T, d, inner, JC_GEMM_ACCUMULATE)))
        return rc;
    // group attention sub-layer (Chronos2Forward.java:273-281)
    if ((rc = launch_rms(ctx, W, x, w->group_norm, hn, T, d, eps))) return rc;
    if ((rc = launch_linear(ctx, W, hn, d, static_cast<const float*>(w->group_qkv), w->group_qkv_bias, big, 3 * inner, T, 3 * inner, d, 0)))
        return rc;
    if ((rc = jc_c2_group_attention(ctx, big, att, live, group_start, group_end, rows, n, heads, dh, inner, JC_F32)))
        return rc;
    if ((rc = launch_linear(ctx, W, att, inner, static_cast<const float*>(w->group_o), w->group_o_bias, x, d, T, d, inner, JC_GEMM_ACCUMULATE)))
        return rc;
    // feed-forward sub-layer (Chronos2Forward.java:283-286)
    if ((rc = launch_rms(ctx, W, x, w->mlp_norm, hn, T, d, eps))) return rc;
    if ((rc = launch_linear(ctx, W, hn, d, static_cast<const float*>(w->wi), w->wi_bias, big, dff, T, dff, d, JC_GEMM_RELU))) return rc;
    return launch_linear(ctx, W, big, dff, static_cast<const float*>(w->wo), w->wo_bias, x, d, T, d, dff, JC_GEMM_ACCUMULATE);
}

int jc_c2_layer(jc_ctx* ctx, float* x, const jc_c2_layer_weights* w, const int32_t* live, const float* table,
                const int32_t* group_start, const int32_t* group_end, void* workspace, int rows, int n, int d, int heads,
                int dh, int dff, float eps, int dtype) {
    return c2_layer(ctx, "jc_c2_layer", x, w, live, table, group_start, group_end, workspace, rows, n, d, heads, dh,
                    dff, eps, dtype);
}

int jc_c2_layer_static(jc_ctx* ctx, float* x, const jc_c2_layer_weights* w, const int32_t* live, const float* table,
                       const int32_t* group_start, const int32_t* group_end, int rows, int n, int d, int heads, int dh,
                       int dff, float eps, int dtype) {
    const char* W = "jc_c2_layer_static";
    if (!ctx) return fail(JC_EINVAL, "%s: null context", W);
    if (rows < 0 || n < 0 || d <= 0 || heads <= 0 || dh <= 0 || dff <= 0)
        return fail(JC_EINVAL, "%s: sizes must be positive (rows=%d n=%d d=%d heads=%d dh=%d dff=%d)", W, rows, n, d,
                    heads, dh, dff);
    if ((int64_t)heads * dh > INT32_MAX / 12) return fail(JC_EINVAL, "%s: heads * dh too large", W);
    const int64_t need = jc_c2_layer_workspace_bytes(rows, n, d, heads * dh, dff, dtype);
    if (need < 0) return fail(JC_EINVAL, "%s: dtype must be JC_F32, JC_BF16, JC_F16 or JC_F16X3 (got %d)", W, dtype);
    if (need > (int64_t)JC_C2_LAYER_STATIC_BYTES)
        return fail(JC_EINVAL,
                    "%s: %d rows x %d tokens need %lld bytes of workspace, past the %lld-byte static scratch "
                    "(split the rows over several calls, or use jc_c2_layer with a caller workspace)",
                    W, rows, n, (long long)need, (long long)JC_C2_LAYER_STATIC_BYTES);
    void* ws = scratch_ptr(ctx->device);
    if (!ws) return fail(JC_EUNSUPPORTED, "%s: no static scratch on device %d", W, ctx->device);
    // the library's own GEMM kernels, so no library routine that could allocate runs: the layer runs
    // on a copy of the context without hipBLASLt, which leaves the caller's context untouched
    jc_ctx own = *ctx;
    own.blas = nullptr;
    // and the group kernel in its fixed order: its tile order would be device memory beyond the
    // static scratch
    own.order = nullptr;
    own.capture_order = nullptr;
    return c2_layer(&own, W, x, w, live, table, group_start, group_end, ws, rows, n, d, heads, dh, dff, eps, dtype);
}

// ---- bf16 / fp16 layer ------------------------------------------------------------------------

static int check_lp_dtype(const char* W, int dtype) {
    if (dtype != JC_BF16 && dtype != JC_F16) return fail(JC_EINVAL, "%s: dtype must be JC_BF16 or JC_F16 (got %d)", W, dtype);
    return JC_OK;
}

static int launch_linear_lp(jc_ctx* ctx, const char* W, const void* a, int lda, const void* w, const float* bias,
                            void* c, int ldc, int m, int n, int k, int flags, int dtype, int c_dtype) {
    int rc = check_lp_dtype(W, dtype);
    if (rc) return rc;
    if (bias) flags |= JC_GEMM_BIAS;
    if (m < 0 || n < 0 || k < 0) return fail(JC_EINVAL, "%s: negative size (m=%d n=%d k=%d)", W, m, n, k);
    if ((size_t)m * n == 0) return JC_OK;
    if (!a || !w || !c) return fail(JC_EINVAL, "%s: null a, w or c", W);
    if (c_dtype != JC_F32 && c_dtype != dtype)
        return fail(JC_EINVAL, "%s: c_dtype must be JC_F32 or the input dtype (got %d)", W, c_dtype);
    if (k % 8 || k == 0) return fail(JC_EINVAL, "%s: k must be a positive multiple of 8 (got %d)", W, k);
    if (lda < k || lda % 8) return fail(JC_EINVAL, "%s: lda must be >= k and a multiple of 8 (got %d)", W, lda);
    if (ldc < n) return fail(JC_EINVAL, "%s: ldc must be >= n (got %d)", W, ldc);
    if (lda >= (1 << 22)) return fail(JC_EINVAL, "%s: lda and k must be below 4194304 (got %d)", W, lda);
    if (!aligned16(a) || !aligned16(w)) return fail(JC_EINVAL, "%s: a and w must be 16-byte aligned", W);
    if (flags & ~(JC_GEMM_BIAS | JC_GEMM_ACCUMULATE | JC_GEMM_SILU | JC_GEMM_RELU))
        return fail(JC_EINVAL, "%s: unknown flags 0x%x", W, flags);
    if ((flags & JC_GEMM_SILU) && (flags & JC_GEMM_RELU)) return fail(JC_EINVAL, "%s: SILU and RELU together", W);
    if ((flags & JC_GEMM_BIAS) && !bias) return fail(JC_EINVAL, "%s: JC_GEMM_BIAS without a bias", W);
    if (c_dtype != JC_F32 && (flags & JC_GEMM_ACCUMULATE))
        return fail(JC_EINVAL, "%s: JC_GEMM_ACCUMULATE needs an fp32 C", W);
    if (use_blas(ctx)) {
        ProfScope ps(ctx, dtype == JC_F16 ? "gemm fp16 (hipBLASLt)" : "gemm bf16 (hipBLASLt)");
        const jc::BlasStatus bs = jc::blas_gemm(ctx->blas, a, lda, w, bias, c, ldc, m, n, k, flags, dtype, c_dtype,
                                                ctx->stream);
        if (bs == jc::kBlasDone) return JC_OK;
        if (bs == jc::kBlasError) return fail(JC_EHIP, "%s: hipblasLtMatmul failed", W);
    }
    jc::GemmLpArgs g{a, w, bias, c, m, n, k, lda, ldc, flags};
    ProfScope ps(ctx, dtype == JC_F16 ? "gemm_lp fp16" : "gemm_lp bf16");
    hipError_t e = jc::gemm_lp_launch(g, dtype == JC_F16, c_dtype != JC_F32, ctx->cus, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_linear_lp(jc_ctx* ctx, const void* a, int lda, const void* w, const float* bias, void* c, int ldc, int m, int n,
                 int k, int flags, int dtype, int c_dtype) {
    const char* W = "jc_linear_lp";
    int rc = use(ctx, W);
    if (rc) return rc;
    return launch_linear_lp(ctx, W, a, lda, w, bias, c, ldc, m, n, k, flags, dtype, c_dtype);
}

static int launch_rms_lp(jc_ctx* ctx, const char* W, const float* x, const float* w, void* y, int rows, int d, float eps,
                         int dtype) {
    int rc = dtype == JC_F16X3 ? JC_OK : check_lp_dtype(W, dtype);
    if (rc) return rc;
    if (rows < 0 || d < 0) return fail(JC_EINVAL, "%s: negative size", W);
    if ((size_t)rows * d == 0) return JC_OK;
    if (!x || !y) return fail(JC_EINVAL, "%s: null x or y", W);
    if (d % 4) return fail(JC_EINVAL, "%s: d must be a multiple of 4 (got %d)", W, d);
    if (!aligned16(x) || !aligned16(y) || (w && !aligned16(w))) return fail(JC_EINVAL, "%s: 16-byte alignment", W);
    ProfScope ps(ctx, dtype == JC_F16X3 ? "rms_norm (split out)" : "rms_norm_lp");
    hipError_t e = dtype == JC_F16X3 ? jc::rms_norm_x3_launch(x, y, w, rows, d, eps, ctx->stream)
                                     : jc::rms_norm_lp_launch(x, y, w, rows, d, eps, dtype == JC_F16, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_rms_norm_lp(jc_ctx* ctx, const float* x, const float* w, void* y, int rows, int d, float eps, int dtype) {
    const char* W = "jc_rms_norm_lp";
    int rc = use(ctx, W);
    if (rc) return rc;
    return launch_rms_lp(ctx, W, x, w, y, rows, d, eps, dtype);
}

static int launch_to_lp(jc_ctx* ctx, const char* W, const float* src, void* dst, int64_t count, int dtype) {
    int rc = check_lp_dtype(W, dtype);
    if (rc) return rc;
    if (count < 0) return fail(JC_EINVAL, "%s: negative count", W);
    if (count == 0) return JC_OK;
    if (!src || !dst) return fail(JC_EINVAL, "%s: null src or dst", W);
    ProfScope ps(ctx, "to_lp");
    hipError_t e = jc::to_lp_launch(src, dst, (uint64_t)count, dtype == JC_F16, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_to_lp(jc_ctx* ctx, const float* src, void* dst, int64_t count, int dtype) {
    const char* W = "jc_to_lp";
    int rc = use(ctx, W);
    if (rc) return rc;
    return launch_to_lp(ctx, W, src, dst, count, dtype);
}

static int layer_lp(jc_ctx* ctx, const char* W, float* x, const jc_c2_layer_weights* w, const int32_t* live,
                    const float* table, const int32_t* group_start, const int32_t* group_end, void* workspace, int rows,
                    int n, int d, int heads, int dh, int dff, float eps, int dtype) {
    const int inner = heads * dh, T = rows * n;
    const size_t t = (size_t)T;
    const size_t big_bytes = (size_t)(12 * inner > 2 * dff ? 12 * inner : 2 * dff);
    char* ws = static_cast<char*>(workspace);
    void* hn = ws;                                                   // [T, d] storage type
    void* big = ws + round256(t * d * 2);                            // qkv [T, 3*inner] (storage type or fp32) or act [T, dff]
    void* att = ws + round256(t * d * 2) + round256(t * big_bytes) + round256(t * (size_t)inner * 4);  // [T, inner]
    int rc;
    // time attention sub-layer (Chronos2Forward.java:260-271), qkv and att in the storage type
    if ((rc = launch_rms_lp(ctx, W, x, w->time_norm, hn, T, d, eps, dtype))) return rc;
    if ((rc = launch_linear_lp(ctx, W, hn, d, w->time_qkv, w->time_qkv_bias, big, 3 * inner, T, 3 * inner, d, 0, dtype,
                               dtype)))
        return rc;
    if ((rc = jc_c2_time_attention(ctx, big, att, live, table, rows, n, heads, dh, inner, dtype))) return rc;
    if ((rc = launch_linear_lp(ctx, W, att, inner, w->time_o, w->time_o_bias, x, d, T, d, inner, JC_GEMM_ACCUMULATE,
                               dtype, JC_F32)))
        return rc;
    // group attention sub-layer (Chronos2Forward.java:273-281), qkv and att in the storage type
    if ((rc = launch_rms_lp(ctx, W, x, w->group_norm, hn, T, d, eps, dtype))) return rc;
    if ((rc = launch_linear_lp(ctx, W, hn, d, w->group_qkv, w->group_qkv_bias, big, 3 * inner, T, 3 * inner, d, 0,
                               dtype, dtype)))
        return rc;
    if ((rc = jc_c2_group_attention(ctx, big, att, live, group_start, group_end, rows, n, heads, dh, inner, dtype)))
        return rc;
    if ((rc = launch_linear_lp(ctx, W, att, inner, w->group_o, w->group_o_bias, x, d, T, d, inner, JC_GEMM_ACCUMULATE,
                               dtype, JC_F32)))
        return rc;
    // feed-forward sub-layer (Chronos2Forward.java:283-286)
    if ((rc = launch_rms_lp(ctx, W, x, w->mlp_norm, hn, T, d, eps, dtype))) return rc;
    if ((rc = launch_linear_lp(ctx, W, hn, d, w->wi, w->wi_bias, big, dff, T, dff, d, JC_GEMM_RELU, dtype, dtype)))
        return rc;
    return launch_linear_lp(ctx, W, big, dff, w->wo, w->wo_bias, x, d, T, d, dff, JC_GEMM_ACCUMULATE, dtype, JC_F32);
}

// ---- fp32 layer on fp16 operand splits (JC_F16X3) ------------------------------------------------

static int launch_split_x3(jc_ctx* ctx, const char* W, const float* src, int ld, void* dst, int rows, int k,
                           int weights) {
    if (rows < 0 || k < 0) return fail(JC_EINVAL, "%s: negative size (rows=%d k=%d)", W, rows, k);
    if ((size_t)rows * k == 0) return JC_OK;
    if (!src || !dst) return fail(JC_EINVAL, "%s: null src or dst", W);
    if (k % 4 || ld < k || ld % 4) return fail(JC_EINVAL, "%s: k and ld must be multiples of 4, ld >= k (k=%d ld=%d)", W, k, ld);
    if (!aligned16(src) || ((uintptr_t)dst & 7u)) return fail(JC_EINVAL, "%s: src 16-byte and dst 8-byte alignment", W);
    if (weights != 0 && weights != 1) return fail(JC_EINVAL, "%s: weights must be 0 or 1 (got %d)", W, weights);
    ProfScope ps(ctx, "split_f16x3");
    hipError_t e = jc::split_x3_launch(src, ld, dst, rows, k, weights == 1, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_split_f16x3(jc_ctx* ctx, const float* src, int ld_src, void* dst, int rows, int k, int weights) {
    const char* W = "jc_split_f16x3";
    int rc = use(ctx, W);
    if (rc) return rc;
    return launch_split_x3(ctx, W, src, ld_src, dst, rows, k, weights);
}

// The JC_F32 layer with every GEMM on the operands' three-term fp16 splits: the norms write the
// A-operand split of hn directly, the attention kernels write the split of their outputs (64-wide
// heads; other widths go through fp32 and a split pass), the MLP activation is split before its
// GEMM, and every GEMM (K = 3k, fp32 accumulation) writes fp32.
static int layer_x3(jc_ctx* ctx, const char* W, float* x, const jc_c2_layer_weights* w, const int32_t* live,
                    const float* table, const int32_t* group_start, const int32_t* group_end, void* workspace, int rows,
                    int n, int d, int heads, int dh, int dff, float eps) {
    const int inner = heads * dh, T = rows * n;
    const size_t t = (size_t)T;
    const size_t big_cols = (size_t)(3 * inner > dff ? 3 * inner : dff);
    char* ws = static_cast<char*>(workspace);
    float* big = reinterpret_cast<float*>(ws);                                  // qkv [T, 3*inner] or act [T, dff]
    float* att = reinterpret_cast<float*>(ws + round256(t * big_cols * 4));    // [T, inner]
    void* a3 = ws + round256(t * big_cols * 4) + round256(t * (size_t)inner * 4);  // [T, 3k] fp16, k <= max(d, inner, dff)
    const int F = JC_F16;
    int rc;
    auto rms3 = [&](const float* nw) -> int {
        ProfScope ps(ctx, "rms_norm (split out)");
        hipError_t e = jc::rms_norm_x3_launch(x, a3, nw, T, d, eps, ctx->stream);
        return e == hipSuccess ? JC_OK : hip_fail(W, e);
    };
    // time attention sub-layer (Chronos2Forward.java:260-271)
    if ((rc = rms3(w->time_norm))) return rc;
    if ((rc = launch_linear_lp(ctx, W, a3, 3 * d, w->time_qkv, w->time_qkv_bias, big, 3 * inner, T, 3 * inner, 3 * d, 0,
                               F, JC_F32)))
        return rc;
    const bool fused = dh == 64;  // the attention kernels write the split themselves
    if (fused) {
        if ((rc = c2_time(ctx, W, big, a3, live, table, rows, n, heads, dh, inner, JC_F32, true))) return rc;
    } else {
        if ((rc = c2_time(ctx, W, big, att, live, table, rows, n, heads, dh, inner, JC_F32, false))) return rc;
        if ((rc = launch_split_x3(ctx, W, att, inner, a3, T, inner, 0))) return rc;
    }
    if ((rc = launch_linear_lp(ctx, W, a3, 3 * inner, w->time_o, w->time_o_bias, x, d, T, d, 3 * inner,
                               JC_GEMM_ACCUMULATE, F, JC_F32)))
        return rc;
    // group attention sub-layer (Chronos2Forward.java:273-281)
    if ((rc = rms3(w->group_norm))) return rc;
    if ((rc = launch_linear_lp(ctx, W, a3, 3 * d, w->group_qkv, w->group_qkv_bias, big, 3 * inner, T, 3 * inner, 3 * d,
                               0, F, JC_F32)))
        return rc;
    if (fused) {
        if ((rc = c2_group(ctx, W, big, a3, live, group_start, group_end, rows, n, heads, dh, inner, JC_F32, true)))
            return rc;
    } else {
        if ((rc = c2_group(ctx, W, big, att, live, group_start, group_end, rows, n, heads, dh, inner, JC_F32, false)))
            return rc;
        if ((rc = launch_split_x3(ctx, W, att, inner, a3, T, inner, 0))) return rc;
    }
    if ((rc = launch_linear_lp(ctx, W, a3, 3 * inner, w->group_o, w->group_o_bias, x, d, T, d, 3 * inner,
                               JC_GEMM_ACCUMULATE, F, JC_F32)))
        return rc;
    // feed-forward sub-layer (Chronos2Forward.java:283-286)
    if ((rc = rms3(w->mlp_norm))) return rc;
    if ((rc = launch_linear_lp(ctx, W, a3, 3 * d, w->wi, w->wi_bias, big, dff, T, dff, 3 * d, JC_GEMM_RELU, F, JC_F32)))
        return rc;
    if ((rc = launch_split_x3(ctx, W, big, dff, a3, T, dff, 0))) return rc;
    return launch_linear_lp(ctx, W, a3, 3 * dff, w->wo, w->wo_bias, x, d, T, d, 3 * dff, JC_GEMM_ACCUMULATE, F, JC_F32);
}

// ---- The rest of the Chronos-2 forward ------------------------------------------------------

int jc_c2_assemble(jc_ctx* ctx, const float* emb, const float* reg, float* x, int rows, int nc, int nreg, int n, int d) {
    const char* W = "jc_c2_assemble";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || nc < 0 || nreg < 0 || nreg > 1 || nc + nreg > n || d <= 0)
        return fail(JC_EINVAL, "%s: sizes (rows=%d nc=%d nreg=%d n=%d d=%d)", W, rows, nc, nreg, n, d);
    if ((size_t)rows * n == 0) return JC_OK;
    if (d % 4) return fail(JC_EINVAL, "%s: d must be a multiple of 4 (got %d)", W, d);
    if (!x || (n > nreg && !emb) || (nreg && !reg)) return fail(JC_EINVAL, "%s: null buffer", W);
    if (!aligned16(x) || (emb && !aligned16(emb)) || (reg && !aligned16(reg)))
        return fail(JC_EINVAL, "%s: 16-byte alignment", W);
    ProfScope ps(ctx, "c2 assemble");
    hipError_t e = jc::assemble_tokens_launch(emb, reg, x, rows, nc, nreg, n, d, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_c2_prep(jc_ctx* ctx, const float* context, int64_t ld_context, int steps, const float* future,
               int64_t ld_future, int future_steps, const int32_t* order, int rows, int context_length, int patch,
               int h, int nreg, float time_scale, int arcsinh, float* tokens, float* loc, float* scale,
               int32_t* live) {
    const char* W = "jc_c2_prep";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || steps < 0 || context_length < 1 || patch < 1 || h < 1 || nreg < 0 || nreg > 1)
        return fail(JC_EINVAL, "%s: sizes (rows=%d steps=%d context_length=%d patch=%d h=%d nreg=%d)", W, rows, steps,
                    context_length, patch, h, nreg);
    if (ld_context < steps || (future && (future_steps < 0 || future_steps > h * patch || ld_future < future_steps)))
        return fail(JC_EINVAL, "%s: row strides (ld_context=%lld steps=%d ld_future=%lld future_steps=%d, h*patch=%d)",
                    W, (long long)ld_context, steps, (long long)ld_future, future_steps, h * patch);
    if (!(time_scale > 0.f)) return fail(JC_EINVAL, "%s: time_scale must be positive", W);
    if (rows == 0) return JC_OK;
    if ((!context && steps > 0) || !tokens || !loc || !scale || !live) return fail(JC_EINVAL, "%s: null buffer", W);
    const int kept = steps < context_length ? steps : context_length;
    const int nc = (kept + patch - 1) / patch;
    ProfScope ps(ctx, "c2 prep");
    hipError_t e = jc::c2_prep_launch(context, ld_context, steps, future, ld_future, future ? future_steps : 0, order,
                                      rows, kept, nc, h, patch, nreg, time_scale, arcsinh, tokens, loc, scale, live,
                                      ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_c2_finish(jc_ctx* ctx, const float* raw, const float* loc, const float* scale, const int32_t* order, int rows,
                 int h, int q, int patch, int arcsinh, float* out) {
    const char* W = "jc_c2_finish";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || h < 1 || q < 1 || patch < 1)
        return fail(JC_EINVAL, "%s: sizes (rows=%d h=%d q=%d patch=%d)", W, rows, h, q, patch);
    if (rows == 0) return JC_OK;
    if (!raw || !loc || !scale || !out) return fail(JC_EINVAL, "%s: null buffer", W);
    ProfScope ps(ctx, "c2 finish");
    hipError_t e = jc::c2_finish_launch(raw, loc, scale, order, rows, h, q, patch, arcsinh, out, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_c2_gather_future(jc_ctx* ctx, const float* y, float* dec, int rows, int fs, int n, int h, int d) {
    const char* W = "jc_c2_gather_future";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || fs < 0 || h < 0 || fs + h > n || d <= 0)
        return fail(JC_EINVAL, "%s: sizes (rows=%d fs=%d h=%d n=%d d=%d)", W, rows, fs, h, n, d);
    if ((size_t)rows * h == 0) return JC_OK;
    if (d % 4) return fail(JC_EINVAL, "%s: d must be a multiple of 4 (got %d)", W, d);
    if (!y || !dec) return fail(JC_EINVAL, "%s: null buffer", W);
    if (!aligned16(y) || !aligned16(dec)) return fail(JC_EINVAL, "%s: 16-byte alignment", W);
    ProfScope ps(ctx, "c2 gather_future");
    hipError_t e = jc::gather_future_launch(y, dec, rows, fs, n, h, d, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

// a residual block as the plans queue it: hidden with the activation into scratch, output into out,
// residual accumulated into out
static int residual_block(jc_ctx* ctx, const char* W, const float* x, int m, int din, const float* w_hidden,
                          const float* b_hidden, const float* w_output, const float* b_output, const float* w_residual,
                          const float* b_residual, int dff, int dout, float* scratch, float* out, int act) {
    int rc = use(ctx, W);
    if (rc) return rc;
    if (!scratch || !w_hidden || !w_output || !w_residual) return fail(JC_EINVAL, "%s: null weight or scratch", W);
    if ((rc = launch_linear(ctx, W, x, din, w_hidden, b_hidden, scratch, dff, m, dff, din, act))) return rc;
    if ((rc = launch_linear(ctx, W, scratch, dff, w_output, b_output, out, dout, m, dout, dff, 0))) return rc;
    return launch_linear(ctx, W, x, din, w_residual, b_residual, out, dout, m, dout, din, JC_GEMM_ACCUMULATE);
}

int jc_c2_residual(jc_ctx* ctx, const float* x, int m, int din, const float* w_hidden, const float* b_hidden,
                   const float* w_output, const float* b_output, const float* w_residual, const float* b_residual, int dff,
                   int dout, float* scratch, float* out) {
    // Chronos2Forward.Plan.residual: ReLU hidden layer
    return residual_block(ctx, "jc_c2_residual", x, m, din, w_hidden, b_hidden, w_output, b_output, w_residual,
                          b_residual, dff, dout, scratch, out, JC_GEMM_RELU);
}

int jc_ts_residual(jc_ctx* ctx, const float* x, int m, int din, const float* w_hidden, const float* b_hidden,
                   const float* w_output, const float* b_output, const float* w_residual, const float* b_residual, int dff,
                   int dout, float* scratch, float* out) {
    // TimestralForward.Plan.residual: SiLU hidden layer
    return residual_block(ctx, "jc_ts_residual", x, m, din, w_hidden, b_hidden, w_output, b_output, w_residual,
                          b_residual, dff, dout, scratch, out, JC_GEMM_SILU);
}

int jc_ts_assemble(jc_ctx* ctx, const float* emb, const float* query, float* x, int rows, int enc, int n, int d) {
    const char* W = "jc_ts_assemble";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || enc < 0 || enc > n || d <= 0)
        return fail(JC_EINVAL, "%s: sizes (rows=%d enc=%d n=%d d=%d)", W, rows, enc, n, d);
    if ((size_t)rows * n == 0) return JC_OK;
    if (d % 4) return fail(JC_EINVAL, "%s: d must be a multiple of 4 (got %d)", W, d);
    if (!x || (enc && !emb) || (n > enc && !query)) return fail(JC_EINVAL, "%s: null buffer", W);
    if (!aligned16(x) || (emb && !aligned16(emb)) || (query && !aligned16(query)))
        return fail(JC_EINVAL, "%s: 16-byte alignment", W);
    ProfScope ps(ctx, "ts assemble");
    hipError_t e = jc::ts_assemble_launch(emb, query, x, rows, enc, n, d, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_ts_gather_decoder(jc_ctx* ctx, const float* y, float* dec, int rows, int enc, int n, int h, int d) {
    const char* W = "jc_ts_gather_decoder";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || enc < 0 || h < 0 || enc + h > n || d <= 0)
        return fail(JC_EINVAL, "%s: sizes (rows=%d enc=%d h=%d n=%d d=%d)", W, rows, enc, h, n, d);
    if ((size_t)rows * h == 0) return JC_OK;
    if (d % 4) return fail(JC_EINVAL, "%s: d must be a multiple of 4 (got %d)", W, d);
    if (!y || !dec) return fail(JC_EINVAL, "%s: null buffer", W);
    if (!aligned16(y) || !aligned16(dec)) return fail(JC_EINVAL, "%s: 16-byte alignment", W);
    ProfScope ps(ctx, "ts gather_decoder");
    hipError_t e = jc::gather_future_launch(y, dec, rows, enc, n, h, d, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_swiglu(jc_ctx* ctx, const void* up, void* act, int64_t tokens, int f, int dtype) {
    const char* W = "jc_swiglu";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (dtype != JC_F32 && dtype != JC_BF16 && dtype != JC_F16 && dtype != JC_F16X3)
        return fail(JC_EINVAL, "%s: unknown dtype %d", W, dtype);
    if (tokens < 0 || f < 0) return fail(JC_EINVAL, "%s: negative size (tokens=%lld f=%d)", W, (long long)tokens, f);
    if (tokens * (int64_t)f == 0) return JC_OK;
    if (!up || !act) return fail(JC_EINVAL, "%s: null up or act", W);
    if (dtype == JC_F16X3 && (f % 4 || !aligned16(up) || !aligned16(act)))
        return fail(JC_EINVAL, "%s: JC_F16X3 needs f a multiple of 4 (got %d) and 16-byte alignment", W, f);
    ProfScope ps(ctx, "swiglu");
    hipError_t e = jc::swiglu_launch(up, act, (uint64_t)tokens, f, dtype, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_ts_prep(jc_ctx* ctx, const float* window, const uint8_t* observed, int rows, int w, int patch,
               const int32_t* known, float minimum_scale, int use_asinh, float* tokens, float* scaled, float* loc,
               float* scale) {
    const char* W = "jc_ts_prep";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || w < 0 || patch < 1 || patch > 64 || w % patch)
        return fail(JC_EINVAL, "%s: sizes (rows=%d w=%d patch=%d; 1 <= patch <= 64 dividing w)", W, rows, w, patch);
    if ((int64_t)rows * w == 0) return JC_OK;
    if (!window || !observed || !tokens || !loc || !scale) return fail(JC_EINVAL, "%s: null buffer", W);
    ProfScope ps(ctx, "ts prep");
    hipError_t e = jc::ts_prep_launch(window, observed, rows, w, patch, known, minimum_scale, use_asinh, tokens, scaled,
                                      loc, scale, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

int jc_ts_finish(jc_ctx* ctx, const float* raw, const float* loc, const float* scale, int rows, int w,
                 int context_patches, int h, int patch, int q, const float* width, int median, int use_asinh,
                 float* out) {
    const char* W = "jc_ts_finish";
    int rc = use(ctx, W);
    if (rc) return rc;
    if (rows < 0 || h < 1 || patch < 1 || q < 1 || q > jc::kTsMaxQuantiles || median < 0 || median >= q)
        return fail(JC_EINVAL, "%s: sizes (rows=%d h=%d patch=%d q=%d median=%d; q <= %d)", W, rows, h, patch, q, median,
                    jc::kTsMaxQuantiles);
    if (context_patches < 1 || (int64_t)context_patches * patch > w)
        return fail(JC_EINVAL, "%s: context_patches=%d * patch=%d exceeds the window w=%d", W, context_patches, patch, w);
    if (rows == 0) return JC_OK;
    if (!raw || !loc || !scale || !out || !width) return fail(JC_EINVAL, "%s: null buffer", W);
    ProfScope ps(ctx, "ts finish");
    hipError_t e = jc::ts_finish_launch(raw, loc, scale, rows, w, (context_patches - 1) * patch, h * patch, q, width,
                                        median, use_asinh, out, ctx->stream);
    return e == hipSuccess ? JC_OK : hip_fail(W, e);
}

}  // extern "C"
