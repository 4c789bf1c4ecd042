// Plain GEMMs on hipBLASLt: C[m, n] (+)= act(A[m, :k] . W[n, :k]^T + bias[n]) with row-major A, W and
// C, the contract of Kernels.gemm (J/tornado/Kernels.java:50-103) and the reference's cuBLAS path
// (Chronos2Forward.java:377-409). Row-major C = A W^T is the column-major product C^T = W A^T, so W
// is hipBLASLt's transposed first operand and A its second.
//
// The epilogue order is the reference's: bias, then the activation, then the accumulation. hipBLASLt
// applies its epilogue after alpha * W A^T + beta * C, so an activation with ACCUMULATE is declined
// (the caller runs its own kernel); BIAS with ACCUMULATE only reorders two additions. C in fp16 is
// declined too: the reference's FP16 twins saturate to +-65504 (Kernels.java:42-46), hipBLASLt's
// conversion does not.
//
// Per context: one handle and one workspace (made by jc_init), and a cache of descriptors and the
// heuristic's first algorithm per GEMM shape, so a call costs one descriptor update and the launch.
#include "jc_blas.hpp"

#include <hipblaslt/hipblaslt.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <unordered_map>
#include <unordered_set>

#include "../../include/jitcast_hip.h"

namespace jc {

namespace {

struct Key {
    int m, n, k, lda, ldc, ab, cd, epi, acc;
    bool operator==(const Key& o) const { return std::memcmp(this, &o, sizeof(Key)) == 0; }
};
struct KeyHash {
    size_t operator()(const Key& k) const {
        size_t h = 1469598103934665603ull;
        const unsigned char* p = reinterpret_cast<const unsigned char*>(&k);
        for (size_t i = 0; i < sizeof(Key); i++) h = (h ^ p[i]) * 1099511628211ull;
        return h;
    }
};

struct Entry {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;  // the heuristic found an algorithm
};

hipDataType hip_type(int dtype) {
    return dtype == JC_BF16 ? HIP_R_16BF : dtype == JC_F16 ? HIP_R_16F : HIP_R_32F;
}

}  // namespace

// an activation without a bias runs as activation-with-bias on zeros (x + 0 = x exactly): hipBLASLt
// has more algorithms for the bias forms
constexpr int kZeroBias = 1 << 16;

struct Blas {
    hipblasLtHandle_t handle = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    size_t ws_limit = 0;  // the most workspace an algorithm may ask for (JITCAST_HIP_BLAS_WORKSPACE)
    float* zeros = nullptr;  // kZeroBias floats
    std::unordered_map<Key, Entry, KeyHash> cache;
    std::unordered_set<uint64_t> reported;  // declined shapes already reported (JITCAST_HIP_BLAS_DEBUG)
};

Blas* blas_create() {
    Blas* b = new (std::nothrow) Blas();
    if (!b) return nullptr;
    if (hipblasLtCreate(&b->handle) != HIPBLAS_STATUS_SUCCESS) {
        delete b;
        return nullptr;
    }
    b->ws_bytes = kBlasWorkspaceBytes;
    b->ws_limit = b->ws_bytes;
    if (const char* e = getenv("JITCAST_HIP_BLAS_WORKSPACE")) {
        const unsigned long long v = strtoull(e, nullptr, 10);
        b->ws_limit = v < b->ws_bytes ? (size_t)v : b->ws_bytes;
    }
    if (hipMalloc(&b->ws, b->ws_bytes) != hipSuccess) {
        (void)hipblasLtDestroy(b->handle);
        delete b;
        return nullptr;
    }
    if (hipMalloc(&b->zeros, kZeroBias * sizeof(float)) != hipSuccess ||
        hipMemset(b->zeros, 0, kZeroBias * sizeof(float)) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(b->zeros);
        (void)hipFree(b->ws);
        (void)hipblasLtDestroy(b->handle);
        delete b;
        return nullptr;
    }
    return b;
}

void blas_destroy(Blas* b) {
    if (!b) return;
    for (auto& kv : b->cache) {
        Entry& e = kv.second;
        if (e.desc) (void)hipblasLtMatmulDescDestroy(e.desc);
        if (e.lw) (void)hipblasLtMatrixLayoutDestroy(e.lw);
        if (e.la) (void)hipblasLtMatrixLayoutDestroy(e.la);
        if (e.lc) (void)hipblasLtMatrixLayoutDestroy(e.lc);
    }
    (void)hipFree(b->zeros);
    (void)hipFree(b->ws);
    (void)hipblasLtDestroy(b->handle);
    delete b;
}

static Entry* entry_for(Blas* b, const Key& key) {
    auto it = b->cache.find(key);
    if (it != b->cache.end()) return &it->second;
    Entry e;
    const hipDataType ab = hip_type(key.ab), cd = hip_type(key.cd);
    bool good = hipblasLtMatmulDescCreate(&e.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    if (good) {
        const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
        const hipblasLtEpilogue_t epi = (hipblasLtEpilogue_t)key.epi;
        good = hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) == 0 &&
               hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) == 0 &&
               hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof epi) == 0;
        if (good && (key.epi & HIPBLASLT_EPILOGUE_BIAS)) {
            const hipDataType bt = HIP_R_32F;
            good = hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof bt) == 0;
        }
    }
    // W: column-major k x n (ld k); A: column-major k x m (ld lda); C: column-major n x m (ld ldc)
    good = good && hipblasLtMatrixLayoutCreate(&e.lw, ab, key.k, key.n, key.k) == 0 &&
           hipblasLtMatrixLayoutCreate(&e.la, ab, key.k, key.m, key.lda) == 0 &&
           hipblasLtMatrixLayoutCreate(&e.lc, cd, key.n, key.m, key.ldc) == 0;
    if (good) {
        hipblasLtMatmulPreference_t pref = nullptr;
        if (hipblasLtMatmulPreferenceCreate(&pref) == 0) {
            const uint64_t wsb = b->ws_limit;
            constexpr int kAsk = 8;
            hipblasLtMatmulHeuristicResult_t res[kAsk];
            int got = 0;
            if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                                      sizeof wsb) == 0 &&
                hipblasLtMatmulAlgoGetHeuristic(b->handle, e.desc, e.lw, e.la, e.lc, e.lc, pref, kAsk, res, &got) == 0) {
                for (int i = 0; i < got; i++) {  // the heuristic's order: the first that fits the workspace
                    if (res[i].workspaceSize <= b->ws_limit) {
                        e.algo = res[i].algo;
                        e.ok = true;
                        break;
                    }
                }
            }
            (void)hipblasLtMatmulPreferenceDestroy(pref);
        }
    }
    try {
        return &b->cache.emplace(key, e).first->second;
    } catch (...) {
        return nullptr;
    }
}

// JITCAST_HIP_BLAS_DEBUG=1 reports on stderr each GEMM shape this path declines, once per shape and context.
static bool debug_on() {
    static const bool on = [] {
        const char* e = getenv("JITCAST_HIP_BLAS_DEBUG");
        return e && *e == '1';
    }();
    return on;
}

static BlasStatus decline(Blas* b, const char* why, int m, int n, int k, int flags, int ab, int cd) {
    if (debug_on()) {
        uint64_t h = 1469598103934665603ull;
        for (int v : {m, n, k, flags, ab, cd}) h = (h ^ (uint32_t)v) * 1099511628211ull;
        bool fresh = true;
        try {
            fresh = b->reported.insert(h).second;
        } catch (...) {
        }
        if (fresh)
            fprintf(stderr, "[jc_blas] declined m=%d n=%d k=%d flags=%d ab=%d c=%d: %s\n", m, n, k, flags, ab, cd, why);
    }
    return kBlasDecline;
}

BlasStatus blas_gemm(Blas* b, const void* a, int lda, const void* w, const float* bias, void* c, int ldc, int m, int n,
                     int k, int flags, int ab_dtype, int c_dtype, hipStream_t stream) {
    if (!b) return kBlasDecline;
    const bool act = flags & (JC_GEMM_RELU | JC_GEMM_SILU);
    const bool acc = flags & JC_GEMM_ACCUMULATE;
    if ((act && acc) || c_dtype == JC_F16) return decline(b, "combination", m, n, k, flags, ab_dtype, c_dtype);
    if (c_dtype != JC_F32 && c_dtype != ab_dtype) return decline(b, "output type", m, n, k, flags, ab_dtype, c_dtype);
    bool has_bias = (flags & JC_GEMM_BIAS) && bias;
    if (act && !has_bias) {
        if (n > kZeroBias) return decline(b, "activation without a bias", m, n, k, flags, ab_dtype, c_dtype);
        bias = b->zeros;
        has_bias = true;
    }
    int epi = HIPBLASLT_EPILOGUE_DEFAULT;
    if (flags & JC_GEMM_RELU) epi = has_bias ? HIPBLASLT_EPILOGUE_RELU_BIAS : HIPBLASLT_EPILOGUE_RELU;
    else if (flags & JC_GEMM_SILU) epi = has_bias ? HIPBLASLT_EPILOGUE_SWISH_BIAS_EXT : HIPBLASLT_EPILOGUE_SWISH_EXT;
    else if (has_bias) epi = HIPBLASLT_EPILOGUE_BIAS;
    const Key key{m, n, k, lda, ldc, ab_dtype, c_dtype, epi, acc ? 1 : 0};
    Entry* e = entry_for(b, key);
    if (!e || !e->ok) return decline(b, "no algorithm", m, n, k, flags, ab_dtype, c_dtype);
    if (has_bias &&
        hipblasLtMatmulDescSetAttribute(e->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof bias) != 0)
        return kBlasError;
    const float alpha = 1.f, beta = acc ? 1.f : 0.f;
    const hipblasStatus_t s = hipblasLtMatmul(b->handle, e->desc, &alpha, w, e->lw, a, e->la, &beta, c, e->lc, c,
                                              e->lc, &e->algo, b->ws, b->ws_bytes, stream);
    return s == HIPBLAS_STATUS_SUCCESS ? kBlasDone : kBlasError;
}

}  // namespace jc
