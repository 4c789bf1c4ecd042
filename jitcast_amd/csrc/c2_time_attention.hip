// Chronos-2 time attention, fused flash-style for gfx950 (FP32 path).
//
// Replaces the reference's per-layer pair Chronos2Kernels.rope + Chronos2Kernels.timeAttention
// (Chronos2Kernels.java:87-116, 118-464; oracle CpuChronos2.java:175-228, 284-304):
// for every (row r, head h, query t), scores s_k = q_t . k_k over the keys k with live[r*n+k]
// (unscaled, both directions), o_t = sum_k softmax(s)_k v_k, and o_t = 0 when no key is live.
// RoPE rotates q and k at load from the host-built table [n, dh] (cos half, then sin half).
//
// Layout: qkv [rows*n, 3*inner] (q | k | v, heads-major per token), out [rows*n, inner], live
// [rows*n] int32. One workgroup = 4 waves = 128 consecutive queries of one (row, head); each wave
// owns 32 queries. Keys stream through LDS in blocks of KB, double-buffered. Blocks start at the
// row's first live key, so left padding costs nothing and dead blocks inside the row (gaps) are
// skipped from a per-block live bitmask.
//
// MFMA mapping (v_mfma_f32_32x32x2_f32, 64 flops/clk/SIMD):
//   S^T[key][q] = K Q^T   A = K  (lane i+32kk: K[key i][kk*dh/2 + s]),  B = Q (same dim map)
//   O^T[e][q]  += V^T P^T A = V^T (lane i+32kk: V[key(kk,c)][e]),        B = P straight from S^T
// The dimension map d(s,kk) = kk*dh/2 + s puts the RoPE pair (e, e+dh/2) in the two lane halves of
// one step, and the accumulator layout of S^T is exactly the B-operand layout P^T needs, so P
// never leaves registers. With queries along lanes, the online-softmax state of a query lives in
// lanes j and j+32: the block max needs one v_permlane32_swap.
//
// K/V/table prefetch uses buffer loads whose per-thread VGPR offset never changes; the block moves
// through the SGPR resource base. Keys past the end of the row fall outside the resource's
// num_records and read as 0 (and are masked), so the load path has no per-lane bounds branches.
#include "jc_common.hpp"
#include "jc_kernels.hpp"

#include <cstdlib>

namespace jc {
namespace {

constexpr int kQ = 32;        // queries per wave
constexpr int kWaves = 4;     // waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxTokens = 4096;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format (gfx9 family)

template <int DH, int KB>
struct TimeF32Lds {
    static constexpr int kPitchK = DH + 4;         // floats per key row of K
    static constexpr int kTiles = (DH + 31) / 32;  // 32-dim output tiles
    static constexpr int kPitchV = KB + 4;         // floats per dim row of V^T
    float k[2][KB * kPitchK];
    float vt[2][kTiles * 32 * kPitchV];
    uint64_t mask[kMaxTokens / KB];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// One KB-key block of K (rotated at store) and V for (row, head), staged through registers:
// item i of thread tid covers key (tid + i*256) / (dh/8) and dims e..e+3 of each half.
template <int DH, int KB, bool ROPE>
struct KvStage {
    static constexpr int kQuads = DH / 8;
    static constexpr int kItems = KB * kQuads;
    static constexpr int kPer = (kItems + kThreads - 1) / kThreads;
    floatx4 k0[kPer], k1[kPer], v0[kPer], v1[kPer], c[kPer], s[kPer];
    uint32_t off_kv[kPer], off_tab[kPer];  // loop-invariant byte offsets

    __device__ __forceinline__ void init(int tid, int inner) {
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            int it = tid + i * kThreads;
            int key = it / kQuads, e = (it % kQuads) * 4;
            off_kv[i] = (uint32_t)((key * 3 * inner + e) * 4);
            off_tab[i] = (uint32_t)((key * DH + e) * 4);
        }
    }

    // rk: resource over k of (row, head) from the block's first key; rt: over the table rows.
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rt, int tid, int inner) {
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            if (kItems % kThreads != 0 && tid + i * kThreads >= kItems) break;
            k0[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off_kv[i], 0, 0);
            k1[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off_kv[i] + DH * 2, 0, 0);
            v0[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off_kv[i] + inner * 4, 0, 0);
            v1[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off_kv[i] + inner * 4 + DH * 2, 0, 0);
            if (ROPE) {
                c[i] = __builtin_amdgcn_raw_buffer_load_b128(rt, off_tab[i], 0, 0);
                s[i] = __builtin_amdgcn_raw_buffer_load_b128(rt, off_tab[i] + DH * 2, 0, 0);
            }
        }
    }

    __device__ __forceinline__ void store(TimeF32Lds<DH, KB>& lds, int buf, int tid) {
        constexpr int PK = TimeF32Lds<DH, KB>::kPitchK, PV = TimeF32Lds<DH, KB>::kPitchV;
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            int it = tid + i * kThreads;
            if (kItems % kThreads != 0 && it >= kItems) break;
            int key = it / kQuads, e = (it % kQuads) * 4;
            floatx4 a0 = k0[i], a1 = k1[i];
            if (ROPE) {
                a0 = k0[i] * c[i] - k1[i] * s[i];
                a1 = k1[i] * c[i] + k0[i] * s[i];
            }
            float* kr = &lds.k[buf][key * PK];
            *reinterpret_cast<floatx4*>(kr + e) = a0;
            *reinterpret_cast<floatx4*>(kr + DH / 2 + e) = a1;
            float* vt = lds.vt[buf];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                vt[(e + u) * PV + key] = v0[i][u];
                vt[(DH / 2 + e + u) * PV + key] = v1[i][u];
            }
        }
    }
};

template <int DH, int KB, bool ROPE>
__global__ __launch_bounds__(kThreads) void c2_time_attention_f32(const float* __restrict__ qkv,
                                                                  float* __restrict__ out,
                                                                  const int32_t* __restrict__ live,
                                                                  const float* __restrict__ table, int rows, int n,
                                                                  int heads, int inner, int qgroups) {
    static_assert(DH % 8 == 0 && DH <= 64, "head width");
    static_assert(KB == 32 || KB == 64, "key block");
    constexpr int kHalf = DH / 2;
    constexpr int kSteps = kHalf;  // K=2 per MFMA step: one dim from each lane half
    constexpr int kTiles = TimeF32Lds<DH, KB>::kTiles;
    constexpr int kSub = KB / 32;  // 32-key S^T tiles per block
    constexpr int PK = TimeF32Lds<DH, KB>::kPitchK, PV = TimeF32Lds<DH, KB>::kPitchV;
    __shared__ TimeF32Lds<DH, KB> lds;
    __shared__ int first_live;

    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int j = lane % 32, g = lane / 32;
    const uint32_t total = (uint32_t)rows * heads * qgroups;
    const uint32_t logical = xcd_remap(blockIdx.x, total);
    const int qg = logical % qgroups;
    const int bh = logical / qgroups;
    const int h = bh % heads, r = bh / heads;
    const int32_t* lrow = live + (size_t)r * n;

    // padded V^T rows (DH not a multiple of 32) feed only discarded output dims; zero them once
    if (DH % 32 != 0) {
        for (int i = tid; i < 2 * kTiles * 32 * PV; i += kThreads) (&lds.vt[0][0])[i] = 0.f;
    }
    // the row's first live key (n if none)
    if (tid == 0) first_live = n;
    __syncthreads();
    for (int base = wave * kWave; base < n; base += kThreads) {
        int k = base + lane;
        uint64_t bits = __ballot(k < n && lrow[k] != 0);
        if (bits && lane == 0) atomicMin(&first_live, base + (int)__builtin_ctzll(bits));
    }
    __syncthreads();
    const int kstart = first_live;
    const int nb = (n - kstart + KB - 1) / KB;
    // per-block live bitmasks from kstart: bit b of mask[kb] = key kstart + kb*KB + b
    for (int kb = wave; kb * KB < n - kstart; kb += kWaves) {
        uint64_t bits = 0;
#pragma unroll
        for (int part = 0; part < KB / 64 + (KB < 64); part++) {
            int k = kstart + kb * KB + part * 64 + lane;
            bool ok = (KB == 64 || lane < 32) && k < n && lrow[k] != 0;
            bits |= __ballot(ok);
        }
        if (lane == 0) lds.mask[kb] = bits;
    }

    // Q in registers: lane (j, g) holds dims g*dh/2 + s of query q0+j, rotated and scaled by log2(e)
    const int q0 = (qg * kWaves + wave) * kQ;
    const int nq = min(max(n - q0, 0), kQ);
    float qreg[kSteps];
    {
        int q = q0 + j;
#pragma unroll
        for (int s = 0; s < kSteps; s++) qreg[s] = 0.f;
        if (j < nq) {
            const float* qp = qkv + ((size_t)r * n + q) * 3 * inner + h * DH;
#pragma unroll
            for (int s4 = 0; s4 < kSteps / 4; s4++) {
                floatx4 a = *reinterpret_cast<const floatx4*>(qp + 4 * s4);
                floatx4 b = *reinterpret_cast<const floatx4*>(qp + kHalf + 4 * s4);
                floatx4 o = g == 0 ? a : b;
                if (ROPE) {
                    floatx4 c = *reinterpret_cast<const floatx4*>(table + (size_t)q * DH + 4 * s4);
                    floatx4 sn = *reinterpret_cast<const floatx4*>(table + (size_t)q * DH + kHalf + 4 * s4);
                    o = g == 0 ? a * c - b * sn : b * c + a * sn;
                }
#pragma unroll
                for (int u = 0; u < 4; u++) qreg[4 * s4 + u] = o[u] * kLog2e;
            }
        }
    }
    __syncthreads();

    // resources: the k of (row, head) from key kstart + kb*KB to the end of the row; the table rows
    const size_t row0 = (size_t)r * n;
    const uint32_t stride_b = 3u * inner * 4u;
    auto rk_at = [&](int kb) {
        int k = kstart + kb * KB;
        const float* p = qkv + (row0 + k) * 3 * inner + inner + h * DH;
        uint32_t bytes = (uint32_t)(n - k) * stride_b - (uint32_t)(inner + h * DH) * 4u;
        return make_rsrc(p, bytes);
    };
    auto rt_at = [&](int kb) {
        int k = kstart + kb * KB;
        return make_rsrc(table + (size_t)k * DH, (uint32_t)((n - k) * DH * 4));
    };

    int kb = 0;
    while (kb < nb && lds.mask[kb] == 0) kb++;

    KvStage<DH, KB, ROPE> stage;
    stage.init(tid, inner);
    if (kb < nb) {
        stage.load(rk_at(kb), ROPE ? rt_at(kb) : rk_at(kb), tid, inner);
        stage.store(lds, 0, tid);
    }
    __syncthreads();

    floatx16 o_acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; t++) o_acc[t] = floatx16{0};
    float m_run = -INFINITY, l_run = 0.f;
    int buf = 0;
    // Settle every prologue load here: the compiler cannot prove that the divergent Q loads were
    // consumed on all paths and would otherwise wait on them (vmcnt(0)) inside every iteration.
    __builtin_amdgcn_s_waitcnt(0);

    while (kb < nb) {
        int next = kb + 1;
        while (next < nb && lds.mask[next] == 0) next++;
        if (next < nb) stage.load(rk_at(next), ROPE ? rt_at(next) : rk_at(next), tid, inner);
        // keep the prefetch above the block's MFMAs (the scheduler would sink it to its use)
        __builtin_amdgcn_sched_barrier(0);

        if (nq > 0) {
            // S^T = K Q^T over this block, one 32x32 tile per 32 keys
            floatx16 s_acc[kSub];
#pragma unroll
            for (int sb = 0; sb < kSub; sb++) {
                s_acc[sb] = floatx16{0};
                const float* kp = &lds.k[buf][(32 * sb + j) * PK + g * kHalf];
#pragma unroll
                for (int s4 = 0; s4 < kSteps / 4; s4++) {
                    floatx4 kv = *reinterpret_cast<const floatx4*>(kp + 4 * s4);
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        s_acc[sb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[u], qreg[4 * s4 + u], s_acc[sb], 0, 0, 0);
                }
            }
            // mask: reg rho of tile sb in lane (j, g) holds key 32sb + 8*(rho/4) + 4g + rho%4 of the block
            uint64_t km = lds.mask[kb];
            if (km != (KB == 64 ? ~0ull : 0xffffffffull)) {
#pragma unroll
                for (int sb = 0; sb < kSub; sb++) {
#pragma unroll
                    for (int rho = 0; rho < 16; rho++) {
                        int bit = 32 * sb + 8 * (rho / 4) + 4 * g + (rho % 4);
                        if (!((km >> bit) & 1ull)) s_acc[sb][rho] = -INFINITY;
                    }
                }
            }
            float mx = s_acc[0][0];
#pragma unroll
            for (int sb = 0; sb < kSub; sb++)
#pragma unroll
                for (int rho = 0; rho < 16; rho++) mx = fmaxf(mx, s_acc[sb][rho]);
            mx = pair_max(mx);
            float m_new = fmaxf(m_run, mx);
            float m_use = m_new == -INFINITY ? 0.f : m_new;
            float alpha = fast_exp2(m_run - m_use);
            m_run = m_new;
            float rs = 0.f;
#pragma unroll
            for (int sb = 0; sb < kSub; sb++)
#pragma unroll
                for (int rho = 0; rho < 16; rho++) {
                    s_acc[sb][rho] = fast_exp2(s_acc[sb][rho] - m_use);
                    rs += s_acc[sb][rho];
                }
            l_run = l_run * alpha + rs;
            // rescale O only when some query's running max moved (wave-uniform branch)
            if (__any(alpha != 1.f)) {
#pragma unroll
                for (int t = 0; t < kTiles; t++) o_acc[t] *= alpha;
            }
            // O^T += V^T P^T: step c = 4a + u of tile sb uses keys 32sb + 8a + 4kk + u, P from s_acc[sb][c]
#pragma unroll
            for (int t = 0; t < kTiles; t++) {
                const float* vp = &lds.vt[buf][(32 * t + j) * PV + 4 * g];
#pragma unroll
                for (int sb = 0; sb < kSub; sb++) {
#pragma unroll
                    for (int a = 0; a < 4; a++) {
                        floatx4 vv = *reinterpret_cast<const floatx4*>(vp + 32 * sb + 8 * a);
#pragma unroll
                        for (int u = 0; u < 4; u++)
                            o_acc[t] =
                                __builtin_amdgcn_mfma_f32_32x32x2f32(vv[u], s_acc[sb][4 * a + u], o_acc[t], 0, 0, 0);
                    }
                }
            }
        }
        if (next < nb) stage.store(lds, buf ^ 1, tid);
        __syncthreads();
        buf ^= 1;
        kb = next;
    }

    // every lane reaches the swap (its partner holds the other half of the same query)
    float l = pair_sum(l_run);
    if (j < nq) {
        float inv = l > 0.f ? 1.f / l : 0.f;
        float* op = out + ((size_t)r * n + q0 + j) * inner + h * DH;
        // O^T reg 4a+u of lane (j, g) is dim 32t + 8a + 4g + u of query j
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
#pragma unroll
            for (int a = 0; a < 4; a++) {
                int e = 32 * t + 8 * a + 4 * g;
                if (e < DH) {
                    floatx4 v;
#pragma unroll
                    for (int u = 0; u < 4; u++) v[u] = o_acc[t][4 * a + u] * inv;
                    *reinterpret_cast<floatx4*>(op + e) = v;
                }
            }
        }
    }
}

}  // namespace

template <int DH, int KB>
static hipError_t launch_f32(const float* qkv, float* out, const int32_t* live, const float* table, int rows, int n,
                             int heads, int inner, hipStream_t stream) {
    int tiles = (n + kQ - 1) / kQ;
    int qgroups = (tiles + kWaves - 1) / kWaves;
    uint64_t grid = (uint64_t)rows * heads * qgroups;
    if (table) {
        hipLaunchKernelGGL((c2_time_attention_f32<DH, KB, true>), dim3((uint32_t)grid), dim3(kThreads), 0, stream,
                           qkv, out, live, table, rows, n, heads, inner, qgroups);
    } else {
        hipLaunchKernelGGL((c2_time_attention_f32<DH, KB, false>), dim3((uint32_t)grid), dim3(kThreads), 0, stream,
                           qkv, out, live, table, rows, n, heads, inner, qgroups);
    }
    return hipGetLastError();
}

// Key-block size: 32 by default; JITCAST_C2_TIME_KB=64 selects 64-key blocks (read once).
static int key_block() {
    static int kb = [] {
        const char* e = getenv("JITCAST_C2_TIME_KB");
        return (e && atoi(e) == 64) ? 64 : 32;
    }();
    return kb;
}

template <int KB>
static hipError_t dispatch_f32(const float* qkv, float* out, const int32_t* live, const float* table, int rows,
                               int n, int heads, int dh, int inner, hipStream_t stream) {
    switch (dh) {
        case 16: return launch_f32<16, KB>(qkv, out, live, table, rows, n, heads, inner, stream);
        case 32: return launch_f32<32, KB>(qkv, out, live, table, rows, n, heads, inner, stream);
        case 48: return launch_f32<48, KB>(qkv, out, live, table, rows, n, heads, inner, stream);
        case 64: return launch_f32<64, KB>(qkv, out, live, table, rows, n, heads, inner, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t c2_time_attention_f32_launch(const float* qkv, float* out, const int32_t* live, const float* table,
                                        int rows, int n, int heads, int dh, int inner, hipStream_t stream) {
    if (key_block() == 64) return dispatch_f32<64>(qkv, out, live, table, rows, n, heads, dh, inner, stream);
    return dispatch_f32<32>(qkv, out, live, table, rows, n, heads, dh, inner, stream);
}

int c2_time_attention_max_tokens() { return kMaxTokens; }

}  // namespace jc
