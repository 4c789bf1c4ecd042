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
// owns 32 queries. Keys stream through LDS in blocks of 32, double-buffered; the blocks are
// aligned to the END of the row (n-32, n-64, ...) so that the always-live [REG]/future tokens share
// a block with the last context patches and left padding fills whole dead blocks, which are
// skipped from a per-block live bitmask.
//
// MFMA mapping (v_mfma_f32_32x32x2_f32, 64 flops/clk/SIMD):
//   S^T[key][q] = K Q^T   A = K  (lane i+32kk: K[key i][kk*dh/2 + s]),  B = Q (same dim map)
//   O^T[e][q]  += V^T P^T A = V^T (lane i+32kk: V[key(kk,c)][e]),        B = P straight from S^T
// The dimension map d(s,kk) = kk*dh/2 + s puts the RoPE pair (e, e+dh/2) in the two lane halves of
// one step, and the accumulator layout of S^T is exactly the B-operand layout P^T needs, so P
// never leaves registers. With queries along lanes, the online-softmax state of a query lives in
// lanes j and j+32: the block max needs one v_permlane32_swap.
#include "jc_common.hpp"
#include "jc_kernels.hpp"

namespace jc {
namespace {

constexpr int kQ = 32;        // queries per wave
constexpr int kKB = 32;       // keys per block
constexpr int kWaves = 4;     // waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxBlocks = 128;  // n <= 4096 keys per row

template <int DH>
struct TimeF32Lds {
    static constexpr int kHalf = DH / 2;
    static constexpr int kPitchK = DH + 4;                 // floats per key row of K
    static constexpr int kTiles = (DH + 31) / 32;          // 32-dim output tiles
    static constexpr int kPitchV = kKB + 4;                // floats per dim row of V^T
    float k[2][kKB * kPitchK];
    float vt[2][kTiles * 32 * kPitchV];
    uint32_t mask[kMaxBlocks];
};

// Loads one 32-key block of K (rotated) and V for (row, head) into registers: thread tid covers
// key tid / (dh/8) and the 4 dims e..e+3 of each half (e = 4 * (tid % (dh/8))).
template <int DH>
struct KvStage {
    static constexpr int kQuads = DH / 8;  // 4-dim quads per half
    static constexpr int kItems = kKB * kQuads;
    floatx4 k0, k1, v0, v1;
    bool valid;
    int key, e;

    __device__ __forceinline__ void load(const float* __restrict__ qkv, const float* __restrict__ table, int r,
                                         int h, int n, int inner, int k0_block, int tid) {
        valid = false;
        if (tid >= kItems) return;
        key = tid / kQuads;
        e = (tid % kQuads) * 4;
        int kg = k0_block + key;
        if (kg < 0 || kg >= n) return;
        valid = true;
        const float* base = qkv + ((size_t)r * n + kg) * 3 * inner + inner + h * DH;
        k0 = *reinterpret_cast<const floatx4*>(base + e);
        k1 = *reinterpret_cast<const floatx4*>(base + DH / 2 + e);
        v0 = *reinterpret_cast<const floatx4*>(base + inner + e);
        v1 = *reinterpret_cast<const floatx4*>(base + inner + DH / 2 + e);
        if (table) {
            floatx4 c = *reinterpret_cast<const floatx4*>(table + (size_t)kg * DH + e);
            floatx4 s = *reinterpret_cast<const floatx4*>(table + (size_t)kg * DH + DH / 2 + e);
            floatx4 a = k0, b = k1;
            k0 = a * c - b * s;
            k1 = b * c + a * s;
        }
    }

    __device__ __forceinline__ void store(TimeF32Lds<DH>& lds, int buf, int tid) {
        if (tid >= kItems) return;
        int kk = tid / kQuads, ee = (tid % kQuads) * 4;
        floatx4 z = {0.f, 0.f, 0.f, 0.f};
        floatx4 a0 = valid ? k0 : z, a1 = valid ? k1 : z, b0 = valid ? v0 : z, b1 = valid ? v1 : z;
        float* kr = &lds.k[buf][kk * TimeF32Lds<DH>::kPitchK];
        *reinterpret_cast<floatx4*>(kr + ee) = a0;
        *reinterpret_cast<floatx4*>(kr + DH / 2 + ee) = a1;
        float* vt = lds.vt[buf];
        constexpr int P = TimeF32Lds<DH>::kPitchV;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            vt[(ee + u) * P + kk] = b0[u];
            vt[(DH / 2 + ee + u) * P + kk] = b1[u];
        }
    }
};

template <int DH>
__global__ __launch_bounds__(kThreads) void c2_time_attention_f32(const float* __restrict__ qkv,
                                                                      float* __restrict__ out,
                                                                      const int32_t* __restrict__ live,
                                                                      const float* __restrict__ table, int rows,
                                                                      int n, int heads, int inner, int qgroups) {
    static_assert(DH % 8 == 0 && DH <= 64, "head width");
    constexpr int kHalf = DH / 2;
    constexpr int kSteps = kHalf;  // K=2 per MFMA step: one dim from each lane half
    constexpr int kTiles = TimeF32Lds<DH>::kTiles;
    constexpr int PK = TimeF32Lds<DH>::kPitchK, PV = TimeF32Lds<DH>::kPitchV;
    __shared__ TimeF32Lds<DH> lds;

    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int j = lane % 32, g = lane / 32;
    const uint32_t total = (uint32_t)rows * heads * qgroups;
    const uint32_t logical = xcd_remap(blockIdx.x, total);
    const int qg = logical % qgroups;
    const int bh = logical / qgroups;
    const int h = bh % heads, r = bh / heads;
    const int nb = (n + kKB - 1) / kKB;
    const int off = nb * kKB - n;  // block kb covers keys [kb*32 - off, kb*32 - off + 32)

    // padded V^T rows (DH not a multiple of 32) feed only discarded output dims; zero them once
    if (DH % 32 != 0) {
        for (int i = tid; i < 2 * kTiles * 32 * PV; i += kThreads) (&lds.vt[0][0])[i] = 0.f;
    }

    // per-block live bitmasks: bit b of mask[kb] = key kb*32 - off + b is live
    for (int c = wave; c * 2 < nb; c += kWaves) {
        int kg = c * 64 - off + lane;
        bool ok = kg >= 0 && kg < n && live[(size_t)r * n + kg] != 0;
        uint64_t bits = __ballot(ok);
        if (lane == 0) {
            lds.mask[2 * c] = (uint32_t)bits;
            if (2 * c + 1 < nb) lds.mask[2 * c + 1] = (uint32_t)(bits >> 32);
        }
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
                if (table) {
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

    // first non-empty block
    int kb = 0;
    while (kb < nb && lds.mask[kb] == 0) kb++;

    KvStage<DH> stage;
    if (kb < nb) {
        stage.load(qkv, table, r, h, n, inner, kb * kKB - off, tid);
        stage.store(lds, 0, tid);
    }
    __syncthreads();

    floatx16 o_acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; t++) o_acc[t] = floatx16{0};
    float m_run = -INFINITY, l_run = 0.f;
    int buf = 0;

    while (kb < nb) {
        int next = kb + 1;
        while (next < nb && lds.mask[next] == 0) next++;
        if (next < nb) stage.load(qkv, table, r, h, n, inner, next * kKB - off, tid);

        if (nq > 0) {
            // S^T = K Q^T over this block
            floatx16 s_acc = floatx16{0};
            const float* kp = &lds.k[buf][j * PK + g * kHalf];
#pragma unroll
            for (int s4 = 0; s4 < kSteps / 4; s4++) {
                floatx4 kv = *reinterpret_cast<const floatx4*>(kp + 4 * s4);
#pragma unroll
                for (int u = 0; u < 4; u++)
                    s_acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[u], qreg[4 * s4 + u], s_acc, 0, 0, 0);
            }
            // mask: reg rho of lane (j, g) holds key 8*(rho/4) + 4g + rho%4 of the block
            uint32_t km = lds.mask[kb];
            if (km != 0xffffffffu) {
#pragma unroll
                for (int rho = 0; rho < 16; rho++) {
                    int bit = 8 * (rho / 4) + 4 * g + (rho % 4);
                    if (!((km >> bit) & 1u)) s_acc[rho] = -INFINITY;
                }
            }
            float mx = s_acc[0];
#pragma unroll
            for (int rho = 1; rho < 16; rho++) mx = fmaxf(mx, s_acc[rho]);
            mx = pair_max(mx);
            float m_new = fmaxf(m_run, mx);
            float m_use = m_new == -INFINITY ? 0.f : m_new;
            float alpha = fast_exp2(m_run - m_use);
            m_run = m_new;
            float rs = 0.f;
#pragma unroll
            for (int rho = 0; rho < 16; rho++) {
                s_acc[rho] = fast_exp2(s_acc[rho] - m_use);
                rs += s_acc[rho];
            }
            l_run = l_run * alpha + rs;
#pragma unroll
            for (int t = 0; t < kTiles; t++) o_acc[t] *= alpha;
            // O^T += V^T P^T: step c = 4a + u uses keys 8a + 4kk + u and P from s_acc[c]
#pragma unroll
            for (int t = 0; t < kTiles; t++) {
                const float* vp = &lds.vt[buf][(32 * t + j) * PV + 4 * g];
#pragma unroll
                for (int a = 0; a < 4; a++) {
                    floatx4 vv = *reinterpret_cast<const floatx4*>(vp + 8 * a);
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        o_acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[u], s_acc[4 * a + u], o_acc[t], 0, 0, 0);
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

template <int DH>
static hipError_t launch_f32(const float* qkv, float* out, const int32_t* live, const float* table, int rows, int n,
                             int heads, int inner, hipStream_t stream) {
    int tiles = (n + kQ - 1) / kQ;
    int qgroups = (tiles + kWaves - 1) / kWaves;
    uint64_t grid = (uint64_t)rows * heads * qgroups;
    hipLaunchKernelGGL(c2_time_attention_f32<DH>, dim3((uint32_t)grid), dim3(kThreads), 0, stream, qkv, out, live,
                       table, rows, n, heads, inner, qgroups);
    return hipGetLastError();
}

hipError_t c2_time_attention_f32_launch(const float* qkv, float* out, const int32_t* live, const float* table,
                                        int rows, int n, int heads, int dh, int inner, hipStream_t stream) {
    switch (dh) {
        case 16: return launch_f32<16>(qkv, out, live, table, rows, n, heads, inner, stream);
        case 32: return launch_f32<32>(qkv, out, live, table, rows, n, heads, inner, stream);
        case 48: return launch_f32<48>(qkv, out, live, table, rows, n, heads, inner, stream);
        case 64: return launch_f32<64>(qkv, out, live, table, rows, n, heads, inner, stream);
        default: return hipErrorInvalidValue;
    }
}

int c2_time_attention_max_tokens() { return kMaxBlocks * kKB; }

}  // namespace jc
