// Time attention, fused flash-style for gfx950: the FP32 path of Chronos-2 and Timestral.
//
// Chronos-2 replaces the per-layer pair Chronos2Kernels.rope + Chronos2Kernels.timeAttention
// (Chronos2Kernels.java:87-116, 118-464; oracle CpuChronos2.java:175-228, 284-304): unscaled scores
// over the row's live keys, both directions; zeros when no key is live.
// Timestral replaces TimestralKernels.rope + timeAttention + gate (TimestralKernels.java:71-100,
// 102-278, 572-578; oracle CpuTimestral.java:190-259, 156-161): scores scaled by 1/sqrt(dh), the
// BlockLayout.timeAllowed mask (time_mask.hpp), RoPE at each token's position pos[t] (a row of the
// host-built table), and the optional sigmoid output gate fused into the epilogue.
//
// Layout: qkv [rows*n, 3*inner] (q | k | v, heads-major per token), out [rows*n, inner]. One
// workgroup = 4 waves = 128 consecutive queries of one (row, head); each wave owns 32 queries.
// Keys stream through LDS in blocks of KB = 32, double-buffered; blocks no query of the workgroup can
// see are skipped, and a block no query of a wave can see costs that wave nothing but the barrier.
//
// MFMA mapping (v_mfma_f32_32x32x2_f32, 64 flops/clk/SIMD):
//   S^T[key][q] = K Q^T   A = K  (lane i+32kk: K[key i][kk*DHP/2 + s]),  B = Q (same dim map)
//   O^T[e][q]  += V^T P^T A = V^T (lane i+32kk: V[key(kk,c)][e]),        B = P straight from S^T
// DHP is the head width padded to a power of two; the real dh (a multiple of 8) fills the first
// dh/2 dims of each half of the padded Q/K layout, so the RoPE pair (e, e+dh/2) sits in the two
// lane halves of one step. The accumulator layout of S^T is exactly the B-operand layout P^T needs,
// so P never leaves registers. One query's softmax state lives in lanes j and j+32.
//
// K/V/table prefetch uses buffer loads; keys past the end of the row fall outside the resource and
// read as 0 (and are masked), so the load path has no per-lane bounds branches.
//
// FOLD (Chronos-2, rows of 128k + 1 tokens: [REG] after 128k patches): the row's last query would
// be alone in a fifth workgroup that stages every K/V block for one query. The last full workgroup
// computes it instead, on VALU beside its MFMA tiles: lane (key 8w + l/8, c = l%8) of wave w takes
// dims 8c..8c+7 of one key of each 32-key block (8 products and an 8-lane DPP sum give the score),
// each wave keeps a lazy online softmax over its 8 keys per block and accumulates its share of the
// output from V^T in LDS, and the four shares are rescaled to a common max once at the end.
//
// The last key (Chronos-2, 64-wide heads, rows of 32k + 1 tokens): key n - 1 would be alone in a
// last 32-key block whose MFMAs and staging cost a full block. It is staged once instead (rotated K
// and V in LDS), and before the block loop each query takes its score against it on VALU (a 32-dim
// dot per lane, summed over the lane pair) as the first step of its online softmax: running max
// = that score, sum = 1, O = V[n - 1]. The folded query adds it in its final combination.
//
// X3 (Chronos-2, 64-wide heads; the JC_F16X3 layer): out is the O projection's A operand, fp16
// rows of 3 * inner values [hi | hi | lo] (the three-term split of each fp32 output value), so the
// layer needs no separate split pass over the attention output.
#include "f32_tail.hpp"
#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "time_mask.hpp"

namespace jc {
namespace {

constexpr int kQ = 32;        // queries per wave
constexpr int kWaves = 4;     // waves per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxTokens = 4096;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format (gfx9 family)

template <int DHP, int KB, bool TS>
struct F32Lds {
    static constexpr int kPitchK = DHP + 4;         // floats per key row of K
    static constexpr int kTiles = (DHP + 31) / 32;  // 32-dim output tiles
    static constexpr int kPitchV = KB + 4;          // floats per dim row of V^T
    float k[2][KB * kPitchK];
    float vt[2][kTiles * 32 * kPitchV];
    uint64_t mask[kMaxTokens / kMaskBlock];  // per 64-key word: key validity bits
    int32_t pos[TS ? kMaxTokens : 1];       // table row of every token of the row (Timestral)
    float fold_q[DHP];                       // FOLD: the folded query, rotated and scaled
    float last_k[DHP], last_v[DHP];          // the last key (rotated, unscaled) and its value
};

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// One KB-key block of K (rotated at store) and V for (row, head), staged through registers:
// item `it` covers key it / (dh/8) and dims e..e+3 of each half, e = 4 * (it % (dh/8)).
template <int DHP, int KB, bool ROPE, bool TS>
struct KvStage {
    static constexpr int kMaxItems = KB * DHP / 8;
    static constexpr int kPer = (kMaxItems + kThreads - 1) / kThreads;
    floatx4 k0[kPer], k1[kPer], v0[kPer], v1[kPer], c[kPer], s[kPer];
    uint32_t off_kv[kPer], off_tab[kPer];  // loop-invariant byte offsets
    int key[kPer], e[kPer];
    int items, half;

    __device__ __forceinline__ void init(int tid, int inner, int dh) {
        half = dh / 2;
        const int quads = dh / 8;
        items = KB * quads;
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            int it = tid + i * kThreads;
            key[i] = it / quads;
            e[i] = (it % quads) * 4;
            off_kv[i] = (uint32_t)((key[i] * 3 * inner + e[i]) * 4);
            off_tab[i] = (uint32_t)((key[i] * dh + e[i]) * 4);
        }
    }

    // rk: resource over k of (row, head) from the block's first key k0. rt: over the table rows
    // from k0 (Chronos-2) or over the whole table (Timestral: row = pos of the key).
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rt, const int32_t* pos,
                                         int kbase, int n, int tid, int inner, int dh) {
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            if (tid + i * kThreads >= items) break;
            k0[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off_kv[i], 0, 0);
            k1[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off_kv[i] + half * 4, 0, 0);
            v0[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off_kv[i] + inner * 4, 0, 0);
            v1[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off_kv[i] + inner * 4 + half * 4, 0, 0);
            if (ROPE) {
                uint32_t ot = off_tab[i];
                if (TS) {
                    const int k = kbase + key[i];
                    ot = (uint32_t)(((k < n ? pos[k] : 0) * dh + e[i]) * 4);
                }
                c[i] = __builtin_amdgcn_raw_buffer_load_b128(rt, ot, 0, 0);
                s[i] = __builtin_amdgcn_raw_buffer_load_b128(rt, ot + half * 4, 0, 0);
            }
        }
    }

    __device__ __forceinline__ void store(F32Lds<DHP, KB, TS>& lds, int buf, int tid) {
        constexpr int PK = F32Lds<DHP, KB, TS>::kPitchK, PV = F32Lds<DHP, KB, TS>::kPitchV;
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            if (tid + i * kThreads >= items) break;
            floatx4 a0 = k0[i], a1 = k1[i];
            if (ROPE) {
                a0 = k0[i] * c[i] - k1[i] * s[i];
                a1 = k1[i] * c[i] + k0[i] * s[i];
            }
            float* kr = &lds.k[buf][key[i] * PK];
            *reinterpret_cast<floatx4*>(kr + e[i]) = a0;
            *reinterpret_cast<floatx4*>(kr + DHP / 2 + e[i]) = a1;
            float* vt = lds.vt[buf];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                vt[(e[i] + u) * PV + key[i]] = v0[i][u];
                vt[(half + e[i] + u) * PV + key[i]] = v1[i][u];
            }
        }
    }
};

// EXACT: the head is exactly DHP wide, so every head-width expression folds to a constant
template <int DHP, int KB, bool ROPE, bool TS, bool EXACT, bool FOLD, bool X3>
__global__ __launch_bounds__(kThreads) void time_attention_f32(const TimeArgs a, int dh_rt) {
    const int dh = EXACT ? DHP : dh_rt;
    static_assert(!X3 || (!TS && EXACT && DHP == 64), "split output: Chronos-2, 64-wide heads");
    static_assert(DHP % 16 == 0 && DHP <= 128, "head width");
    static_assert(!FOLD || (!TS && EXACT && DHP == 64 && KB == 32), "the folded query: Chronos-2, 64-wide heads");
    static_assert(KB == 32 || KB == 64, "key block");
    constexpr int kHalfP = DHP / 2;
    constexpr int kSteps = kHalfP;  // K=2 per MFMA step: one dim from each lane half
    constexpr int kTiles = F32Lds<DHP, KB, TS>::kTiles;
    constexpr int kSub = KB / 32;  // 32-key S^T tiles per block
    constexpr int PK = F32Lds<DHP, KB, TS>::kPitchK, PV = F32Lds<DHP, KB, TS>::kPitchV;
    constexpr uint64_t kFull = KB == 64 ? ~0ull : 0xffffffffull;
    __shared__ F32Lds<DHP, KB, TS> lds;

    const float* __restrict__ qkv = static_cast<const float*>(a.qkv);
    const int n = a.n, inner = a.inner, half = dh / 2;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int j = lane % 32, g = lane / 32;
    const uint32_t items = (uint32_t)a.rows * a.heads;
    // With tail workgroups (q_tail > 0), every 4 (row, head) items get their qgroups main
    // workgroups followed by one tail workgroup whose 4 waves take the items' last R queries; the
    // neighbouring logical workgroups run on one XCD, so the tail's K/V reads find them in its L2.
    constexpr bool kTailOk = !TS && !FOLD && EXACT && DHP == 64 && KB == 32;  // FOLD rows have R = 1
    const bool tails = kTailOk && a.q_tail > 0;
    const uint32_t per_group = 4 * a.qgroups + 1;
    const uint32_t total = tails ? (items + 3) / 4 * per_group : items * a.qgroups;
    const uint32_t logical = xcd_remap(blockIdx.x, total);
    int qg, bh;
    if (tails) {
        const uint32_t grp = logical / per_group, s = logical % per_group;
        if (s == 4 * (uint32_t)a.qgroups) {
            const uint32_t item = 4 * grp + tid / kWave;
            if constexpr (kTailOk) {
                if (item < items)
                    f32_tail_item<ROPE, X3>(a, item / a.heads, item % a.heads, a.q_tail, tid % kWave);
            }
            return;  // the whole workgroup: tail workgroups take no barrier
        }
        const uint32_t item = 4 * grp + s / a.qgroups;
        if (item >= items) return;  // the last group's missing items: before any barrier
        qg = s % a.qgroups;
        bh = item;
    } else {
        qg = logical % a.qgroups;
        bh = logical / a.qgroups;
    }
    const int h = bh % a.heads, r = bh / a.heads;
    const bool fold = FOLD && qg == a.qgroups - 1;  // this workgroup also computes query n - 1
    // key n - 1 alone in the last block: taken on VALU after the loop
    constexpr bool kLastOk = !TS && EXACT && DHP == 64 && KB == 32;
    const bool lastk = kLastOk && a.n > 1 && a.n % KB == 1;
    TimeMask<TS> mask;
    mask.init(a, r);
    const int32_t* vrow = a.valid + (size_t)r * (TS ? a.enc : n);

    // The wave's queries are requested first, so their latency overlaps the validity scan.
    // Lane (j, g) holds dims g*dh/2 + s (s < dh/2) of query q0+j; the rest of its DHP/2 are zero.
    const int q0 = (qg * kWaves + wave) * kQ;
    const int nq = min(max(n - q0, 0), kQ);
    floatx4 qa[kSteps / 4], qb[kSteps / 4], qc[kSteps / 4], qs[kSteps / 4];
    if (j < nq) {
        const int q = q0 + j;
        const float* qp = qkv + ((size_t)r * n + q) * 3 * inner + h * dh;
        int trow = q;
        if (TS && ROPE && a.pos) trow = min(max(a.pos[(size_t)r * n + q], 0), a.table_rows - 1);
#pragma unroll
        for (int s4 = 0; s4 < kSteps / 4; s4++) {
            if (4 * s4 < half) {
                qa[s4] = *reinterpret_cast<const floatx4*>(qp + 4 * s4);
                qb[s4] = *reinterpret_cast<const floatx4*>(qp + half + 4 * s4);
                if (ROPE) {
                    qc[s4] = *reinterpret_cast<const floatx4*>(a.table + (size_t)trow * dh + 4 * s4);
                    qs[s4] = *reinterpret_cast<const floatx4*>(a.table + (size_t)trow * dh + half + 4 * s4);
                }
            }
        }
    }

    // zero the padding of the K and V^T tiles once (staging never writes it)
    if (dh < DHP) {
        for (int i = tid; i < 2 * KB; i += kThreads) {
            float* kr = &lds.k[i / KB][(i % KB) * PK];
            for (int c = half; c < kHalfP; c++) kr[c] = kr[kHalfP + c] = 0.f;
        }
    }
    if (dh < kTiles * 32) {
        for (int i = tid; i < 2 * (kTiles * 32 - dh) * PV; i += kThreads) {
            const int b = i / ((kTiles * 32 - dh) * PV), rest = i % ((kTiles * 32 - dh) * PV);
            lds.vt[b][dh * PV + rest] = 0.f;
        }
    }
    // key validity of every 64-key word of the row, and (Timestral) every token's table row
    const int nwords = (n + kMaskBlock - 1) / kMaskBlock;
    for (int w = wave; w < nwords; w += kWaves) {
        const uint64_t bits = __ballot(mask.key_valid(vrow, w * kMaskBlock + lane));
        if (lane == 0) lds.mask[w] = bits;
    }
    if (TS) {
        for (int t = tid; t < n; t += kThreads)
            lds.pos[t] = a.pos ? min(max(a.pos[(size_t)r * n + t], 0), a.table_rows - 1) : t;
    }
    if (FOLD && fold && wave == 0 && lane < DHP / 2) {
        // the folded query's dims e and e + 32, rotated at table row n - 1 like the tiles' queries
        const int qf = n - 1, e = lane;
        const float* qp = qkv + ((size_t)r * n + qf) * 3 * inner + h * dh;
        float x = qp[e], y = qp[DHP / 2 + e];
        if (ROPE) {
            const float c = a.table[(size_t)qf * dh + e], sn = a.table[(size_t)qf * dh + DHP / 2 + e];
            const float rx = x * c - y * sn, ry = y * c + x * sn;
            x = rx;
            y = ry;
        }
        lds.fold_q[e] = x * a.qscale;
        lds.fold_q[DHP / 2 + e] = y * a.qscale;
    }
    __syncthreads();
    // 64-key words any query of the workgroup can see (the same in every wave)
    const int qlo = qg * kWaves * kQ, qhi = min(qlo + kWaves * kQ, n) - 1;
    const uint64_t need = __ballot(lane < nwords && mask.any_allowed(lds.mask[lane], lane * kMaskBlock, qlo, qhi));
    const int nblk = (n - (lastk ? 1 : 0) + KB - 1) / KB;
    auto next_block = [&](int after) {
        const int b = after + 1;
        const int w = b * KB / kMaskBlock;
        const uint64_t rest = (b >= nblk || w >= 64) ? 0ull : need & (~0ull << w);
        if (!rest) return nblk;
        const int wn = (int)__builtin_ctzll(rest);
        return wn == w ? b : wn * kMaskBlock / KB;
    };

    // Q operands: rotated, scaled by qscale (log2(e) times the score scale)
    float qreg[kSteps];
#pragma unroll
    for (int s4 = 0; s4 < kSteps / 4; s4++) {
        floatx4 o = floatx4{0.f, 0.f, 0.f, 0.f};
        if (j < nq && 4 * s4 < half) {
            o = g == 0 ? qa[s4] : qb[s4];
            if (ROPE) o = g == 0 ? qa[s4] * qc[s4] - qb[s4] * qs[s4] : qb[s4] * qc[s4] + qa[s4] * qs[s4];
            o *= a.qscale;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) qreg[4 * s4 + u] = o[u];
    }

    const size_t row0 = (size_t)r * n;
    const uint32_t stride_b = 3u * inner * 4u;
    auto rk_at = [&](int b) {
        const int k = b * KB;
        const float* p = qkv + (row0 + k) * 3 * inner + inner + h * dh;
        const uint32_t bytes = (uint32_t)(n - k) * stride_b - (uint32_t)(inner + h * dh) * 4u;
        return make_rsrc(p, bytes);
    };
    auto rt_at = [&](int b) {
        if (TS) return make_rsrc(a.table, (uint32_t)a.table_rows * dh * 4u);
        const int k = b * KB;
        return make_rsrc(a.table + (size_t)k * dh, (uint32_t)((n - k) * dh * 4));
    };

    int kb = next_block(-1);
    KvStage<DHP, KB, ROPE, TS> stage;
    stage.init(tid, inner, dh);
    if (kb < nblk) {
        stage.load(rk_at(kb), ROPE ? rt_at(kb) : rk_at(kb), lds.pos, kb * KB, n, tid, inner, dh);
        stage.store(lds, 0, tid);
    }
    if (kLastOk && lastk && wave == 1) {
        // key n - 1's dims e and e + 32, rotated at its table row as staging rotates every key (loaded
        // here, after Q's prologue registers are free, beside the first block's staging)
        const int kl = n - 1;
        const float* kp = qkv + ((size_t)r * n + kl) * 3 * inner + inner + h * dh;
        if (lane < DHP / 2) {
            const int e = lane;
            float x = kp[e], y = kp[DHP / 2 + e];
            if (ROPE) {
                const float c = a.table[(size_t)kl * dh + e], sn = a.table[(size_t)kl * dh + DHP / 2 + e];
                const float rx = x * c - y * sn, ry = y * c + x * sn;
                x = rx;
                y = ry;
            }
            lds.last_k[e] = x;
            lds.last_k[DHP / 2 + e] = y;
        }
        lds.last_v[lane] = kp[inner + lane];
    }
    __syncthreads();

    floatx16 o_acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; t++) o_acc[t] = floatx16{0};
    float m_run = -INFINITY, l_run = 0.f;
    if (kLastOk && lastk && ((lds.mask[(n - 1) / kMaskBlock] >> ((n - 1) % kMaskBlock)) & 1ull)) {
        // the live last key opens the online softmax (uniform over the workgroup): m = its score,
        // P = 1, O = its value. Lane (j, g) holds dims 32g..32g+31 of query j, so the pair sum of
        // the lane's partial dot is the whole score.
        const float* kp = &lds.last_k[g * kHalfP];
        float d = 0.f;
#pragma unroll
        for (int s4 = 0; s4 < kSteps / 4; s4++) {
            const floatx4 kv = *reinterpret_cast<const floatx4*>(kp + 4 * s4);
#pragma unroll
            for (int u = 0; u < 4; u++) d += qreg[4 * s4 + u] * kv[u];
        }
        m_run = pair_sum(d);
        l_run = g == 0 ? 1.f : 0.f;  // the pair sum at the end counts it once
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++) {
                const floatx4 vv = *reinterpret_cast<const floatx4*>(&lds.last_v[32 * t + 8 * a4 + 4 * g]);
#pragma unroll
                for (int u = 0; u < 4; u++) o_acc[t][4 * a4 + u] = vv[u];
            }
        }
    }
    // FOLD: this wave's softmax state for the folded query over its keys (8 per block)
    float f_m = -INFINITY, f_l = 0.f;
    floatx4 f_oa = floatx4{0.f, 0.f, 0.f, 0.f}, f_ob = f_oa;
    int buf = 0;
    // Settle every prologue load here: the compiler cannot prove that the divergent Q loads were
    // consumed on all paths and would otherwise wait on them (vmcnt(0)) inside every iteration.
    __builtin_amdgcn_s_waitcnt(0);

    while (kb < nblk) {
        const int next = next_block(kb);
        if (next < nblk) stage.load(rk_at(next), ROPE ? rt_at(next) : rk_at(next), lds.pos, next * KB, n, tid, inner, dh);
        // keep the prefetch above the block's MFMAs (the scheduler would sink it to its use)
        __builtin_amdgcn_sched_barrier(0);

        // the keys of this block the lane's query may see (bit i = key kb*KB + i)
        const int k0 = kb * KB;
        const uint64_t word = lds.mask[k0 / kMaskBlock];
        const uint64_t allowed =
            (mask.allowed(word, k0 & ~(kMaskBlock - 1), q0 + j) >> (k0 % kMaskBlock)) & kFull;
        if (nq > 0 && __any(j < nq && allowed != 0)) {
            // S^T = K Q^T over this block, one 32x32 tile per 32 keys
            floatx16 s_acc[kSub];
#pragma unroll
            for (int sb = 0; sb < kSub; sb++) {
                s_acc[sb] = floatx16{0};
                const float* kp = &lds.k[buf][(32 * sb + j) * PK + g * kHalfP];
#pragma unroll
                for (int s4 = 0; s4 < kSteps / 4; s4++) {
                    if (4 * s4 < half) {
                        floatx4 kv = *reinterpret_cast<const floatx4*>(kp + 4 * s4);
#pragma unroll
                        for (int u = 0; u < 4; u++)
                            s_acc[sb] =
                                __builtin_amdgcn_mfma_f32_32x32x2f32(kv[u], qreg[4 * s4 + u], s_acc[sb], 0, 0, 0);
                    }
                }
            }
            // mask: reg rho of tile sb in lane (j, g) holds key 32sb + 8*(rho/4) + 4g + rho%4 of the block
            if (__any(j < nq && allowed != kFull)) {
#pragma unroll
                for (int sb = 0; sb < kSub; sb++) {
#pragma unroll
                    for (int rho = 0; rho < 16; rho++) {
                        int bit = 32 * sb + 8 * (rho / 4) + 4 * g + (rho % 4);
                        if (!((allowed >> bit) & 1ull)) s_acc[sb][rho] = -INFINITY;
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
                if (32 * t < dh) {
                    const float* vp = &lds.vt[buf][(32 * t + j) * PV + 4 * g];
#pragma unroll
                    for (int sb = 0; sb < kSub; sb++) {
#pragma unroll
                        for (int a4 = 0; a4 < 4; a4++) {
                            floatx4 vv = *reinterpret_cast<const floatx4*>(vp + 32 * sb + 8 * a4);
#pragma unroll
                            for (int u = 0; u < 4; u++)
                                o_acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[u], s_acc[sb][4 * a4 + u], o_acc[t],
                                                                                0, 0, 0);
                        }
                    }
                }
            }
        }
        if (FOLD && fold) {
            // the folded query against key 8w + l/8 of the block: dims 8c..8c+7 in this lane
            const int fkey = 8 * wave + lane / 8, c8 = 8 * (lane % 8);
            const float* kr = &lds.k[buf][fkey * PK + c8];
            const floatx4 ka = *reinterpret_cast<const floatx4*>(kr);
            const floatx4 kb4 = *reinterpret_cast<const floatx4*>(kr + 4);
            const floatx4 qa4 = *reinterpret_cast<const floatx4*>(&lds.fold_q[c8]);
            const floatx4 qb4 = *reinterpret_cast<const floatx4*>(&lds.fold_q[c8 + 4]);
            float sc = 0.f;
#pragma unroll
            for (int u = 0; u < 4; u++) sc += ka[u] * qa4[u] + kb4[u] * qb4[u];
            sc += dpp_f<0xB1>(sc);   // quad_perm [1,0,3,2]
            sc += dpp_f<0x4E>(sc);   // quad_perm [2,3,0,1]
            sc += dpp_f<0x141>(sc);  // row_half_mirror: the key's 8 lanes hold its score
            const bool live = (word >> ((k0 % kMaskBlock) + fkey)) & 1ull;
            const float fs = live ? sc : -INFINITY;
            // the reference max moves only when a score passes it by 2^64 (or at the first live key),
            // so P stays below 2^64
            if (__any(fs - f_m > 64.f)) {
                float mx = fmaxf(fs, dpp_f<0x128>(fs));  // row_ror:8: the row's other key
                auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
                mx = pair_max(fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])));
                const float m_new = fmaxf(f_m, mx);
                const float alpha = fast_exp2(f_m - m_new);  // f_m = -inf: 0
                f_l *= alpha;
                f_oa *= alpha;
                f_ob *= alpha;
                f_m = m_new;
            }
            const float p = live ? fast_exp2(fs - f_m) : 0.f;
            f_l += p;
            const float* vp = &lds.vt[buf][c8 * PV + fkey];  // V[key][c8 + u] at row c8 + u of V^T
#pragma unroll
            for (int u = 0; u < 4; u++) {
                f_oa[u] += p * vp[u * PV];
                f_ob[u] += p * vp[(4 + u) * PV];
            }
        }
        if (next < nblk) stage.store(lds, buf ^ 1, tid);
        __syncthreads();
        buf ^= 1;
        kb = next;
    }

    if (FOLD && fold) {
        // each wave's share: dims 8c..8c+7 summed over its 8 keys' lanes (c, c+8, ..., c+56), with its
        // max and sum (each key's P counted in 8 lanes), into the K buffers (free after the loop)
        floatx4 fo[2] = {f_oa, f_ob};
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float v = fo[i][u];
                v += dpp_f<0x128>(v);  // row_ror:8
                auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
                fo[i][u] = pair_sum(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
            }
        }
        float lw = f_l;
        lw += dpp_f<0xB1>(lw);
        lw += dpp_f<0x4E>(lw);
        lw += dpp_f<0x124>(lw);  // row_ror:4
        lw += dpp_f<0x128>(lw);  // row_ror:8
        {
            auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(lw), __float_as_uint(lw), false, false);
            lw = pair_sum(__uint_as_float(sw[0]) + __uint_as_float(sw[1])) * 0.125f;
        }
        float* part = &lds.k[0][wave * (DHP + 2)];
        if (lane < 8) {
            *reinterpret_cast<floatx4*>(&part[8 * lane]) = fo[0];
            *reinterpret_cast<floatx4*>(&part[8 * lane + 4]) = fo[1];
        }
        if (lane == 0) {
            part[DHP] = f_m;
            part[DHP + 1] = lw;
        }
        __syncthreads();
        if (wave == 0) {
            float mw[kWaves], mx = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                mw[w] = lds.k[0][w * (DHP + 2) + DHP];
                mx = fmaxf(mx, mw[w]);
            }
            // the folded query against the last key, when the loop left it out and it is live
            float sl = -INFINITY;
            if (lastk && ((lds.mask[(n - 1) / kMaskBlock] >> ((n - 1) % kMaskBlock)) & 1ull)) {
                float d = lds.fold_q[lane] * lds.last_k[lane];
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off);
                sl = d;
                mx = fmaxf(mx, sl);
            }
            float o = 0.f, l = 0.f;
            if (mx != -INFINITY) {
#pragma unroll
                for (int w = 0; w < kWaves; w++) {
                    const float f = fast_exp2(mw[w] - mx);
                    o += f * lds.k[0][w * (DHP + 2) + lane];
                    l += f * lds.k[0][w * (DHP + 2) + DHP + 1];
                }
                const float f = fast_exp2(sl - mx);  // 0 without the last key
                o += f * lds.last_v[lane];
                l += f;
            }
            const float res = l > 0.f ? o / l : 0.f;
            if constexpr (X3) {
                store_split_one(static_cast<_Float16*>(a.out) + ((size_t)r * n + n - 1) * 3 * inner, inner,
                                h * dh + lane, res);
            } else {
                float* op = static_cast<float*>(a.out) + ((size_t)r * n + n - 1) * inner + h * dh;
                op[lane] = res;
            }
        }
    }

    // every lane reaches the swap (its partner holds the other half of the same query)
    const float l = pair_sum(l_run);
    if constexpr (X3) {
        // Lanes (j, 0) and (j, 1) trade halves of each 16-dim run (v_permlane32_swap), so each holds 8
        // consecutive dims: 32t + 16p + 8g + (0..7), from O^T regs 8p + u (dims 32t + 16p + 4g + u) and
        // 8p + 4 + u (dims 32t + 16p + 8 + 4g + u). Each piece of the split then goes out as one
        // 16-byte store.
        const float inv = l > 0.f ? 1.f / l : 0.f;
        _Float16* orow = static_cast<_Float16*>(a.out) + ((size_t)r * n + q0 + j) * 3 * inner + h * dh;
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
#pragma unroll
            for (int p = 0; p < 2; p++) {
                floatx4 d0, d4;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(o_acc[t][8 * p + u] * inv),
                                                                     __float_as_uint(o_acc[t][8 * p + 4 + u] * inv),
                                                                     false, false);
                    d0[u] = __uint_as_float(sw[0]);
                    d4[u] = __uint_as_float(sw[1]);
                }
                if (j < nq) store_split_row8(orow, inner, 32 * t + 16 * p + 8 * g, d0, d4);
            }
        }
        return;
    }
    if (j < nq) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const size_t tok = (size_t)r * n + q0 + j;
        float* op = static_cast<float*>(a.out) + tok * inner + h * dh;
        const float* gp = a.gate ? static_cast<const float*>(a.gate) + tok * inner + h * dh : nullptr;
        // O^T reg 4a+u of lane (j, g) is dim 32t + 8a + 4g + u of query j
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++) {
                const int e = 32 * t + 8 * a4 + 4 * g;
                if (e < dh) {
                    floatx4 v;
#pragma unroll
                    for (int u = 0; u < 4; u++) v[u] = o_acc[t][4 * a4 + u] * inv;
                    if (gp) {
                        // the output gate: att * sigmoid(g) (CpuTimestral.java:156-161)
                        const floatx4 gv = *reinterpret_cast<const floatx4*>(gp + e);
#pragma unroll
                        for (int u = 0; u < 4; u++) v[u] *= 1.f / (1.f + fast_exp2(-gv[u] * kLog2e));
                    }
                    *reinterpret_cast<floatx4*>(op + e) = v;
                }
            }
        }
    }
}

}  // namespace

template <int DHP, int KB, bool TS, bool EXACT, bool FOLD, bool X3>
static void launch_f32_rope(const TimeArgs& a, int dh, uint64_t grid, hipStream_t stream) {
    if (a.table) {
        hipLaunchKernelGGL((time_attention_f32<DHP, KB, true, TS, EXACT, FOLD, X3>), dim3((uint32_t)grid),
                           dim3(kThreads), 0, stream, a, dh);
    } else {
        hipLaunchKernelGGL((time_attention_f32<DHP, KB, false, TS, EXACT, FOLD, X3>), dim3((uint32_t)grid),
                           dim3(kThreads), 0, stream, a, dh);
    }
}

// R when a row of 128k + R tokens, 2 <= R <= 16, takes tail workgroups for its last R queries
// (Chronos-2, 64-wide heads, no gate), else 0
static int tail_rows(const TimeArgs& a, int dh) {
    if (dh != 64 || a.gate || a.q_begin != 0 || a.n <= kWaves * kQ) return 0;
    if (a.table && a.table_rows < a.n) return 0;
    const int R = a.n % (kWaves * kQ);
    return R >= 2 && R <= kTailT ? R : 0;
}

template <int DHP, bool TS, bool EXACT, bool X3 = false>
static hipError_t launch_f32(TimeArgs a, int dh, hipStream_t stream) {
    constexpr int KB = 32;  // 32-key blocks (64 measured slower on config 1)
    const int tiles = (a.n + kQ - 1) / kQ;
    // a last query alone after whole workgroups (n = 128k + 1) is folded into the last of them
    constexpr bool kCanFold = !TS && EXACT && DHP == 64;
    const bool fold = kCanFold && a.n > 1 && a.n % (kWaves * kQ) == 1;
    a.qgroups = fold ? (a.n - 1) / (kWaves * kQ) : (tiles + kWaves - 1) / kWaves;
    // rows of 128k + R tokens, 2 <= R <= 16 (Chronos-2, 64-wide heads): the main workgroups take the
    // first 128k queries and tail workgroups (f32_tail.hpp) the last R, instead of a fifth main
    // workgroup that stages every block for one partly filled wave
    int tail = 0;
    if constexpr (kCanFold) tail = tail_rows(a, dh);
    if (tail) {
        a.qgroups = (a.n - tail) / (kWaves * kQ);
        a.q_tail = a.n - tail;
    }
    const uint64_t items = (uint64_t)a.rows * a.heads;
    const uint64_t grid = tail ? (items + 3) / 4 * (4 * a.qgroups + 1) : items * a.qgroups;
    if constexpr (kCanFold) {
        if (fold) {
            launch_f32_rope<DHP, KB, TS, EXACT, true, X3>(a, dh, grid, stream);
            return hipGetLastError();
        }
    }
    launch_f32_rope<DHP, KB, TS, EXACT, false, X3>(a, dh, grid, stream);
    return hipGetLastError();
}

template <int DHP, bool TS>
static hipError_t launch_f32_width(const TimeArgs& a, int dh, hipStream_t stream) {
    return dh == DHP ? launch_f32<DHP, TS, true>(a, dh, stream) : launch_f32<DHP, TS, false>(a, dh, stream);
}

template <bool TS>
static hipError_t dispatch_f32(const TimeArgs& a, int dh, hipStream_t stream) {
    if (dh <= 16) return launch_f32_width<16, TS>(a, dh, stream);
    if (dh <= 32) return launch_f32_width<32, TS>(a, dh, stream);
    if (dh <= 64 || !TS) return launch_f32_width<64, TS>(a, dh, stream);
    if constexpr (TS) return launch_f32_width<128, TS>(a, dh, stream);  // Chronos-2 heads are at most 64 wide
    return hipErrorInvalidValue;
}

hipError_t time_attention_f32_launch(const TimeArgs& a, int dh, bool ts, hipStream_t stream) {
    if (dh < 8 || dh > 128 || dh % 8) return hipErrorInvalidValue;
    return ts ? dispatch_f32<true>(a, dh, stream) : dispatch_f32<false>(a, dh, stream);
}

hipError_t time_attention_f32_x3_launch(const TimeArgs& a, int dh, hipStream_t stream) {
    if (dh != 64) return hipErrorInvalidValue;
    return launch_f32<64, false, true, true>(a, dh, stream);
}

int time_attention_max_tokens() { return kMaxTokens; }

}  // namespace jc
