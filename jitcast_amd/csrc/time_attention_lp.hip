// Time attention, fused flash-style for gfx950: the bf16 / fp16 path of Chronos-2 and Timestral
// (fp32 accumulation, fp32 softmax).
//
// Same contracts as the fp32 kernels (time_attention_f32.hip): Chronos-2's Chronos2Kernels.rope +
// timeAttention (Chronos2Kernels.java:87-116, 118-464; oracle CpuChronos2.java:175-228, 284-304) and
// Timestral's TimestralKernels.rope + timeAttention + gate (TimestralKernels.java:71-100, 102-278,
// 572-578; oracle CpuTimestral.java:156-161, 190-259). RoPE rotates q and k at load from the fp32
// table (the rotation runs in fp32, then rounds to the storage type); qkv, gate and out are bf16 or
// fp16; scores, softmax and accumulation are fp32.
//
// Layout: qkv [rows*n, 3*inner], out [rows*n, inner]. One workgroup = NW waves = NW*32 consecutive
// queries of one (row, head); keys stream through LDS in 64-key blocks aligned to 64,
// double-buffered; blocks no query of the workgroup sees are skipped.
//
// MFMA mapping (v_mfma_f32_32x32x16_{bf16,f16}: A lane i+32g holds A[i][8g..8g+7], B lane j+32g
// holds B[8g..8g+7][j], D lane j+32g reg r = D[8(r/4)+4g+r%4][j]):
//   S^T[key][q] = K Q^T   step s contracts padded dims 16s+8g..+7: A = K rows from LDS (one 16-byte
//                         read), B = the wave's rotated queries, resident in registers. The head is
//                         padded to DHP (a power of two): the real dh (a multiple of 16) fills the
//                         first dh/2 dims of each half, so RoPE pairs stay chunk-aligned.
//   O^T[e][q] += V^T P^T  16 keys per MFMA: B = P^T straight from S^T's accumulators (regs 8c..8c+7
//                         of a 32-key tile are keys 16c+4g+{0..3} and 16c+8+4g+{0..3}); A = V^T
//                         rows, stored in LDS with the keys of each 16-key group permuted
//                         (16c+8a+4g+u -> 16c+8g+4a+u) so the same 8 keys are one 16-byte read.
// Queries along lanes put one query's softmax state in lanes j and j+32: the block max is one
// v_permlane32_swap.
#include <type_traits>

#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "lp_common.hpp"
#include "time_mask.hpp"

namespace jc {
namespace {

using namespace lp;

constexpr int kQ = 32;    // queries per wave
constexpr int kKB = 64;   // keys per block
constexpr int kMaxTokens = 4096;



template <int DHP, bool TS>
struct LpLds {
    static constexpr int kPitchK = DHP + 8;         // elements per key row of K (16-byte aligned rows)
    static constexpr int kTiles = (DHP + 31) / 32;  // 32-dim output tiles
    static constexpr int kPitchV = kKB + 8;         // elements per dim row of V^T
    uint16_t k[2][kKB * kPitchK];
    uint16_t vt[2][kTiles * 32 * kPitchV];
    uint64_t mask[kMaxTokens / kKB];  // per 64-key block: key validity bits
    int32_t pos[TS ? kMaxTokens : 1];  // table row of every token of the row (Timestral)
};



// One 64-key block of K (rotated, then rounded) and V for (row, head), staged through registers.
//   K item (key, chunk c < dh/16): real dims 8c..8c+7 and dh/2+8c..+7 (two 16-byte loads, the RoPE
//     pair), written to padded dims 8c and DHP/2+8c
//   V item (4 keys, 4 dims): four 8-byte loads, written transposed as four 8-byte V^T row pieces
template <typename T, int DHP, int NT, bool ROPE, bool TS>
struct LpStage {
    static constexpr int kPerK = (kKB * DHP / 16 + NT - 1) / NT;
    static constexpr int kPerV = ((kKB / 4) * (DHP / 4) + NT - 1) / NT;
    u32x4 k0[kPerK], k1[kPerK];
    floatx4 c0[kPerK], c1[kPerK], s0[kPerK], s1[kPerK];
    u32x2 v[kPerV][4];
    uint32_t off_k[kPerK], off_t[kPerK], off_v[kPerV];
    int key[kPerK], ck[kPerK], kv4[kPerV], ev4[kPerV];
    int items_k, items_v, half;

    // V items start 256 threads after K items (mod NT), so a workgroup of more than 256 threads
    // spreads the two kinds of work over different waves
    static __device__ __forceinline__ int vtid(int tid) { return NT > 256 ? (tid + 256) % NT : tid; }

    __device__ __forceinline__ void init(int tid, int inner, int dh) {
        const uint32_t stride = 3u * inner * 2u;
        half = dh / 2;
        const int chunks = dh / 16, quads = dh / 4;
        items_k = kKB * chunks;
        items_v = (kKB / 4) * quads;
#pragma unroll
        for (int i = 0; i < kPerK; i++) {
            const int it = tid + i * NT;
            key[i] = it / chunks;
            ck[i] = it % chunks;
            off_k[i] = key[i] * stride + ck[i] * 16;
            off_t[i] = (uint32_t)((key[i] * dh + 8 * ck[i]) * 4);
        }
#pragma unroll
        for (int i = 0; i < kPerV; i++) {
            const int it = vtid(tid) + i * NT;
            kv4[i] = it / quads;
            ev4[i] = it % quads;
            off_v[i] = 4 * kv4[i] * stride + inner * 2 + ev4[i] * 8;
        }
    }

    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rt, const int32_t* pos,
                                         int k0b, int n, int tid, int inner, int dh) {
        const uint32_t stride = 3u * inner * 2u;
#pragma unroll
        for (int i = 0; i < kPerK; i++) {
            if (tid + i * NT >= items_k) break;
            k0[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off_k[i], 0, 0));
            k1[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off_k[i] + half * 2, 0, 0));
            if (ROPE) {
                uint32_t ot = off_t[i];
                if (TS) {
                    const int k = k0b + key[i];
                    ot = (uint32_t)(((k < n ? pos[k] : 0) * dh + 8 * ck[i]) * 4);
                }
                c0[i] = __builtin_amdgcn_raw_buffer_load_b128(rt, ot, 0, 0);
                c1[i] = __builtin_amdgcn_raw_buffer_load_b128(rt, ot + 16, 0, 0);
                s0[i] = __builtin_amdgcn_raw_buffer_load_b128(rt, ot + half * 4, 0, 0);
                s1[i] = __builtin_amdgcn_raw_buffer_load_b128(rt, ot + half * 4 + 16, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < kPerV; i++) {
            if (vtid(tid) + i * NT >= items_v) break;
#pragma unroll
            for (int u = 0; u < 4; u++)
                v[i][u] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rk, off_v[i] + u * stride, 0, 0));
        }
    }

    __device__ __forceinline__ void store(LpLds<DHP, TS>& lds, int buf, int tid) {
        constexpr int PK = LpLds<DHP, TS>::kPitchK, PV = LpLds<DHP, TS>::kPitchV;
#pragma unroll
        for (int i = 0; i < kPerK; i++) {
            if (tid + i * NT >= items_k) break;
            u32x4 w0 = k0[i], w1 = k1[i];
            if (ROPE) {
                floatx4 a0, a1, b0, b1;
                widen8<T>(k0[i], a0, a1);
                widen8<T>(k1[i], b0, b1);
                w0 = narrow8<T>(a0 * c0[i] - b0 * s0[i], a1 * c1[i] - b1 * s1[i]);
                w1 = narrow8<T>(b0 * c0[i] + a0 * s0[i], b1 * c1[i] + a1 * s1[i]);
            }
            uint16_t* kr = &lds.k[buf][key[i] * PK];
            *reinterpret_cast<u32x4*>(kr + 8 * ck[i]) = w0;
            *reinterpret_cast<u32x4*>(kr + DHP / 2 + 8 * ck[i]) = w1;
        }
#pragma unroll
        for (int i = 0; i < kPerV; i++) {
            if (vtid(tid) + i * NT >= items_v) break;
            const int pos = vt_pos(4 * kv4[i]);
            // v[u] holds keys 4kq+u, dims 4e4..4e4+3 (two per dword); row e of V^T takes the four keys
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;  // v_perm: high or low halves
                const int w = e >> 1;
                u32x2 row;
                row[0] = __builtin_amdgcn_perm(v[i][1][w], v[i][0][w], sel);
                row[1] = __builtin_amdgcn_perm(v[i][3][w], v[i][2][w], sel);
                *reinterpret_cast<u32x2*>(&lds.vt[buf][(4 * ev4[i] + e) * PV + pos]) = row;
            }
        }
    }
};

// 3 waves per SIMD where the kernel fits 168 VGPRs without spilling (Timestral's fp16 instance
// would spill 12 bytes per lane)
template <typename T, bool TS>
constexpr bool kLp3Waves = !TS || std::is_same_v<T, __bf16>;

template <typename T, int DHP, int NW, bool ROPE, bool TS, bool EXACT>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(NW >= 4 && DHP <= 64 && kLp3Waves<T, TS> ? 3 : 2)))
void time_attention_lp(const TimeArgs a, int dh_rt) {
    const int dh = EXACT ? DHP : dh_rt;
    static_assert(DHP % 16 == 0 && DHP <= 128, "head width");
    constexpr int NT = NW * kWave;
    constexpr int kHalfP = DHP / 2;
    constexpr int kSteps = DHP / 16;  // QK^T MFMA steps (16 dims each), plus the bias step
    constexpr int kTiles = LpLds<DHP, TS>::kTiles;
    constexpr int kSub = kKB / 32;   // 32-key S^T tiles per block
    constexpr int PK = LpLds<DHP, TS>::kPitchK, PV = LpLds<DHP, TS>::kPitchV;
    typedef typename Lp<T>::x8 x8;
    typedef Enc<T> E;
    __shared__ LpLds<DHP, TS> lds;

    const T* __restrict__ qkv = static_cast<const T*>(a.qkv);
    const int n = a.n, inner = a.inner, half = dh / 2;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int j = lane % 32, g = lane / 32;
    const uint32_t total = (uint32_t)a.rows * a.heads * a.qgroups;
    const uint32_t logical = xcd_remap(blockIdx.x, total);
    const int qg = logical % a.qgroups;
    const int bh = logical / a.qgroups;
    const int h = bh % a.heads, r = bh / a.heads;
    TimeMask<TS> mask;
    mask.init(a, r);
    const int32_t* vrow = a.valid + (size_t)r * (TS ? a.enc : n);

    // The prologue has two load latencies, not four: the wave's raw queries (and their RoPE partner
    // chunks and table rows) are requested first, so they arrive while the validity row is scanned.
    // Lane (j, g) of step s holds padded dims 16s+8g..+7 of query q0+j. (A 128-wide head converts its
    // queries before the scan instead: holding them raw would take 192 VGPRs.)
    const int q0 = a.q_begin + (qg * NW + wave) * kQ;
    const int nq = min(max(n - q0, 0), kQ);
    constexpr bool kEarly = DHP <= 64;
    u32x4 q_own[kSteps], q_par[kSteps];
    floatx4 t_c0[kSteps], t_c1[kSteps], t_s0[kSteps], t_s1[kSteps];
    x8 qreg[kSteps];
    auto load_q = [&](int s) {
        const int q = q0 + j;
        const T* qp = qkv + ((size_t)r * n + q) * 3 * inner + h * dh;
        int trow = q;
        if (TS && ROPE && a.pos) trow = min(max(a.pos[(size_t)r * n + q], 0), a.table_rows - 1);
        const int d0 = 16 * s + 8 * g;
        const bool first = d0 < kHalfP;
        const int e0 = first ? d0 : d0 - kHalfP;  // position within the half
        if (j < nq && e0 < half) {
            // own chunk and its rotation partner half a head away (real dims)
            q_own[s] = *reinterpret_cast<const u32x4*>(qp + (first ? e0 : half + e0));
            if (ROPE) {
                q_par[s] = *reinterpret_cast<const u32x4*>(qp + (first ? half + e0 : e0));
                const float* tp = a.table + (size_t)trow * dh + e0;
                t_c0[s] = *reinterpret_cast<const floatx4*>(tp);
                t_c1[s] = *reinterpret_cast<const floatx4*>(tp + 4);
                t_s0[s] = *reinterpret_cast<const floatx4*>(tp + half);
                t_s1[s] = *reinterpret_cast<const floatx4*>(tp + half + 4);
            }
        }
    };
    // Q operands: rotated, scaled by qscale (log2(e) times the score scale), rounded to T
    auto convert_q = [&](int s) {
        floatx4 lo = floatx4{0.f, 0.f, 0.f, 0.f}, hi = lo;
        const int d0 = 16 * s + 8 * g;
        const bool first = d0 < kHalfP;
        if (j < nq && (first ? d0 : d0 - kHalfP) < half) {
            widen8<T>(q_own[s], lo, hi);
            if (ROPE) {
                floatx4 plo, phi;
                widen8<T>(q_par[s], plo, phi);
                if (first) {
                    lo = lo * t_c0[s] - plo * t_s0[s];
                    hi = hi * t_c1[s] - phi * t_s1[s];
                } else {
                    lo = lo * t_c0[s] + plo * t_s0[s];
                    hi = hi * t_c1[s] + phi * t_s1[s];
                }
            }
            lo *= a.qscale;
            hi *= a.qscale;
        }
        qreg[s] = __builtin_bit_cast(x8, narrow8<T>(lo, hi));
    };
#pragma unroll
    for (int s = 0; s < kSteps; s++) {
        load_q(s);
        if (!kEarly) convert_q(s);
    }

    // zero the padding of the K and V^T tiles once (staging never writes it)
    if (dh < DHP) {
        for (int i = tid; i < 2 * kKB; i += NT) {
            uint16_t* kr = &lds.k[i / kKB][(i % kKB) * PK];
            for (int c = half; c < kHalfP; c++) kr[c] = kr[kHalfP + c] = 0;
        }
    }
    if (dh < kTiles * 32) {
        const int pad = (kTiles * 32 - dh) * PV;
        for (int i = tid; i < 2 * pad; i += NT) lds.vt[i / pad][dh * PV + i % pad] = 0;
    }
    // key validity of every 64-key block of the row, and (Timestral) every token's table row
    const int nblk = (n + kKB - 1) / kKB;
    for (int b = wave; b < nblk; b += NW) {
        const uint64_t bits = __ballot(mask.key_valid(vrow, b * kKB + lane));
        if (lane == 0) lds.mask[b] = bits;
    }
    if (TS) {
        for (int t = tid; t < n; t += NT)
            lds.pos[t] = a.pos ? min(max(a.pos[(size_t)r * n + t], 0), a.table_rows - 1) : t;
    }
    __syncthreads();
    // blocks any query of the workgroup can see (bit b = block b), the same in every wave
    const int qlo = a.q_begin + qg * NW * kQ, qhi = min(qlo + NW * kQ, n) - 1;
    const uint64_t need = __ballot(lane < nblk && mask.any_allowed(lds.mask[lane], lane * kKB, qlo, qhi));
    auto next_block = [&](int after) {
        const uint64_t rest = after + 1 >= 64 ? 0ull : need & (~0ull << (after + 1));
        return rest ? (int)__builtin_ctzll(rest) : nblk;
    };

    if (kEarly) {
#pragma unroll
        for (int s = 0; s < kSteps; s++) convert_q(s);
    }

    const size_t row0 = (size_t)r * n;
    const uint32_t stride_b = 3u * inner * 2u;
    // resources over k (and v) of (row, head) from the block's first key to the end of the row, and
    // over the table (rows from that key, or all rows for Timestral): keys past n read as zero
    auto rk_at = [&](int b) {
        const int k = b * kKB;
        const T* p = qkv + (row0 + k) * 3 * inner + inner + h * dh;
        const uint32_t bytes = (uint32_t)(n - k) * stride_b - (uint32_t)(inner + h * dh) * 2u;
        return make_rsrc(p, bytes);
    };
    auto rt_at = [&](int b) {
        if (TS) return make_rsrc(a.table, (uint32_t)a.table_rows * dh * 4u);
        const int k = b * kKB;
        return make_rsrc(a.table + (size_t)k * dh, (uint32_t)((n - k) * dh * 4));
    };

    int kb = next_block(-1);

    LpStage<T, DHP, NT, ROPE, TS> stage;
    stage.init(tid, inner, dh);
    if (kb < nblk) {
        stage.load(rk_at(kb), ROPE ? rt_at(kb) : rk_at(kb), lds.pos, kb * kKB, n, tid, inner, dh);
        stage.store(lds, 0, tid);
    }
    __syncthreads();

    floatx16 o_acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; t++) o_acc[t] = floatx16{0};
    // softmax state of query j (equal in lanes j and j+32): the reference max m_tot, the part of it
    // the MFMA subtracts (m_mfma = -b_m exactly), their difference (non-zero only when -m_tot does
    // not fit T), the running sum l relative to m_tot, and whether the query has a reference yet
    float m_tot = 0.f, m_mfma = 0.f, resid = 0.f, l_run = 0.f;
    bool has_ref = false, any_resid = false;
    uint32_t qx0 = g == 0 ? E::kBigQ : 0u;  // Q' dims 0,1 = (kBigQ, b_m = 0)
    int buf = 0;
    __builtin_amdgcn_s_waitcnt(0);

    while (kb < nblk) {
        const int next = next_block(kb);
        if (next < nblk) stage.load(rk_at(next), ROPE ? rt_at(next) : rk_at(next), lds.pos, next * kKB, n, tid, inner, dh);
        __builtin_amdgcn_sched_barrier(0);

        // the keys of this block the lane's query may see (bit i = key 64kb + i); lanes past the
        // row's last query take lane 0's keys so they never decide a wave-wide branch
        const uint64_t word = lds.mask[kb];
        uint64_t allowed = mask.allowed(word, kb * kKB, q0 + j);
        // (readfirstlane returns int: widen through uint32_t, or bit 31 would sign-extend)
        const uint64_t ref = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)allowed) |
                             ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(allowed >> 32)) << 32);
        if (j >= nq) allowed = ref;
        const bool lane_keys = allowed != 0;
        if (nq > 0 && __any(lane_keys)) {
            // the bias step masks by key when every query sees the same keys; otherwise (the causal
            // diagonal) it masks nothing and the per-element select below does the work
            const bool uniform = TS ? !__any(allowed != ref) : true;
            const uint64_t kmask = uniform ? ref : ~0ull;
            const x8 qx = __builtin_bit_cast(x8, u32x4{qx0, 0u, 0u, 0u});
            floatx16 s_acc[kSub];
#pragma unroll
            for (int sb = 0; sb < kSub; sb++) {
                s_acc[sb] = floatx16{0};
                const uint16_t* kp = &lds.k[buf][(32 * sb + j) * PK + 8 * g];
#pragma unroll
                for (int s = 0; s < kSteps; s++) {
                    if ((16 * s) % kHalfP < half) {
                        x8 kv = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(kp + 16 * s));
                        s_acc[sb] = Lp<T>::mfma(kv, qreg[s], s_acc[sb]);
                    }
                }
                // the bias step: A row i = key 32sb + i
                const uint32_t kx0 = g == 0 ? (((kmask >> (32 * sb + j)) & 1ull) ? E::kLive : E::kDead) : 0u;
                s_acc[sb] = Lp<T>::mfma(__builtin_bit_cast(x8, u32x4{kx0, 0u, 0u, 0u}), qx, s_acc[sb]);
            }
            // reg rho of tile sb in lane (j, g) holds key 32sb + 8*(rho/4) + 4g + rho%4 of the block
            if (!uniform) {
                // one 32-bit word per sub-tile, shifted to the lane's keys: the 64-bit word tested
                // per score held so many registers that Timestral's instance ran 2 waves per SIMD
#pragma unroll
                for (int sb = 0; sb < kSub; sb++) {
                    // bits 8k + u of w: key 32sb + 8k + 4g + u, i.e. reg rho = 4k + u
                    const uint32_t w = (uint32_t)(allowed >> (32 * sb)) >> (4 * g);
#pragma unroll
                    for (int rho = 0; rho < 16; rho++)
                        if (!((w >> (8 * (rho / 4) + rho % 4)) & 1u)) s_acc[sb][rho] = -INFINITY;
                }
            }
            x8 p[kSub][2];
            auto exps = [&](float shift) {
#pragma unroll
                for (int sb = 0; sb < kSub; sb++)
#pragma unroll
                    for (int c = 0; c < 2; c++) {
                        floatx4 lo, hi;
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            lo[u] = fast_exp2(s_acc[sb][8 * c + u] - shift);
                            hi[u] = fast_exp2(s_acc[sb][8 * c + 4 + u] - shift);
                        }
                        p[sb][c] = __builtin_bit_cast(x8, narrow8<T>(lo, hi));
                    }
            };
            auto block_sum = [&]() {
                float acc = 0.f;
#pragma unroll
                for (int sb = 0; sb < kSub; sb++)
#pragma unroll
                    for (int c = 0; c < 2; c++) {
                        u32x4 w = __builtin_bit_cast(u32x4, p[sb][c]);
#pragma unroll
                        for (int d = 0; d < 4; d++) acc = E::dot2(w[d], acc);
                    }
                return pair_sum(acc);
            };
            if (!any_resid) {
#pragma unroll
                for (int sb = 0; sb < kSub; sb++)
#pragma unroll
                    for (int c = 0; c < 2; c++) {
                        floatx4 lo, hi;
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            lo[u] = fast_exp2(s_acc[sb][8 * c + u]);
                            hi[u] = fast_exp2(s_acc[sb][8 * c + 4 + u]);
                        }
                        p[sb][c] = __builtin_bit_cast(x8, narrow8<T>(lo, hi));
                    }
            } else {
                exps(resid);
            }
            float lb = block_sum();
            const bool bad = !(lb <= kSumHi) || (!has_ref && lane_keys && !(lb >= kSumLo));
            if (__any(bad)) {
                // the exact block max (relative to m_mfma), a new reference rounded to T; a query
                // that sees no key of this block keeps its state
                float mx = s_acc[0][0];
#pragma unroll
                for (int sb = 0; sb < kSub; sb++)
#pragma unroll
                    for (int rho = 0; rho < 16; rho++) mx = fmaxf(mx, s_acc[sb][rho]);
                mx = pair_max(mx);
                const float s_max = m_mfma + mx;
                float m_new = !lane_keys ? m_tot : (has_ref ? fmaxf(m_tot, s_max) : s_max);
                const uint32_t bm = to_bits<T>(fminf(fmaxf(-m_new, -E::kMax), E::kMax));
                const float m_enc = -from_bits<T>(bm);
                if (fabsf(m_new) <= E::kMax) m_new = m_enc;  // keep the reference exactly encodable
                exps(m_new - m_mfma);
                lb = block_sum();
                if (has_ref) {
                    const float alpha = fast_exp2(m_tot - m_new);
#pragma unroll
                    for (int t = 0; t < kTiles; t++) o_acc[t] *= alpha;
                    l_run *= alpha;
                }
                m_tot = m_new;
                m_mfma = m_enc;
                resid = m_tot - m_mfma;
                any_resid = __any(resid != 0.f);
                qx0 = g == 0 ? (E::kBigQ | (bm << 16)) : 0u;
            }
            l_run += lb;
            has_ref = has_ref || lane_keys;
            // O^T += V^T P^T, 16 keys per MFMA
#pragma unroll
            for (int t = 0; t < kTiles; t++) {
                if (32 * t < dh) {
                    const uint16_t* vp = &lds.vt[buf][(32 * t + j) * PV + 8 * g];
#pragma unroll
                    for (int cc = 0; cc < kKB / 16; cc++) {
                        x8 vv = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(vp + 16 * cc));
                        o_acc[t] = Lp<T>::mfma(vv, p[cc / 2][cc % 2], o_acc[t]);
                    }
                }
            }
        }
        if (next < nblk) stage.store(lds, buf ^ 1, tid);
        __syncthreads();
        buf ^= 1;
        kb = next;
    }

    if (j < nq) {
        const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
        const size_t tok = (size_t)r * n + q0 + j;
        T* op = static_cast<T*>(a.out) + tok * inner + h * dh;
        const T* gp = a.gate ? static_cast<const T*>(a.gate) + tok * inner + h * dh : nullptr;
        // O^T reg 4a+u of lane (j, g) in tile t is dim 32t + 8a + 4g + u of query j
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
                        floatx4 gv, gz;
                        widen8<T>(u32x4{(*reinterpret_cast<const u32x2*>(gp + e))[0],
                                        (*reinterpret_cast<const u32x2*>(gp + e))[1], 0u, 0u},
                                  gv, gz);
#pragma unroll
                        for (int u = 0; u < 4; u++) v[u] *= 1.f / (1.f + fast_exp2(-gv[u] * kLog2e));
                    }
                    *reinterpret_cast<u32x2*>(op + e) = narrow4<T>(v);
                }
            }
        }
    }
}

template <typename T, int DHP, int NW, bool TS, bool EXACT>
hipError_t launch_lp_nw(TimeArgs a, int dh, hipStream_t stream) {
    const int tiles = (a.n - a.q_begin + kQ - 1) / kQ;
    a.qgroups = (tiles + NW - 1) / NW;
    const uint64_t grid = (uint64_t)a.rows * a.heads * a.qgroups;
    if (a.table) {
        hipLaunchKernelGGL((time_attention_lp<T, DHP, NW, true, TS, EXACT>), dim3((uint32_t)grid), dim3(NW * kWave), 0,
                           stream, a, dh);
    } else {
        hipLaunchKernelGGL((time_attention_lp<T, DHP, NW, false, TS, EXACT>), dim3((uint32_t)grid), dim3(NW * kWave), 0,
                           stream, a, dh);
    }
    return hipGetLastError();
}

// Waves per workgroup: 4 (2 when the row has at most 2 query tiles). Measured on config 1
// (n = 513, 17 tiles): 4 waves 0.511 ms, 6 waves 0.634 ms, 8 waves 0.611 ms. The kernel is bound by
// the latency of each workgroup's prologue and per-block loads; three 4-wave workgroups per CU
// overlap those better than two 6-wave ones, which outweighs the extra idle query slots. Rows of 5
// tiles (config 4's 133 tokens) as one 5-wave workgroup per (row, head), each K/V block loaded once
// and no idle wave: 2.94 ms per call against 2.65 ms for two 4-wave workgroups.
template <typename T, int DHP, bool TS, bool EXACT>
hipError_t launch_lp(const TimeArgs& a, int dh, hipStream_t stream) {
    if ((a.n + kQ - 1) / kQ <= 2) return launch_lp_nw<T, DHP, 2, TS, EXACT>(a, dh, stream);
    return launch_lp_nw<T, DHP, 4, TS, EXACT>(a, dh, stream);
}

template <typename T, int DHP, bool TS>
hipError_t launch_lp_width(const TimeArgs& a, int dh, hipStream_t stream) {
    return dh == DHP ? launch_lp<T, DHP, TS, true>(a, dh, stream) : launch_lp<T, DHP, TS, false>(a, dh, stream);
}

template <typename T, bool TS>
hipError_t dispatch_lp(const TimeArgs& a, int dh, hipStream_t stream) {
    if (dh <= 16) return launch_lp_width<T, 16, TS>(a, dh, stream);
    if (dh <= 32) return launch_lp_width<T, 32, TS>(a, dh, stream);
    if (dh <= 64 || !TS) return launch_lp_width<T, 64, TS>(a, dh, stream);
    if constexpr (TS) return launch_lp_width<T, 128, TS>(a, dh, stream);  // Chronos-2 heads are at most 64 wide
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t time_attention_lp_launch(const TimeArgs& a, int dh, bool ts, bool fp16, hipStream_t stream) {
    if (dh < 16 || dh > 128 || dh % 16) return hipErrorInvalidValue;
    if (fp16) return ts ? dispatch_lp<_Float16, true>(a, dh, stream) : dispatch_lp<_Float16, false>(a, dh, stream);
    return ts ? dispatch_lp<__bf16, true>(a, dh, stream) : dispatch_lp<__bf16, false>(a, dh, stream);
}

}  // namespace jc
