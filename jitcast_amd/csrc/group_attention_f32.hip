// Group (cross-series) attention for gfx950, FP32 path: Chronos-2's group attention and
// Timestral's variate attention.
//
// Chronos-2 replaces Chronos2Kernels.groupAttention(qkv, out, live, groupStart, groupEnd, rows, n,
// heads, dh, inner) (Chronos2Kernels.java:466-682; oracle CpuChronos2.java:230-282): at every token
// slot t, row i attends the rows j of its group (groupStart[i] <= j < groupEnd[i], groups are
// contiguous runs of rows) whose token at t is live; unscaled scores, no positional encoding; zeros
// when no key is live.
// Timestral replaces TimestralKernels.variateAttention(qkv, out, keyValid, groupStart, groupEnd,
// role, covariates, rows, enc, n, heads, dh, d) and the gate (TimestralKernels.java:280-446,
// 572-578; oracle CpuTimestral.java:156-161, 261-314): scores scaled by 1/sqrt(dh) under
// BlockLayout.variateAllowed (BlockLayout.java:223-243): an encoder slot only where the key row's
// patch is a valid key; with covariates a covariate row never reads a target row and a known row
// reads only known rows; a row always reads itself. The optional sigmoid gate is fused.
//
// Storage types: q|k|v, the gate and out are fp32, or (T = bf16 / fp16, the layers' FP16 GEMM mode)
// 16-bit values rounded once at the store. The products: fp32 values as fp16 pairs (three fp16 MFMA
// products per product, fp32 MFMA for values beyond fp16's range), 16-bit values as stored (exact
// products on the MFMA of their type, P as a hi + lo pair of the type); scores, softmax and
// accumulation are fp32 either way.
//
// The stage reads q|k|v once and writes out once, about 10 flop per byte: it is HBM-bound, so the
// kernel is built around the memory stream. One wave per (16-row tile, slot) owns the groups that
// START in its tile (found by a ballot on groupStart[i] == i), so each row's q, k and v are fetched
// from HBM once; everything lives in registers (no LDS, no barriers). A one-workgroup kernel
// (group_tile_order) first sorts the tiles by work, and the grid dispatches the heaviest first, so
// the launch ends on light waves. The wave's work is a flat
// stream of jobs (group, chunk of up to 4 query tiles (2 for heads over 64 wide), head, 16-key
// tile): the chunk's queries and output accumulators stay in registers while the group's key tiles
// stream past, each K/V tile used by every query tile right after it lands, and the next job's K/V loads are issued before this
// job's MFMAs (register double-buffering). The online softmax across key tiles makes any group size
// work; a group past 64 rows re-streams its keys once per further 64-row chunk.
//
// Operand layouts (16x16x4 f32: A lane i+16kk = A[i][kk], B lane j+16kk = B[kk][j]; 16x16x16
// f16 / bf16: A lane i+16kk = A[i][4kk..4kk+3], B likewise by column; D lane j+16g reg r =
// D[4g+r][j] for both):
//   S^T[key][q] = K Q^T: each lane holds dims 16m + 4kk .. +3 of its key and of its query (one 16-
//                        or 8-byte load per m, a 64-byte run per row per load): 4 fp32 steps per m,
//                        or one 16x16x16 product per m and term.
//   O^T[e][q] += V^T P^T: keys 4kk + c (c = 0..3), whose P^T is S^T's reg c in the same lane; V^T
//                        is loaded per lane as V[key][e] (16 rows x 64 contiguous bytes per load):
//                        4 fp32 steps, or one 16x16x16 product per term.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "f16_split.hpp"
#include "lp_common.hpp"

namespace jc {
namespace {

constexpr int kRT = 16;  // rows per tile (queries and keys)
constexpr int kModeF32 = 0, kModeSplit = 1, kModeNative = 2;  // the job stream's MFMA forms

// v_mfma_f32_16x16x16 of the storage type T (bf16 or fp16): A lane i+16kk = A[i][4kk..4kk+3], B lane
// j+16kk = B[4kk..4kk+3][j], 4 values of T per operand
template <typename T>
__device__ __forceinline__ floatx4 mfma16(lp::u32x2 a, lp::u32x2 b, floatx4 c) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    if constexpr (std::is_same_v<T, __bf16>) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(halfx4, a), __builtin_bit_cast(halfx4, b), c, 0, 0,
                                                     0);
    }
}

// p = hi + lo in T, both rounded to nearest: within 2^-16 |p| (bf16) or 2^-22 |p| + 2^-25 (fp16)
template <typename T>
__device__ __forceinline__ void split_lp(floatx4 p, lp::u32x2& hi, lp::u32x2& lo) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    const t4 h = __builtin_convertvector(p, t4);
    const t4 l = __builtin_convertvector(p - __builtin_convertvector(h, floatx4), t4);
    hi = __builtin_bit_cast(lp::u32x2, h);
    lo = __builtin_bit_cast(lp::u32x2, l);
}

// four consecutive storage values as fp32 (one 16- or 8-byte load), and back
template <typename T>
__device__ __forceinline__ floatx4 load4(const T* p) {
    if constexpr (std::is_same_v<T, float>) {
        return *reinterpret_cast<const floatx4*>(p);
    } else {
        typedef T t4 __attribute__((ext_vector_type(4)));
        const t4 v = __builtin_bit_cast(t4, *reinterpret_cast<const lp::u32x2*>(p));
        floatx4 r;
#pragma unroll
        for (int u = 0; u < 4; u++) r[u] = (float)v[u];
        return r;
    }
}
template <typename T>
__device__ __forceinline__ void store4(T* p, floatx4 v) {
    if constexpr (std::is_same_v<T, float>) {
        *reinterpret_cast<floatx4*>(p) = v;
    } else {
        *reinterpret_cast<lp::u32x2*>(p) = lp::narrow4<T>(v);
    }
}

// A position in the wave's job stream: rows [gs, ge) (one group, or a pack of consecutive groups
// spanning at most 16 rows), query chunk qc (up to kQT tiles of 16 rows), head h, key tile kt.
struct Job {
    int gs, ge, qc, h, kt;
    uint32_t pb;    // group starts of the job relative to gs (bit i = row gs + i); 1 for one group
    uint32_t rest;  // starts of the tile's remaining groups (bit b = row r0 + b)
    bool valid;
};


// X3 (Chronos-2, 64-wide heads; the JC_F16X3 layer): out holds fp16 rows of 3 * inner values, the
// O projection's A operand [hi | hi | lo] (the three-term split of each fp32 output value).
// T: the storage type of q|k|v, the gate and out (float, __bf16 or _Float16).
template <typename T, int DHP, bool TS, bool EXACT, bool X3>
__global__ __launch_bounds__(kWave) void group_attention_f32(const GroupArgs a, int dh_rt) {
    static_assert(!X3 || (!TS && EXACT && DHP == 64 && std::is_same_v<T, float>),
                  "split output: Chronos-2, 64-wide heads, fp32");
    static_assert(DHP % 16 == 0 && DHP <= 128, "head width");
    constexpr int kM = DHP / 16;            // 16-dim groups: K/Q loads per lane, and output dim tiles
    constexpr int kQT = DHP <= 64 ? 4 : 2;  // query tiles held in registers at once
    const int dh = EXACT ? DHP : dh_rt;
    const T* __restrict__ qkv = static_cast<const T*>(a.qkv);
    const T* __restrict__ gate = static_cast<const T*>(a.gate);
    T* __restrict__ out = static_cast<T*>(a.out);
    const int rows = a.rows, n = a.n, heads = a.heads, inner = a.inner;
    const int lane = threadIdx.x;
    const int j = lane % 16, g = lane / 16;
    const uint32_t total = (uint32_t)a.rtiles * n * a.hsplit;
    // With a tile order: blocks in that order (tile, then slot, then head range), heaviest first, so
    // the last waves of the launch are light ones; consecutive blocks go to different XCDs, which
    // balances them. Without: tiles fastest within each slot, each XCD a contiguous range.
    const uint32_t logical = a.order ? blockIdx.x : xcd_remap(blockIdx.x, total);
    const uint32_t tile_slot = logical / a.hsplit;
    const int t = a.order ? (int)(tile_slot % n) : (int)(tile_slot / a.rtiles);
    const int rt = a.order ? a.order[tile_slot / n] : (int)(tile_slot % a.rtiles);
    // this wave's heads [h_lo, h_hi): a (tile, slot)'s heads are split over hsplit waves, so the
    // tiles where long groups start do not hold one wave for all heads while their neighbours idle
    const int hs = logical % a.hsplit;
    const int h_lo = heads * hs / a.hsplit, h_hi = heads * (hs + 1) / a.hsplit;
    const int r0 = rt * kRT;
    const int nr = min(kRT, rows - r0);
    const size_t stride = 3 * (size_t)inner;  // floats per token of qkv
    const size_t tok_n = (size_t)n;
    const bool enc_slot = TS && t < a.enc;
    const bool cov = TS && a.covariates != 0 && a.role != nullptr;

    // the groups starting in this tile (both bounds loaded at once: one round trip)
    const int gs_l = lane < nr ? a.gstart[r0 + lane] : -1;
    const int ge_l = lane < nr ? a.gend[r0 + lane] : 0;
    const uint32_t starts = (uint32_t)__ballot(gs_l == r0 + lane) & 0xffffu;
    if (starts == 0) return;

    // A tile of one-row groups (every series of the block univariate): a row's only key is itself,
    // so its softmax weight is exactly 1 for a finite score and its output is its own v (gated),
    // which a stream over (row, head) pairs writes without MFMA work. The outcomes are the job
    // stream's below: 0 where the row may not read itself (Chronos-2: its token is not live) or its
    // score is -inf, NaN where the score is NaN or +inf, v otherwise.
    const bool single = lane >= nr || (gs_l == r0 + lane && (ge_l <= r0 + lane + 1 || r0 + lane + 1 >= rows));
    if (__ballot(!single) == 0) {
        const int pj = lane % 16;  // 16 lanes per (row, head) pair, 4 dims each per 64-dim step
        const int hn = h_hi - h_lo;
        for (int pr = lane / 16; pr < nr * hn; pr += kWave / 16) {
            const int row = r0 + pr / hn, h = h_lo + pr % hn;
            const T* tokp = qkv + ((size_t)row * tok_n + t) * stride + h * dh;
            float sc = 0.f;
            for (int e = 4 * pj; e < dh; e += 64) {
                const floatx4 q4 = load4(tokp + e);
                const floatx4 k4 = load4(tokp + inner + e);
#pragma unroll
                for (int u = 0; u < 4; u++) sc += (q4[u] * a.qscale) * k4[u];
            }
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) sc += __shfl_xor(sc, o, 16);
            const bool self_ok = TS || a.valid[(size_t)row * tok_n + t] != 0;
            const bool zero = !self_ok || sc == -INFINITY;
            const bool nan = !zero && !(sc < INFINITY);  // NaN or +inf
            const size_t off = ((size_t)row * tok_n + t) * inner + h * dh;
            for (int e = 4 * pj; e < dh; e += 64) {
                floatx4 v = load4(tokp + 2 * inner + e);
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = zero ? 0.f : nan ? __builtin_nanf("") : v[u];
                if (gate) {
                    const floatx4 gv = load4(gate + off + e);
#pragma unroll
                    for (int u = 0; u < 4; u++) v[u] *= 1.f / (1.f + fast_exp2(-gv[u] * kLog2e));
                }
                if constexpr (X3) {
                    store_split_row(static_cast<_Float16*>(a.out) + ((size_t)row * tok_n + t) * 3 * inner, inner,
                                    h * dh + e, v);
                } else {
                    store4(out + off + e, v);
                }
            }
        }
        return;
    }

    auto first_of = [&](uint32_t rest) {
        Job jb;
        jb.valid = rest != 0;
        int b = jb.valid ? __builtin_ctz(rest) : 0;
        jb.gs = r0 + b;
        // clamped into [gs+1, rows]: a group always holds its first row and only rows that exist.
        // Its end comes from the prologue's load (lane b holds gend[r0 + b]; b is wave-uniform), not
        // from memory: a load here would stall every group change on its latency.
        jb.ge = jb.valid ? min(max(__builtin_amdgcn_readlane(ge_l, b), jb.gs + 1), rows) : jb.gs + 1;
        jb.qc = 0;
        jb.h = h_lo;
        jb.kt = 0;
        jb.pb = 1u;
        jb.rest = jb.valid ? rest & (rest - 1) : 0;
        // small groups starting in the tile share one job while they span at most 16 rows: one
        // 16 x 16 score tile, masked block-diagonally, instead of one mostly empty tile per group
        while (jb.rest != 0) {
            const int b2 = __builtin_ctz(jb.rest);
            if (r0 + b2 != jb.ge) break;
            const int e2 = min(max(__builtin_amdgcn_readlane(ge_l, b2), jb.ge + 1), rows);
            if (e2 - jb.gs > kRT) break;
            jb.pb |= 1u << (jb.ge - jb.gs);
            jb.ge = e2;
            jb.rest &= jb.rest - 1;
        }
        return jb;
    };
    // key tiles innermost, so a K/V tile is used by every resident query tile right after it lands
    auto advance = [&](Job jb) {
        const int tiles = (jb.ge - jb.gs + kRT - 1) / kRT;
        if (++jb.kt < tiles) return jb;
        jb.kt = 0;
        if (++jb.h < h_hi) return jb;
        jb.h = h_lo;
        if (++jb.qc * kQT < tiles) return jb;
        return first_of(jb.rest);
    };
    // K (A operand) and V^T (A operand of PV) of a job's key tile; rows past the group are clamped
    // (finite, masked). In lanes j < 16: the validity of key 16kt + j and (Timestral) its role.
    struct Kv {
        floatx4 k[kM];
        float v[kM][4];
        int valid, role;
    };
    // (bf16 / fp16 storage, NATIVE below) the same operands as stored: K's 4 dims per m and, per m,
    // V[key 4g + c][16m + j] for c = 0..3 packed as one 4-value operand
    struct KvN {
        lp::u32x2 k[kM];
        lp::u32x2 v[kM];
        int valid, role;
    };
    auto load_kv = [&](const Job& jb, auto& d) {
        constexpr bool kRaw = std::is_same_v<std::decay_t<decltype(d)>, KvN>;
        const int kbase = jb.gs + kRT * jb.kt;
        const int krow = min(kbase + j, jb.ge - 1);
        const T* kp = qkv + ((size_t)krow * tok_n + t) * stride + inner + jb.h * dh + 4 * g;
        const bool in_group = g == 0 && kbase + j < jb.ge;
        if (TS) {
            d.valid = in_group && (!enc_slot || a.valid[(size_t)krow * a.enc + t] != 0);
            d.role = cov ? a.role[krow] : 0;
        } else {
            d.valid = in_group ? a.valid[(size_t)krow * tok_n + t] : 0;
            d.role = 0;
        }
        if constexpr (kRaw) {
            uint16_t vb[kM][4];
#pragma unroll
            for (int m = 0; m < kM; m++)
                d.k[m] = (EXACT || 16 * m + 4 * g < dh) ? *reinterpret_cast<const lp::u32x2*>(kp + 16 * m) : lp::u32x2{0u, 0u};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int vrow = min(kbase + 4 * g + c, jb.ge - 1);
                const uint16_t* vp = reinterpret_cast<const uint16_t*>(qkv + ((size_t)vrow * tok_n + t) * stride +
                                                                      2 * inner + jb.h * dh + j);
#pragma unroll
                for (int m = 0; m < kM; m++) vb[m][c] = (EXACT || 16 * m + j < dh) ? vp[16 * m] : (uint16_t)0;
            }
#pragma unroll
            for (int m = 0; m < kM; m++)
                d.v[m] = lp::u32x2{vb[m][0] | ((uint32_t)vb[m][1] << 16), vb[m][2] | ((uint32_t)vb[m][3] << 16)};
        } else {
#pragma unroll
            for (int m = 0; m < kM; m++)
                d.k[m] = (EXACT || 16 * m + 4 * g < dh) ? load4(kp + 16 * m) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int vrow = min(kbase + 4 * g + c, jb.ge - 1);
                const T* vp = qkv + ((size_t)vrow * tok_n + t) * stride + 2 * inner + jb.h * dh + j;
#pragma unroll
                for (int m = 0; m < kM; m++) d.v[m][c] = (EXACT || 16 * m + j < dh) ? (float)vp[16 * m] : 0.f;
            }
        }
    };

    // The job stream, in one of three modes:
    //   kModeF32    v_mfma_f32_16x16x4f32 on fp32 values (widened from the storage type);
    //   kModeSplit  fp32 storage: QK^T and PV as three fp16 MFMA products each (split_f16), a quarter
    //               of the fp32 MFMA cycles. It gives up, returning false, at the first query, key or
    //               value outside fp16's range (or infinite); the wave then runs its whole stream
    //               again in kModeF32, which writes every output of the wave anew;
    //   kModeNative bf16 / fp16 storage: K and Q as stored on the 16x16x16 MFMA of their type (exact
    //               products; qscale applied to the fp32 scores), and P as a pair of the storage
    //               type, hi + lo, against V as stored: two products per value tile.
    auto stream = [&](auto mode_tag) -> bool {
        constexpr int MODE = decltype(mode_tag)::value;
        constexpr bool SPLIT = MODE == kModeSplit, NATIVE = MODE == kModeNative;
        Job cur = first_of(starts);
        std::conditional_t<NATIVE, KvN, Kv> dc, dn;
        load_kv(cur, dc);

        // resident query tiles (B operand): fp32 scaled by qscale, (SPLIT) their fp16 pairs, or
        // (NATIVE) the stored values, unscaled
        float qreg[MODE == kModeF32 ? kQT : 1][4 * kM];
        halfx4 qhi[SPLIT ? kQT : 1][kM], qlo[SPLIT ? kQT : 1][kM];
        lp::u32x2 qn[NATIVE ? kQT : 1][kM];
        floatx4 o_acc[kQT][kM];
        float m_run[kQT], l_run[kQT];
        int q_role[kQT];
        uint32_t gmask = ~0u;  // a pack's keys in the group of the lane's query row (bit i = row gs + i)
        while (cur.valid) {
            const int tiles = (cur.ge - cur.gs + kRT - 1) / kRT;
            const int nq = min(kQT, tiles - kQT * cur.qc);  // query tiles in this chunk
            if (cur.kt == 0) {
                // a pack spans one tile: the lane's query row gs + j reads the rows of its own group
                if (cur.pb != 1u) {
                    const uint32_t upto = (2u << j) - 1u;
                    const int s_q = 31 - __builtin_clz(cur.pb & upto);
                    const uint32_t above = cur.pb & ~upto;
                    gmask = (above ? (1u << __builtin_ctz(above)) - 1u : 0xffffu) & ~((1u << s_q) - 1u);
                } else {
                    gmask = ~0u;
                }
                // a new (group, chunk, head): load its query tiles and reset the softmax state
                float q_abs = 0.f;
#pragma unroll
                for (int qi = 0; qi < kQT; qi++) {
                    if (qi < nq) {
                        const int qrow = min(cur.gs + kRT * (kQT * cur.qc + qi) + j, cur.ge - 1);
                        const T* qp = qkv + ((size_t)qrow * tok_n + t) * stride + cur.h * dh + 4 * g;
#pragma unroll
                        for (int m = 0; m < kM; m++) {
                            if constexpr (NATIVE) {
                                qn[qi][m] = (EXACT || 16 * m + 4 * g < dh) ? *reinterpret_cast<const lp::u32x2*>(qp + 16 * m)
                                                                          : lp::u32x2{0u, 0u};
                                continue;
                            }
                            const floatx4 x = ((EXACT || 16 * m + 4 * g < dh) ? load4(qp + 16 * m)
                                                                             : floatx4{0.f, 0.f, 0.f, 0.f}) *
                                              a.qscale;
                            if constexpr (SPLIT) {
                                q_abs = abs_max4(q_abs, x);
                                split_f16(x, qhi[qi][m], qlo[qi][m]);
                            } else {
#pragma unroll
                                for (int u = 0; u < 4; u++) qreg[qi][4 * m + u] = x[u];
                            }
                        }
                        if (cov) q_role[qi] = a.role[qrow];
                    }
#pragma unroll
                    for (int m = 0; m < kM; m++) o_acc[qi][m] = floatx4{0.f, 0.f, 0.f, 0.f};
                    m_run[qi] = -INFINITY;
                    l_run[qi] = 0.f;
                }
                if constexpr (SPLIT) {
                    if (__ballot(!(q_abs <= kF16Max)) != 0) return false;
                }
            }
            const Job nxt = advance(cur);
            load_kv(nxt, dn);  // in flight under this job's MFMAs (an invalid job reloads in-bounds rows)
            __builtin_amdgcn_sched_barrier(0);

            // bit b: key gs + 16kt + b is valid (and, for Timestral, a target / known-covariate row)
            const uint32_t vbits = (uint32_t)__ballot(dc.valid != 0) & 0xffffu;
            const uint32_t tbits = cov ? (uint32_t)__ballot(g == 0 && dc.role == 0) & 0xffffu : 0u;
            const uint32_t kbits = cov ? (uint32_t)__ballot(g == 0 && dc.role == 2) & 0xffffu : 0u;
            const int kbase = cur.gs + kRT * cur.kt;
            // query tile qi's scores s (reg r of lane (j, g): key 16kt + 4g + r) to the online
            // softmax's weights, in place; returns the factor that rescales the tile's earlier sums
            auto softmax = [&](int qi, floatx4& s) {
                // the keys query row qrow may read (BlockLayout.variateAllowed for Timestral)
                uint32_t allowed = vbits & gmask;
                if (TS) {
                    const int qrow = cur.gs + kRT * (kQT * cur.qc + qi) + j;
                    uint32_t forbid = 0;
                    if (cov) {
                        if (q_role[qi] != 0) forbid |= tbits;             // covariate rows never read targets
                        if (q_role[qi] == 2) forbid |= ~kbits & 0xffffu;  // known rows read known rows only
                    }
                    const int self = qrow - kbase;
                    allowed = ((vbits & ~forbid) | ((self >= 0 && self < kRT) ? (1u << self) : 0u)) & gmask;
                }
#pragma unroll
                for (int r = 0; r < 4; r++) s[r] = ((allowed >> (4 * g + r)) & 1u) ? s[r] : -INFINITY;
                const float mx = quad_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
                const float m_new = fmaxf(m_run[qi], mx);
                const float m_use = m_new == -INFINITY ? 0.f : m_new;
                const float alpha = fast_exp2(m_run[qi] - m_use);
                m_run[qi] = m_new;
#pragma unroll
                for (int r = 0; r < 4; r++) s[r] = fast_exp2(s[r] - m_use);
                l_run[qi] = l_run[qi] * alpha + (s[0] + s[1]) + (s[2] + s[3]);
                return alpha;
            };
            if constexpr (SPLIT) {
                float kv_abs = 0.f;
#pragma unroll
                for (int m = 0; m < kM; m++) kv_abs = abs_max4(abs_max4(kv_abs, dc.k[m]), v4(dc.v[m]));
                if (__ballot(!(kv_abs <= kF16Max)) != 0) return false;
                halfx4 khi[kM], klo[kM], vhi[kM], vlo[kM];
#pragma unroll
                for (int m = 0; m < kM; m++) {
                    split_f16(dc.k[m], khi[m], klo[m]);
                    split_f16(v4(dc.v[m]), vhi[m], vlo[m]);
                }
#pragma unroll
                for (int qi = 0; qi < kQT; qi++) {
                    if (qi < nq) {
                        // S^T = K_hi Q_hi + K_hi Q_lo + K_lo Q_hi
                        floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int m = 0; m < kM; m++) {
                            if (EXACT || 16 * m < dh) {
                                s = __builtin_amdgcn_mfma_f32_16x16x16f16(khi[m], qhi[qi][m], s, 0, 0, 0);
                                s = __builtin_amdgcn_mfma_f32_16x16x16f16(khi[m], qlo[qi][m], s, 0, 0, 0);
                                s = __builtin_amdgcn_mfma_f32_16x16x16f16(klo[m], qhi[qi][m], s, 0, 0, 0);
                            }
                        }
                        const float alpha = softmax(qi, s);
                        // O^T += V_hi P_hi + V_hi P_lo + V_lo P_hi (P in [0, 1])
                        halfx4 phi, plo;
                        split_f16(s, phi, plo);
#pragma unroll
                        for (int m = 0; m < kM; m++) {
                            if (EXACT || 16 * m < dh) {
                                floatx4 acc = o_acc[qi][m] * alpha;
                                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(vhi[m], phi, acc, 0, 0, 0);
                                acc = __builtin_amdgcn_mfma_f32_16x16x16f16(vhi[m], plo, acc, 0, 0, 0);
                                o_acc[qi][m] = __builtin_amdgcn_mfma_f32_16x16x16f16(vlo[m], phi, acc, 0, 0, 0);
                            }
                        }
                    }
                }
            } else if constexpr (NATIVE) {
#pragma unroll
                for (int qi = 0; qi < kQT; qi++) {
                    if (qi < nq) {
                        floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int m = 0; m < kM; m++) {
                            if (EXACT || 16 * m < dh) s = mfma16<T>(dc.k[m], qn[qi][m], s);
                        }
                        s *= a.qscale;
                        const float alpha = softmax(qi, s);
                        // O^T += V^T P_hi + V^T P_lo, P = P_hi + P_lo in the storage type (P in [0, 1])
                        lp::u32x2 phi, plo;
                        split_lp<T>(s, phi, plo);
#pragma unroll
                        for (int m = 0; m < kM; m++) {
                            if (EXACT || 16 * m < dh) {
                                floatx4 acc = o_acc[qi][m] * alpha;
                                acc = mfma16<T>(dc.v[m], phi, acc);
                                o_acc[qi][m] = mfma16<T>(dc.v[m], plo, acc);
                            }
                        }
                    }
                }
            } else {
#pragma unroll
                for (int qi = 0; qi < kQT; qi++) {
                    if (qi < nq) {
                        floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int m = 0; m < kM; m++) {
                            if (EXACT || 16 * m < dh) {
#pragma unroll
                                for (int u = 0; u < 4; u++)
                                    s = __builtin_amdgcn_mfma_f32_16x16x4f32(dc.k[m][u], qreg[qi][4 * m + u], s, 0, 0, 0);
                            }
                        }
                        const float alpha = softmax(qi, s);
#pragma unroll
                        for (int m = 0; m < kM; m++) {
                            if (EXACT || 16 * m < dh) {
                                o_acc[qi][m] *= alpha;
#pragma unroll
                                for (int c = 0; c < 4; c++)
                                    o_acc[qi][m] =
                                        __builtin_amdgcn_mfma_f32_16x16x4f32(dc.v[m][c], s[c], o_acc[qi][m], 0, 0, 0);
                            }
                        }
                    }
                }
            }

            if (cur.kt == tiles - 1) {
#pragma unroll
                for (int qi = 0; qi < kQT; qi++) {
                    if (qi < nq) {
                        const float l = quad_sum(l_run[qi]);
                        const int qrow = cur.gs + kRT * (kQT * cur.qc + qi) + j;
                        if (qrow < cur.ge) {
                            const float inv = l > 0.f ? 1.f / l : 0.f;
                            const size_t off = ((size_t)qrow * tok_n + t) * inner + cur.h * dh + 4 * g;
                            // O^T reg r of lane (j, g) in dim tile m is dim 16m + 4g + r of the query
#pragma unroll
                            for (int m = 0; m < kM; m++) {
                                if (EXACT || 16 * m + 4 * g < dh) {
                                    floatx4 v = o_acc[qi][m] * inv;
                                    if (gate) {
                                        // the output gate: att * sigmoid(g) (CpuTimestral.java:156-161)
                                        const floatx4 gv = load4(gate + off + 16 * m);
#pragma unroll
                                        for (int u = 0; u < 4; u++) v[u] *= 1.f / (1.f + fast_exp2(-gv[u] * kLog2e));
                                    }
                                    if constexpr (X3) {
                                        store_split_row(
                                            static_cast<_Float16*>(a.out) + ((size_t)qrow * tok_n + t) * 3 * inner,
                                            inner, cur.h * dh + 4 * g + 16 * m, v);
                                    } else {
                                        store4(out + off + 16 * m, v);
                                    }
                                }
                            }
                        }
                    }
                }
            }
            cur = nxt;
            dc = dn;
        }
        return true;
    };
    if constexpr (std::is_same_v<T, float>) {
        if (a.f32_mfma || !stream(std::integral_constant<int, kModeSplit>{}))
            stream(std::integral_constant<int, kModeF32>{});
    } else {
        stream(std::integral_constant<int, kModeNative>{});
    }
}

}  // namespace

// Waves per (16-row tile, slot), each taking a range of the heads. A tile's work is that of the
// groups starting in it, so with one wave per tile the tiles where long groups start run several
// times the mean while covered tiles return at once, and the last waves of a launch set its end.
// Splitting the heads over 4 waves moves no extra bytes (heads own disjoint q, k and v).
// JITCAST_HIP_GROUP_SPLIT (1..16) overrides it; read at every launch.
static int group_head_split() {
    const char* e = getenv("JITCAST_HIP_GROUP_SPLIT");
    const int v = e ? atoi(e) : 0;
    return v >= 1 && v <= 16 ? v : 4;
}

// JITCAST_HIP_GROUP_F32MMA=1 runs fp32 storage on fp32 MFMA throughout (the three-term fp16 products
// are the default); read at every launch.
static int group_f32_mfma() {
    const char* e = getenv("JITCAST_HIP_GROUP_F32MMA");
    return e && e[0] == '1' ? 1 : 0;
}

constexpr int kOrderBuckets = 64;

// A counting sort of the tiles by work into buckets, 0 for the most: a group's jobs per head are its
// key tiles times its query tiles, (ceil(g / 16))^2 for a group of g rows (bounds clamped as the
// kernel clamps them), summed over the groups starting in the tile. One row per lane (16 lanes a
// tile, summed by shuffles), the buckets in LDS, one wave's scan of the counts, then the scatter.
// Ties come out in any order: which block runs a tile changes nothing in its results.
__global__ __launch_bounds__(1024) void group_tile_order(const int32_t* gstart, const int32_t* gend, int rows,
                                                         int32_t* order) {
    __shared__ int slot[kOrderBuckets];
    __shared__ uint8_t bucket[kGroupOrderTiles];
    const int tid = threadIdx.x, rtiles = (rows + kRT - 1) / kRT;
    if (tid < kOrderBuckets) slot[tid] = 0;
    __syncthreads();
    for (int r = tid; r < rtiles * kRT; r += blockDim.x) {  // blockDim.x is a multiple of 16
        int w = 0;
        if (r < rows) {
            const int gs = gstart[r], ge = gend[r];
            if (gs == r) {
                const int kt = min((min(max(ge, r + 1), rows) - r + kRT - 1) / kRT, kOrderBuckets);
                w = kt * kt;
            }
        }
#pragma unroll
        for (int o = kRT / 2; o > 0; o >>= 1) w += __shfl_xor(w, o, kRT);
        if (r % kRT == 0) {
            const int b = kOrderBuckets - 1 - min(w, kOrderBuckets - 1);
            bucket[r / kRT] = (uint8_t)b;
            atomicAdd(&slot[b], 1);
        }
    }
    __syncthreads();
    if (tid < kOrderBuckets) {  // wave 0: exclusive prefix sum of the counts
        const int c = slot[tid];
        int x = c;
#pragma unroll
        for (int o = 1; o < kOrderBuckets; o <<= 1) {
            const int y = __shfl_up(x, o);
            if (tid >= o) x += y;
        }
        slot[tid] = x - c;
    }
    __syncthreads();
    for (int tile = tid; tile < rtiles; tile += blockDim.x) order[atomicAdd(&slot[bucket[tile]], 1)] = tile;
}

template <typename T, int DHP, bool TS, bool EXACT, bool X3 = false>
static hipError_t launch_group(GroupArgs a, int dh, hipStream_t stream) {
    a.rtiles = (a.rows + kRT - 1) / kRT;
    a.hsplit = std::min(group_head_split(), a.heads);
    a.f32_mfma = group_f32_mfma();
    if (a.rtiles > kGroupOrderTiles) a.order = nullptr;
    const uint64_t grid = (uint64_t)a.rtiles * a.n * a.hsplit;
    if (grid > 0xffffffffull) return hipErrorInvalidValue;
    hipLaunchKernelGGL((group_attention_f32<T, DHP, TS, EXACT, X3>), dim3((uint32_t)grid), dim3(kWave), 0, stream, a,
                       dh);
    return hipGetLastError();
}

template <typename T, int DHP, bool TS>
static hipError_t launch_group_width(const GroupArgs& a, int dh, hipStream_t stream) {
    return dh == DHP ? launch_group<T, DHP, TS, true>(a, dh, stream) : launch_group<T, DHP, TS, false>(a, dh, stream);
}

template <typename T, bool TS>
static hipError_t dispatch_group(const GroupArgs& a, int dh, hipStream_t stream) {
    if (dh <= 16) return launch_group_width<T, 16, TS>(a, dh, stream);
    if (dh <= 32) return launch_group_width<T, 32, TS>(a, dh, stream);
    if (dh == 48) return launch_group<T, 48, TS, true>(a, dh, stream);
    if (dh <= 64 || !TS) return launch_group_width<T, 64, TS>(a, dh, stream);
    if constexpr (TS) return launch_group_width<T, 128, TS>(a, dh, stream);  // Chronos-2 heads are at most 64 wide
    return hipErrorInvalidValue;
}

template <typename T>
static hipError_t dispatch_group_type(const GroupArgs& a, int dh, bool ts, hipStream_t stream) {
    return ts ? dispatch_group<T, true>(a, dh, stream) : dispatch_group<T, false>(a, dh, stream);
}

hipError_t group_attention_launch(const GroupArgs& a, int dh, bool ts, int dtype, hipStream_t stream) {
    if (dh < 8 || dh > 128 || dh % 8) return hipErrorInvalidValue;
    switch (dtype) {  // the jc_dtype codes: 0 fp32, 1 bf16, 2 fp16
        case 0: return dispatch_group_type<float>(a, dh, ts, stream);
        case 1: return dispatch_group_type<__bf16>(a, dh, ts, stream);
        case 2: return dispatch_group_type<_Float16>(a, dh, ts, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t group_tile_order_launch(const int32_t* gstart, const int32_t* gend, int rows, int32_t* order,
                                   hipStream_t stream) {
    if (rows <= 0 || (rows + kRT - 1) / kRT > kGroupOrderTiles || !gstart || !gend || !order) return hipErrorInvalidValue;
    hipLaunchKernelGGL(group_tile_order, dim3(1), dim3(1024), 0, stream, gstart, gend, rows, order);
    return hipGetLastError();
}

hipError_t group_attention_f32_x3_launch(const GroupArgs& a, int dh, hipStream_t stream) {
    if (dh != 64) return hipErrorInvalidValue;
    return launch_group<float, 64, false, true, true>(a, dh, stream);
}

}  // namespace jc
