// Time attention for gfx950, bf16 / fp16: the row-wide kernel. One 8-wave workgroup covers 256
// queries (8 tiles of 32) of one (row, head), so each K/V block is loaded, rotated and transposed
// once per 256 queries; two workgroups share a CU and run out of phase.
//
// Same contracts as time_attention_lp.hip (Chronos-2's Chronos2Kernels.rope + timeAttention,
// Chronos2Kernels.java:87-116, 118-464; Timestral's TimestralKernels.rope + timeAttention + gate,
// TimestralKernels.java:71-100, 102-278, 572-578; oracles CpuChronos2.java:175-228, 284-304 and
// CpuTimestral.java:156-161, 190-259).
//
// Work split: wave w owns queries 32w..32w+31 of the part (its 32x32 S^T tile stays in registers);
// the workgroup streams the row's 64-key blocks through a double-buffered LDS block, with one block
// in flight in registers, and one barrier per block. Staging is spread over all 512 threads:
//   K item (key, 8-dim chunk of one half): a 16-byte load; lanes l and l+32 hold the two halves of a
//     RoPE pair and exchange them with v_permlane32_swap. The rotation's cos/sin for position p are
//     composed in fp32 from two LDS tables taken from rows of the host table: T_lo (positions
//     0..63) and T_hi (positions 64a), cos(p f) = cos(64a f) cos(b f) - sin(64a f) sin(b f) for
//     p = 64a + b, so no table rows stream per block. Table rows are padded to DH+4 floats: the 8
//     lanes of one 128-byte LDS cycle read 8 consecutive positions, which then fall on distinct
//     banks (at a 256-byte pitch every row starts on the same bank: an 8-way conflict).
//   V item (4 keys, 2 dims): four 4-byte loads written as two 8-byte rows of V^T, keys permuted
//     within 16-key groups as in time_attention_lp.hip.
// Each wave computes its tile in 32-key sub-blocks (S^T 16 VGPRs, P 8), which keeps the kernel
// within 128 VGPRs: four waves per SIMD (two workgroups per CU) overlap one wave's softmax with
// another's MFMAs.
// The softmax is time_attention_lp.hip's: the key mask and the running max ride in an extra MFMA
// step, P = exp2(S) rounded to T, v_dot2 row sums, and a wave-uniform slow path for stale maxima.
#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "lp_common.hpp"
#include "time_mask.hpp"

namespace jc {
namespace {

using namespace lp;

constexpr int kQ = 32;    // queries per wave
constexpr int kKB = 64;   // keys per staged block
constexpr int kW = 8;     // waves per workgroup (256 queries)
constexpr int kThreads = kW * kWave;
constexpr int kMaxTokens = 4096;
constexpr int kMaxHi = 72;  // T_hi rows held in LDS: table rows up to 64 * 72

template <int DH, bool TS>
struct WideLds {
    static constexpr int kPitchK = DH + 8;   // elements per key row of K
    static constexpr int kPitchV = kKB + 8;  // elements per dim row of V^T
    uint16_t k[2][kKB * kPitchK];
    uint16_t vt[2][DH * kPitchV];
    static constexpr int kPitchT = DH + 4;  // floats per table row (rows of consecutive positions on distinct banks)
    float tlo[kKB * kPitchT];     // cos | sin of b * invFreq, b < 64
    float thi[kMaxHi * kPitchT];  // cos | sin of the angle of table row 64a
    uint64_t mask[kMaxTokens / kKB];
    int32_t pos[TS ? kMaxTokens : 1];
};

template <typename T, int DH, bool ROPE, bool TS>
struct WideStage {
    static constexpr int CPH = DH / 16;                 // 8-dim chunks per half
    static constexpr int KPW = 32 / CPH;                // keys per wave
    static constexpr int KWAVES = kKB / KPW;            // waves with a K item
    static constexpr int VITEMS = (kKB / 4) * (DH / 2);  // (4 keys, 2 dims) items
    static constexpr int VFIRST = kThreads - VITEMS;     // V items sit on the last threads
    static_assert(KWAVES <= kW && VITEMS <= kThreads, "staging items");
    bool has_k, has_v, first_half;
    int kk, kcol, tcol, vkey, vdim;
    uint32_t off_k, off_v;
    u32x4 kraw[2];
    uint32_t vraw[2][4];

    __device__ __forceinline__ void init(int tid, int inner) {
        const uint32_t stride = 3u * inner * 2u;
        const int wave = tid / kWave, lane = tid % kWave;
        has_k = wave < KWAVES;
        first_half = lane < 32;
        const int idx = lane & 31;
        kk = wave * KPW + idx / CPH;
        tcol = 8 * (idx % CPH);
        kcol = (first_half ? 0 : DH / 2) + tcol;
        off_k = kk * stride + kcol * 2;
        const int it = tid - VFIRST;
        has_v = it >= 0;
        const int kq = has_v ? it / (DH / 2) : 0, ep = has_v ? it % (DH / 2) : 0;
        vkey = 4 * kq;
        vdim = 2 * ep;
        off_v = vkey * stride + inner * 2 + vdim * 2;
    }

    template <int SET>
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rk, int inner) {
        const uint32_t stride = 3u * inner * 2u;
        if (has_k) kraw[SET] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off_k, 0, 0));
        if (has_v) {
#pragma unroll
            for (int u = 0; u < 4; u++) vraw[SET][u] = __builtin_amdgcn_raw_buffer_load_b32(rk, off_v + u * stride, 0, 0);
        }
    }

    // kbase: the block's first key; the K item's table position is kbase + kk (Chronos-2) or the
    // token's table row pos[kbase + kk] (Timestral)
    template <int SET>
    __device__ __forceinline__ void store(WideLds<DH, TS>& lds, int buf, int kbase, int n) {
        constexpr int PK = WideLds<DH, TS>::kPitchK, PV = WideLds<DH, TS>::kPitchV;
        constexpr int PT = WideLds<DH, TS>::kPitchT;
        if (has_k) {
            u32x4 w = kraw[SET];
            if (ROPE) {
                // the RoPE partner (the other half of the same key) is in lane l ^ 32
                u32x4 part;
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    auto sw = __builtin_amdgcn_permlane32_swap(w[d], w[d], false, false);
                    part[d] = first_half ? sw[1] : sw[0];
                }
                floatx4 x0, x1, y0, y1;
                widen8<T>(w, x0, x1);
                widen8<T>(part, y0, y1);
                const int k = kbase + kk;
                const int p = TS ? (k < n ? lds.pos[k] : 0) : k;
                const float* hi = &lds.thi[(p >> 6) * PT + tcol];
                const float* lo = &lds.tlo[(p & 63) * PT + tcol];
                floatx4 r[2];
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const floatx4 ch = *reinterpret_cast<const floatx4*>(hi + 4 * q);
                    const floatx4 sh = *reinterpret_cast<const floatx4*>(hi + DH / 2 + 4 * q);
                    const floatx4 cl = *reinterpret_cast<const floatx4*>(lo + 4 * q);
                    const floatx4 sl = *reinterpret_cast<const floatx4*>(lo + DH / 2 + 4 * q);
                    const floatx4 c = ch * cl - sh * sl;
                    const floatx4 sn = sh * cl + ch * sl;
                    const floatx4 x = q ? x1 : x0, y = q ? y1 : y0;
                    r[q] = first_half ? x * c - y * sn : x * c + y * sn;
                }
                w = narrow8<T>(r[0], r[1]);
            }
            *reinterpret_cast<u32x4*>(&lds.k[buf][kk * PK + kcol]) = w;
        }
        if (has_v) {
            const int posv = vt_pos(vkey);
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t sel = e ? 0x07060302u : 0x05040100u;  // v_perm: high or low halves
                u32x2 row;
                row[0] = __builtin_amdgcn_perm(vraw[SET][1], vraw[SET][0], sel);
                row[1] = __builtin_amdgcn_perm(vraw[SET][3], vraw[SET][2], sel);
                *reinterpret_cast<u32x2*>(&lds.vt[buf][(vdim + e) * PV + posv]) = row;
            }
        }
    }
};

template <typename T, int DH, bool ROPE, bool TS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void time_attention_lpw(const TimeArgs a) {
    static_assert(DH == 32 || DH == 64, "head width");
    constexpr int kSteps = DH / 16;  // QK^T MFMA steps (16 dims each), plus the bias step
    constexpr int kTiles = DH / 32;  // 32-dim output tiles
    constexpr int PK = WideLds<DH, TS>::kPitchK, PV = WideLds<DH, TS>::kPitchV;
    constexpr int PT = WideLds<DH, TS>::kPitchT;
    typedef typename Lp<T>::x8 x8;
    typedef Enc<T> E;
    __shared__ WideLds<DH, TS> lds;

    const T* __restrict__ qkv = static_cast<const T*>(a.qkv);
    const int n = a.n, inner = a.inner, half = DH / 2;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int j = lane % 32, g = lane / 32;
    const uint32_t total = (uint32_t)a.rows * a.heads * a.qgroups;
    const uint32_t logical = xcd_remap(blockIdx.x, total);
    const int part = logical % a.qgroups;  // the workgroup's 256-query part of the row
    const uint32_t bh = logical / a.qgroups;
    const int h = bh % a.heads, r = bh / a.heads;
    TimeMask<TS> mask;
    mask.init(a, r);
    const int32_t* vrow = a.valid + (size_t)r * (TS ? a.enc : n);
    const int qbase = part * kW * kQ;  // the workgroup's first query

    // the wave's raw queries (and their RoPE partner chunks), requested first so they arrive
    // during the prologue; their rotation uses the same composed cos/sin as the keys
    const int q0 = qbase + wave * kQ;
    const int nq = min(max(n - q0, 0), kQ);
    u32x4 q_own[kSteps], q_par[kSteps];
    if (j < nq) {
        const T* qp = qkv + ((size_t)r * n + q0 + j) * 3 * inner + h * DH;
#pragma unroll
        for (int s = 0; s < kSteps; s++) {
            const int d0 = 16 * s + 8 * g;
            const bool first = d0 < half;
            q_own[s] = *reinterpret_cast<const u32x4*>(qp + d0);
            if (ROPE) q_par[s] = *reinterpret_cast<const u32x4*>(qp + (first ? d0 + half : d0 - half));
        }
    }

    // the RoPE composition tables (rows of the host table), key validity, positions
    if (ROPE) {
        // 16-byte pieces, all requested before any is stored, so the copy costs one load latency
        constexpr int kLo = kKB * DH / 4;                          // float4 pieces of T_lo
        constexpr int kLoPer = (kLo + kThreads - 1) / kThreads;
        constexpr int kHiPer = (kMaxHi * DH / 4 + kThreads - 1) / kThreads;
        const int enc0 = TS ? a.enc : 0;  // the table row of position 0
        const floatx4* t4 = reinterpret_cast<const floatx4*>(a.table);
        const int nhi4 = (a.table_rows + kKB - 1) / kKB * (DH / 4);
        floatx4 lo4[kLoPer], hi4[kHiPer];
#pragma unroll
        for (int i = 0; i < kLoPer; i++) {
            const int f = tid + i * kThreads;
            if (f < kLo) lo4[i] = t4[(size_t)enc0 * (DH / 4) + f];
        }
#pragma unroll
        for (int i = 0; i < kHiPer; i++) {
            const int f = tid + i * kThreads;  // piece f: row 64 * (f / (DH/4)), column 4 * (f % (DH/4))
            if (f < nhi4) hi4[i] = t4[(size_t)(f / (DH / 4)) * kKB * (DH / 4) + f % (DH / 4)];
        }
#pragma unroll
        for (int i = 0; i < kLoPer; i++) {
            const int f = tid + i * kThreads;
            if (f < kLo) *reinterpret_cast<floatx4*>(&lds.tlo[(f / (DH / 4)) * PT + 4 * (f % (DH / 4))]) = lo4[i];
        }
#pragma unroll
        for (int i = 0; i < kHiPer; i++) {
            const int f = tid + i * kThreads;
            if (f < nhi4) *reinterpret_cast<floatx4*>(&lds.thi[(f / (DH / 4)) * PT + 4 * (f % (DH / 4))]) = hi4[i];
        }
    }
    const int nblk = (n + kKB - 1) / kKB;
    for (int b = wave; b < nblk; b += kW) {
        const uint64_t bits = __ballot(mask.key_valid(vrow, b * kKB + lane));
        if (lane == 0) lds.mask[b] = bits;
    }
    if (TS) {
        for (int t = tid; t < n; t += kThreads)
            lds.pos[t] = a.pos ? min(max(a.pos[(size_t)r * n + t], 0), a.table_rows - 1) : t;
    }
    __syncthreads();
    const uint64_t need = __ballot(lane < nblk && mask.any_allowed(lds.mask[lane], lane * kKB, qbase, min(qbase + kW * kQ, n) - 1));
    auto next_block = [&](int after) __attribute__((always_inline)) {
        const uint64_t rest = after + 1 >= 64 ? 0ull : need & (~0ull << (after + 1));
        return rest ? (int)__builtin_ctzll(rest) : nblk;
    };

    // Q operands: rotated, scaled by qscale (log2(e) times the score scale), rounded to T
    x8 qreg[kSteps];
    {
        const int q = q0 + j;
        const int p = TS ? (j < nq ? lds.pos[q] : 0) : q;
#pragma unroll
        for (int s = 0; s < kSteps; s++) {
            floatx4 lo = floatx4{0.f, 0.f, 0.f, 0.f}, hi = lo;
            if (j < nq) {
                widen8<T>(q_own[s], lo, hi);
                if (ROPE) {
                    const int d0 = 16 * s + 8 * g;
                    const bool first = d0 < half;
                    const int e0 = first ? d0 : d0 - half;
                    floatx4 plo, phi;
                    widen8<T>(q_par[s], plo, phi);
                    const float* th = &lds.thi[(p >> 6) * PT + e0];
                    const float* tl = &lds.tlo[(p & 63) * PT + e0];
#pragma unroll
                    for (int part = 0; part < 2; part++) {
                        const floatx4 ch = *reinterpret_cast<const floatx4*>(th + 4 * part);
                        const floatx4 sh = *reinterpret_cast<const floatx4*>(th + half + 4 * part);
                        const floatx4 cl = *reinterpret_cast<const floatx4*>(tl + 4 * part);
                        const floatx4 sl = *reinterpret_cast<const floatx4*>(tl + half + 4 * part);
                        const floatx4 c = ch * cl - sh * sl, sn = sh * cl + ch * sl;
                        floatx4& x = part ? hi : lo;
                        const floatx4 y = part ? phi : plo;
                        x = first ? x * c - y * sn : x * c + y * sn;
                    }
                }
                lo *= a.qscale;
                hi *= a.qscale;
            }
            qreg[s] = __builtin_bit_cast(x8, narrow8<T>(lo, hi));
        }
    }

    const size_t row0 = (size_t)r * n;
    const uint32_t stride_b = 3u * inner * 2u;
    auto rk_at = [&](int b) __attribute__((always_inline)) {
        const int k = b * kKB;
        const T* p = qkv + (row0 + k) * 3 * inner + inner + h * DH;
        const uint32_t bytes = (uint32_t)(n - k) * stride_b - (uint32_t)(inner + h * DH) * 2u;
        return make_rsrc(p, bytes);
    };

    // the pipeline: block i is computed from LDS buffer i % 2 while block i+1 waits in register
    // set (i+1) % 2 and block i+2 is requested into set i % 2
    WideStage<T, DH, ROPE, TS> stage;
    stage.init(tid, inner);
    int b0 = next_block(-1);
    int b1 = b0 < nblk ? next_block(b0) : nblk;
    if (b0 < nblk) stage.template load<0>(rk_at(b0), inner);
    if (b1 < nblk) stage.template load<1>(rk_at(b1), inner);
    if (b0 < nblk) stage.template store<0>(lds, 0, b0 * kKB, n);
    __syncthreads();

    floatx16 o_acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; t++) o_acc[t] = floatx16{0};
    // softmax state of query j (equal in lanes j and j+32), as in time_attention_lp.hip
    float m_tot = 0.f, m_mfma = 0.f, resid = 0.f, l_run = 0.f;
    bool has_ref = false, any_resid = false;
    uint32_t qx0 = g == 0 ? E::kBigQ : 0u;

    // one 32-key sub-block: S^T, P, the row sum check (and slow path), PV
    auto sub_block = [&](int buf, int sb, uint32_t allowed32, uint32_t kmask32, bool uniform) __attribute__((always_inline)) {
        const bool lane_keys = allowed32 != 0;
        const x8 qx = __builtin_bit_cast(x8, u32x4{qx0, 0u, 0u, 0u});
        floatx16 s_acc = floatx16{0};
        const uint16_t* kp = &lds.k[buf][(32 * sb + j) * PK + 8 * g];
#pragma unroll
        for (int s = 0; s < kSteps; s++) {
            x8 kv = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(kp + 16 * s));
            s_acc = Lp<T>::mfma(kv, qreg[s], s_acc);
        }
        const uint32_t kx0 = g == 0 ? (((kmask32 >> j) & 1u) ? E::kLive : E::kDead) : 0u;
        s_acc = Lp<T>::mfma(__builtin_bit_cast(x8, u32x4{kx0, 0u, 0u, 0u}), qx, s_acc);
        // reg rho in lane (j, g) holds key 32sb + 8*(rho/4) + 4g + rho%4 of the block
        if (!uniform) {
#pragma unroll
            for (int rho = 0; rho < 16; rho++) {
                const int bit = 8 * (rho / 4) + 4 * g + (rho % 4);
                if (!((allowed32 >> bit) & 1u)) s_acc[rho] = -INFINITY;
            }
        }
        x8 p[2];
        auto exps = [&](float shift) __attribute__((always_inline)) {
#pragma unroll
            for (int c = 0; c < 2; c++) {
                floatx4 lo, hi;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    lo[u] = fast_exp2(s_acc[8 * c + u] - shift);
                    hi[u] = fast_exp2(s_acc[8 * c + 4 + u] - shift);
                }
                p[c] = __builtin_bit_cast(x8, narrow8<T>(lo, hi));
            }
        };
        auto block_sum = [&]() __attribute__((always_inline)) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                u32x4 w = __builtin_bit_cast(u32x4, p[c]);
#pragma unroll
                for (int d = 0; d < 4; d++) acc = E::dot2(w[d], acc);
            }
            return pair_sum(acc);
        };
        if (!any_resid) {
#pragma unroll
            for (int c = 0; c < 2; c++) {
                floatx4 lo, hi;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    lo[u] = fast_exp2(s_acc[8 * c + u]);
                    hi[u] = fast_exp2(s_acc[8 * c + 4 + u]);
                }
                p[c] = __builtin_bit_cast(x8, narrow8<T>(lo, hi));
            }
        } else {
            exps(resid);
        }
        float lb = block_sum();
        const bool bad = !(lb <= kSumHi) || (!has_ref && lane_keys && !(lb >= kSumLo));
        if (__any(bad)) {
            float mx = s_acc[0];
#pragma unroll
            for (int rho = 1; rho < 16; rho++) mx = fmaxf(mx, s_acc[rho]);
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
            const uint16_t* vp = &lds.vt[buf][(32 * t + j) * PV + 32 * sb + 8 * g];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                x8 vv = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(vp + 16 * c));
                o_acc[t] = Lp<T>::mfma(vv, p[c], o_acc[t]);
            }
        }
    };

    auto compute = [&](int kb, int buf) __attribute__((always_inline)) {
        // the keys of this block the lane's query may see (bit i = key 64kb + i); lanes past the
        // last query take lane 0's keys so they never decide a wave-wide branch
        const uint64_t word = lds.mask[kb];
        uint64_t allowed = mask.allowed(word, kb * kKB, q0 + j);
        // (readfirstlane returns int: widen through uint32_t, or bit 31 would sign-extend)
        const uint64_t ref = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)allowed) |
                             ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(allowed >> 32)) << 32);
        if (j >= nq) allowed = ref;
        const bool uniform = TS ? !__any(allowed != ref) : true;
        const uint64_t kmask = uniform ? ref : ~0ull;
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            const uint32_t a32 = (uint32_t)(allowed >> (32 * sb));
            if (__any(a32 != 0)) sub_block(buf, sb, a32, (uint32_t)(kmask >> (32 * sb)), uniform);
        }
    };

    // one pipeline step with compile-time register sets: compute block `cur` (buffer SET), store
    // block `nxt` (held in set 1-SET) into buffer 1-SET, request block `far` into set SET
    int cur = b0, nxt = b1;
    __builtin_amdgcn_s_waitcnt(0);
    auto step = [&](auto set_tag) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_tag)::value;
        const int far = nxt < nblk ? next_block(nxt) : nblk;
        if (far < nblk) stage.template load<SET>(rk_at(far), inner);
        __builtin_amdgcn_sched_barrier(0);
        if (nq > 0) compute(cur, SET);
        if (nxt < nblk) stage.template store<1 - SET>(lds, 1 - SET, nxt * kKB, n);
        __syncthreads();
        cur = nxt;
        nxt = far;
    };
    while (cur < nblk) {
        step(std::integral_constant<int, 0>{});
        if (cur >= nblk) break;
        step(std::integral_constant<int, 1>{});
    }

    if (j < nq) {
        const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
        const size_t tok = (size_t)r * n + q0 + j;
        T* op = static_cast<T*>(a.out) + tok * inner + h * DH;
        const T* gp = a.gate ? static_cast<const T*>(a.gate) + tok * inner + h * DH : nullptr;
        // O^T reg 4a+u of lane (j, g) in tile t is dim 32t + 8a + 4g + u of query j
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++) {
                const int e = 32 * t + 8 * a4 + 4 * g;
                floatx4 v;
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = o_acc[t][4 * a4 + u] * inv;
                if (gp) {
                    // the output gate: att * sigmoid(g) (CpuTimestral.java:156-161)
                    floatx4 gv, gz;
                    const u32x2 graw = *reinterpret_cast<const u32x2*>(gp + e);
                    widen8<T>(u32x4{graw[0], graw[1], 0u, 0u}, gv, gz);
#pragma unroll
                    for (int u = 0; u < 4; u++) v[u] *= 1.f / (1.f + fast_exp2(-gv[u] * kLog2e));
                }
                *reinterpret_cast<u32x2*>(op + e) = narrow4<T>(v);
            }
        }
    }
}

template <typename T, int DH, bool TS>
hipError_t launch_lpw(TimeArgs a, hipStream_t stream) {
    a.qgroups = (a.n + kW * kQ - 1) / (kW * kQ);
    const uint64_t grid = (uint64_t)a.rows * a.heads * a.qgroups;
    if (a.table) {
        hipLaunchKernelGGL((time_attention_lpw<T, DH, true, TS>), dim3((uint32_t)grid), dim3(kThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL((time_attention_lpw<T, DH, false, TS>), dim3((uint32_t)grid), dim3(kThreads), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace

bool time_attention_lpw_fits(const TimeArgs& a, int dh) {
    if (dh != 32 && dh != 64) return false;
    if (a.n < 256) return false;  // 8 tiles or more: short rows keep the streaming kernel
    if (a.table && (a.table_rows + kKB - 1) / kKB > kMaxHi) return false;
    return true;
}

hipError_t time_attention_lpw_launch(const TimeArgs& a, int dh, bool ts, bool fp16, hipStream_t stream) {
    if (fp16) {
        if (dh == 32) return ts ? launch_lpw<_Float16, 32, true>(a, stream) : launch_lpw<_Float16, 32, false>(a, stream);
        return ts ? launch_lpw<_Float16, 64, true>(a, stream) : launch_lpw<_Float16, 64, false>(a, stream);
    }
    if (dh == 32) return ts ? launch_lpw<__bf16, 32, true>(a, stream) : launch_lpw<__bf16, 32, false>(a, stream);
    return ts ? launch_lpw<__bf16, 64, true>(a, stream) : launch_lpw<__bf16, 64, false>(a, stream);
}

}  // namespace jc
