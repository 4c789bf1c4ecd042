// Chronos-2 time attention for gfx950, bf16 / fp16: the persistent kernel for short rows (65..160
// tokens; config 4's forecasts run 133 = 128 patches + [REG] + 4 future patches).
//
// Same contract as time_attention_lp.hip for Chronos-2 (Chronos2Kernels.rope + timeAttention,
// Chronos2Kernels.java:87-116, 118-464; oracle CpuChronos2.java:175-228, 284-304): every query of a
// row sees the row's live keys, scores are unscaled, RoPE at token positions.
//
// Why a kernel of its own. A short row has 2 or 3 64-key blocks. The streaming kernel gives each
// (row, head) one or two workgroups whose life is a chain of dependent loads (the validity row,
// every block, each behind a barrier) with little compute in between, and a row of 133 tokens
// spends a second workgroup on its last 5 queries. Here the loads of one item overlap the compute
// of the items before it:
//   - A workgroup has two halves of HW waves (HW = query tiles of the row, 3..5). Each half walks
//     its own list of (row, head) items, wave w of the half owning queries 32w..32w+31 of every
//     item, and streams the items' blocks back to back through a ring of three LDS slots. The two
//     halves step in lockstep (every item has the same number of blocks; blocks without a live key
//     are masked, not skipped) and share the RoPE tables and one barrier per step.
//   - Step e of a half: wait until element e + 1 landed, barrier, issue element e + 2 into the
//     slot element e - 1 left, rotate element e + 1's K in place, compute element e. So a block's
//     loads have a whole step to land, and no LDS slot is written while it is read.
//   - K and V arrive by direct-to-LDS loads into swizzled 128-byte key rows; K is rotated in place
//     (cos / sin composed from two LDS tables of host-table rows, as in time_attention_lpp.hip); V
//     stays row-major and the PV operand comes from transposing LDS reads. The next item's Q tiles
//     are prefetched into a per-wave LDS area during the current item's first step.
//   - The kernel is bound by instruction issue, not by HBM (the loads alone run in 75% of its
//     time), so per-step bookkeeping is kept off the VALU and SALU: cursors instead of divisions,
//     each lane's load offsets computed once, and with 5 or 3 waves per half (SIMDs holding 3, 3,
//     2, 2 waves) the K rotation done by the waves of the two less loaded SIMDs.
// The softmax is time_attention_lp.hip's: the key mask and the running max ride in an extra MFMA
// step, P = exp2(S) rounded to T, v_dot2 row sums, and a wave-uniform slow path for stale maxima.
#include <algorithm>

#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "lp_common.hpp"
#include "lp_stream.hpp"

namespace jc {
namespace {

using namespace lp;

constexpr int kDH = 64;
constexpr int kQ = 32;        // queries per tile
constexpr int kKB = 64;       // keys per block
constexpr int kSlots = 3;     // LDS ring slots per half (K and V of one block each)
constexpr int kMaxBlk = 3;    // 64-key blocks per row at most
constexpr int kMaxHW = 5;     // query tiles per row at most (n <= 160)
constexpr int kIpw = 24;      // items per workgroup at most (both halves)
constexpr int kPT = kDH + 4;  // floats per RoPE table row in LDS

template <int HW>
struct SLds {
    uint16_t kv[2][kSlots][2][kKB * kDH];  // [half][slot][K | V][key * 64 + swizzled dim]
    uint16_t q[2][HW][kQ * kDH];           // prefetched raw Q of the half's next item, per wave
    float tlo[kKB * kPT];                  // cos | sin of b * invFreq, b < 64
    float thi[kMaxBlk * kPT];              // cos | sin of 64a * invFreq
    uint64_t mask[kIpw][kMaxBlk];          // live bits per item and block
};

template <typename T, bool ROPE, int HW>
__global__ __launch_bounds__(2 * HW * kWave) __attribute__((amdgpu_waves_per_eu(HW > 4 ? 3 : 2))) void
time_attention_lps(const TimeArgs a, int items, int groups) {
    typedef typename Lp<T>::x8 x8;
    typedef Enc<T> E;
    constexpr int kThreads = 2 * HW * kWave;
    __shared__ SLds<HW> lds;

    const T* __restrict__ qkv = static_cast<const T*>(a.qkv);
    const int n = a.n, inner = a.inner, heads = a.heads;
    const int tid = threadIdx.x, lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int half = wave / HW, hw = wave % HW;  // the wave's half and its place in the half
    const int j = lane % 32, g = lane / 32;
    const int wg = blockIdx.x;
    const int K = min(kIpw, (items - wg + groups - 1) / groups);  // items wg + k * groups
    const int nblk = (n + kKB - 1) / kKB;
    const size_t rs = 3 * (size_t)inner;  // elements per token of qkv
    // the half's items are k = 2i + half; both halves run steps for ceil(K / 2) items
    const int kh = (K - half + 1) / 2;
    const int steps = ((K + 1) / 2) * nblk;

    // ---- prologue: RoPE composition tables, live words of every item -------------------------
    if (ROPE) {
        const floatx4* t4 = reinterpret_cast<const floatx4*>(a.table);
        constexpr int kLo = kKB * kDH / 4;  // float4 pieces of T_lo
        const int nhi = nblk * (kDH / 4);
        for (int f = tid; f < kLo; f += kThreads)
            *reinterpret_cast<floatx4*>(&lds.tlo[(f / (kDH / 4)) * kPT + 4 * (f % (kDH / 4))]) = t4[f];
        for (int f = tid; f < nhi; f += kThreads)
            *reinterpret_cast<floatx4*>(&lds.thi[(f / (kDH / 4)) * kPT + 4 * (f % (kDH / 4))]) =
                t4[(size_t)(f / (kDH / 4)) * kKB * (kDH / 4) + f % (kDH / 4)];
    }
    {
        constexpr int kW = 2 * HW;
        constexpr int kPer = (kIpw * kMaxBlk + kW - 1) / kW;
        const int pairs = K * nblk;
        int32_t lv[kPer];
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const int pi = wave + kW * i;
            lv[i] = 0;
            if (pi < pairs) {
                const int k = pi / nblk, b = pi % nblk, r = (wg + k * groups) / heads, key = b * kKB + lane;
                if (key < n) lv[i] = a.valid[(size_t)r * n + key];
            }
        }
#pragma unroll
        for (int i = 0; i < kPer; i++) {
            const int pi = wave + kW * i;
            const uint64_t bits = __ballot(lv[i] != 0);
            if (pi < pairs && lane == 0) lds.mask[pi / nblk][pi % nblk] = bits;
        }
    }

    // ---- the half's stream of (item, block) elements: element e is block e % nblk of the half's
    // item e / nblk, i.e. item 2 (e / nblk) + half of the workgroup. Cursors follow the element
    // computed, the one rotated and the next one loaded (no divisions per step).
    struct Cur {
        int i, b, slot;  // the half's item index, block, ring slot
    };
    auto adv = [&](Cur& c) __attribute__((always_inline)) {
        c.slot = c.slot + 1 == kSlots ? 0 : c.slot + 1;
        if (++c.b == nblk) {
            c.b = 0;
            c.i++;
        }
    };
    auto item_rh = [&](int k, int& r, int& h) __attribute__((always_inline)) {
        const int it = wg + k * groups;
        r = it / heads;
        h = it % heads;
    };
    // loads per element and wave: the block's 16 1-KB pieces (8 key rows of K or of V each), piece
    // d taken by wave d % HW of the half; each lane's key and column offset are fixed per piece
    constexpr int kMaxP = (16 + HW - 1) / HW;
    const int kv_loads = (16 - hw + HW - 1) / HW;
    int p_key[kMaxP], p_col[kMaxP];
#pragma unroll
    for (int p = 0; p < kMaxP; p++) {
        const int d = hw + p * HW, key = 8 * (d % 8) + lane / 8;
        p_key[p] = key;
        p_col[p] = (1 + d / 8) * inner + 8 * ((lane % 8) ^ (key & 7));
    }
    const T* ld_base = qkv;  // q|k|v of (row, head) of the item the load cursor is in
    int ld_item = -1;
    auto issue_kv = [&](const Cur& c) __attribute__((always_inline)) {
        if (c.i != ld_item) {
            int r, h;
            item_rh(2 * c.i + half, r, h);
            ld_item = c.i;
            ld_base = qkv + (size_t)r * n * rs + h * kDH;
        }
#pragma unroll
        for (int p = 0; p < kMaxP; p++) {
            if (p < kv_loads) {
                const int d = hw + p * HW;
                const uint32_t tok = (uint32_t)min(c.b * kKB + p_key[p], n - 1);
                dma16(ld_base + (tok * (uint32_t)rs + (uint32_t)p_col[p]),
                      &lds.kv[half][c.slot][d / 8][8 * (d % 8) * kDH]);
            }
        }
    };
    // the wave's Q tile of item k: 4 loads
    auto issue_q = [&](int k) __attribute__((always_inline)) {
        const int ln = opaque(lane);
        int r, h;
        item_rh(k, r, h);
        const T* base = qkv + (size_t)r * n * rs + h * kDH;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int jq = 8 * i + ln / 8;
            const int q = min(32 * hw + jq, n - 1);
            const int c = (ln % 8) ^ (jq & 7);
            dma16(base + (size_t)q * rs + 8 * c, &lds.q[half][hw][8 * i * kDH]);
        }
    };

    // RoPE cos / sin of position p for freqs f0..f0+3, composed from the two tables
    auto cs4 = [&](int p, int f0, floatx4& c, floatx4& s) __attribute__((always_inline)) {
        const float* hi = &lds.thi[(p >> 6) * kPT + f0];
        const float* lo = &lds.tlo[(p & 63) * kPT + f0];
        const floatx4 ch = *reinterpret_cast<const floatx4*>(hi);
        const floatx4 sh = *reinterpret_cast<const floatx4*>(hi + kDH / 2);
        const floatx4 cl = *reinterpret_cast<const floatx4*>(lo);
        const floatx4 sl = *reinterpret_cast<const floatx4*>(lo + kDH / 2);
        c = ch * cl - sh * sl;
        s = sh * cl + ch * sl;
    };
    // K of element c rotated in place: lane = (key 8kg + l/8, chunk pair cp, half-chunk hh). With 5
    // or 3 waves per half the workgroup's waves sit 3, 3, 2, 2 (2, 2, 1, 1) to a SIMD (wave w on
    // SIMD w % 4), so the 8 key groups go to the waves of SIMDs 2 and 3; with 4 they go round.
    int rot_first = hw, rot_stride = HW;
    bool rotator = true;
    if (HW != 4) {
        int rank = 0, cnt = 0;
        for (int w = 0; w < HW; w++) {
            const bool rot = (half * HW + w) % 4 >= 2;
            rank += rot && w < hw ? 1 : 0;
            cnt += rot ? 1 : 0;
        }
        rotator = (half * HW + hw) % 4 >= 2;
        rot_first = rank;
        rot_stride = cnt;
    }
    auto rotate_k = [&](const Cur& cu) __attribute__((always_inline)) {
        if (!ROPE || !rotator) return;
        const int cp = (lane % 8) / 2, hh = lane % 2;
        for (int kg = rot_first; kg < 8; kg += rot_stride) {
            const int key = 8 * kg + lane / 8;
            uint16_t* p0 = &lds.kv[half][cu.slot][0][swz(key, cp) + 4 * hh];
            uint16_t* p1 = &lds.kv[half][cu.slot][0][swz(key, cp + 4) + 4 * hh];
            const floatx4 x = widen4<T>(*reinterpret_cast<const u32x2*>(p0));
            const floatx4 y = widen4<T>(*reinterpret_cast<const u32x2*>(p1));
            floatx4 c, s;
            cs4(cu.b * kKB + key, 8 * cp + 4 * hh, c, s);
            *reinterpret_cast<u32x2*>(p0) = narrow4<T>(x * c - y * s);
            *reinterpret_cast<u32x2*>(p1) = narrow4<T>(y * c + x * s);
        }
    };

    Tile tl;
    x8 qreg[4];
    // item start: the wave's Q tile from LDS, rotated, scaled, rounded; state reset
    auto start_item = [&]() __attribute__((always_inline)) {
        const int ln = opaque(lane), jj = ln % 32, gg = ln / 32;
        const int q = 32 * hw + jj;
#pragma unroll
        for (int sp = 0; sp < 2; sp++) {
            const int c0 = 2 * sp + gg;
            floatx4 x0, x1, y0, y1;
            widen8<T>(*reinterpret_cast<const u32x4*>(&lds.q[half][hw][swz(jj, c0)]), x0, x1);
            widen8<T>(*reinterpret_cast<const u32x4*>(&lds.q[half][hw][swz(jj, c0 + 4)]), y0, y1);
            if (ROPE) {
                const int f0 = 16 * sp + 8 * gg;
                floatx4 ca, sa, cb, sb;
                cs4(q, f0, ca, sa);
                cs4(q, f0 + 4, cb, sb);
                const floatx4 rx0 = x0 * ca - y0 * sa, ry0 = y0 * ca + x0 * sa;
                const floatx4 rx1 = x1 * cb - y1 * sb, ry1 = y1 * cb + x1 * sb;
                x0 = rx0; y0 = ry0; x1 = rx1; y1 = ry1;
            }
            const float sc = q < n ? a.qscale : 0.f;
            qreg[sp] = __builtin_bit_cast(x8, narrow8<T>(x0 * sc, x1 * sc));
            qreg[sp + 2] = __builtin_bit_cast(x8, narrow8<T>(y0 * sc, y1 * sc));
        }
        tl.o[0] = floatx16{0};
        tl.o[1] = floatx16{0};
        tl.m_tot = 0.f;
        tl.m_mfma = 0.f;
        tl.resid = 0.f;
        tl.l_run = 0.f;
        tl.has_ref = false;
        tl.any_resid = false;
        tl.qx0 = gg == 0 ? E::kBigQ : 0u;
    };

    // the softmax slow path: the exact block max, a new reference rounded to T, P recomputed, the
    // O/l rescale (a wave-uniform branch, taken when a block's sums leave the fast path's range)
    auto softmax_slow = [&](floatx16& s_acc, x8 (&p)[2], float& lb) __attribute__((always_inline)) {
        lp::softmax_slow<T>(tl, s_acc, p, lb, g);
    };
    // the fast path: P = exp2(S) against the current reference; true when a block's sum leaves
    // the range it can carry (the slow path then recomputes it)
    auto sm_fast = [&](const floatx16& s_acc, x8 (&p)[2], float& lb) __attribute__((always_inline)) {
        return lp::softmax_fast<T>(tl, s_acc, p, lb);
    };
    // the wave's tile against element e's block, per 32-key half: QK^T (4 steps and the mask /
    // reference step), the softmax, PV from transposing reads of V; halves without a live key are
    // skipped (uniform across the wave)
    auto compute = [&](int slot, uint64_t kmask) __attribute__((always_inline)) {
        const uint16_t* kb = lds.kv[half][slot][0];
        const uint16_t* vb = lds.kv[half][slot][1];
        const int G = lane / 16, rr = lane % 16;
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            const uint32_t a32 = (uint32_t)(kmask >> (32 * sb));
            if (a32 == 0u) continue;
            x8 kop[4];
#pragma unroll
            for (int s = 0; s < 4; s++)
                kop[s] = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(&kb[swz(32 * sb + j, 2 * s + g)]));
            const uint32_t kx0 = g == 0 ? (((a32 >> j) & 1u) ? E::kLive : E::kDead) : 0u;
            floatx16 sacc = floatx16{0};
#pragma unroll
            for (int s = 0; s < 4; s++) sacc = Lp<T>::mfma(kop[s], qreg[s], sacc);
            sacc = Lp<T>::mfma(__builtin_bit_cast(x8, u32x4{kx0, 0u, 0u, 0u}),
                               __builtin_bit_cast(x8, u32x4{tl.qx0, 0u, 0u, 0u}), sacc);
            x8 vop[2][2];
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const int key = 32 * sb + 16 * c + 4 * g + rr / 4;
                    const int ch = 4 * dt + 2 * (G % 2) + (rr % 4) / 2, off = 4 * (rr % 2);
                    const u32x2 v0 = read_tr(&vb[swz(key, ch) + off]);
                    const u32x2 v1 = read_tr(&vb[swz(key + 8, ch) + off]);
                    vop[dt][c] = __builtin_bit_cast(x8, u32x4{v0[0], v0[1], v1[0], v1[1]});
                }
            }
            x8 p[2];
            float lb = 0.f;
            // a tile without a reference yet (its first live keys) goes straight to the exact max
            const bool bad = tl.has_ref ? sm_fast(sacc, p, lb) : true;
            if (bad || tl.any_resid) softmax_slow(sacc, p, lb);
            tl.l_run += lb;
            tl.has_ref = true;
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
#pragma unroll
                for (int c = 0; c < 2; c++) tl.o[dt] = Lp<T>::mfma(vop[dt][c], p[c], tl.o[dt]);
            }
        }
    };

    // item end: the normalized outputs of the wave's tile
    auto finish_item = [&](int r, int h) __attribute__((always_inline)) {
        const int ln = opaque(lane), jj = ln % 32, gg = ln / 32;
        const int q = 32 * hw + jj;
        if (q >= n) return;
        const float inv = tl.l_run > 0.f ? 1.f / tl.l_run : 0.f;
        T* op = static_cast<T*>(a.out) + ((size_t)r * n + q) * inner + h * kDH;
        // O^T reg 4a+u of lane (j, g) in dim tile dt is dim 32dt + 8a + 4g + u of query j
#pragma unroll
        for (int dt = 0; dt < 2; dt++) {
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++) {
                floatx4 v;
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = tl.o[dt][4 * a4 + u] * inv;
                *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * a4 + 4 * gg) = narrow4<T>(v);
            }
        }
    };

    // ---- prologue loads: Q of the half's first item, elements 0 and 1 --------------------------
    const int helems = kh * nblk;  // elements of this half (kh items); later steps idle
    Cur cc{0, 0, 0}, rc{0, 0, 0}, lc{0, 0, 0};  // computed, rotated, loaded next
    int issued = 0;
    if (kh > 0) {
        issue_q(half);
        issue_kv(lc);
        adv(lc);
        issued = 1;
        if (helems > 1) {
            issue_kv(lc);
            adv(lc);
            issued = 2;
        }
    }
    // element 0 and the Q tile before it landed (element 1's loads may still be in flight), and the
    // live words and tables written
    if (helems > 1) wait_vm_rt(kv_loads);
    else wait_vm<0>();
    lds_barrier();
    if (kh > 0) rotate_k(rc);
    adv(rc);
    bool fin = false;     // the previous item's tile still to be written
    bool q_prev = false;  // the previous step issued the next item's Q tile
    int pr = 0, ph = 0;
    for (int e = 0; e < steps; e++) {
        const bool active = e < helems;
        const bool item_start = cc.b == 0, item_end = cc.b == nblk - 1;
        // element e + 1 landed: its loads were issued at step e - 1, before that step's output
        // stores and its Q loads (4, at an item start), which the next item needs only later.
        // Loads complete in order among themselves, so at most 4 outstanding leaves none of e + 1's.
        if (q_prev) wait_vm<4>();
        else wait_vm<0>();
        lds_barrier();
        // element e + 2 into the slot element e - 1 left (every wave is past its compute)
        if (issued < helems) {
            issue_kv(lc);
            adv(lc);
            issued++;
        }
        // the previous item's output stores go out after this step's wait: s_waitcnt vmcnt counts
        // stores too, so stores issued at the end of the item would hold up that wait
        if (fin) finish_item(pr, ph);
        fin = false;
        q_prev = false;
        if (!active) continue;
        if (item_start) start_item();
        if (e + 1 < helems) rotate_k(rc);
        compute(cc.slot, lds.mask[2 * cc.i + half][cc.b]);
        if (item_end) {
            item_rh(2 * cc.i + half, pr, ph);
            fin = true;
        }
        // the next item's Q tile into the area start_item read (after the compute, which consumed
        // those reads); the next item starts nblk - 1 >= 1 steps later
        if (item_start && cc.i + 1 < kh) {
            issue_q(2 * (cc.i + 1) + half);
            q_prev = true;
        }
        adv(cc);
        adv(rc);
    }
    if (fin) finish_item(pr, ph);
}

template <typename T, bool ROPE>
hipError_t launch_lps_hw(int hw, const TimeArgs& a, dim3 grid, int items, int groups, hipStream_t stream) {
    switch (hw) {
        case 3:
            hipLaunchKernelGGL((time_attention_lps<T, ROPE, 3>), grid, dim3(2 * 3 * kWave), 0, stream, a, items, groups);
            break;
        case 4:
            hipLaunchKernelGGL((time_attention_lps<T, ROPE, 4>), grid, dim3(2 * 4 * kWave), 0, stream, a, items, groups);
            break;
        default:
            hipLaunchKernelGGL((time_attention_lps<T, ROPE, 5>), grid, dim3(2 * 5 * kWave), 0, stream, a, items, groups);
            break;
    }
    return hipGetLastError();
}

}  // namespace

bool time_attention_lps_fits(const TimeArgs& a, int dh, bool ts) {
    if (ts || dh != kDH || a.gate || a.q_begin != 0) return false;
    if (a.n <= kKB || a.n > kMaxHW * kQ) return false;
    if (a.table && a.table_rows < a.n) return false;
    return true;
}

hipError_t time_attention_lps_launch(const TimeArgs& a, bool fp16, int cus, hipStream_t stream) {
    const uint64_t items = (uint64_t)a.rows * a.heads;
    if (items == 0) return hipSuccess;
    // as many workgroups as make the last round of the CUs full: items spread evenly, at most kIpw
    // per workgroup, a multiple of the CU count where that keeps every workgroup busy
    uint64_t groups = (items + kIpw - 1) / kIpw;
    const uint64_t rounds = (groups + cus - 1) / cus;
    if (rounds * cus <= items) groups = rounds * cus;
    const dim3 grid((uint32_t)groups);
    const int hw = (a.n + kQ - 1) / kQ, it = (int)items, gr = (int)groups;
    if (fp16) {
        return a.table ? launch_lps_hw<_Float16, true>(hw, a, grid, it, gr, stream)
                       : launch_lps_hw<_Float16, false>(hw, a, grid, it, gr, stream);
    }
    return a.table ? launch_lps_hw<__bf16, true>(hw, a, grid, it, gr, stream)
                   : launch_lps_hw<__bf16, false>(hw, a, grid, it, gr, stream);
}

}  // namespace jc
