// Chronos-2 time attention for gfx950, bf16 / fp16: the persistent kernel.
//
// Same contract as time_attention_lp.hip for Chronos-2 (Chronos2Kernels.rope + timeAttention,
// Chronos2Kernels.java:87-116, 118-464; oracle CpuChronos2.java:175-228, 284-304): every query of a
// row sees the row's live keys, scores are unscaled, RoPE at token positions.
//
// One 8-wave workgroup per CU walks a fixed list of (row, head) items. Wave w owns two 32-query
// tiles of every item (queries 32w.. and 256+32w..), so 512 queries share each K/V block. Query 512
// (Chronos-2's [REG] token at the end of a 512-patch context) is spread over all waves: its scores
// come out of the K rotation, every wave runs the same scalar online softmax over a block's 64
// scores and accumulates its 8 keys' share of the output, and the shares are added once per item.
//
// The workgroup streams the 64-key blocks of its items, back to back across items, through a ring
// of four LDS slots:
//   - K and V of a block arrive by direct-to-LDS loads (global_load_lds_dwordx4, no VGPRs),
//     issued three blocks ahead. Each key row is 128 bytes with its 16-byte chunks XOR-swizzled by
//     the key's low 3 bits, which keeps both MFMA operand reads and the DMA writes conflict-free.
//   - K is rotated in place one block ahead (RoPE: cos/sin composed from two LDS tables of
//     host-table rows, cos((64a+b)f) = cos(64af)cos(bf) - sin(64af)sin(bf)).
//   - V stays row-major: the PV operand V^T comes from ds_read_b64_tr_b16 (transposing 16-bit
//     reads), so V costs no VALU work at all.
//   - The next item's Q is prefetched the same way into a per-wave LDS area while the current item
//     runs.
// One barrier per block. Wait counts are explicit: every load of the stream is a direct-to-LDS
// load, loads complete in order among themselves, so waiting until no more than (loads issued
// after X) are outstanding guarantees X has landed, whatever stores are pending. Pending stores
// still hold such a wait up (the counter counts them too), so an item's output stores go out right
// after the next step's wait instead of at the end of its last step.
//
// The softmax is time_attention_lp.hip's: the key mask and the running max ride in an extra MFMA
// step, P = exp2(S) rounded to T, v_dot2 row sums, and a wave-uniform slow path for stale maxima.
#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "lp_common.hpp"
#include "lp_stream.hpp"
#include "time_mask.hpp"

namespace jc {
namespace {

using namespace lp;

constexpr int kDH = 64;
constexpr int kQ = 32;                   // queries per tile
constexpr int kKB = 64;                  // keys per block
constexpr int kW = 8;                    // waves per workgroup
constexpr int kThreads = kW * kWave;
constexpr int kTiles = 2;                // query tiles per wave
constexpr int kPart = kW * kTiles * kQ;  // queries the tiles cover (512)
constexpr int kSlots = 4;                // LDS ring slots (K and V of one block each)
constexpr int kAhead = 3;                // blocks between a block's load and its compute
constexpr int kIpw = 12;                 // items per workgroup at most
constexpr int kMaxBlk = 9;               // 64-key blocks per row at most (n <= 576)
constexpr int kPT = kDH + 4;             // floats per RoPE table row in LDS
constexpr int kMaxN = kPart + 1;         // rows up to 512 tokens plus the [REG] token

struct PLds {
    uint16_t kv[kSlots][2][kKB * kDH];  // [slot][K | V][key * 64 + swizzled dim]
    uint16_t q[kW][kTiles][kQ * kDH];   // prefetched raw Q of the next item, per wave and tile
    uint16_t reg_raw[3][kDH];           // raw q of query 512, by item mod 3 (loaded two items ahead)
    float tlo[kKB * kPT];               // cos | sin of b * invFreq, b < 64
    float thi[kMaxBlk * kPT];           // cos | sin of 64a * invFreq
    uint64_t mask[kIpw][kMaxBlk];       // live bits per item and block
    uint32_t need[kIpw];                // blocks of an item with a live key
    float reg_part[2][kW][kDH + 2];     // query 512: each wave's share of the output, its max and sum
};

template <typename T, bool ROPE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void time_attention_lpp(
    const TimeArgs a, int items, int groups) {
    typedef typename Lp<T>::x8 x8;
    typedef Enc<T> E;
    __shared__ PLds lds;

    const T* __restrict__ qkv = static_cast<const T*>(a.qkv);
    const int n = a.n, inner = a.inner, heads = a.heads;
    const int tid = threadIdx.x, lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int j = lane % 32, g = lane / 32;
    const int wg = blockIdx.x;
    const int K = min(kIpw, (items - wg + groups - 1) / groups);  // items wg + k * groups
    const int nblk = (n + kKB - 1) / kKB;
    const size_t rs = 3 * (size_t)inner;  // elements per token of qkv
    const bool has_reg = n > kPart;

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
    __syncthreads();
    if (tid < K) {
        uint32_t nd = 0;
        for (int b = 0; b < nblk; b++) nd |= (lds.mask[tid][b] != 0ull ? 1u : 0u) << b;
        lds.need[tid] = nd ? nd : 1u;  // an item without live keys still runs one (dead) block
    }
    __syncthreads();

    // ---- the stream of (item, block) elements ------------------------------------------------
    auto first_blk = [&](int k) __attribute__((always_inline)) { return (int)__builtin_ctz(lds.need[k]); };
    // next element after (k, b): returns false at the end of the stream
    auto advance = [&](int& k, int& b) __attribute__((always_inline)) {
        const uint32_t rest = lds.need[k] & ~((2u << b) - 1u);
        if (rest) {
            b = (int)__builtin_ctz(rest);
        } else {
            k++;
            b = k < K ? first_blk(k) : 0;
        }
        return k < K;
    };
    auto item_rh = [&](int k, int& r, int& h) __attribute__((always_inline)) {
        const int it = wg + k * groups;
        r = it / heads;
        h = it % heads;
    };

    // direct-to-LDS loads: K and V of element (k, b) into `slot` (keys 8w..8w+7 of the block per
    // wave); 2 loads per wave
    auto issue_kv = [&](int k, int b, int slot) __attribute__((always_inline)) {
        int r, h;
        item_rh(k, r, h);
        const int key = 8 * wave + lane / 8;
        const int tok = min(b * kKB + key, n - 1);
        const int c = (lane % 8) ^ (key & 7);
        const T* src = qkv + ((size_t)r * n + tok) * rs + inner + h * kDH + 8 * c;
        dma16(src, &lds.kv[slot][0][8 * wave * kDH]);
        dma16(src + inner, &lds.kv[slot][1][8 * wave * kDH]);
    };
    // the wave's two Q tiles of item k: 8 loads
    auto issue_q = [&](int k) __attribute__((always_inline)) {
        const int ln = opaque(lane);
        int r, h;
        item_rh(k, r, h);
        const T* base = qkv + (size_t)r * n * rs + h * kDH;
#pragma unroll
        for (int i = 0; i < 2 * kTiles * 2; i++) {
            const int t = i / 4, jq = 8 * (i % 4) + ln / 8;
            const int q = min(32 * wave + kW * kQ * t + jq, n - 1);
            const int c = (ln % 8) ^ (jq & 7);
            dma16(base + (size_t)q * rs + 8 * c, &lds.q[wave][t][8 * (i % 4) * kDH]);
        }
    };
    // query 512's raw q of item k into reg_raw[k % 3] (wave 0: 1 load)
    auto issue_reg_raw = [&](int k) __attribute__((always_inline)) {
        const int ln = opaque(lane);
        int r, h;
        item_rh(k, r, h);
        if (ln < 8) dma16(qkv + ((size_t)r * n + kPart) * rs + h * kDH + 8 * ln, lds.reg_raw[k % 3]);
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

    // Query 512 ([REG]) is spread over all waves. Lane (key 8w + l/8, chunk pair cp, half hh) holds
    // the scaled, rotated q of query 512 at the dims it rotates for K (rq_lo: f0..f0+3, rq_hi: the
    // partners f0+32..), so scores come out of the K rotation: 8 products per lane, summed over the
    // 8 lanes of a key, and stay in those lanes until the block is computed one step later. Each
    // wave runs its own online softmax over its 8 keys per block (a lazy reference max, fp32 P),
    // lane (key, c) accumulating dims 8c..8c+7 of the output; the waves' shares are rescaled to a
    // common max and added once per item.
    floatx4 rq_lo = floatx4{0.f, 0.f, 0.f, 0.f}, rq_hi = rq_lo;
    auto load_reg_q = [&](int k) __attribute__((always_inline)) {
        const int ln = opaque(lane), f0 = 8 * ((ln % 8) / 2) + 4 * (ln % 2);
        floatx4 x = widen4<T>(*reinterpret_cast<const u32x2*>(&lds.reg_raw[k % 3][f0]));
        floatx4 y = widen4<T>(*reinterpret_cast<const u32x2*>(&lds.reg_raw[k % 3][f0 + kDH / 2]));
        if (ROPE) {
            floatx4 c, s;
            cs4(kPart, f0, c, s);
            const floatx4 rx = x * c - y * s, ry = y * c + x * s;
            x = rx;
            y = ry;
        }
        rq_lo = x * a.qscale;
        rq_hi = y * a.qscale;
    };

    // K of block b in `slot` rotated in place: lane = (key 8w + l/8, chunk pair cp, half hh); with
    // `reg`, query 512's score of the lane's key into rs_next
    float rs_next = 0.f;  // query 512's score of this lane's key in the block rotated this step
    auto rotate_k = [&](int b, int slot, bool reg) __attribute__((always_inline)) {
        if (!ROPE && !reg) return;
        const int key = 8 * wave + lane / 8, cp = (lane % 8) / 2, hh = lane % 2;
        uint16_t* p0 = &lds.kv[slot][0][swz(key, cp) + 4 * hh];
        uint16_t* p1 = &lds.kv[slot][0][swz(key, cp + 4) + 4 * hh];
        floatx4 x = widen4<T>(*reinterpret_cast<const u32x2*>(p0));
        floatx4 y = widen4<T>(*reinterpret_cast<const u32x2*>(p1));
        if (ROPE) {
            floatx4 c, s;
            cs4(b * kKB + key, 8 * cp + 4 * hh, c, s);
            const floatx4 rx = x * c - y * s, ry = y * c + x * s;
            x = rx;
            y = ry;
            *reinterpret_cast<u32x2*>(p0) = narrow4<T>(x);
            *reinterpret_cast<u32x2*>(p1) = narrow4<T>(y);
        }
        if (reg) {
            float sc = 0.f;
#pragma unroll
            for (int u = 0; u < 4; u++) sc += x[u] * rq_lo[u] + y[u] * rq_hi[u];
            sc += dpp<0xB1>(sc);   // quad_perm [1,0,3,2]
            sc += dpp<0x4E>(sc);   // quad_perm [2,3,0,1]
            sc += dpp<0x141>(sc);  // row_half_mirror: every lane of the 8 holds the key's sum
            rs_next = sc;
        }
    };

    Tile tl[kTiles];
    x8 qreg[kTiles][4];

    // item start: the wave's Q tiles from LDS, rotated, scaled, rounded; state reset
    auto start_item = [&]() __attribute__((always_inline)) {
        const int ln = opaque(lane), jj = ln % 32, gg = ln / 32;
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
            const int q = 32 * wave + kW * kQ * t + jj;
#pragma unroll
            for (int sp = 0; sp < 2; sp++) {
                const int c0 = 2 * sp + gg;
                floatx4 x0, x1, y0, y1;
                widen8<T>(*reinterpret_cast<const u32x4*>(&lds.q[wave][t][swz(jj, c0)]), x0, x1);
                widen8<T>(*reinterpret_cast<const u32x4*>(&lds.q[wave][t][swz(jj, c0 + 4)]), y0, y1);
                if (ROPE) {
                    const int f0 = 16 * sp + 8 * gg;
                    floatx4 ca, sa, cb, sb;
                    cs4(q, f0, ca, sa);
                    cs4(q, f0 + 4, cb, sb);
                    const floatx4 rx0 = x0 * ca - y0 * sa, ry0 = y0 * ca + x0 * sa;
                    const floatx4 rx1 = x1 * cb - y1 * sb, ry1 = y1 * cb + x1 * sb;
                    x0 = rx0; y0 = ry0; x1 = rx1; y1 = ry1;
                }
                const bool ok = q < n;
                const float sc = ok ? a.qscale : 0.f;
                qreg[t][sp] = __builtin_bit_cast(x8, narrow8<T>(x0 * sc, x1 * sc));
                qreg[t][sp + 2] = __builtin_bit_cast(x8, narrow8<T>(y0 * sc, y1 * sc));
            }
            tl[t].o[0] = floatx16{0};
            tl[t].o[1] = floatx16{0};
            tl[t].m_tot = 0.f;
            tl[t].m_mfma = 0.f;
            tl[t].resid = 0.f;
            tl[t].l_run = 0.f;
            tl[t].has_ref = false;
            tl[t].any_resid = false;
            tl[t].qx0 = gg == 0 ? E::kBigQ : 0u;
        }
    };

    // the softmax slow path: the exact block max, a new reference rounded to T, P recomputed, the
    // O/l rescale (a wave-uniform branch, taken when a block's sums leave the fast path's range)
    auto softmax_slow = [&](Tile& st, floatx16& s_acc, x8 (&p)[2], float& lb) __attribute__((always_inline)) {
        lp::softmax_slow<T>(st, s_acc, p, lb, g);
    };

    // The two tiles against one block. The softmax fast path assumes a reference without residual
    // (always, short of scores beyond the storage type's range); a tile carrying one takes the
    // slow path, which applies it.
    auto sm_fast = [&](Tile& st, const floatx16& s_acc, x8 (&p)[2], float& lb) __attribute__((always_inline)) {
        return lp::softmax_fast<T>(st, s_acc, p, lb);
    };
    auto compute = [&](int slot, uint64_t kmask) __attribute__((always_inline)) {
        const uint16_t* kb = lds.kv[slot][0];
        const uint16_t* vb = lds.kv[slot][1];
        const int G = lane / 16, rr = lane % 16;
        auto read_k = [&](int sb, x8 (&kop)[4]) __attribute__((always_inline)) {
#pragma unroll
            for (int s = 0; s < 4; s++)
                kop[s] = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(&kb[swz(32 * sb + j, 2 * s + g)]));
        };
        auto read_v = [&](int sb, x8 (&vop)[2][2]) __attribute__((always_inline)) {
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
        };
        auto kx_of = [&](int sb) __attribute__((always_inline)) {
            const uint32_t a32 = (uint32_t)(kmask >> (32 * sb));
            const uint32_t kx0 = g == 0 ? (((a32 >> j) & 1u) ? E::kLive : E::kDead) : 0u;
            return __builtin_bit_cast(x8, u32x4{kx0, 0u, 0u, 0u});
        };
        auto qk = [&](int t, const x8 (&kop)[4], x8 kx) __attribute__((always_inline)) {
            floatx16 acc = floatx16{0};
#pragma unroll
            for (int s = 0; s < 4; s++) acc = Lp<T>::mfma(kop[s], qreg[t][s], acc);
            return Lp<T>::mfma(kx, __builtin_bit_cast(x8, u32x4{tl[t].qx0, 0u, 0u, 0u}), acc);
        };
        auto pv = [&](int t, const x8 (&vop)[2][2], const x8 (&p)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
#pragma unroll
                for (int c = 0; c < 2; c++) tl[t].o[dt] = Lp<T>::mfma(vop[dt][c], p[c], tl[t].o[dt]);
            }
        };
        auto finish_unit = [&](Tile& st, floatx16& s_acc, x8 (&p)[2], float& lb, bool bad, int sb) __attribute__((always_inline)) {
            const bool live = (uint32_t)(kmask >> (32 * sb)) != 0u;
            if (live && (bad || st.any_resid)) softmax_slow(st, s_acc, p, lb);
            st.l_run += lb;
            st.has_ref = st.has_ref || live;
        };
        // per 32-key half: QK^T of both tiles (they share the K operands), then each tile's
        // softmax and PV (they share the V^T operands); halves without live keys are skipped
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            if ((uint32_t)(kmask >> (32 * sb)) == 0u) continue;  // uniform across the workgroup
            x8 kop[4], vop[2][2];
            read_k(sb, kop);
            const x8 kx = kx_of(sb);
            floatx16 sacc[kTiles];
#pragma unroll
            for (int t = 0; t < kTiles; t++) sacc[t] = qk(t, kop, kx);
            read_v(sb, vop);
#pragma unroll
            for (int t = 0; t < kTiles; t++) {
                x8 p[2];
                float lb = 0.f;
                // a tile without a reference yet (its first live keys) goes straight to the exact
                // max: the fast path would fail there on all but tiny scores
                const bool bad = tl[t].has_ref ? sm_fast(tl[t], sacc[t], p, lb) : true;
                finish_unit(tl[t], sacc[t], p, lb, bad, sb);
                pv(t, vop, p);
            }
        }
    };

    // query 512 against block `slot`: this wave's reference max rm (uniform), per-lane sums rl (8
    // copies of each key's P) and output dims ro (8c..8c+7 for lane (key, c)); rs_cur holds the
    // scores of the wave's 8 keys
    float rm = -INFINITY, rl = 0.f, rs_cur = 0.f;
    floatx4 ro_lo = floatx4{0.f, 0.f, 0.f, 0.f}, ro_hi = ro_lo;
    auto reg_update = [&](int slot, uint64_t kmask) __attribute__((always_inline)) {
        const int key = 8 * wave + lane / 8;
        const bool live = (kmask >> key) & 1ull;
        const float sc = live ? rs_cur : -INFINITY;
        // the reference moves only when a score exceeds it by 2^64 (or on the first live key):
        // P stays below 2^64, well inside fp32
        if (__any(sc - rm > 64.f)) {
            float mx = sc;
            mx = fmaxf(mx, dpp<0x128>(mx));  // row_ror:8: the other key of the row
            auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = pair_max(fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])));
            const float m_new = fmaxf(rm, mx);
            const float alpha = fast_exp2(rm - m_new);  // rm = -inf: 0
            rl *= alpha;
            ro_lo *= alpha;
            ro_hi *= alpha;
            rm = m_new;
        }
        const float pk = live ? fast_exp2(sc - rm) : 0.f;  // a live key makes rm finite above
        rl += pk;
        floatx4 v0, v1;
        widen8<T>(*reinterpret_cast<const u32x4*>(&lds.kv[slot][1][swz(key, lane % 8)]), v0, v1);
        ro_lo += pk * v0;
        ro_hi += pk * v1;
    };
    // item end: this wave's share (dims from the 8 keys' lanes added), its max and sum into reg_part
    auto reg_flush = [&](int par) __attribute__((always_inline)) {
        floatx4 o[2] = {ro_lo, ro_hi};
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float v = o[i][u];
                v += dpp<0x128>(v);  // row_ror:8
                auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
                o[i][u] = pair_sum(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
            }
        }
        const float l = wave_sum(rl) * 0.125f;
        float* dst = lds.reg_part[par][wave];
        if (lane < 8) {
            *reinterpret_cast<floatx4*>(&dst[8 * lane]) = o[0];
            *reinterpret_cast<floatx4*>(&dst[8 * lane + 4]) = o[1];
        }
        if (lane == 0) {
            dst[kDH] = rm;
            dst[kDH + 1] = l;
        }
    };
    // query 512's output of item (r, h): the waves' shares rescaled to the largest max
    auto reg_combine = [&](int par, int r, int h) __attribute__((always_inline)) {
        const int ln = opaque(lane);
        float mw[kW], mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kW; w++) {
            mw[w] = lds.reg_part[par][w][kDH];
            mx = fmaxf(mx, mw[w]);
        }
        float o = 0.f, l = 0.f;
        if (mx != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kW; w++) {
                const float f = fast_exp2(mw[w] - mx);
                o += f * lds.reg_part[par][w][ln];
                l += f * lds.reg_part[par][w][kDH + 1];
            }
        }
        T* op = static_cast<T*>(a.out) + ((size_t)r * n + kPart) * inner + h * kDH + ln;
        *op = (T)(l > 0.f ? o / l : 0.f);
    };

    // item end: normalized outputs of the wave's tiles
    auto finish_item = [&](int r, int h) __attribute__((always_inline)) {
        const int ln = opaque(lane), jj = ln % 32, gg = ln / 32;
#pragma unroll
        for (int t = 0; t < kTiles; t++) {
            const int q = 32 * wave + kW * kQ * t + jj;
            if (q >= n) continue;
            const float inv = tl[t].l_run > 0.f ? 1.f / tl[t].l_run : 0.f;
            T* op = static_cast<T*>(a.out) + ((size_t)r * n + q) * inner + h * kDH;
            // O^T reg 4a+u of lane (j, g) in dim tile dt is dim 32dt + 8a + 4g + u of query j
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
#pragma unroll
                for (int a4 = 0; a4 < 4; a4++) {
                    floatx4 v;
#pragma unroll
                    for (int u = 0; u < 4; u++) v[u] = tl[t].o[dt][4 * a4 + u] * inv;
                    *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * a4 + 4 * gg) = narrow4<T>(v);
                }
            }
        }
    };

    // ---- prologue loads: Q of item 0, query 512's q of items 0 and 1, the first kAhead elements
    int lk = 0, lbk = first_blk(0);  // load iterator
    bool lvalid = true;
    int lslot = 0;
    issue_q(0);
    if (has_reg && wave == 0) {
        issue_reg_raw(0);
        if (K > 1) issue_reg_raw(1);
    }
    int issued[kAhead] = {0, 0, 0};  // loads issued for elements 0..kAhead-1
#pragma unroll
    for (int i = 0; i < kAhead; i++) {
        if (lvalid) {
            issue_kv(lk, lbk, lslot);
            issued[i] = 2;
            lvalid = advance(lk, lbk);
        }
        lslot = (lslot + 1) % kSlots;
    }
    // element 0 and the Q loads before it landed
    wait_vm_rt(issued[1] + issued[2]);
    lds_barrier();
    int ck = 0, cb = first_blk(0), cslot = 0;
    if (has_reg) load_reg_q(0);
    rotate_k(cb, cslot, has_reg);
    int prev_e = issued[2];  // loads issued (elements) at the end of the previous step
    int prev_q = 0;          // loads issued (Q, query 512) at the end of the previous step, before prev_e
    int eidx = 0;            // element index within the current item
    bool more = true;
    bool pending = false;    // query 512 of the previous item still to be combined
    bool fin = false;        // the previous item's tiles still to be written
    int pc_par = 0, pc_r = 0, pc_h = 0;
    while (more) {
        // next compute element (k1, b1) to know whether this one ends its item
        int k1 = ck, b1 = cb;
        const bool has_next = advance(k1, b1);
        const bool item_start = eidx == 0;
        const bool item_end = !has_next || k1 != ck;
        // element e+1 landed; at an item start (its Q tiles) or an item end (the next item's
        // query-512 q) right after a step that issued Q loads, those too
        wait_vm_rt(prev_q && (item_start || item_end) ? prev_e : prev_q + prev_e);
        lds_barrier();
        // the previous item's output stores go out here, after this step's wait: s_waitcnt vmcnt
        // counts stores too, so stores issued at the end of the item would hold up this wait
        if (fin) finish_item(pc_r, pc_h);
        fin = false;
        if (pending && wave == kW - 1) reg_combine(pc_par, pc_r, pc_h);
        pending = false;
        if (item_start) {
            start_item();
            rm = -INFINITY;
            rl = 0.f;
            ro_lo = floatx4{0.f, 0.f, 0.f, 0.f};
            ro_hi = ro_lo;
        }
        rs_cur = rs_next;
        const uint64_t kmask = lds.mask[ck][cb];
        // the two waves of a SIMD (w and w + 4) run the step's VALU-only work (the next block's
        // rotation, query 512) at opposite ends of the tile compute, so one wave's MFMAs overlap
        // the other's VALU instead of both contending for the same pipe at once
        auto side_work = [&]() __attribute__((always_inline)) {
            if (has_next) {
                if (has_reg && item_end) load_reg_q(k1);
                rotate_k(b1, (cslot + 1) % kSlots, has_reg);
            }
            if (has_reg) reg_update(cslot, kmask);
        };
        if (wave >= kW / 2) side_work();
        compute(cslot, kmask);
        if (wave < kW / 2) side_work();
        if (item_end) {
            item_rh(ck, pc_r, pc_h);
            fin = true;
            if (has_reg) {
                reg_flush(ck & 1);
                pending = true;
                pc_par = ck & 1;
            }
        }
        // loads for later: the next item's Q tiles and the query-512 q two items ahead (after this
        // item's reads of both), then element e + kAhead
        prev_q = 0;
        if (item_start) {
            if (ck + 1 < K) {
                issue_q(ck + 1);
                prev_q = 2 * kTiles * 2;
            }
            if (has_reg && wave == 0 && ck + 2 < K) {
                issue_reg_raw(ck + 2);
                prev_q += 1;
            }
        }
        prev_e = 0;
        if (lvalid) {
            issue_kv(lk, lbk, lslot);
            prev_e = 2;
            lvalid = advance(lk, lbk);
            lslot = (lslot + 1) % kSlots;
        }
        eidx = item_end ? 0 : eidx + 1;
        ck = k1;
        cb = b1;
        cslot = (cslot + 1) % kSlots;
        more = has_next;
    }
    if (fin) finish_item(pc_r, pc_h);
    if (pending) {
        lds_barrier();
        if (wave == kW - 1) reg_combine(pc_par, pc_r, pc_h);
    }
}

}  // namespace

bool time_attention_lpp_fits(const TimeArgs& a, int dh, bool ts) {
    if (ts || dh != 64 || a.gate || a.q_begin != 0) return false;
    if (a.n <= 256 || a.n > kMaxN) return false;
    if (a.table && a.table_rows < a.n) return false;
    return true;
}

hipError_t time_attention_lpp_launch(const TimeArgs& a, bool fp16, int cus, hipStream_t stream) {
    const uint64_t items = (uint64_t)a.rows * a.heads;
    if (items == 0) return hipSuccess;
    uint64_t groups = (items + kIpw - 1) / kIpw;
    if (groups < (uint64_t)cus) groups = std::min<uint64_t>(items, (uint64_t)cus);
    const dim3 grid((uint32_t)groups), block(kThreads);
    const int it = (int)items, gr = (int)groups;
    if (fp16) {
        if (a.table) hipLaunchKernelGGL((time_attention_lpp<_Float16, true>), grid, block, 0, stream, a, it, gr);
        else hipLaunchKernelGGL((time_attention_lpp<_Float16, false>), grid, block, 0, stream, a, it, gr);
    } else {
        if (a.table) hipLaunchKernelGGL((time_attention_lpp<__bf16, true>), grid, block, 0, stream, a, it, gr);
        else hipLaunchKernelGGL((time_attention_lpp<__bf16, false>), grid, block, 0, stream, a, it, gr);
    }
    return hipGetLastError();
}

}  // namespace jc
