// Building blocks of the bf16 / fp16 time-attention kernels that stream K/V blocks through LDS
// with direct-to-LDS loads (time_attention_lpp.hip, time_attention_lps.hip): swizzled 64-element
// rows, the loads, waits and barriers as inline assembly, cross-lane reductions, transposing LDS
// reads, and one query tile's online-softmax state and steps.
#pragma once

#include "lp_common.hpp"

namespace jc {
namespace lp {

typedef short shortx4 __attribute__((ext_vector_type(4)));

// element index of (key, 16-byte chunk c) in a block of 128-byte key rows (64 16-bit values), the
// chunks XOR-swizzled by the key's low 3 bits: conflict-free DMA writes, operand reads and
// transposing reads
__device__ __forceinline__ int swz(int key, int c) { return key * 64 + ((c ^ (key & 7)) << 3); }

// The stream's loads, waits and barriers are inline assembly, so the compiler neither sees the
// direct-to-LDS loads (it would otherwise wait for all of them before any LDS read it cannot prove
// disjoint) nor moves LDS accesses across a wait or a barrier ("memory" clobbers).
// 16 bytes per lane from gptr to lds_base + 16 * lane (M0 holds the wave-uniform LDS address).
__device__ __forceinline__ void dma16(const void* gptr, const void* lds_base) {
    const uint32_t off = (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)lds_base;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(off) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// waits until at most n loads are outstanding, rounded down to 0, 2, 4 or 8 (a wait for fewer is
// always safe: it only waits longer)
__device__ __forceinline__ void wait_vm_rt(int n) {
    if (n >= 8) {
        wait_vm<8>();
    } else if (n >= 4) {
        wait_vm<4>();
    } else if (n >= 2) {
        wait_vm<2>();
    } else {
        wait_vm<0>();
    }
}
// waits until at most n loads are outstanding, exactly for n < 16 (n >= 16 waits for 15)
__device__ __forceinline__ void wait_vm_n(int n) {
    switch (n) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<1>(); break;
        case 2: wait_vm<2>(); break;
        case 3: wait_vm<3>(); break;
        case 4: wait_vm<4>(); break;
        case 5: wait_vm<5>(); break;
        case 6: wait_vm<6>(); break;
        case 7: wait_vm<7>(); break;
        case 8: wait_vm<8>(); break;
        case 9: wait_vm<9>(); break;
        case 10: wait_vm<10>(); break;
        case 11: wait_vm<11>(); break;
        case 12: wait_vm<12>(); break;
        case 13: wait_vm<13>(); break;
        case 14: wait_vm<14>(); break;
        default: wait_vm<15>(); break;
    }
}
// this wave's LDS writes done, then the workgroup barrier
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// a copy of x the compiler cannot see through: values derived from it inside a rarely taken path
// are computed there instead of being hoisted out of the stream loop into long-lived registers
__device__ __forceinline__ int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// over the 64 lanes of the wave, result in every lane: quad exchanges and row rotations (DPP),
// then the row pairs and the wave halves (v_permlane16_swap, v_permlane32_swap)
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
    v = fmaxf(v, dpp<0x128>(v));  // row_ror:8
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return pair_max(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x124>(v);
    v += dpp<0x128>(v);
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return pair_sum(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

template <typename T>
__device__ __forceinline__ floatx4 widen4(u32x2 raw) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    t4 v = __builtin_bit_cast(t4, raw);
    floatx4 r;
#pragma unroll
    for (int u = 0; u < 4; u++) r[u] = (float)v[u];
    return r;
}

// ds_read_b64_tr_b16: in each group of 16 lanes, lane 4a + c receives element c of the 8-byte rows
// addressed by lanes a, a+4, a+8, a+12
__device__ __forceinline__ u32x2 read_tr(const uint16_t* p) {
    auto v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) shortx4*)((__attribute__((address_space(3))) void*)p));
    return __builtin_bit_cast(u32x2, v);
}

// per 32-query tile: output accumulators (two 32-dim tiles of O^T) and the online-softmax state of
// time_attention_lp.hip
struct Tile {
    floatx16 o[2];
    float m_tot, m_mfma, resid, l_run;
    bool has_ref, any_resid;
    uint32_t qx0;
};

// The online softmax of one 32-query tile against a 32-key half block, the scores s_acc (16 per
// lane, already relative to the tile's reference max m_mfma: the extra QK^T step) to P rounded to
// T (two 8-value operands) and the half block's row sum lb (v_dot2 over those same values).
// The fast path: P = exp2(S) against the current reference; true when some lane's sum leaves the
// range it can carry (the slow path then recomputes P).
template <typename T>
__device__ __forceinline__ bool softmax_fast(const Tile& st, const floatx16& s_acc, typename Lp<T>::x8 (&p)[2],
                                             float& lb) {
    typedef typename Lp<T>::x8 x8;
    typedef Enc<T> E;
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
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        u32x4 w = __builtin_bit_cast(u32x4, p[c]);
#pragma unroll
        for (int d = 0; d < 4; d++) acc = E::dot2(w[d], acc);
    }
    lb = pair_sum(acc);
    const bool bad = !(lb <= kSumHi) || (!st.has_ref && !(lb >= kSumLo));
    return (bool)__any(bad);
}

// The slow path: the exact block max, a new reference rounded to T (so the extra QK^T step encodes
// it exactly; qx0 carries it for lanes g == 0), P against it, and the rescale of O and l.
template <typename T>
__device__ __forceinline__ void softmax_slow(Tile& st, const floatx16& s_acc, typename Lp<T>::x8 (&p)[2], float& lb,
                                             int g) {
    typedef typename Lp<T>::x8 x8;
    typedef Enc<T> E;
    float mx = s_acc[0];
#pragma unroll
    for (int rho = 1; rho < 16; rho++) mx = fmaxf(mx, s_acc[rho]);
    mx = pair_max(mx);
    const float s_max = st.m_mfma + mx;
    float m_new = st.has_ref ? fmaxf(st.m_tot, s_max) : s_max;
    const uint32_t bm = to_bits<T>(fminf(fmaxf(-m_new, -E::kMax), E::kMax));
    const float m_enc = -from_bits<T>(bm);
    if (fabsf(m_new) <= E::kMax) m_new = m_enc;  // keep the reference exactly encodable
    const float shift = m_new - st.m_mfma;
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
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        u32x4 w = __builtin_bit_cast(u32x4, p[c]);
#pragma unroll
        for (int d = 0; d < 4; d++) acc = E::dot2(w[d], acc);
    }
    lb = pair_sum(acc);
    if (st.has_ref) {
        const float alpha = fast_exp2(st.m_tot - m_new);
        st.o[0] *= alpha;
        st.o[1] *= alpha;
        st.l_run *= alpha;
    }
    st.m_tot = m_new;
    st.m_mfma = m_enc;
    st.resid = st.m_tot - st.m_mfma;
    st.any_resid = __any(st.resid != 0.f);
    st.qx0 = g == 0 ? (E::kBigQ | (bm << 16)) : 0u;
}

}  // namespace lp
}  // namespace jc
