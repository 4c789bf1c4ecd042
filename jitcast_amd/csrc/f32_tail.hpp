// The tail queries of Chronos-2 fp32 time attention: the last R queries (2 <= R <= 16) of rows of
// 128k + R tokens, for one (row, head) per wave, without LDS or barriers (time_attention_f32.hip
// runs them in tail workgroups beside its main ones).
//
// Same contract as the main kernel (Chronos2Kernels.rope + timeAttention, Chronos2Kernels.java:87-116,
// 118-464; oracle CpuChronos2.java:175-228, 284-304). Operand layouts of v_mfma_f32_16x16x4f32
// (A lane i+16kk = A[i][kk], B lane j+16kk = B[kk][j], D lane j+16g reg r = D[4g+r][j]):
//   S^T[key][q] = K Q^T   step (m, u) contracts dim 16m + 4kk + u, so a lane holds 4 consecutive dims
//                         per m (one 16-byte load) and the RoPE pair of dim e < 32, e + 32, sits in
//                         the same lane (m and m + 2): the rotation is lane-local.
//   O^T[e][q] += V^T P^T  step c contracts keys 4kk + c, whose P^T is S^T's reg c in the same lane;
//                         V^T comes per lane as V[key][16t + i].
// The R queries are one 16-query operand; keys stream in 16-key tiles loaded straight into these
// layouts, the next tile's loads issued before this tile's MFMAs.
#pragma once

#include "jc_common.hpp"
#include "jc_kernels.hpp"

namespace jc {

constexpr int kTailT = 16;  // tail queries at most, and keys per tile

struct TailTile {
    floatx4 k[4];       // K dims 16m + 4kk .. +3 of key 16kt + i
    floatx4 c[2], s[2]; // cos / sin of dims 16m + 4kk .. +3 (m = 0, 1) at the key's position
    float v[4][4];      // [t][c]: V[key 16kt + 4kk + c][dim 16t + i]
    int valid;          // lanes i < 16 (kk = 0): key 16kt + i is live
};

template <bool ROPE, bool X3>
__device__ __forceinline__ void f32_tail_item(const TimeArgs& a, int r, int h, int q0, int lane) {
    constexpr int kDH = 64;
    const int n = a.n, inner = a.inner, R = n - q0;
    const int i = lane % 16, kk = lane / 16;  // also (j, g) of the accumulator layouts
    const size_t ts = 3 * (size_t)inner;      // floats per token of qkv
    const float* base = static_cast<const float*>(a.qkv) + (size_t)r * n * ts + h * kDH;
    const float* table = a.table;

    // Q: lane (j, kk) holds dims 16m + 4kk .. +3 of query q0 + j, rotated at its position and scaled
    // (zeros for the operand's rows past the row's last query)
    floatx4 qv[4];
    {
        const int q = min(q0 + i, n - 1);
        const float* qp = base + (size_t)q * ts + 4 * kk;
#pragma unroll
        for (int m = 0; m < 4; m++) qv[m] = *reinterpret_cast<const floatx4*>(qp + 16 * m);
        if (ROPE) {
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const floatx4 c = *reinterpret_cast<const floatx4*>(table + (size_t)q * kDH + 16 * m + 4 * kk);
                const floatx4 s = *reinterpret_cast<const floatx4*>(table + (size_t)q * kDH + kDH / 2 + 16 * m + 4 * kk);
                const floatx4 x = qv[m], y = qv[m + 2];
                qv[m] = x * c - y * s;
                qv[m + 2] = y * c + x * s;
            }
        }
        const float sc = q0 + i < n ? a.qscale : 0.f;
#pragma unroll
        for (int m = 0; m < 4; m++) qv[m] *= sc;
    }

    const int32_t* live = a.valid + (size_t)r * n;
    auto load = [&](int kt, TailTile& d) {
        const int key = min(kTailT * kt + i, n - 1);
        const float* kp = base + (size_t)key * ts + inner + 4 * kk;
#pragma unroll
        for (int m = 0; m < 4; m++) d.k[m] = *reinterpret_cast<const floatx4*>(kp + 16 * m);
        if (ROPE) {
#pragma unroll
            for (int m = 0; m < 2; m++) {
                d.c[m] = *reinterpret_cast<const floatx4*>(table + (size_t)key * kDH + 16 * m + 4 * kk);
                d.s[m] = *reinterpret_cast<const floatx4*>(table + (size_t)key * kDH + kDH / 2 + 16 * m + 4 * kk);
            }
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int vkey = min(kTailT * kt + 4 * kk + c, n - 1);
            const float* vp = base + (size_t)vkey * ts + 2 * inner + i;
#pragma unroll
            for (int t = 0; t < 4; t++) d.v[t][c] = vp[16 * t];
        }
        d.valid = (kk == 0 && kTailT * kt + i < n) ? live[kTailT * kt + i] : 0;
    };

    float m_run = -INFINITY, l_run = 0.f;
    floatx4 o[4];
#pragma unroll
    for (int t = 0; t < 4; t++) o[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const TailTile& d) {
        floatx4 kr[4] = {d.k[0], d.k[1], d.k[2], d.k[3]};
        if (ROPE) {
#pragma unroll
            for (int m = 0; m < 2; m++) {
                kr[m] = d.k[m] * d.c[m] - d.k[m + 2] * d.s[m];
                kr[m + 2] = d.k[m + 2] * d.c[m] + d.k[m] * d.s[m];
            }
        }
        floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; m++) {
#pragma unroll
            for (int u = 0; u < 4; u++) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[m][u], qv[m][u], s, 0, 0, 0);
        }
        // reg r of lane (j, g) is key 16kt + 4g + r
        const uint32_t vbits = (uint32_t)__ballot(d.valid != 0) & 0xffffu;
#pragma unroll
        for (int q = 0; q < 4; q++) s[q] = ((vbits >> (4 * kk + q)) & 1u) ? s[q] : -INFINITY;
        const float mx = quad_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        m_run = m_new;
#pragma unroll
        for (int q = 0; q < 4; q++) s[q] = fast_exp2(s[q] - m_use);
        l_run = l_run * alpha + (s[0] + s[1]) + (s[2] + s[3]);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            o[t] *= alpha;
#pragma unroll
            for (int c = 0; c < 4; c++) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(d.v[t][c], s[c], o[t], 0, 0, 0);
        }
    };

    const int tiles = (n + kTailT - 1) / kTailT;
    TailTile cur, nxt;
    load(0, cur);
    for (int kt = 0; kt < tiles; kt++) {
        if (kt + 1 < tiles) load(kt + 1, nxt);  // in flight under this tile's MFMAs
        compute(cur);
        cur = nxt;
    }

    // O^T reg r of lane (j, g) in dim tile t is dim 16t + 4g + r of query q0 + j
    const float l = quad_sum(l_run);
    if (i < R) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const size_t tok = (size_t)r * n + q0 + i;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const floatx4 v = o[t] * inv;
            if constexpr (X3) {
                store_split_row(static_cast<_Float16*>(a.out) + tok * 3 * inner, inner, h * kDH + 16 * t + 4 * kk, v);
            } else {
                *reinterpret_cast<floatx4*>(static_cast<float*>(a.out) + tok * inner + h * kDH + 16 * t + 4 * kk) = v;
            }
        }
    }
}

}  // namespace jc
