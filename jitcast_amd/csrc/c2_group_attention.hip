// Chronos-2 group (cross-series) attention for gfx950 (FP32 path).
//
// Replaces Chronos2Kernels.groupAttention(qkv, out, live, groupStart, groupEnd, rows, n, heads, dh,
// inner) (Chronos2Kernels.java:466-682; oracle CpuChronos2.java:230-282): at every token slot t,
// row i attends the rows j of its group (groupStart[i] <= j < groupEnd[i], groups are contiguous
// runs of rows) whose token at t is live; unscaled scores, no positional encoding; zeros when no
// key is live.
//
// The stage reads q|k|v once and writes out once, about 10 flop per byte: it is HBM-bound, so the
// kernel is built around the memory stream. One wave per (16-row tile, slot) loops over the heads
// with everything in registers (no LDS, no barriers): per head it loads the tile's queries and the
// keys/values of the union of the tile's groups straight into MFMA operand layout, and runs
// v_mfma_f32_16x16x4_f32 tiles with an online softmax over 16-key tiles, so any group size works.
//
// Operand layouts (16x16x4 f32: A lane i+16kk = A[i][kk], B lane j+16kk = B[kk][j],
// D lane j+16g reg r = D[4g+r][j]):
//   S^T[key][q] = K Q^T: step s = 4m+u contracts dim 16m + 4kk + u, so each lane's K and Q come
//                        from one 16-byte load per m and a 64-byte run per row per load.
//   O^T[e][q] += V^T P^T: step c contracts key 4kk + c, whose P^T is S^T's reg c; V^T is loaded
//                        per lane as V[key][e] (16 rows x 64 contiguous bytes per load).
#include "jc_common.hpp"
#include "jc_kernels.hpp"

namespace jc {
namespace {

constexpr int kRT = 16;  // rows (queries) per tile

// max / sum over the four lanes j, j+16, j+32, j+48 (v_permlane16_swap then v_permlane32_swap)
__device__ __forceinline__ float quad_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    return pair_max(v);
}

__device__ __forceinline__ float quad_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    return pair_sum(v);
}

template <int DH>
__global__ __launch_bounds__(kWave) void c2_group_attention_f32(const float* __restrict__ qkv, float* __restrict__ out,
                                                                const int32_t* __restrict__ live,
                                                                const int32_t* __restrict__ gstart,
                                                                const int32_t* __restrict__ gend, int rows, int n,
                                                                int heads, int inner, int rtiles) {
    static_assert(DH % 16 == 0 && DH <= 64, "head width");
    constexpr int kM = DH / 16;  // 16-dim groups: K/Q loads per lane, and output dim tiles
    const int lane = threadIdx.x;
    const int j = lane % 16, g = lane / 16;
    const uint32_t total = (uint32_t)rtiles * n;
    const uint32_t logical = xcd_remap(blockIdx.x, total);
    const int t = logical / rtiles, rt = logical % rtiles;
    const int r0 = rt * kRT;
    const int nr = min(kRT, rows - r0);
    const size_t stride = 3 * (size_t)inner;  // floats per token of qkv
    const size_t tok_n = (size_t)n;

    // this lane's query row and its group; the key range is the union of the tile's groups
    const bool qvalid = j < nr;
    const int qrow = r0 + (qvalid ? j : nr - 1);
    const int gs_q = gstart[qrow], ge_q = gend[qrow];
    // clamped into [0, rows]: group bounds only ever select rows that exist
    const int ks = min(max(gstart[r0], 0), rows);
    const int ke = min(max(gend[r0 + nr - 1], ks), rows);

    for (int h = 0; h < heads; h++) {
        // Q tile: lane (j, g) holds q[r0+j][16m + 4g + u], scaled by log2(e)
        float qreg[4 * kM];
        {
            const float* qp = qkv + ((size_t)qrow * tok_n + t) * stride + h * DH + 4 * g;
#pragma unroll
            for (int m = 0; m < kM; m++) {
                floatx4 a = *reinterpret_cast<const floatx4*>(qp + 16 * m);
#pragma unroll
                for (int u = 0; u < 4; u++) qreg[4 * m + u] = qvalid ? a[u] * kLog2e : 0.f;
            }
        }
        floatx4 o_acc[kM];
#pragma unroll
        for (int m = 0; m < kM; m++) o_acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
        float m_run = -INFINITY, l_run = 0.f;

        for (int kt = ks; kt < ke; kt += 16) {
            // K tile (A operand): lane (i, g) holds k[kt+i][16m + 4g + u]; rows past ke are clamped
            // (finite, masked below)
            const int krow = min(kt + j, ke - 1);
            const float* kp = qkv + ((size_t)krow * tok_n + t) * stride + inner + h * DH + 4 * g;
            floatx4 kreg[kM];
#pragma unroll
            for (int m = 0; m < kM; m++) kreg[m] = *reinterpret_cast<const floatx4*>(kp + 16 * m);
            // V^T (A operand of PV): lane (i, g) holds v[key 4g + c][16m + i] for step c, dim tile m
            float vreg[kM][4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int vrow = min(kt + 4 * g + c, ke - 1);
                const float* vp = qkv + ((size_t)vrow * tok_n + t) * stride + 2 * inner + h * DH + j;
#pragma unroll
                for (int m = 0; m < kM; m++) vreg[m][c] = vp[16 * m];
            }
            // live keys of the tile: bit b = key kt + b
            const int lk = kt + j;
            const uint32_t lbits =
                (uint32_t)__ballot(g == 0 && lk < ke && live[(size_t)lk * tok_n + t] != 0) & 0xffffu;

            floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < kM; m++)
#pragma unroll
                for (int u = 0; u < 4; u++) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kreg[m][u], qreg[4 * m + u], s, 0, 0, 0);

            // reg r of lane (j, g) is key kt + 4g + r for query r0 + j
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = kt + 4 * g + r;
                const bool ok = qvalid && ((lbits >> (4 * g + r)) & 1u) && key >= gs_q && key < ge_q;
                s[r] = ok ? s[r] : -INFINITY;
            }
            float mx = quad_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
            const float m_new = fmaxf(m_run, mx);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float alpha = fast_exp2(m_run - m_use);
            m_run = m_new;
#pragma unroll
            for (int r = 0; r < 4; r++) s[r] = fast_exp2(s[r] - m_use);
            l_run = l_run * alpha + (s[0] + s[1]) + (s[2] + s[3]);
#pragma unroll
            for (int m = 0; m < kM; m++) {
                o_acc[m] *= alpha;
#pragma unroll
                for (int c = 0; c < 4; c++) o_acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(vreg[m][c], s[c], o_acc[m], 0, 0, 0);
            }
        }

        const float l = quad_sum(l_run);
        if (qvalid) {
            const float inv = l > 0.f ? 1.f / l : 0.f;
            float* op = out + ((size_t)(r0 + j) * tok_n + t) * inner + h * DH + 4 * g;
            // O^T reg r of lane (j, g) in dim tile m is dim 16m + 4g + r of query r0 + j
#pragma unroll
            for (int m = 0; m < kM; m++) *reinterpret_cast<floatx4*>(op + 16 * m) = o_acc[m] * inv;
        }
    }
}

}  // namespace

template <int DH>
static hipError_t launch_group_f32(const float* qkv, float* out, const int32_t* live, const int32_t* gs,
                                   const int32_t* ge, int rows, int n, int heads, int inner, hipStream_t stream) {
    int rtiles = (rows + kRT - 1) / kRT;
    uint64_t grid = (uint64_t)rtiles * n;
    hipLaunchKernelGGL(c2_group_attention_f32<DH>, dim3((uint32_t)grid), dim3(kWave), 0, stream, qkv, out, live, gs, ge,
                       rows, n, heads, inner, rtiles);
    return hipGetLastError();
}

hipError_t c2_group_attention_f32_launch(const float* qkv, float* out, const int32_t* live, const int32_t* gs,
                                         const int32_t* ge, int rows, int n, int heads, int dh, int inner,
                                         hipStream_t stream) {
    switch (dh) {
        case 16: return launch_group_f32<16>(qkv, out, live, gs, ge, rows, n, heads, inner, stream);
        case 32: return launch_group_f32<32>(qkv, out, live, gs, ge, rows, n, heads, inner, stream);
        case 48: return launch_group_f32<48>(qkv, out, live, gs, ge, rows, n, heads, inner, stream);
        case 64: return launch_group_f32<64>(qkv, out, live, gs, ge, rows, n, heads, inner, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace jc
