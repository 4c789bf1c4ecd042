// Chronos-2 group (cross-series) attention for gfx950 (FP32 path).
//
// Replaces Chronos2Kernels.groupAttention(qkv, out, live, groupStart, groupEnd, rows, n, heads, dh,
// inner) (Chronos2Kernels.java:466-682; oracle CpuChronos2.java:230-282): at every token slot t,
// row i attends the rows j of its group (groupStart[i] <= j < groupEnd[i], groups are contiguous
// runs of rows) whose token at t is live; unscaled scores, no positional encoding; zeros when no
// key is live.
//
// The stage reads q|k|v once and writes out once, about 10 flop per byte: it is HBM-bound, so the
// kernel is built around the memory stream. One wave per (16-row tile, slot) owns the groups that
// START in its tile (found by a ballot on groupStart[i] == i), so each row's q, k and v are fetched
// from HBM once; everything lives in registers (no LDS, no barriers). The wave's work is a flat
// stream of jobs (group, chunk of up to 4 query tiles, head, 16-key tile): the chunk's queries and
// output accumulators stay in registers while the group's key tiles stream past, each K/V tile used
// by every query tile right after it lands, and the next job's K/V loads are issued before this
// job's MFMAs (register double-buffering). The online softmax across key tiles makes any group size
// work; a group past 64 rows re-streams its keys once per further 64-row chunk.
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

constexpr int kRT = 16;  // rows per tile (queries and keys)

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

// A position in the wave's job stream: group [gs, ge), query chunk qc (up to kQT tiles of 16
// rows), head h, key tile kt.
struct Job {
    int gs, ge, qc, h, kt;
    uint32_t rest;  // starts of the tile's remaining groups (bit b = row r0 + b)
    bool valid;
};

constexpr int kQT = 4;  // query tiles held in registers at once (64 rows)

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

    // the groups starting in this tile
    const uint32_t starts = (uint32_t)__ballot(lane < nr && gstart[r0 + lane] == r0 + lane) & 0xffffu;
    if (starts == 0) return;

    auto first_of = [&](uint32_t rest) {
        Job jb;
        jb.valid = rest != 0;
        int b = jb.valid ? __builtin_ctz(rest) : 0;
        jb.gs = r0 + b;
        // clamped into [gs+1, rows]: a group always holds its first row and only rows that exist
        jb.ge = jb.valid ? min(max(gend[jb.gs], jb.gs + 1), rows) : jb.gs + 1;
        jb.qc = 0;
        jb.h = 0;
        jb.kt = 0;
        jb.rest = jb.valid ? rest & (rest - 1) : 0;
        return jb;
    };
    // key tiles innermost, so a K/V tile is used by every resident query tile right after it lands
    auto advance = [&](Job jb) {
        const int tiles = (jb.ge - jb.gs + kRT - 1) / kRT;
        if (++jb.kt < tiles) return jb;
        jb.kt = 0;
        if (++jb.h < heads) return jb;
        jb.h = 0;
        if (++jb.qc * kQT < tiles) return jb;
        return first_of(jb.rest);
    };
    // K (A operand) and V^T (A operand of PV) of a job's key tile; rows past the group are clamped
    // (finite, masked). live bit of key 16kt + j in lanes j < 16.
    struct Kv {
        floatx4 k[kM];
        float v[kM][4];
        int live;
    };
    auto load_kv = [&](const Job& jb, Kv& d) {
        const int kbase = jb.gs + kRT * jb.kt;
        const int krow = min(kbase + j, jb.ge - 1);
        const float* kp = qkv + ((size_t)krow * tok_n + t) * stride + inner + jb.h * DH + 4 * g;
        d.live = (g == 0 && kbase + j < jb.ge) ? live[(size_t)krow * tok_n + t] : 0;
#pragma unroll
        for (int m = 0; m < kM; m++) d.k[m] = *reinterpret_cast<const floatx4*>(kp + 16 * m);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int vrow = min(kbase + 4 * g + c, jb.ge - 1);
            const float* vp = qkv + ((size_t)vrow * tok_n + t) * stride + 2 * inner + jb.h * DH + j;
#pragma unroll
            for (int m = 0; m < kM; m++) d.v[m][c] = vp[16 * m];
        }
    };

    Job cur = first_of(starts);
    Kv dc, dn;
    load_kv(cur, dc);

    float qreg[kQT][4 * kM];  // resident query tiles (B operand), scaled by log2(e)
    floatx4 o_acc[kQT][kM];
    float m_run[kQT], l_run[kQT];
    while (cur.valid) {
        const int tiles = (cur.ge - cur.gs + kRT - 1) / kRT;
        const int nq = min(kQT, tiles - kQT * cur.qc);  // query tiles in this chunk
        if (cur.kt == 0) {
            // a new (group, chunk, head): load its query tiles and reset the softmax state
#pragma unroll
            for (int qi = 0; qi < kQT; qi++) {
                if (qi < nq) {
                    const int qrow = min(cur.gs + kRT * (kQT * cur.qc + qi) + j, cur.ge - 1);
                    const float* qp = qkv + ((size_t)qrow * tok_n + t) * stride + cur.h * DH + 4 * g;
#pragma unroll
                    for (int m = 0; m < kM; m++) {
                        floatx4 a = *reinterpret_cast<const floatx4*>(qp + 16 * m);
#pragma unroll
                        for (int u = 0; u < 4; u++) qreg[qi][4 * m + u] = a[u] * kLog2e;
                    }
                }
#pragma unroll
                for (int m = 0; m < kM; m++) o_acc[qi][m] = floatx4{0.f, 0.f, 0.f, 0.f};
                m_run[qi] = -INFINITY;
                l_run[qi] = 0.f;
            }
        }
        const Job nxt = advance(cur);
        load_kv(nxt, dn);  // in flight under this job's MFMAs (an invalid job reloads in-bounds rows)
        __builtin_amdgcn_sched_barrier(0);

        const uint32_t lbits = (uint32_t)__ballot(dc.live != 0) & 0xffffu;  // bit b: key gs + 16kt + b
#pragma unroll
        for (int qi = 0; qi < kQT; qi++) {
            if (qi < nq) {
                floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int m = 0; m < kM; m++)
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        s = __builtin_amdgcn_mfma_f32_16x16x4f32(dc.k[m][u], qreg[qi][4 * m + u], s, 0, 0, 0);
                // reg r of lane (j, g) is key 16kt + 4g + r of the group (every row of the job is in it)
#pragma unroll
                for (int r = 0; r < 4; r++) s[r] = ((lbits >> (4 * g + r)) & 1u) ? s[r] : -INFINITY;
                const float mx = quad_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
                const float m_new = fmaxf(m_run[qi], mx);
                const float m_use = m_new == -INFINITY ? 0.f : m_new;
                const float alpha = fast_exp2(m_run[qi] - m_use);
                m_run[qi] = m_new;
#pragma unroll
                for (int r = 0; r < 4; r++) s[r] = fast_exp2(s[r] - m_use);
                l_run[qi] = l_run[qi] * alpha + (s[0] + s[1]) + (s[2] + s[3]);
#pragma unroll
                for (int m = 0; m < kM; m++) {
                    o_acc[qi][m] *= alpha;
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        o_acc[qi][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(dc.v[m][c], s[c], o_acc[qi][m], 0, 0, 0);
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
                        float* op = out + ((size_t)qrow * tok_n + t) * inner + cur.h * DH + 4 * g;
                        // O^T reg r of lane (j, g) in dim tile m is dim 16m + 4g + r of the query
#pragma unroll
                        for (int m = 0; m < kM; m++) *reinterpret_cast<floatx4*>(op + 16 * m) = o_acc[qi][m] * inv;
                    }
                }
            }
        }
        cur = nxt;
        dc = dn;
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
