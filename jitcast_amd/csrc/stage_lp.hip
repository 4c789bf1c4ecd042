// The bf16 / fp16 kernels of the Chronos-2 encoder layer for gfx950: the GEMM with fp32
// accumulation (the reference's FP16 GEMM modes: Kernels.gemmHalf and GemmEx FP16->FP32,
// Kernels.java:115-232, Chronos2Forward.java:377-409, with Kernels.gemm's epilogue flags,
// Kernels.java:50-103), RMSNorm writing the storage-type twin of its output (Kernels.rmsNorm's
// `twin`, Kernels.java:800-829), and the fp32 -> storage-type conversion (Kernels.toHalf).
//
// GEMM: C[m, n] (+)= act(A[m, :k] . W[n, :k] + b[n]) with A and W in bf16 (or fp16), fp32 MFMA
// accumulation (v_mfma_f32_32x32x16_{bf16,f16}) and C either fp32 (any flags, ACCUMULATE included:
// the residual stream stays fp32) or the storage type (the next GEMM's or the attention's input).
// Storage-type outputs saturate to the type's finite range, as the reference's FP16 twins do
// (Kernels.java:42-46).
//
// Tiling: a 512-thread workgroup owns a 256x256 tile of C; wave w owns the 128x64 block
// (w / 4, w % 4) as 4x2 MFMA tiles of 32x32 (128 accumulators per lane), which reads 6 KB of
// operands from LDS per 8 MFMAs. K advances 64 at a time through two LDS stages (A and W tiles of
// 256 rows x 64 elements, 128 KB in all). The tiles arrive by direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds, 1 KB per wave instruction): a row of 64 elements is 8 chunks of
// 16 bytes, and chunk c of row r sits at position c ^ ((r >> 1) & 7), so the MFMA operand reads (16
// bytes of 32 consecutive rows, 16 lanes per LDS cycle over 64 banks) hit distinct banks. Out-of-range rows and k columns read as zero through
// the buffer descriptor's range check, so any m, n and k (a multiple of 8) need no clamping.
// The grid is persistent (one workgroup per CU): a workgroup walks its tiles, and the first stage
// of its next tile loads while the epilogue of the current one stores. Tiles that share a row
// block of A run at the same time on one XCD, so A is read from HBM about once.
// MFMA layouts (32x32x16): A lane i+32g = A[i][8g..8g+7], B lane j+32g = B[8g..8g+7][j],
// D lane j+32g reg r = D[8(r/4) + 4g + r%4][j].
#include "jc_common.hpp"
#include "jc_kernels.hpp"
#include "lp_common.hpp"

namespace jc {
namespace {

using namespace lp;

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kWM = 2, kWN = 4;  // waves along M and N
constexpr int kThreads = kWM * kWN * kWave;
constexpr int kWaves = kWM * kWN;
constexpr int kTM = kBM / kWM / 32, kTN = kBN / kWN / 32;  // 32x32 tiles per wave: 4 x 2
static_assert(kTN * 32 == 64 && kWaves / 2 * 2048 * 4 == kBM * kBK * 2, "epilogue staging: 32 x 64 floats per wave");
constexpr int kLoads = kBM * kBK * 2 / 1024 / (kWM * kWN);  // 1 KB loads per wave, operand and stage: 4
constexpr uint32_t kOob = 0x80000000u;                      // a buffer offset past every range: reads 0

struct alignas(16) LpTile {  // 16-byte aligned, so operand reads stay ds_read_b128
    uint16_t a[2][kBM * kBK];
    uint16_t w[2][kBN * kBK];
    float bias[2][kBN];  // the bias of the tile in flight, by tile parity
};

// element offset of chunk c (8 elements) of row r in a swizzled stage
// chunk c of row r sits at position c ^ skey(r): rows r and r + 8 of a 16-lane read phase land in
// different 16-byte bank groups
__device__ __forceinline__ int skey(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int gswz(int r, int c) { return r * kBK + ((c ^ skey(r)) << 3); }

// raw buffer descriptor of `bytes` bytes at p (the base fits 48 bits, stride 0)
__device__ __forceinline__ u32x4 buf_desc(const void* p, uint32_t bytes) {
    const uint64_t a = (uint64_t)p;
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xFFFFu, bytes, kRsrcWord3};
}

// 16 bytes per lane from rsrc + voff into LDS at lds + 16 * lane (zero when out of range)
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t voff, const void* lds) {
    const uint32_t m0 = (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)lds;
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "s"(m0)
                 : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// a copy of x the compiler cannot see through (values derived from it are not hoisted)
__device__ __forceinline__ int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
}
// 4 bytes per lane from rsrc + voff into LDS at lds + 4 * lane (zero when out of range)
__device__ __forceinline__ void dma4(u32x4 rsrc, uint32_t voff, const void* lds) {
    const uint32_t m0 = (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)lds;
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "s"(m0)
                 : "memory", "m0");
}
// this wave's LDS accesses done, then the workgroup barrier
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// clamp to the storage type's finite range, keeping NaN (TornadoMath.clamp propagates it)
__device__ __forceinline__ float clamp_finite(float v, float m) { return v != v ? v : fminf(fmaxf(v, -m), m); }

template <typename T>
__device__ __forceinline__ T saturate(float v) {
    return (T)clamp_finite(v, Enc<T>::kMax);
}

// bias, then the activation (0 none, 1 SiLU, 2 ReLU keeping NaN), in Kernels.gemm's order
template <int ACT>
__device__ __forceinline__ floatx4 activate(floatx4 v, floatx4 b) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
        v[u] += b[u];
        if (ACT == 1) v[u] = v[u] / (1.f + __expf(-v[u]));
        if (ACT == 2) v[u] = (v[u] > 0.f || v[u] != v[u]) ? v[u] : 0.f;
    }
    return v;
}

template <typename T, bool OUT_LP>
__global__ __launch_bounds__(kThreads, 1) void gemm_lp(const GemmLpArgs g, uint32_t tiles_n, uint32_t total, int vec) {
    typedef typename Lp<T>::x8 x8;
    __shared__ LpTile lds;
    const T* __restrict__ A = static_cast<const T*>(g.a);
    const T* __restrict__ W = static_cast<const T*>(g.w);
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int j = lane % 32, hg = lane / 32;
    const int wm = wave / kWN, wn = wave % kWN;
    const int stages = (g.k + kBK - 1) / kBK;
    // staging: load u of this wave fills rows 8(kLoads * wave + u) .. +7; lane -> row lane / 8,
    // position lane % 8, which holds chunk (lane % 8) ^ (lane / 8)
    const uint32_t a_row = (uint32_t)g.lda * 2u, w_row = (uint32_t)g.k * 2u;

    // loads u0 .. u1 - 1 of stage st of a tile into stage buffer buf; with stage 0 and u0 = 0, the
    // tile's bias into bias slot bslot
    auto issue = [&](uint32_t tile, int st, int buf, int bslot, int u0, int u1) __attribute__((always_inline)) {
        const int m0 = (int)(tile / tiles_n) * kBM, n0 = (int)(tile % tiles_n) * kBN;
        if (st == 0 && u0 == 0 && wave == 0 && (g.flags & kGemmBias)) {
            const u32x4 rb = buf_desc(g.bias + n0, (uint32_t)min(kBN, g.n - n0) * 4u);
#pragma unroll
            for (int u = 0; u < kBN / kWave; u++) dma4(rb, 4u * (uint32_t)(kWave * u + opaque(lane)), &lds.bias[bslot][kWave * u]);
        }
        const u32x4 ra = buf_desc(A + (size_t)m0 * g.lda, (uint32_t)min(kBM, g.m - m0) * a_row);
        const u32x4 rw = buf_desc(W + (size_t)n0 * g.k, (uint32_t)min(kBN, g.n - n0) * w_row);
        // recomputed per call from an opaque lane id, not hoisted into long-lived registers
        const int ln = opaque(lane), srow = ln / 8;
#pragma unroll
        for (int u = u0; u < u1; u++) {
            const int r = 8 * (kLoads * wave + u) + srow;
            const int kc = st * kBK + 8 * ((ln % 8) ^ skey(r));  // the chunk this lane's position holds
            const bool kin = kc < g.k;
            dma16(ra, kin ? (uint32_t)r * a_row + 2u * kc : kOob, &lds.a[buf][8 * (kLoads * wave + u) * kBK]);
            dma16(rw, kin ? (uint32_t)r * w_row + 2u * kc : kOob, &lds.w[buf][8 * (kLoads * wave + u) * kBK]);
        }
    };

    // persistent walk: round i takes tiles i * gridDim.x + (this workgroup's slot in XCD order)
    const uint32_t slot = xcd_remap(blockIdx.x, gridDim.x);
    uint32_t tile = slot;
    if (tile >= total) return;
    issue(tile, 0, 0, 0, 0, kLoads);
    // VMEM instructions the previous tile's epilogue issued after this tile's first-stage loads
    // (whole tiles only; 0 = wait for everything). Vector memory operations retire in issue order,
    // so waiting until at most that many are outstanding waits for the loads and leaves the
    // epilogue's stores draining behind the next MFMAs.
    int younger = 0;
    const bool accumulate = !OUT_LP && (g.flags & kGemmAccumulate);
    for (int it = 0;; it++) {
        const int m0 = (int)(tile / tiles_n) * kBM, n0 = (int)(tile % tiles_n) * kBN;
        const int er = lane / 16, ec = 4 * (lane % 16);
        const int col0 = n0 + 64 * wn + ec;  // this lane's 4 output columns in the epilogue
        floatx16 acc[kTM][kTN];
#pragma unroll
        for (int ti = 0; ti < kTM; ti++)
#pragma unroll
            for (int tj = 0; tj < kTN; tj++) acc[ti][tj] = floatx16{0};

        for (int st = 0; st < stages; st++) {
            const int buf = st & 1;
            // stage st has landed everywhere, and every wave is done with stage st - 1's buffer
            if (st == 0 && younger == 63) {
                wait_vm<63>();
            } else if (st == 0 && younger == 32) {
                wait_vm<32>();
            } else {
                wait_vm<0>();
            }
            lds_barrier();
            // the next stage's loads are spread over the first two k-steps, so the per-CU address
            // unit works through them while the MFMAs run instead of stalling every wave at once
            // operands of k-step kk sit in registers set kk % 2: the next k-step's LDS reads are
            // issued before this k-step's MFMAs (the scheduling barrier keeps them there), so their
            // latency runs under 8 MFMAs instead of stalling the first one
            x8 av[2][kTM], wv[2][kTN];
            auto operands = [&](int kk, int s) __attribute__((always_inline)) {
                const int c = 2 * kk + hg;
#pragma unroll
                for (int ti = 0; ti < kTM; ti++)
                    av[s][ti] = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(&lds.a[buf][gswz(128 * wm + 32 * ti + j, c)]));
#pragma unroll
                for (int tj = 0; tj < kTN; tj++)
                    wv[s][tj] = __builtin_bit_cast(x8, *reinterpret_cast<const u32x4*>(&lds.w[buf][gswz(64 * wn + 32 * tj + j, c)]));
            };
            operands(0, 0);
#pragma unroll
            for (int kk = 0; kk < kBK / 16; kk++) {
                if (kk < 2 && st + 1 < stages) issue(tile, st + 1, buf ^ 1, 0, kk * kLoads / 2, (kk + 1) * kLoads / 2);
                if (kk + 1 < kBK / 16) operands(kk + 1, (kk + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int ti = 0; ti < kTM; ti++)
#pragma unroll
                    for (int tj = 0; tj < kTN; tj++) acc[ti][tj] = Lp<T>::mfma(av[kk & 1][ti], wv[kk & 1][tj], acc[ti][tj]);
            }
        }
        // every wave is done with both stages: the next tile's first stage may load
        const uint32_t next = tile + gridDim.x;
        wait_vm<0>();
        lds_barrier();
        if (next < total) issue(next, 0, 0, (it + 1) & 1, 0, kLoads);

        // epilogue, 32 rows of the wave's block at a time through the wave's 8 KB of the stage the
        // next tile does not load into: the MFMA layout in (reg r of lane (j, hg) in tile (ti, tj)
        // is row 8(r/4) + 4hg + r%4, column 32tj + j of the block), rows of 4 consecutive columns
        // out, so each lane stores 16 bytes (fp32) or 8 bytes (storage type) of one row. Bias,
        // activation, accumulate, in Kernels.gemm's order.
        float* ep = reinterpret_cast<float*>(wave < kWaves / 2 ? lds.a[1] : lds.w[1]) + (wave % (kWaves / 2)) * 2048;
        // the bias came with the tile's first stage (zero past n)
        const floatx4 b4 = (g.flags & kGemmBias) ? *reinterpret_cast<const floatx4*>(&lds.bias[it & 1][64 * wn + ec])
                                                 : floatx4{0.f, 0.f, 0.f, 0.f};
        // block ti through LDS: write it, then read back rows vv[q - q0] = row 4q + lane / 16,
        // columns 4 (lane % 16) .. + 3 for q in [q0, q0 + nq) (the reads issued before any use)
        auto to_lds = [&](int ti) __attribute__((always_inline)) {
#pragma unroll
            for (int tj = 0; tj < kTN; tj++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int R = 8 * (r / 4) + 4 * hg + r % 4;
                    ep[R * 64 + ((32 * tj + j) ^ ((R & 4) << 3))] = acc[ti][tj][r];
                }
            __builtin_amdgcn_wave_barrier();
            asm volatile("" ::: "memory");
        };
        auto rows = [&](int q0, int nq, floatx4* vv) __attribute__((always_inline)) {
#pragma unroll
            for (int q = q0; q < q0 + nq; q++) {
                const int R = 4 * q + er;
                vv[q - q0] = *reinterpret_cast<const floatx4*>(&ep[R * 64 + (ec ^ ((R & 4) << 3))]);
            }
        };
        auto to_rows = [&](int ti, floatx4* vv) __attribute__((always_inline)) {
            to_lds(ti);
            rows(0, 8, vv);
        };
        auto finish = [&](floatx4 v) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                v[u] += b4[u];
                if (g.flags & kGemmSilu) v[u] = v[u] / (1.f + __expf(-v[u]));
                if (g.flags & kGemmRelu) v[u] = (v[u] > 0.f || v[u] != v[u]) ? v[u] : 0.f;
            }
            return v;
        };
        const int row0 = m0 + 128 * wm + er;  // + 32 ti + 4 q
        const bool whole = vec && m0 + kBM <= g.m && n0 + kBN <= g.n;
        // whole tiles: one epilogue per activation, so no flag test sits in the per-element code
        auto whole_epi = [&](auto act_tag) __attribute__((always_inline)) {
            constexpr int ACT = decltype(act_tag)::value;
            // every access in range: one 16- or 8-byte store (and load) per lane and 4 rows, no
            // branches, so the instruction count below is exact
            // (a scalar base per row group plus a 32-bit lane offset, so each access takes one VGPR
            // of address)
            constexpr size_t kElt = OUT_LP ? 2u : 4u;
            char* const tb = static_cast<char*>(g.c) + (size_t)(m0 + 128 * wm) * g.ldc * kElt;
            const uint32_t lo = ((uint32_t)er * (uint32_t)g.ldc + (uint32_t)col0) * (uint32_t)kElt;
            // row 32 ti + 4 q of the wave's block
            auto at = [&](int ti, int q) __attribute__((always_inline)) {
                return tb + (size_t)(32 * ti + 4 * q) * g.ldc * kElt + lo;
            };
            if (accumulate) {
                // C in halves of 4 row groups, each half's loads issued before the previous half's
                // stores (a load waited for behind older stores would wait for them too)
                u32x4 cv[2][4];
#pragma unroll
                for (int q = 0; q < 4; q++) cv[0][q] = *reinterpret_cast<const u32x4*>(at(0, q));
#pragma unroll
                for (int ti = 0; ti < kTM; ti++) {
                    to_lds(ti);  // frees acc[ti] before more loads take registers
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const int hx = 2 * ti + h;  // this half; the next is hx + 1
                        if (hx + 1 < 2 * kTM) {
#pragma unroll
                            for (int q = 0; q < 4; q++)
                                cv[(hx + 1) & 1][q] = *reinterpret_cast<const u32x4*>(at((hx + 1) / 2, 4 * ((hx + 1) % 2) + q));
                        }
                        floatx4 vv[4];
                        rows(4 * h, 4, vv);
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const floatx4 v = activate<ACT>(vv[q], b4) + __builtin_bit_cast(floatx4, cv[hx & 1][q]);
                            *reinterpret_cast<floatx4*>(at(ti, 4 * h + q)) = v;
                        }
                    }
                    asm volatile("" ::: "memory");
                }
                younger = 63;  // 32 loads and 32 stores (the wait is capped at 63)
            } else {
#pragma unroll
                for (int ti = 0; ti < kTM; ti++) {
                    floatx4 vv[8];
                    to_rows(ti, vv);
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        const floatx4 v = activate<ACT>(vv[q], b4);
                        if (OUT_LP) {
                            floatx4 sv;
#pragma unroll
                            for (int u = 0; u < 4; u++) sv[u] = clamp_finite(v[u], Enc<T>::kMax);
                            *reinterpret_cast<u32x2*>(at(ti, q)) = narrow4<T>(sv);
                        } else {
                            *reinterpret_cast<floatx4*>(at(ti, q)) = v;
                        }
                    }
                    asm volatile("" ::: "memory");
                }
                younger = 32;  // 32 stores
            }
        };
        if (whole) {
            if (g.flags & kGemmSilu) {
                whole_epi(std::integral_constant<int, 1>{});
            } else if (g.flags & kGemmRelu) {
                whole_epi(std::integral_constant<int, 2>{});
            } else {
                whole_epi(std::integral_constant<int, 0>{});
            }
        } else {
#pragma unroll
            for (int ti = 0; ti < kTM; ti++) {
                floatx4 vv[8];
                to_rows(ti, vv);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const floatx4 v = finish(vv[q]);
                    const int row = row0 + 32 * ti + 4 * q;
                    if (row >= g.m || col0 >= g.n) continue;
                    const size_t ci = (size_t)row * g.ldc + col0;
                    if (vec && col0 + 3 < g.n) {
                        if (OUT_LP) {
                            floatx4 sv;
#pragma unroll
                            for (int u = 0; u < 4; u++) sv[u] = clamp_finite(v[u], Enc<T>::kMax);
                            *reinterpret_cast<u32x2*>(static_cast<T*>(g.c) + ci) = narrow4<T>(sv);
                        } else {
                            floatx4* cp = reinterpret_cast<floatx4*>(static_cast<float*>(g.c) + ci);
                            *cp = accumulate ? v + *cp : v;
                        }
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            if (col0 + u >= g.n) break;
                            if (OUT_LP) {
                                static_cast<T*>(g.c)[ci + u] = saturate<T>(v[u]);
                            } else {
                                float* cp = static_cast<float*>(g.c) + ci + u;
                                *cp = accumulate ? v[u] + *cp : v[u];
                            }
                        }
                    }
                }
                // this block's reads are issued before the next block's writes (LDS keeps a wave's order)
                asm volatile("" ::: "memory");
            }
            younger = 0;
        }
        if (next >= total) break;
        tile = next;
    }
}

// y = twin(x * (1 / sqrt(mean(x^2) + eps)) * w), one wave per row, x fp32, y in the storage type
template <typename T>
__global__ __launch_bounds__(256) void rms_norm_lp(const float* __restrict__ x, T* __restrict__ y,
                                                   const float* __restrict__ w, int rows, int d, float eps) {
    const int row = blockIdx.x * 4 + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (row >= rows) return;
    const floatx4* xr = reinterpret_cast<const floatx4*>(x + (size_t)row * d);
    float ss = 0.f;
    for (int i = lane; i < d / 4; i += kWave) {
        const floatx4 v = xr[i];
        ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float inv = 1.f / sqrtf(ss / d + eps);
    const floatx4* wr = reinterpret_cast<const floatx4*>(w);
    T* yr = y + (size_t)row * d;
    for (int i = lane; i < d / 4; i += kWave) {
        const floatx4 v = xr[i] * inv * (w ? wr[i] : floatx4{1.f, 1.f, 1.f, 1.f});
        floatx4 s;
#pragma unroll
        for (int u = 0; u < 4; u++) s[u] = clamp_finite(v[u], Enc<T>::kMax);
        *reinterpret_cast<u32x2*>(yr + 4 * i) = narrow4<T>(s);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void to_lp(const float* __restrict__ x, T* __restrict__ y, uint64_t count) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride)
        y[i] = saturate<T>(x[i]);
}

// The three-term fp16 split (dtype JC_F16X3). hi = fp16(v), saturated to +-65504 as the FP16
// twins, and lo = fp16(v - hi). A row of k values becomes 3k fp16 values, [hi | hi | lo] for a
// GEMM's A operand or [hi | lo | hi] for its W operand, so one fp16 GEMM over K = 3k with fp32
// accumulation sums a_hi w_hi + a_hi w_lo + a_lo w_hi (fp16 products are exact in fp32).
// hi + lo = v within 2^-22 |v| + 2^-25 (lo's rounding; below 2^-14 its subnormal spacing 2^-24
// sets the absolute term), so with the dropped a_lo w_lo each product is within about
// 2^-20 |a w| + 2^-25 (|a| + |w|), against 2^-11 |a w| for a single fp16 product. Values beyond
// +-65504 saturate, as in the FP16 GEMM mode. split_f16x4 (jc_common.hpp) makes the pieces.

// x [rows, ldx] fp32 (k a multiple of 4, ldx of 4, 16-byte aligned) -> y [rows, 3k] fp16
__global__ __launch_bounds__(256) void split_x3(const float* __restrict__ x, int ldx, _Float16* __restrict__ y,
                                                int rows, int k, int weights) {
    const int q = k / 4;
    const uint64_t total = (uint64_t)rows * q;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int r = (int)(i / q), c = (int)(i % q) * 4;
        halfx4 hi, lo;
        split_f16x4(*reinterpret_cast<const floatx4*>(x + (size_t)r * ldx + c), hi, lo);
        _Float16* yr = y + (size_t)r * 3 * k;
        *reinterpret_cast<halfx4*>(yr + c) = hi;
        *reinterpret_cast<halfx4*>(yr + k + c) = weights ? lo : hi;
        *reinterpret_cast<halfx4*>(yr + 2 * k + c) = weights ? hi : lo;
    }
}

// rms_norm_f32's y, written as the A-operand split [hi | hi | lo] of 3d fp16 per row
__global__ __launch_bounds__(256) void rms_norm_x3(const float* __restrict__ x, _Float16* __restrict__ y,
                                                   const float* __restrict__ w, int rows, int d, float eps) {
    const int row = blockIdx.x * 4 + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (row >= rows) return;
    const floatx4* xr = reinterpret_cast<const floatx4*>(x + (size_t)row * d);
    float ss = 0.f;
    for (int i = lane; i < d / 4; i += kWave) {
        const floatx4 v = xr[i];
        ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float inv = 1.f / sqrtf(ss / d + eps);
    const floatx4* wr = reinterpret_cast<const floatx4*>(w);
    _Float16* yr = y + (size_t)row * 3 * d;
    for (int i = lane; i < d / 4; i += kWave) {
        halfx4 hi, lo;
        split_f16x4(xr[i] * inv * (w ? wr[i] : floatx4{1.f, 1.f, 1.f, 1.f}), hi, lo);
        *reinterpret_cast<halfx4*>(yr + 4 * i) = hi;
        *reinterpret_cast<halfx4*>(yr + d + 4 * i) = hi;
        *reinterpret_cast<halfx4*>(yr + 2 * d + 4 * i) = lo;
    }
}

}  // namespace

hipError_t gemm_lp_launch(const GemmLpArgs& g, bool fp16, bool out_lp, int cus, hipStream_t stream) {
    const uint64_t tiles_n = (uint64_t)((g.n + kBN - 1) / kBN);
    const uint64_t total = (uint64_t)((g.m + kBM - 1) / kBM) * tiles_n;
    const uint32_t grid = (uint32_t)(total < (uint64_t)cus ? total : (uint64_t)cus);
    const uint32_t tn = (uint32_t)tiles_n, tt = (uint32_t)total;
    // whole-quad stores need every row start aligned: 16 bytes (fp32 C) or 8 (storage-type C)
    // (and a 256-row block of C addressable with 32-bit offsets)
    const int vec = g.ldc % 4 == 0 && g.ldc < (1 << 22) && (size_t)g.c % (out_lp ? 8 : 16) == 0;
    if (fp16) {
        if (out_lp) hipLaunchKernelGGL((gemm_lp<_Float16, true>), dim3(grid), dim3(kThreads), 0, stream, g, tn, tt, vec);
        else hipLaunchKernelGGL((gemm_lp<_Float16, false>), dim3(grid), dim3(kThreads), 0, stream, g, tn, tt, vec);
    } else {
        if (out_lp) hipLaunchKernelGGL((gemm_lp<__bf16, true>), dim3(grid), dim3(kThreads), 0, stream, g, tn, tt, vec);
        else hipLaunchKernelGGL((gemm_lp<__bf16, false>), dim3(grid), dim3(kThreads), 0, stream, g, tn, tt, vec);
    }
    return hipGetLastError();
}

hipError_t rms_norm_lp_launch(const float* x, void* y, const float* w, int rows, int d, float eps, bool fp16,
                              hipStream_t stream) {
    const dim3 grid((uint32_t)((rows + 3) / 4));
    if (fp16) hipLaunchKernelGGL(rms_norm_lp<_Float16>, grid, dim3(256), 0, stream, x, (_Float16*)y, w, rows, d, eps);
    else hipLaunchKernelGGL(rms_norm_lp<__bf16>, grid, dim3(256), 0, stream, x, (__bf16*)y, w, rows, d, eps);
    return hipGetLastError();
}

hipError_t split_x3_launch(const float* x, int ldx, void* y, int rows, int k, bool weights, hipStream_t stream) {
    const uint64_t blocks = (uint64_t)rows * (k / 4) / 256 + 1;
    const dim3 grid((uint32_t)(blocks < 8192 ? blocks : 8192));
    hipLaunchKernelGGL(split_x3, grid, dim3(256), 0, stream, x, ldx, (_Float16*)y, rows, k, weights ? 1 : 0);
    return hipGetLastError();
}

hipError_t rms_norm_x3_launch(const float* x, void* y, const float* w, int rows, int d, float eps, hipStream_t stream) {
    hipLaunchKernelGGL(rms_norm_x3, dim3((uint32_t)((rows + 3) / 4)), dim3(256), 0, stream, x, (_Float16*)y, w, rows, d,
                       eps);
    return hipGetLastError();
}

hipError_t to_lp_launch(const float* x, void* y, uint64_t count, bool fp16, hipStream_t stream) {
    const uint64_t blocks = count / 256 + 1;
    const dim3 grid((uint32_t)(blocks < 8192 ? blocks : 8192));
    if (fp16) hipLaunchKernelGGL(to_lp<_Float16>, grid, dim3(256), 0, stream, x, (_Float16*)y, count);
    else hipLaunchKernelGGL(to_lp<__bf16>, grid, dim3(256), 0, stream, x, (__bf16*)y, count);
    return hipGetLastError();
}

}  // namespace jc
