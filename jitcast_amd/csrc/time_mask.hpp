// The attention masks of the time-attention kernels, over 64-key blocks aligned to 64.
//
// Chronos-2 (Chronos2Kernels.timeAttention, Chronos2Kernels.java:118-464; CpuChronos2.java:190-211):
//   a key is visible to every query of its row when live[r*n + k] != 0 (bidirectional, key-only).
// Timestral (BlockLayout.timeAllowed, BlockLayout.java:209-221; TimestralKernels.timeAttention,
// TimestralKernels.java:102-278):
//   encoder query q < enc:  k < enc and (k == q or (keyValid[r][k] and (k <= q or known[r])))
//   decoder query q >= enc: k < enc ? (k < ll and keyValid[r][k]) : k <= q
//
// Each block b carries one 64-bit word of per-key validity (bit i = key 64b + i): Chronos-2's live
// bits, or Timestral's keyValid bits of encoder keys (0 for k >= enc). A query's visible keys in
// the block are derived from that word by a few 64-bit operations (allowed()), and a workgroup's
// query range [qlo, qhi] marks the blocks any of its queries can see (any_allowed()).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jc {

constexpr int kMaskBlock = 64;

// Bits of the keys k0 + i with k < lim (i < 64).
__device__ __forceinline__ uint64_t bits_below(int lim, int k0) {
    int c = lim - k0;
    return c <= 0 ? 0ull : (c >= 64 ? ~0ull : ((1ull << c) - 1ull));
}

// The arguments every time-attention kernel takes (by value).
struct TimeArgs {
    const void* qkv;        // [rows*n, 3*inner] of the storage type
    void* out;              // [rows*n, inner]
    const int32_t* valid;   // Chronos-2: live [rows*n]; Timestral: keyValid [rows*enc]
    const int32_t* known;   // Timestral: [rows] (a known-covariate row sees every valid key); else null
    const int32_t* pos;     // RoPE table row of each token [rows*n], or null (row = token index)
    const float* table;     // [table_rows, dh] cos | sin, or null (q and k already rotated)
    const void* gate;       // [rows*n, inner] of the storage type: out *= sigmoid(gate); or null
    int rows, n, heads, inner;
    int enc, ll;            // Timestral's encoder tokens and context patches (Chronos-2: enc = n)
    int table_rows;         // rows of the table a pos value may address
    float qscale;           // score scale times log2(e), folded into q
    int qgroups;            // workgroups per (row, head)
    int q_begin;            // the first query the launch covers (0: all of them)
    int q_tail;             // fp32 Chronos-2 rows of 128k + R: the first query of the tail workgroups
                            // (0: none), set by the fp32 launcher
};

template <bool TS>
struct TimeMask {
    int enc, ll, n;
    bool known;

    __device__ __forceinline__ void init(const TimeArgs& a, int r) {
        n = a.n;
        enc = TS ? a.enc : a.n;
        ll = TS ? a.ll : a.n;
        known = TS && a.known != nullptr && a.known[r] != 0;
    }

    // validity word of block b from the row's mask array (one lane per key: lane i reads key 64b+i)
    __device__ __forceinline__ bool key_valid(const int32_t* row_valid, int k) const {
        return TS ? (k < enc && row_valid[k] != 0) : (k < n && row_valid[k] != 0);
    }

    // keys of block k0 visible to query q, from the block's validity word vb
    __device__ __forceinline__ uint64_t allowed(uint64_t vb, int k0, int q) const {
        if (!TS) return vb;
        const uint64_t le = bits_below(q + 1, k0);
        if (q < enc) {
            const uint64_t self = (q >= k0 && q < k0 + 64) ? (1ull << (q - k0)) : 0ull;
            return bits_below(enc, k0) & (self | (vb & (known ? ~0ull : le)));
        }
        return (vb & bits_below(ll, k0)) | (~bits_below(enc, k0) & le);
    }

    // whether any query of [qlo, qhi] sees a key of block k0
    __device__ __forceinline__ bool any_allowed(uint64_t vb, int k0, int qlo, int qhi) const {
        if (!TS) return vb != 0;
        if (qlo > qhi) return false;
        uint64_t u = 0;
        if (qlo < enc) {
            const int ez = min(qhi, enc - 1);
            const uint64_t selfs = bits_below(ez + 1, k0) & ~bits_below(qlo, k0);
            u |= bits_below(enc, k0) & (selfs | (vb & (known ? ~0ull : bits_below(ez + 1, k0))));
        }
        if (qhi >= enc) u |= (vb & bits_below(ll, k0)) | (~bits_below(enc, k0) & bits_below(qhi + 1, k0));
        return u != 0;
    }
};

}  // namespace jc
