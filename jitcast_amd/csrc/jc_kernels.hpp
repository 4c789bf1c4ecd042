// Internal launchers of the gfx950 kernels (host side). Each validates nothing: the C-ABI layer
// (jc_abi.cpp) checks shapes, pointers and alignment before calling them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "time_mask.hpp"

namespace jc {

// Chronos-2 (ts = false) or Timestral (ts = true) time attention (time_mask.hpp); a.qgroups is set
// by the launcher. fp32: dh a multiple of 8, at most 128; bf16/fp16: a multiple of 16, at most 128.
hipError_t time_attention_f32_launch(const TimeArgs& a, int dh, bool ts, hipStream_t stream);
// Chronos-2 with 64-wide heads only (else hipErrorInvalidValue): out is fp16 [rows*n, 3*inner], each
// output value's three-term split [hi | hi | lo] (the JC_F16X3 layer's A operand of the O projection).
hipError_t time_attention_f32_x3_launch(const TimeArgs& a, int dh, hipStream_t stream);
hipError_t time_attention_lp_launch(const TimeArgs& a, int dh, bool ts, bool fp16, hipStream_t stream);
int time_attention_max_tokens();
// The row-wide bf16/fp16 kernel: 8-wave workgroups of 256 queries of one (row, head); dh 32 or 64;
// rows of at least 256 tokens.
bool time_attention_lpw_fits(const TimeArgs& a, int dh);
hipError_t time_attention_lpw_launch(const TimeArgs& a, int dh, bool ts, bool fp16, hipStream_t stream);
// The persistent bf16/fp16 kernel (Chronos-2, dh 64, 257..513 tokens per row, no gate): one
// 8-wave workgroup per CU streams its (row, head) items; `cus` sizes the grid.
bool time_attention_lpp_fits(const TimeArgs& a, int dh, bool ts);
hipError_t time_attention_lpp_launch(const TimeArgs& a, bool fp16, int cus, hipStream_t stream);
bool time_attention_lps_fits(const TimeArgs& a, int dh, bool ts);
hipError_t time_attention_lps_launch(const TimeArgs& a, bool fp16, int cus, hipStream_t stream);
// att[i] *= sigmoid(g[i]) for i < count (dtype: 0 fp32, 1 bf16, 2 fp16)
hipError_t gate_launch(void* att, const void* g, uint64_t count, int dtype, hipStream_t stream);
// The arguments of the group-attention kernels (by value).
struct GroupArgs {
    const void* qkv;        // [rows*n, 3*inner] of the storage type
    void* out;              // [rows*n, inner] of the storage type
    const int32_t* valid;   // Chronos-2: live [rows*n]; Timestral: keyValid [rows*enc]
    const int32_t* gstart;  // [rows]
    const int32_t* gend;    // [rows]
    const int32_t* role;    // Timestral: [rows] TARGET 0 / PAST 1 / KNOWN 2, or null
    const void* gate;       // [rows*n, inner] of the storage type: out *= sigmoid(gate); or null
    int rows, n, heads, inner;
    int enc;                // Timestral's encoder slots (keyValid applies to t < enc)
    int covariates;         // Timestral: whether the block runs the covariate rules
    float qscale;           // score scale times log2(e), folded into q
    int rtiles;             // 16-row tiles, set by the launcher
    int hsplit;             // head ranges per (tile, slot), one wave each; set by the launcher
    const int32_t* order;   // [rtiles] the tiles by descending work (group_tile_order_launch), or null
    int f32_mfma;           // fp32 storage on fp32 MFMA instead of three-term fp16 products; set by the launcher
};

// Capacity, in 16-row tiles, of the buffers group_tile_order_launch fills.
constexpr int kGroupOrderTiles = 16384;

// The order in which the group kernel dispatches its tiles: by descending work, (16-row key tiles)^2
// summed over the groups starting in the tile (bucketed), so the launch ends on light waves. One
// workgroup; order gets the ceil(rows / 16) tile indices (rows <= 16 * kGroupOrderTiles).
hipError_t group_tile_order_launch(const int32_t* gstart, const int32_t* gend, int rows, int32_t* order,
                                   hipStream_t stream);

// Chronos-2 group attention (ts = false) or Timestral variate attention (ts = true); a.rtiles is
// set by the launcher. dh a multiple of 8, at most 128 (64 for Chronos-2). dtype (0 fp32, 1 bf16,
// 2 fp16) is the storage type of qkv, the gate and out; the arithmetic is fp32.
hipError_t group_attention_launch(const GroupArgs& a, int dh, bool ts, int dtype, hipStream_t stream);
// Chronos-2 with 64-wide heads only (else hipErrorInvalidValue): a.out is read as fp16 [rows*n, 3*inner],
// each output value's three-term split [hi | hi | lo].
hipError_t group_attention_f32_x3_launch(const GroupArgs& a, int dh, hipStream_t stream);

hipError_t fill_normal_launch(float* out, uint64_t count, uint64_t stream_seed, double mean, double stdv,
                              hipStream_t stream);
hipError_t fill_uniform_launch(float* out, uint64_t count, uint64_t stream_seed, double lo, double hi,
                               hipStream_t stream);

// C[m, n] (+)= act(A[m, :k] . W[n, :k] + b[n]) in fp32 (Kernels.gemm's flags, Kernels.java:50-56).
constexpr int kGemmBias = 1, kGemmAccumulate = 2, kGemmSilu = 4, kGemmRelu = 16;
struct GemmArgs {
    const float* a;     // [m, lda]
    const float* w;     // [n, k]
    const float* bias;  // [n] when flags & kGemmBias
    float* c;           // [m, ldc]
    int m, n, k, lda, ldc, flags;
};
// k a multiple of 16; lda a multiple of 4; a, w 16-byte aligned
hipError_t gemm_f32_launch(const GemmArgs& g, hipStream_t stream);
// y = x * (1 / sqrt(mean(x^2) + eps)) * w per row of d (d a multiple of 4; w may be null)
hipError_t rms_norm_f32_launch(const float* x, float* y, const float* w, int rows, int d, float eps, hipStream_t stream);

// bf16/fp16 GEMM with fp32 accumulation: C (+)= act(A . W^T + b), A [m, lda] and W [n, k] in the
// storage type, C fp32 (out_lp false: any flags) or the storage type (out_lp true: no ACCUMULATE),
// saturated to its finite range. k a multiple of 8; a, w 16-byte aligned, lda a multiple of 8.
struct GemmLpArgs {
    const void* a;
    const void* w;
    const float* bias;
    void* c;
    int m, n, k, lda, ldc, flags;
};
// persistent: at most `cus` workgroups; m, n < 2^31 tiles; lda and k below 2^22 (a 256-row block of
// either operand spans less than 2^31 bytes)
hipError_t gemm_lp_launch(const GemmLpArgs& g, bool fp16, bool out_lp, int cus, hipStream_t stream);
// y (storage type) = x * (1 / sqrt(mean(x^2) + eps)) * w per row of d (d a multiple of 4)
hipError_t rms_norm_lp_launch(const float* x, void* y, const float* w, int rows, int d, float eps, bool fp16,
                              hipStream_t stream);
// y[i] = x[i] rounded to the storage type, saturated to its finite range
hipError_t to_lp_launch(const float* x, void* y, uint64_t count, bool fp16, hipStream_t stream);
// the three-term fp16 split of x [rows, ldx] fp32 into y [rows, 3k] fp16: [hi | hi | lo] (A operand)
// or, with weights, [hi | lo | hi] (W operand); k and ldx multiples of 4, x 16-byte aligned
hipError_t split_x3_launch(const float* x, int ldx, void* y, int rows, int k, bool weights, hipStream_t stream);
// rms_norm_f32's output as the A-operand split [rows, 3d] fp16
hipError_t rms_norm_x3_launch(const float* x, void* y, const float* w, int rows, int d, float eps, hipStream_t stream);

// Chronos-2 token moves (d a multiple of 4, 16-byte aligned): the encoder input from the patch
// embeddings and [REG] (reg may be null when nreg = 0), and the future tokens of the encoder output
hipError_t assemble_tokens_launch(const float* emb, const float* reg, float* x, int rows, int nc, int nreg, int n, int d,
                                  hipStream_t stream);
hipError_t gather_future_launch(const float* y, float* dec, int rows, int fs, int n, int h, int d, hipStream_t stream);

// The Timestral block's elementwise stages (ts_block.hip): token assembly (d a multiple of 4,
// 16-byte aligned) and SwiGLU (dtype_code 0 fp32, 1 bf16, 2 fp16 for both up and act)
hipError_t ts_assemble_launch(const float* emb, const float* query, float* x, int rows, int enc, int n, int d,
                              hipStream_t stream);
hipError_t swiglu_launch(const void* up, void* act, uint64_t tokens, int f, int dtype_code, hipStream_t stream);

// The Chronos-2 host ends (c2_prep.hip): ModelLayout's cut and live mask plus ModelPrep.of from the
// raw context rows; ModelPrep.finish into [rows][Q][h*P]. order (nullable) gathers input rows /
// scatters output rows.
hipError_t c2_prep_launch(const float* ctx, int64_t ld_ctx, int steps, const float* fut, int64_t ld_fut, int fut_steps,
                          const int32_t* order, int rows, int kept, int nc, int h, int patch, int nreg, float time_scale,
                          int arcsinh, float* tok, float* loc, float* scale, int32_t* live, hipStream_t stream);
hipError_t c2_finish_launch(const float* raw, const float* loc, const float* scale, const int32_t* order, int rows,
                            int h, int q, int patch, int arcsinh, float* out, hipStream_t stream);

constexpr int kTsMaxQuantiles = 32;
hipError_t ts_prep_launch(const float* window, const uint8_t* observed, int rows, int w, int patch,
                          const int32_t* known, float minimum_scale, int use_asinh, float* tok, float* scaled,
                          float* loc, float* scale, hipStream_t stream);
hipError_t ts_finish_launch(const float* raw, const float* loc, const float* scale, int rows, int w, int anchor,
                            int steps, int q, const float* width, int median, int use_asinh, float* out,
                            hipStream_t stream);

}  // namespace jc
