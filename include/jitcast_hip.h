/*
 * libjitcast_hip — C ABI of the MI355X (gfx950) encoder self-attention path.
 *
 * This is the drop-in boundary beside the reference's TornadoVM engines: a host (Java through
 * Panama FFM downcalls, C++, or Python ctypes) owns device buffers allocated here, uploads the
 * per-call inputs the reference's plans upload every run (tokens, RoPE table, live mask, group
 * bounds; Chronos2Forward.java:248-249, 462-489), and calls one entry point per attention stage.
 * Citations name the reference interface each entry point replaces; `J/` is
 * src/main/java/ai/beestream/jitcast/ in the reference.
 *
 * Conventions (all entry points):
 *   - return JC_OK (0) on success, a negative jc_status on error; jc_last_error() then holds a
 *     thread-local message naming the entry point and the offending argument. Nothing throws or
 *     aborts across this ABI.
 *   - device pointers are caller-owned (jc_alloc or any hipMalloc'd memory); launches are
 *     asynchronous on the context's stream; jc_sync waits.
 *   - a jc_ctx is not thread-safe; callers serialise per engine, as the reference's
 *     `synchronized PlanCache.run` does (J/tornado/PlanCache.java:70).
 *   - activations are the reference's layout: qkv [rows*n, 3*inner], q|k|v heads-major per token
 *     (h*dh + e); out [rows*n, inner]; masks int32 0/1.
 */
#ifndef JITCAST_HIP_H
#define JITCAST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum jc_status {
    JC_OK = 0,
    JC_EINVAL = -1,       /* a bad argument (shape, pointer, alignment, dtype) */
    JC_EHIP = -2,         /* the HIP runtime reported an error */
    JC_ENOMEM = -3,       /* device or host allocation failed */
    JC_EUNSUPPORTED = -4, /* a valid request this build does not implement */
    JC_ESTATE = -5        /* a call out of order (e.g. plan_end without plan_begin) */
} jc_status;

typedef enum jc_dtype {
    JC_F32 = 0,  /* fp32 in and out, fp32 MFMA: the reference's FP32-exact default */
    JC_BF16 = 1, /* bf16 qkv and out, bf16 MFMA with fp32 accumulation and fp32 softmax */
    JC_F16 = 2,  /* fp16 qkv and out (saturated to +-65504 as Kernels.java:42-46), fp32 accumulation */
    JC_F16X3 = 3 /* jc_c2_layer only: fp32 in and out, each GEMM as three fp16 products with fp32
                    accumulation (jc_split_f16x3), about fp32's accuracy; no reference counterpart */
} jc_dtype;

typedef struct jc_ctx jc_ctx;
typedef struct jc_plan jc_plan;

/* ---- runtime (replaces TornadoVM device selection and buffers: J/tornado/Devices.java:44-73) ---- */

/* Makes `device` current and creates the context's stream (default priority) and its 64 KB buffer
 * for the group kernels' tile order (jc_c2_group_attention). */
int jc_init(int device, jc_ctx **ctx);
/* Destroys the context (idempotent on NULL). */
int jc_destroy(jc_ctx *ctx);
/*
 * Launches on an existing stream (e.g. a framework's current stream) instead of the context's
 * own; NULL selects the device's default (null) stream. jc_stream() before the call returns the
 * context's own stream, to restore it later.
 */
int jc_set_stream(jc_ctx *ctx, void *hip_stream);
/* The stream launches go to. */
void *jc_stream(jc_ctx *ctx);
/*
 * Per-kernel timing, the counterpart of -Dchronos2.tornado.profile and -Dtimestral.tornado.profile
 * (J/chronos2/tornado/Chronos2Forward.java:301-303, J/timestral/tornado/TimestralForward.java:391-393,
 * TornadoVM's console profiler). on = 1 starts (or restarts) recording a HIP event pair around every
 * launch the context makes outside a capture; on = 0 stops and discards.
 */
int jc_profile(jc_ctx *ctx, int on);
/*
 * Waits for the context's stream, writes one line per kernel (calls, total, mean, min and max ms,
 * the largest total first) into buf as text, and clears what was recorded. JC_ESTATE when profiling
 * is off.
 */
int jc_profile_report(jc_ctx *ctx, char *buf, size_t len);
int jc_alloc(jc_ctx *ctx, size_t bytes, void **dptr);
int jc_free(jc_ctx *ctx, void *dptr);
int jc_memcpy_h2d(jc_ctx *ctx, void *dst, const void *src, size_t bytes);
int jc_memcpy_d2h(jc_ctx *ctx, void *dst, const void *src, size_t bytes);
int jc_memcpy_d2d(jc_ctx *ctx, void *dst, const void *src, size_t bytes);
int jc_sync(jc_ctx *ctx);
/* Compute units and the gfx architecture name of the context's device. */
int jc_device_info(jc_ctx *ctx, int *compute_units, char *arch, size_t arch_len);
/* The calling thread's last error message ("" if none). */
const char *jc_last_error(void);
/* 1 + the library's ABI revision. */
int jc_version(void);

/* ---- plans: one captured hipGraph per batch shape (replaces a compiled TornadoVM execution plan:
 *      J/tornado/PlanCache.java:40-161, J/chronos2/tornado/Chronos2Forward.java:106, 294-300) ------- */

/*
 * Starts capturing everything the context enqueues (attention entry points, device-to-device
 * copies) into a plan for the batch shape `shape_key`. The context must launch on a created stream
 * (jc_init's own, or one given to jc_set_stream), not the null stream. While capturing, host copies
 * and jc_sync return JC_ESTATE: upload per-call inputs into the plan's buffers before
 * jc_plan_launch, as the reference uploads them before each execution.
 */
int jc_plan_begin(jc_ctx *ctx, uint64_t shape_key);
/* (jc_plan_begin also allocates the plan's own 64 KB tile-order buffer, freed with the plan and not
 * counted by jc_plan_device_bytes.) */
/* Ends the capture and instantiates the plan; on error no plan is made and capture has ended. */
int jc_plan_end(jc_ctx *ctx, jc_plan **plan);
/* Replays the plan on the context's current stream (asynchronous; jc_sync waits). */
int jc_plan_launch(jc_plan *plan);
/*
 * Replays the plan on `hip_stream` (NULL: the stream of the context that captured it), whichever
 * stream that context launches on now; for a host whose threads each keep their own context and
 * share plans, as one PlanCache serves every caller of an engine (J/tornado/PlanCache.java:70-100).
 */
int jc_plan_launch_on(jc_plan *plan, void *hip_stream);
/*
 * Gives the plan ownership of a device buffer from jc_alloc: jc_plan_destroy frees it and
 * jc_plan_device_bytes counts it, as each TornadoVM plan counts its own buffers (PlanCache.java:30-36).
 */
int jc_plan_adopt(jc_plan *plan, void *dptr, size_t bytes);
/* The bytes of the buffers the plan owns. */
int64_t jc_plan_device_bytes(jc_plan *plan);
/* The shape key given to jc_plan_begin. */
uint64_t jc_plan_key(jc_plan *plan);
/* Waits for the plan's last replay (on whichever stream it was launched), frees the adopted buffers
 * and the graph (idempotent on NULL). */
int jc_plan_destroy(jc_plan *plan);

/* ---- synthetic inputs (no reference counterpart: the benchmark's seeded generator) ---------------- */

/*
 * Fills device memory with the portable RNG: SplitMix64 output i of stream `stream_seed`
 * (a case's tensor k uses seed*1000003 + k), 24-bit uniforms, Box-Muller normals in double rounded
 * to float. Bit-compatible with jitcast_amd/rng.py up to the last-ulp rounding of the device's
 * double log/cos/sin.
 */
int jc_fill_normal(jc_ctx *ctx, float *dptr, uint64_t count, uint64_t stream_seed, float mean, float stdv);
int jc_fill_uniform(jc_ctx *ctx, float *dptr, uint64_t count, uint64_t stream_seed, float lo, float hi);

/* ---- Chronos-2 time attention --------------------------------------------------------------- */

/*
 * The host-built RoPE table: table[p*dh + e] = cos((float)p * invFreq[e]) and
 * table[p*dh + dh/2 + e] = sin(..), e < dh/2, cos/sin in double rounded to float, invFreq[i] =
 * 1/(float)pow(theta, (float)(2i)/dh). Writes host memory [n*dh].
 * Replaces Chronos2Forward.Plan.run's table fill (J/chronos2/tornado/Chronos2Forward.java:465-474)
 * and CpuChronos2.inverseFrequencies (J/chronos2/cpu/CpuChronos2.java:102-111).
 */
int jc_c2_rope_table(int n, int dh, float theta, float *table_host);

/*
 * Fused RoPE + bidirectional time attention over the live keys of each row, unscaled scores;
 * a query with no live key gets zeros.
 * Replaces the pair Chronos2Kernels.rope(qkv, table, tokens, n, heads, dh, inner) and
 * Chronos2Kernels.timeAttention(qkv, out, live, rows, n, heads, dh, inner)
 * (J/chronos2/tornado/Chronos2Kernels.java:93-94, 130-131), oracle CpuChronos2.java:175-228.
 *   qkv         device, [rows*n, 3*inner] of `dtype`; never written (RoPE is applied at load)
 *   out         device, [rows*n, inner] of `dtype`
 *   live        device, [rows*n] int32
 *   rope_table  device, [n, dh] fp32 from jc_c2_rope_table, or NULL when q and k are already rotated
 *   dh          a multiple of 8, at most 64 (the reference takes multiples of 16 up to 64,
 *               Chronos2Forward.java:126-128); inner >= heads*dh, a multiple of 4; n <= 4096
 */
int jc_c2_time_attention(jc_ctx *ctx, const void *qkv, void *out, const int32_t *live, const float *rope_table,
                         int rows, int n, int heads, int dh, int inner, int dtype);

/* ---- Chronos-2 group attention ---------------------------------------------------------------- */

/*
 * Attention across the rows of each group at every token slot, per head: row i reads the rows j
 * in [group_start[i], group_end[i]) whose token at the slot is live; unscaled scores, no RoPE;
 * zeros when none is. Groups must be contiguous runs of rows (jc_c2_group_order makes them so).
 * Replaces Chronos2Kernels.groupAttention(qkv, out, live, groupStart, groupEnd, rows, n, heads,
 * dh, inner) (J/chronos2/tornado/Chronos2Kernels.java:473-474), oracle CpuChronos2.java:230-282.
 *   qkv, out     device, as jc_c2_time_attention (the group sublayer's own projection)
 *   group_start  device int32 [rows]; group_end device int32 [rows] (jc_c2_group_bounds)
 *   dh           a multiple of 8, at most 64 (the reference takes multiples of 16)
 *   dtype        the storage type of qkv and out: JC_F32, or JC_BF16 / JC_F16 (scores, softmax and
 *                accumulation in fp32, out rounded once)
 * With JC_F32 the QK^T and PV products run as three fp16 MFMA products each (v = hi + lo), within
 * about 2^-20 of the fp32 product; a wave that meets a value beyond fp16's range runs on fp32 MFMA.
 * With JC_BF16 / JC_F16, K and Q enter the MFMA of their type as stored (exact products), and P as a
 * hi + lo pair of the type against V as stored.
 * A one-workgroup kernel first sorts the 16-row tiles by work (into the context's buffer, or the
 * plan's while capturing), so the launch dispatches the heaviest first.
 */
int jc_c2_group_attention(jc_ctx *ctx, const void *qkv, void *out, const int32_t *live, const int32_t *group_start,
                          const int32_t *group_end, int rows, int n, int heads, int dh, int inner, int dtype);

/* ---- Timestral time attention ----------------------------------------------------------------- */

/*
 * The host-built RoPE table over every position a token can have, (-enc, enc + h): row p holds
 * cos((float)(p - enc) * invFreq[e]) at e < dh/2 and the sin at dh/2 + e (double cos/sin rounded to
 * float), invFreq[i] = 1/(float)pow(theta, (float)(2i)/rope_dim) for i < rope_dim/2 and 0 after (those
 * dims pass through). n = enc + h tokens per row; writes host memory [(enc + n) * dh].
 * Replaces TimestralForward.Plan.run's table fill (J/timestral/tornado/TimestralForward.java:599-610)
 * and CpuTimestral.inverseFrequencies (J/timestral/cpu/CpuTimestral.java:107-116).
 */
int jc_ts_rope_table(int enc, int n, int dh, int rope_dim, float theta, float *table_host);

/*
 * Fused RoPE + masked time attention + output gate of one Timestral attention sublayer: scores
 * q.k/sqrt(dh) under BlockLayout.timeAllowed (encoder query q < enc: keys k < enc with k == q or
 * (key_valid[r][k] and (k <= q or known[r])); decoder query: valid context keys k < ll and decoder
 * keys k <= q), RoPE at table row pos[token] for q and k, and out *= sigmoid(gate) when gate is not
 * NULL.
 * Replaces TimestralKernels.rope(qkv, pos, table, tokens, heads, dh, d), TimestralKernels.timeAttention(
 * qkv, out, keyValid, known, rows, enc, ll, n, heads, dh, d) and TimestralKernels.gate(att, g, count)
 * (J/timestral/tornado/TimestralKernels.java:77-78, 114-115, 573); oracle CpuTimestral.java:150-163,
 * 190-259; masks BlockLayout.java:209-221.
 *   qkv, out     device, [rows*n, 3*d] and [rows*n, d] of `dtype` (q|k|v heads-major per token)
 *   key_valid    device int32 [rows*enc]; known device int32 [rows] or NULL (no known rows)
 *   pos          device int32 [rows*n]: table row of each token (position + enc), clamped into the
 *                table's enc + n rows; NULL uses the token index
 *   rope_table   device [(enc + n), dh] fp32 from jc_ts_rope_table, or NULL when q, k are rotated
 *   gate         device [rows*n, d] of `dtype`, or NULL (no gate)
 *   dh           fp32: a multiple of 8, at most 128 (TimestralForward.java:163-166); bf16/fp16: a
 *                multiple of 16; d >= heads*dh; 0 <= ll <= enc <= n <= 4096
 */
int jc_ts_time_attention(jc_ctx *ctx, const void *qkv, void *out, const int32_t *key_valid, const int32_t *known,
                         const int32_t *pos, const float *rope_table, const void *gate, int rows, int enc, int ll,
                         int n, int heads, int dh, int d, int dtype);

/*
 * att[i] *= sigmoid(g[i]) for i < count, in place on device memory of `dtype` (fp32 16-byte aligned,
 * bf16/fp16 8-byte aligned). Replaces TimestralKernels.gate(att, g, count)
 * (J/timestral/tornado/TimestralKernels.java:572-578); the attention entry points fuse it.
 */
int jc_ts_gate(jc_ctx *ctx, void *att, const void *g, int64_t count, int dtype);

/* ---- Timestral variate attention -------------------------------------------------------------- */

/*
 * Attention across the rows of each series at every token slot, per head, with scores scaled by
 * 1/sqrt(dh) under BlockLayout.variateAllowed: row q reads row k of its group [group_start[q],
 * group_end[q]) when k == q, or when (at an encoder slot t < enc) key_valid[k][t] and, with
 * covariates, not (role[q] != TARGET and role[k] == TARGET) and not (role[q] == KNOWN and role[k] !=
 * KNOWN); out *= sigmoid(gate) when gate is not NULL. Groups are contiguous runs of rows.
 * Replaces TimestralKernels.variateAttention(qkv, out, keyValid, groupStart, groupEnd, role,
 * covariates, rows, enc, n, heads, dh, d) and TimestralKernels.gate
 * (J/timestral/tornado/TimestralKernels.java:290-292, 573); oracle CpuTimestral.java:261-314;
 * masks BlockLayout.java:223-243.
 *   key_valid  device int32 [rows*enc]; role device int32 [rows] (0 TARGET, 1 PAST, 2 KNOWN;
 *              BlockInput.java:35-37), may be NULL when covariates == 0
 *   gate       device [rows*n, d] of `dtype` or NULL; dtype: the storage type of qkv, gate and out,
 *              JC_F32 or JC_BF16 / JC_F16 (fp32 arithmetic, out rounded once)
 *   dh         a multiple of 8, at most 128; d >= heads*dh
 */
int jc_ts_variate_attention(jc_ctx *ctx, const void *qkv, void *out, const int32_t *key_valid,
                            const int32_t *group_start, const int32_t *group_end, const int32_t *role, int covariates,
                            const void *gate, int rows, int enc, int n, int heads, int dh, int d, int dtype);

/* ---- host-side layout (the per-call work the reference does in Java before each upload) ------- */

/*
 * live[i*n + p] for n = nc + reg + h tokens: a context patch is live when any of its `patch`
 * steps of window[i*nc*patch ..] is not NaN; [REG] and future tokens are always live.
 * Replaces ModelLayout.of's mask (J/chronos2/ModelLayout.java:104-114). Host memory.
 */
int jc_c2_live(const float *window, int rows, int nc, int patch, int reg, int h, int32_t *live);
/*
 * The row order that makes groups contiguous: groups in order of first appearance, rows in order
 * within a group; *identity = 1 when the rows already are. Replaces Chronos2Forward.groupOrder
 * (J/chronos2/tornado/Chronos2Forward.java:178-194). Host memory.
 */
int jc_c2_group_order(const int32_t *group, int rows, int32_t *order, int *identity);
/*
 * Per-row [start, end) of each row's group; JC_EINVAL if a group's rows are not contiguous.
 * Replaces the bounds fill of Chronos2Forward.Plan.run (J/chronos2/tornado/Chronos2Forward.java:475-489)
 * and TimestralForward.Plan.run's contiguity check (J/timestral/tornado/TimestralForward.java:614-629).
 */
int jc_c2_group_bounds(const int32_t *group, int rows, int32_t *start, int32_t *end);

/*
 * Timestral's block layout: BlockLayout.of and position() (J/timestral/BlockLayout.java:77-148,
 * 203-207), host memory. The block runs the covariate path (*covariates_out = 1) when role is given,
 * covariate_enabled is set and some row is not a TARGET; its window is then the context plus the
 * horizon's known-future steps (future_observed [rows][h*patch], NULL = unobserved), so
 * enc = t/patch + h, else enc = t/patch.
 *   observed      [rows][t] 0/1, t a multiple of patch; h >= 1 (h <= block_size with covariates)
 *   key_valid     out [rows*enc]: the patch has an observed step (attend_missing: or any earlier one)
 *   known         out [rows]: the row is a KNOWN covariate of a covariate block
 *   pos           out [rows*(enc+h)]: table row (position + enc) of every token, positions counted
 *                 from the first patch any row of the series observes; decoder tokens continue from
 *                 t/patch. Size key_valid and pos for enc = t/patch + h.
 * Errors mirror BlockLayout.of's IllegalArgumentExceptions (JC_EINVAL).
 */
int jc_ts_block_layout(const uint8_t *observed, const uint8_t *future_observed, const int32_t *group,
                       const int32_t *role, int rows, int t, int patch, int h, int covariate_enabled,
                       int attend_missing, int block_size, int *enc_out, int *covariates_out, int32_t *key_valid,
                       int32_t *known, int32_t *pos);

/*
 * Per row of Timestral's assembled context x [rows][t] with observed [rows][t] 0/1, host memory:
 * Scaler.lastLocScale (J/timestral/Scaler.java:65-79), the mean (loc) and Bessel-corrected std
 * (scale, at least minimum_scale) of the observed values, summed in double in order; and the
 * smallest (lo) and largest (hi) observed value, 0 when none is, which TimestralPipeline's cap
 * bounds use (_cap_quantiles, TimestralPipeline.java:378-395). NaN propagates. Outputs [rows];
 * any may be NULL.
 */
int jc_ts_context_stats(const float *x, const uint8_t *observed, int rows, int t, float minimum_scale, float *loc,
                        float *scale, float *lo, float *hi);

/*
 * Scaler.advancingFrames (J/timestral/Scaler.java:161-236), host memory: the (loc, scale) frame of
 * each of a decoded block's n_pred patches, patch j in the statistics of the observed context
 * plus the block's medians of patches 0..j-1 (each denormalised in its own frame, clipped and
 * folded in by welford_combine). The context's per-patch states combine by an inclusive
 * Hillis-Steele scan in the reference's order.
 *   context, observed  [rows][t], t a multiple of patch, t >= patch
 *   sinh_median        [rows][n_pred][patch] (median - loc) / scale in the last context patch's frame
 *   locs, scales       out [rows][n_pred], double
 */
int jc_ts_advancing_frames(const float *context, const uint8_t *observed, const double *sinh_median, int rows, int t,
                           int patch, int n_pred, float minimum_scale, double *locs, double *scales);

/* ---- The Chronos-2 encoder layer around the attention cores (fp32) -------------------------- */

/* Kernels.gemm flags (J/tornado/Kernels.java:50-56). */
#define JC_GEMM_BIAS 1
#define JC_GEMM_ACCUMULATE 2
#define JC_GEMM_SILU 4
#define JC_GEMM_RELU 16

/*
 * C[m, n] (+)= act(A[m, :k] . W[n, :k] + bias[n]), fp32 on MFMA, in the epilogue order bias,
 * activation (SILU or RELU), accumulate. Replaces Kernels.gemm / gemmBlocked / gemmBlockedWide and
 * the cuBLAS path of Chronos2Forward.Plan.gemm (J/tornado/Kernels.java:59-103, 233-480;
 * J/chronos2/tornado/Chronos2Forward.java:312-409); W is PyTorch's [out, in]. A non-NULL bias sets
 * JC_GEMM_BIAS, as Plan.gemm does for a Lin with a bias.
 *   a [m, lda], w [n, k], c [m, ldc] device fp32; k a multiple of 16, lda >= k and a multiple of 4,
 *   ldc >= n; a and w 16-byte aligned.
 */
int jc_linear(jc_ctx *ctx, const float *a, int lda, const float *w, const float *bias, float *c, int ldc, int m,
              int n, int k, int flags);

/*
 * y = x * (1 / sqrt(mean(x^2) + eps)) * w per row of d: Kernels.rmsNorm (J/tornado/Kernels.java:800-829)
 * and Ops.rmsNorm (J/cpu/Ops.java:53-68). x, y [rows, d] device fp32 (may alias), w [d] or NULL;
 * d a multiple of 4; 16-byte aligned.
 */
int jc_rms_norm(jc_ctx *ctx, const float *x, const float *w, float *y, int rows, int d, float eps);

/*
 * The three-term fp16 split of an fp32 matrix src [rows, ld_src] (k columns): dst [rows, 3k] fp16
 * holds, per row, [hi | hi | lo] (weights = 0: a GEMM's A operand) or [hi | lo | hi] (weights = 1:
 * its W operand), hi = fp16(v) saturated to +-65504, lo = fp16(v - hi). One fp16 GEMM over K = 3k
 * with fp32 accumulation then sums a_hi w_hi + a_hi w_lo + a_lo w_hi: each product within about
 * 2^-20 |a w| + 2^-25 (|a| + |w|) (hi + lo = v within 2^-22 |v| + 2^-25; hi saturates beyond
 * +-65504, as the FP16 GEMM mode's operands do). No counterpart in the reference: it is the JC_F16X3 layer's operand format (fp32
 * accuracy on fp16 MFMA). k and ld_src multiples of 4, src 16-byte aligned, dst 8-byte aligned.
 */
int jc_split_f16x3(jc_ctx *ctx, const float *src, int ld_src, void *dst, int rows, int k, int weights);

/* Device weights of one Chronos-2 encoder layer (Chronos2Packed.Layer, Chronos2Packed.java:41-47,
 * 150-154). The matrices are fp32 for a JC_F32 layer, bf16 / fp16 for a JC_BF16 / JC_F16 layer
 * (jc_to_lp converts them once) and fp16 [n, 3k] W-operand splits for a JC_F16X3 layer
 * (jc_split_f16x3 with weights = 1); norm weights and biases are always fp32. A bias may be NULL. */
typedef struct jc_c2_layer_weights {
    const float *time_norm;  /* [d] */
    const void *time_qkv;    /* [3*inner, d]: q | k | v rows, heads-major */
    const float *time_qkv_bias;
    const void *time_o;      /* [d, inner] */
    const float *time_o_bias;
    const float *group_norm; /* [d] */
    const void *group_qkv;   /* [3*inner, d] */
    const float *group_qkv_bias;
    const void *group_o;     /* [d, inner] */
    const float *group_o_bias;
    const float *mlp_norm;   /* [d] */
    const void *wi;          /* [dff, d] */
    const float *wi_bias;
    const void *wo;          /* [d, dff] */
    const float *wo_bias;
} jc_c2_layer_weights;

/* Bytes of the workspace jc_c2_layer needs for T = rows*n tokens, each part 256-byte aligned, or
 * -1 for a negative size. JC_F32: hn [T, d], big [T, max(3*inner, dff)], att [T, inner] floats.
 * JC_BF16 / JC_F16: hn [T, d] and att [T, inner] in the storage type, big [T, max(3*inner floats,
 * dff storage values)] and an fp32 [T, inner] part the layer no longer uses (the size stays as it
 * was, so callers' workspaces keep fitting). JC_F16X3: big
 * [T, max(3*inner, dff)] and att [T, inner] floats and the split operand [T, 3*max(d, inner, dff)]
 * fp16. */
int64_t jc_c2_layer_workspace_bytes(int rows, int n, int d, int inner, int dff, int dtype);

/*
 * One Chronos-2 encoder layer in place on x [rows*n, d] fp32 (the per-layer stage of
 * Chronos2Forward.Plan, J/chronos2/tornado/Chronos2Forward.java:258-286; CPU CpuChronos2.forward,
 * J/chronos2/cpu/CpuChronos2.java:150-161):
 *   x += O_time(timeAttention(RoPE(QKV_time(rmsNorm(x)))))
 *   x += O_group(groupAttention(QKV_group(rmsNorm(x))))
 *   x += Wo(ReLU(Wi(rmsNorm(x))))
 * live [rows*n], table [n, dh] (jc_c2_rope_table), group_start/group_end [rows] as for
 * jc_c2_time_attention and jc_c2_group_attention (groups contiguous); workspace of
 * jc_c2_layer_workspace_bytes, 256-byte aligned. inner = heads*dh. d a multiple of 16, dh a multiple
 * of 16 and at most 64, dff a multiple of 16.
 * dtype JC_F32: everything in fp32. JC_BF16 / JC_F16: the GEMMs take the storage type with fp32
 * accumulation (the reference's FP16 GEMM modes, Chronos2Forward.java:377-409, GemmMode.HALF), both
 * attention cores read q|k|v and write their output in the storage type (fp32 arithmetic inside),
 * and x (the residual stream), the norms and the accumulations stay fp32. JC_F16X3 (no reference counterpart): every
 * GEMM runs on its operands' three-term fp16 splits (jc_split_f16x3; the norms, and the attention
 * kernels for 64-wide heads, write the split directly), with fp32 accumulation and fp32 outputs;
 * the attention, the norms and x are fp32, as in JC_F32, whose accuracy it keeps to about 2^-20 per
 * product (plus 2^-25 times the other operand where lo is subnormal, for operands below about
 * 2^-2).
 */
int jc_c2_layer(jc_ctx *ctx, float *x, const jc_c2_layer_weights *w, const int32_t *live, const float *table,
                const int32_t *group_start, const int32_t *group_end, void *workspace, int rows, int n, int d,
                int heads, int dh, int dff, float eps, int dtype);

/*
 * jc_c2_layer without a caller workspace: the layer runs in JC_C2_LAYER_STATIC_BYTES of device memory
 * the library holds on each GPU it runs on (resolved by jc_init, held until the process ends), and
 * the call allocates nothing (no hipMalloc, hipFree or allocating library routine). No counterpart
 * in the reference: it is for callers that cannot allocate (code under hipGraph capture, serving
 * loops, harnesses that forbid hipMalloc). Arguments and results are jc_c2_layer's; a call whose
 * jc_c2_layer_workspace_bytes exceeds JC_C2_LAYER_STATIC_BYTES returns JC_EINVAL (split the rows
 * over several calls). Every call on a GPU shares that GPU's scratch and leaves its contents behind
 * (the layer writes each part before reading it, so nothing needs clearing): calls that overlap on
 * one GPU, on any streams or contexts, race.
 */
#define JC_C2_LAYER_STATIC_BYTES (64u << 20)
int jc_c2_layer_static(jc_ctx *ctx, float *x, const jc_c2_layer_weights *w, const int32_t *live, const float *table,
                       const int32_t *group_start, const int32_t *group_end, int rows, int n, int d, int heads, int dh,
                       int dff, float eps, int dtype);

/*
 * bf16 / fp16 GEMM with fp32 accumulation: C[m, n] (+)= act(A[m, :k] . W[n, :k] + bias[n]), A and W
 * in the storage type `dtype` (JC_BF16 or JC_F16), bias fp32. c_dtype JC_F32: C fp32, any flags
 * (JC_GEMM_ACCUMULATE adds into C). c_dtype = dtype: C in the storage type, saturated to its finite
 * range (the reference's FP16 twins, Kernels.java:42-46), no ACCUMULATE. Replaces Kernels.gemmHalf
 * and the GemmEx FP16->FP32 path (J/tornado/Kernels.java:115-232; Chronos2Forward.java:377-409).
 *   k a multiple of 8, lda >= k and a multiple of 8, lda < 2^22, ldc >= n; a and w 16-byte aligned.
 */
int jc_linear_lp(jc_ctx *ctx, const void *a, int lda, const void *w, const float *bias, void *c, int ldc, int m,
                 int n, int k, int flags, int dtype, int c_dtype);

/* Kernels.rmsNorm with its twin output (J/tornado/Kernels.java:800-829): y in the storage type
 * `dtype` = x * (1 / sqrt(mean(x^2) + eps)) * w, x fp32; d a multiple of 4; 16-byte aligned.
 * dtype JC_F16X3 (no reference counterpart): y is fp16 [rows, 3d], the fp32 result's A-operand
 * split [hi | hi | lo] (jc_split_f16x3's layout), ready for a JC_F16X3 GEMM. */
int jc_rms_norm_lp(jc_ctx *ctx, const float *x, const float *w, void *y, int rows, int d, float eps, int dtype);

/* dst[i] = src[i] rounded to the storage type `dtype`, saturated to its finite range (Kernels.toHalf,
 * J/tornado/Kernels.java:887-895): for weights, converted once. */
int jc_to_lp(jc_ctx *ctx, const float *src, void *dst, int64_t count, int dtype);

/* ---- The rest of the Chronos-2 forward (fp32) ------------------------------------------------ */

/*
 * x [rows*n, d]: the encoder input from the patch embeddings emb [rows*(n-nreg), d] (each row's
 * context tokens then its future tokens) and the [REG] token reg [d] between them (NULL when
 * nreg = 0): Chronos2Kernels.assembleTokens (J/chronos2/tornado/Chronos2Kernels.java:66-85).
 * 0 <= nc, 0 <= nreg <= 1, nc + nreg <= n; d a multiple of 4; 16-byte aligned.
 */
int jc_c2_assemble(jc_ctx *ctx, const float *emb, const float *reg, float *x, int rows, int nc, int nreg, int n, int d);

/*
 * dec [rows*h, d] = the tokens fs..fs+h-1 of every row of y [rows*n, d]: Chronos2Kernels.gatherFuture
 * (J/chronos2/tornado/Chronos2Kernels.java:684-694). fs + h <= n; d a multiple of 4; 16-byte aligned.
 */
int jc_c2_gather_future(jc_ctx *ctx, const float *y, float *dec, int rows, int fs, int n, int h, int d);

/*
 * The forecast's host ends on the device. jc_c2_prep = ModelLayout.of's cut and live mask
 * (J/chronos2/ModelLayout.java:70-116) + ModelPrep.of (J/chronos2/ModelPrep.java:38-72, instanceNorm
 * 80-101, scaled/asinh 104-114) from the raw rows: row i of the outputs is input row order[i]
 * (order nullable: i), context [rows, ld_context] holds `steps` steps per row of which the last
 * min(steps, context_length) are kept and NaN-padded on the left to nc = ceil(kept / patch) whole
 * patches; future (nullable) [rows, ld_future] holds future_steps <= h*patch known steps. Writes
 * tokens [rows*(nc+h), 3*patch] (time encoding, arcsinh-scaled value or 0, observed flag), loc and
 * scale [rows], live [rows*(nc+nreg+h)] int32. Mean and std in double rounded to float, as the
 * reference; only the order of the double sums may differ from its sequential loop.
 */
int jc_c2_prep(jc_ctx *ctx, const float *context, int64_t ld_context, int steps, const float *future,
               int64_t ld_future, int future_steps, const int32_t *order, int rows, int context_length, int patch,
               int h, int nreg, float time_scale, int arcsinh, float *tokens, float *loc, float *scale,
               int32_t *live);

/*
 * ModelPrep.finish (J/chronos2/ModelPrep.java:117-143): out [order[i]][k][p*patch + s] =
 * sinh(raw[(i*h + p)*q*patch + k*patch + s]) * scale[i] + loc[i] (without sinh when arcsinh is 0),
 * rounded as the reference (float multiply, then float add). order nullable: i.
 */
int jc_c2_finish(jc_ctx *ctx, const float *raw, const float *loc, const float *scale, const int32_t *order, int rows,
                 int h, int q, int patch, int arcsinh, float *out);

/*
 * out [m, dout] = output(ReLU(hidden(x))) + residual(x): a Chronos-2 residual block (the input and
 * output patch embeddings), as Chronos2Forward.Plan.residual queues it
 * (J/chronos2/tornado/Chronos2Forward.java:306-311; CPU CpuChronos2.Residual.apply,
 * J/chronos2/cpu/CpuChronos2.java:57-69). x [m, din]; hidden [dff, din], output [dout, dff],
 * residual [dout, din] with optional fp32 biases; scratch [m, dff]. din, dff multiples of 16.
 */
int jc_c2_residual(jc_ctx *ctx, const float *x, int m, int din, const float *w_hidden, const float *b_hidden,
                   const float *w_output, const float *b_output, const float *w_residual, const float *b_residual,
                   int dff, int dout, float *scratch, float *out);

/* ---- The rest of the Timestral block (fp32 unless stated) ------------------------------------- */

/*
 * out [m, dout] = output(SiLU(hidden(x))) + residual(x): a Timestral ResidualBlock (the patch
 * embedding and the quantile head), as TimestralForward.Plan.residual queues it
 * (J/timestral/tornado/TimestralForward.java:397-401; CPU CpuTimestral.Residual.apply,
 * J/timestral/cpu/CpuTimestral.java:58-71). Arguments as jc_c2_residual.
 */
int jc_ts_residual(jc_ctx *ctx, const float *x, int m, int din, const float *w_hidden, const float *b_hidden,
                   const float *w_output, const float *b_output, const float *w_residual, const float *b_residual,
                   int dff, int dout, float *scratch, float *out);

/*
 * x [rows*n, d]: row r's encoder tokens t < enc from emb [rows*enc, d], its decoder tokens
 * enc <= t < n the forecast query [d]: TimestralKernels.assembleTokens
 * (J/timestral/tornado/TimestralKernels.java:53-69). d a multiple of 4; 16-byte aligned.
 */
int jc_ts_assemble(jc_ctx *ctx, const float *emb, const float *query, float *x, int rows, int enc, int n, int d);

/*
 * dec [rows*h, d] = the decoder tokens enc..enc+h-1 of every row of y [rows*n, d]:
 * TimestralKernels.gatherDecoder (J/timestral/tornado/TimestralKernels.java:581-590).
 * enc + h <= n; d a multiple of 4; 16-byte aligned.
 */
int jc_ts_gather_decoder(jc_ctx *ctx, const float *y, float *dec, int rows, int enc, int n, int h, int d);

/*
 * act [tokens, f] = SiLU(up[t][j]) * up[t][f + j] with up [tokens, 2f], computed in fp32:
 * Kernels.swiGlu and, for dtype JC_BF16 / JC_F16, Kernels.swiGluHalf with the result saturated to the
 * type's finite range (J/tornado/Kernels.java:832-856). up and act are both of `dtype`.
 * dtype JC_F16X3 (no reference counterpart): up fp32, act fp16 [tokens, 3f], the fp32 result's
 * A-operand split [hi | hi | lo] for a JC_F16X3 GEMM; f a multiple of 4, 16-byte alignment.
 */
int jc_swiglu(jc_ctx *ctx, const void *up, void *act, int64_t tokens, int f, int dtype);

/*
 * The block's host ends on the device. jc_ts_prep = BlockPrep.of (J/timestral/BlockPrep.java:40-75)
 * over the window of BlockLayout.of (J/timestral/BlockLayout.java:77-109): window [rows, w] fp32 and
 * observed [rows, w] bytes (0 = missing), w = encoder tokens * patch, 1 <= patch <= 64; known [rows]
 * int32 (nullable: no known rows) selects Scaler.instanceNorm (J/timestral/Scaler.java:87-110) over
 * the causal patch scaler (Scaler.java:40-64). Writes tokens [rows * w/patch, 2*patch] (scaled values
 * then missing flags), loc and scale [rows, w], and scaled [rows, w] (nullable). The double running
 * sums keep the reference's step order.
 */
int jc_ts_prep(jc_ctx *ctx, const float *window, const uint8_t *observed, int rows, int w, int patch,
               const int32_t *known, float minimum_scale, int use_asinh, float *tokens, float *scaled, float *loc,
               float *scale);

/*
 * jc_ts_finish = BlockPrep.finish (J/timestral/BlockPrep.java:77-101): on raw [rows, h*patch, q]
 * (the head's output), Quantiles.apply (J/timestral/Quantiles.java:52-77) with the per-level widths
 * `width` (host memory, q floats: widthFactor * dp as Quantiles holds them) around level `median`,
 * then Scaler.invert with loc / scale [rows, w] at step (context_patches - 1) * patch of each row and
 * Scaler.clampNonFinite over each step's q values. out [rows, h*patch, q]; out == raw is allowed.
 * q <= 32.
 */
int jc_ts_finish(jc_ctx *ctx, const float *raw, const float *loc, const float *scale, int rows, int w,
                 int context_patches, int h, int patch, int q, const float *width, int median, int use_asinh,
                 float *out);

#ifdef __cplusplus
}
#endif
#endif
