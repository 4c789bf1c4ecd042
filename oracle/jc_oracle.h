/*
 * jc_oracle — CPU FP32 restatement of the reference's attention-stage oracle.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for libjitcast_hip: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it. Nothing in the product path
 * (jitcast_amd/, include/) may call it.
 *
 * Semantics follow the reference's CPU engines, which compute in FP32 storage with double
 * accumulation (dots, exp, sums in double; outputs rounded to float):
 *   - CpuChronos2.java:102-111   inverse frequencies
 *   - CpuChronos2.java:175-228   time attention with RoPE (unscaled scores), 284-304 softmaxValues
 *   - CpuChronos2.java:230-282   group attention (members by group id, ModelLayout.java:169-180)
 *   - Chronos2Forward.java:467-474  the host-built RoPE table
 *   - ModelLayout.java:70-116    the live mask
 *   - CpuTimestral.java:107-116  partial-RoPE inverse frequencies
 *   - CpuTimestral.java:190-259  time attention (1/sqrt(dh) scale, BlockLayout.timeAllowed 209-221)
 *   - CpuTimestral.java:261-314  variate attention (BlockLayout.variateAllowed 223-243)
 *   - CpuTimestral.java:156-161  the sigmoid output gate
 *   - Ops.java:33-88             linear, rmsNorm, relu, add
 *
 * One deliberate, documented difference: a Chronos-2 time-attention query with no live key at all
 * gets zeros (what the reference's device kernel writes, Chronos2Kernels.java:407-462), where the
 * CPU loop would divide 0 by 0. The reference model can never produce that case (REG and future
 * tokens are always live, ModelLayout.java:104-114); isolated-stage tests can.
 *
 * Build with -ffp-contract=off: Java never fuses a*b+c, and neither may this restatement.
 */
#ifndef JC_ORACLE_H
#define JC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* threads <= 0 means one per online CPU. */

/* Chronos-2 ------------------------------------------------------------------------------ */
void jco_c2_inv_freq(int dh, float theta, float *inv /* [dh/2] */);
void jco_c2_rope_table(int n, int dh, float theta, float *table /* [n*dh] */);
int jco_c2_time_attention(const float *qkv, float *out, const int32_t *live, int rows, int n, int heads, int dh,
                          int inner, float theta, int threads);
int jco_c2_group_attention(const float *qkv, float *out, const int32_t *live, const int32_t *group, int rows, int n,
                           int heads, int dh, int inner, int threads);
/* ModelLayout.of's live mask: window [rows * nc * patch] (NaN = missing), reg 0/1, h output patches. */
void jco_c2_live(const float *window, int rows, int nc, int patch, int reg, int h, int32_t *live /* [rows*n] */);

/* Timestral ------------------------------------------------------------------------------ */
void jco_ts_inv_freq(int dh, int rope_dim, float theta, float *inv /* [dh/2] */);
int jco_ts_time_attention(const float *qkv, float *out, const int32_t *key_valid /* [rows*enc] */,
                          const int32_t *known /* [rows] */, const int32_t *pos /* [rows*n], signed */, int rows,
                          int enc, int ll, int n, int heads, int dh, int d, int rope_dim, float theta, int threads);
int jco_ts_variate_attention(const float *qkv, float *out, const int32_t *key_valid, const int32_t *group,
                             const int32_t *role, int covariates, int rows, int enc, int n, int heads, int dh, int d,
                             int threads);
void jco_ts_gate(float *att, const float *g, int64_t count);

/* Shared operators (Ops.java) -------------------------------------------------------------- */
void jco_linear(const float *x, int rows, const float *w, const float *b, int in, int out, float *y, int threads);
void jco_rms_norm(const float *x, int rows, int cols, const float *w, float eps, float *y);
void jco_relu(float *x, int64_t count);
void jco_add(float *acc, const float *x, int64_t count);

#ifdef __cplusplus
}
#endif
#endif
