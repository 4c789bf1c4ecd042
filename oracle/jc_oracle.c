/*
 * jc_oracle.c — CPU FP32 restatement of the reference's attention-stage oracle.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product). Each function cites the reference
 * file:line whose semantics it restates; the header lists them all. Compile with
 * -ffp-contract=off so no a*b+c is fused (Java evaluates them separately).
 */
#include "jc_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---- a parallel-for over [0, jobs), like the reference's IntStream.range(..).parallel() ---- */

typedef void (*job_fn)(void *arg, int64_t job);

typedef struct {
    job_fn fn;
    void *arg;
    int64_t jobs;
    int64_t next; /* claimed with __atomic_fetch_add */
} pool_t;

static void *pool_worker(void *p) {
    pool_t *pool = (pool_t *)p;
    for (;;) {
        int64_t j = __atomic_fetch_add(&pool->next, 1, __ATOMIC_RELAXED);
        if (j >= pool->jobs) {
            return NULL;
        }
        pool->fn(pool->arg, j);
    }
}

static int resolve_threads(int threads) {
    if (threads > 0) {
        return threads;
    }
    /* the process's CPU share when the environment states it (a GPU box's per-GPU share), else
       every online CPU */
    const char *env = getenv("OMP_NUM_THREADS");
    if (env && atoi(env) > 0) {
        return atoi(env);
    }
    long c = sysconf(_SC_NPROCESSORS_ONLN);
    return c > 0 ? (int)c : 1;
}

static void parallel_for(int64_t jobs, int threads, job_fn fn, void *arg) {
    pool_t pool = {fn, arg, jobs, 0};
    int t = resolve_threads(threads);
    if (t > jobs) {
        t = (int)(jobs > 0 ? jobs : 1);
    }
    if (t <= 1) {
        pool_worker(&pool);
        return;
    }
    pthread_t *tids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)(t - 1));
    int started = 0;
    for (int i = 0; i < t - 1; i++) {
        if (pthread_create(&tids[i], NULL, pool_worker, &pool) == 0) {
            started++;
        } else {
            break;
        }
    }
    pool_worker(&pool);
    for (int i = 0; i < started; i++) {
        pthread_join(tids[i], NULL);
    }
    free(tids);
}

/* ---- Chronos-2 -------------------------------------------------------------------------- */

/* CpuChronos2.java:102-111: invFreq[i] = 1 / (float) pow(theta, (float)(2i) / (float) dh), in float. */
void jco_c2_inv_freq(int dh, float theta, float *inv) {
    for (int i = 0; i < dh / 2; i++) {
        float e = (float)(2 * i) / (float)dh;
        inv[i] = 1.0f / (float)pow((double)theta, (double)e);
    }
}

/* Chronos2Forward.java:467-474: table[p*dh + e] = cos((float)p * invFreq[e]), [.. + dh/2 + e] = sin. */
void jco_c2_rope_table(int n, int dh, float theta, float *table) {
    int half = dh / 2;
    float *inv = (float *)malloc(sizeof(float) * (size_t)half);
    jco_c2_inv_freq(dh, theta, inv);
    for (int p = 0; p < n; p++) {
        for (int e = 0; e < half; e++) {
            float a = (float)p * inv[e];
            table[(size_t)p * dh + e] = (float)cos((double)a);
            table[(size_t)p * dh + half + e] = (float)sin((double)a);
        }
    }
    free(inv);
}

/*
 * CpuChronos2.java:215-228 / CpuTimestral.java:250-259: x*cos + rotate_half(x)*sin on one head
 * vector; dims e and e+dh/2 rotate together by (float)pos * inv[e] (cos and sin in double, rounded).
 */
static void rope_vec(const float *src, float *dst, int dh, const float *inv, int pos) {
    int half = dh / 2;
    for (int e = 0; e < half; e++) {
        float f = (float)pos * inv[e];
        float c = (float)cos((double)f), s = (float)sin((double)f);
        float a = src[e], b = src[half + e];
        dst[e] = a * c + -b * s;
        dst[half + e] = b * c + a * s;
    }
}

typedef struct {
    const float *qkv;
    const float *q; /* rotated q, [rows*n*inner] */
    const float *k; /* rotated k */
    float *out;
    const int32_t *live;
    int n, heads, dh, inner;
} c2_time_args;

/* CpuChronos2.java:190-211 for one (row, head) job, with softmaxValues (284-304). */
static void c2_time_job(void *p, int64_t job) {
    const c2_time_args *a = (const c2_time_args *)p;
    int n = a->n, heads = a->heads, dh = a->dh, inner = a->inner;
    int i = (int)(job / heads), hh = (int)(job % heads);
    double *pr = (double *)malloc(sizeof(double) * (size_t)n);
    for (int t = 0; t < n; t++) {
        double max = -INFINITY;
        size_t qo = ((size_t)i * n + t) * inner + (size_t)hh * dh;
        for (int s = 0; s < n; s++) {
            if (!a->live[(size_t)i * n + s]) {
                pr[s] = -INFINITY;
                continue;
            }
            size_t ko = ((size_t)i * n + s) * inner + (size_t)hh * dh;
            double dot = 0;
            for (int e = 0; e < dh; e++) {
                dot += (double)a->q[qo + e] * (double)a->k[ko + e];
            }
            pr[s] = dot;
            if (dot > max) {
                max = dot;
            }
        }
        /* softmaxValues: base = i*n*3*inner, stride 3*inner, vOff = 2*inner + hh*dh */
        double sum = 0;
        for (int s = 0; s < n; s++) {
            pr[s] = pr[s] == -INFINITY ? 0 : exp(pr[s] - max);
            sum += pr[s];
        }
        size_t base = (size_t)i * n * 3 * inner + 2 * (size_t)inner + (size_t)hh * dh;
        for (int e = 0; e < dh; e++) {
            double acc = 0;
            for (int s = 0; s < n; s++) {
                if (pr[s] != 0) {
                    acc += pr[s] * (double)a->qkv[base + (size_t)s * 3 * inner + e];
                }
            }
            /* no live key: zeros, as the reference's device kernel writes (see header) */
            a->out[qo + e] = sum > 0 ? (float)(acc / sum) : 0.0f;
        }
    }
    free(pr);
}

/* CpuChronos2.java:175-213: RoPE into separate q and k, then attention per (row, head). */
int jco_c2_time_attention(const float *qkv, float *out, const int32_t *live, int rows, int n, int heads, int dh,
                          int inner, float theta, int threads) {
    if (rows < 0 || n < 0 || heads < 1 || dh < 2 || dh % 2 || inner < heads * dh) {
        return -1;
    }
    size_t tokens = (size_t)rows * n;
    float *q = (float *)malloc(sizeof(float) * tokens * inner);
    float *k = (float *)malloc(sizeof(float) * tokens * inner);
    float *inv = (float *)malloc(sizeof(float) * (size_t)(dh / 2));
    if (!q || !k || !inv) {
        free(q);
        free(k);
        free(inv);
        return -2;
    }
    jco_c2_inv_freq(dh, theta, inv);
    for (int i = 0; i < rows; i++) {
        for (int t = 0; t < n; t++) {
            size_t o = ((size_t)i * n + t) * 3 * inner;
            size_t d = ((size_t)i * n + t) * inner;
            for (int hh = 0; hh < heads; hh++) {
                rope_vec(qkv + o + (size_t)hh * dh, q + d + (size_t)hh * dh, dh, inv, t);
                rope_vec(qkv + o + inner + (size_t)hh * dh, k + d + (size_t)hh * dh, dh, inv, t);
            }
        }
    }
    memset(out, 0, sizeof(float) * tokens * inner);
    c2_time_args a = {qkv, q, k, out, live, n, heads, dh, inner};
    parallel_for((int64_t)rows * heads, threads, c2_time_job, &a);
    free(q);
    free(k);
    free(inv);
    return 0;
}

typedef struct {
    const float *qkv;
    float *out;
    const int32_t *live;
    const int32_t *mstart; /* members of row i: mlist[mstart[i] .. mstart[i]+mcount[i]) */
    const int32_t *mcount;
    const int32_t *mlist;
    int rows, n, heads, dh, inner;
} c2_group_args;

/* CpuChronos2.java:239-280 for one token slot t. */
static void c2_group_job(void *p, int64_t job) {
    const c2_group_args *a = (const c2_group_args *)p;
    int t = (int)job, n = a->n, heads = a->heads, dh = a->dh, inner = a->inner;
    size_t stride = 3 * (size_t)inner;
    double *pr = (double *)malloc(sizeof(double) * (size_t)(a->rows > 0 ? a->rows : 1));
    for (int i = 0; i < a->rows; i++) {
        const int32_t *m = a->mlist + a->mstart[i];
        int mc = a->mcount[i];
        for (int hh = 0; hh < heads; hh++) {
            size_t qo = ((size_t)i * n + t) * stride + (size_t)hh * dh;
            double max = -INFINITY;
            for (int jj = 0; jj < mc; jj++) {
                int j = m[jj];
                if (!a->live[(size_t)j * n + t]) {
                    pr[jj] = -INFINITY;
                    continue;
                }
                size_t ko = ((size_t)j * n + t) * stride + inner + (size_t)hh * dh;
                double dot = 0;
                for (int e = 0; e < dh; e++) {
                    dot += (double)a->qkv[qo + e] * (double)a->qkv[ko + e];
                }
                pr[jj] = dot;
                if (dot > max) {
                    max = dot;
                }
            }
            size_t oo = ((size_t)i * n + t) * inner + (size_t)hh * dh;
            if (max == -INFINITY) {
                continue; /* no valid key in the group at this slot: zeros */
            }
            double sum = 0;
            for (int jj = 0; jj < mc; jj++) {
                pr[jj] = pr[jj] == -INFINITY ? 0 : exp(pr[jj] - max);
                sum += pr[jj];
            }
            for (int e = 0; e < dh; e++) {
                double acc = 0;
                for (int jj = 0; jj < mc; jj++) {
                    if (pr[jj] != 0) {
                        acc += pr[jj] * (double)a->qkv[((size_t)m[jj] * n + t) * stride + 2 * (size_t)inner +
                                                       (size_t)hh * dh + e];
                    }
                }
                a->out[oo + e] = (float)(acc / sum);
            }
        }
    }
    free(pr);
}

/*
 * The rows of each row's group in ascending order (ModelLayout.java:169-180), as a CSR list:
 * rows with equal ids share one member list.
 */
static int build_members(const int32_t *group, int rows, int32_t **mstart, int32_t **mcount, int32_t **mlist) {
    int32_t *order = (int32_t *)malloc(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
    *mstart = (int32_t *)malloc(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
    *mcount = (int32_t *)malloc(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
    *mlist = order;
    if (!order || !*mstart || !*mcount) {
        return -2;
    }
    /* stable order by group id, then row: an insertion-free counting pass over distinct ids */
    int32_t *seen = (int32_t *)malloc(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
    int ng = 0, k = 0;
    for (int i = 0; i < rows; i++) {
        int found = 0;
        for (int g = 0; g < ng; g++) {
            if (seen[g] == group[i]) {
                found = 1;
                break;
            }
        }
        if (found) {
            continue;
        }
        seen[ng++] = group[i];
        int start = k;
        for (int j = i; j < rows; j++) {
            if (group[j] == group[i]) {
                order[k++] = j;
            }
        }
        for (int j = start; j < k; j++) {
            (*mstart)[order[j]] = start;
            (*mcount)[order[j]] = k - start;
        }
    }
    free(seen);
    return 0;
}

/* CpuChronos2.java:230-282: attention across the rows of each group, per slot; no RoPE. */
int jco_c2_group_attention(const float *qkv, float *out, const int32_t *live, const int32_t *group, int rows, int n,
                           int heads, int dh, int inner, int threads) {
    if (rows < 0 || n < 0 || heads < 1 || dh < 1 || inner < heads * dh) {
        return -1;
    }
    int32_t *mstart, *mcount, *mlist;
    if (build_members(group, rows, &mstart, &mcount, &mlist) != 0) {
        free(mstart);
        free(mcount);
        free(mlist);
        return -2;
    }
    memset(out, 0, sizeof(float) * (size_t)rows * n * inner);
    c2_group_args a = {qkv, out, live, mstart, mcount, mlist, rows, n, heads, dh, inner};
    parallel_for(n, threads, c2_group_job, &a);
    free(mstart);
    free(mcount);
    free(mlist);
    return 0;
}

/* ModelLayout.java:104-114: a context patch is live if any of its steps is observed; REG and future always. */
void jco_c2_live(const float *window, int rows, int nc, int patch, int reg, int h, int32_t *live) {
    int n = nc + reg + h;
    for (int i = 0; i < rows; i++) {
        for (int p = 0; p < nc; p++) {
            int any = 0;
            for (int s = p * patch; s < (p + 1) * patch; s++) {
                any |= !isnan(window[(size_t)i * nc * patch + s]);
            }
            live[(size_t)i * n + p] = any;
        }
        for (int p = nc; p < n; p++) {
            live[(size_t)i * n + p] = 1;
        }
    }
}

/* ---- Timestral -------------------------------------------------------------------------- */

/* CpuTimestral.java:107-116: the first rope_dim/2 frequencies 1/(float)pow(theta, 2i/rope_dim), 0 after. */
void jco_ts_inv_freq(int dh, int rope_dim, float theta, float *inv) {
    for (int i = 0; i < dh / 2; i++) {
        inv[i] = 0.0f;
    }
    for (int i = 0; i < rope_dim / 2; i++) {
        float e = (float)(2 * i) / (float)rope_dim;
        inv[i] = 1.0f / (float)pow((double)theta, (double)e);
    }
}

/* BlockLayout.java:209-221 (known = covariates && role == KNOWN, passed per row). */
static int ts_time_allowed(const int32_t *key_valid, const int32_t *known, int row, int q, int k, int enc, int ll) {
    if (q < enc) {
        if (k >= enc) {
            return 0;
        }
        return k == q || (key_valid[(size_t)row * enc + k] && (k <= q || known[row]));
    }
    if (k < enc) {
        return k < ll && key_valid[(size_t)row * enc + k];
    }
    return k <= q;
}

typedef struct {
    const float *qkv, *q, *k;
    float *out;
    const int32_t *key_valid, *known;
    int n, enc, ll, heads, dh, d;
} ts_time_args;

/* CpuTimestral.java:207-241 for one (row, head) job. */
static void ts_time_job(void *p, int64_t job) {
    const ts_time_args *a = (const ts_time_args *)p;
    int n = a->n, heads = a->heads, dh = a->dh, d = a->d;
    int i = (int)(job / heads), hh = (int)(job % heads);
    double scale = 1.0 / sqrt((double)dh);
    double *pr = (double *)malloc(sizeof(double) * (size_t)n);
    for (int t = 0; t < n; t++) {
        double max = -INFINITY;
        size_t qo = ((size_t)i * n + t) * d + (size_t)hh * dh;
        for (int s = 0; s < n; s++) {
            if (!ts_time_allowed(a->key_valid, a->known, i, t, s, a->enc, a->ll)) {
                pr[s] = -INFINITY;
                continue;
            }
            size_t ko = ((size_t)i * n + s) * d + (size_t)hh * dh;
            double dot = 0;
            for (int e = 0; e < dh; e++) {
                dot += (double)a->q[qo + e] * (double)a->k[ko + e];
            }
            pr[s] = dot * scale;
            if (pr[s] > max) {
                max = pr[s];
            }
        }
        double sum = 0;
        for (int s = 0; s < n; s++) {
            pr[s] = pr[s] == -INFINITY ? 0 : exp(pr[s] - max);
            sum += pr[s];
        }
        for (int e = 0; e < dh; e++) {
            double acc = 0;
            for (int s = 0; s < n; s++) {
                if (pr[s] != 0) {
                    acc += pr[s] * (double)a->qkv[((size_t)i * n + s) * 3 * d + 2 * (size_t)d + (size_t)hh * dh + e];
                }
            }
            a->out[qo + e] = (float)(acc / sum);
        }
    }
    free(pr);
}

/* CpuTimestral.java:190-243: RoPE at each token's position, then masked attention per (row, head). */
int jco_ts_time_attention(const float *qkv, float *out, const int32_t *key_valid, const int32_t *known,
                          const int32_t *pos, int rows, int enc, int ll, int n, int heads, int dh, int d, int rope_dim,
                          float theta, int threads) {
    if (rows < 0 || n < enc || heads < 1 || dh < 2 || dh % 2 || d < heads * dh || ll > enc) {
        return -1;
    }
    size_t tokens = (size_t)rows * n;
    float *q = (float *)malloc(sizeof(float) * tokens * d);
    float *k = (float *)malloc(sizeof(float) * tokens * d);
    float *inv = (float *)malloc(sizeof(float) * (size_t)(dh / 2));
    if (!q || !k || !inv) {
        free(q);
        free(k);
        free(inv);
        return -2;
    }
    jco_ts_inv_freq(dh, rope_dim, theta, inv);
    for (int i = 0; i < rows; i++) {
        for (int t = 0; t < n; t++) {
            int ps = pos[(size_t)i * n + t];
            size_t o = ((size_t)i * n + t) * 3 * d;
            size_t dd = ((size_t)i * n + t) * d;
            for (int hh = 0; hh < heads; hh++) {
                rope_vec(qkv + o + (size_t)hh * dh, q + dd + (size_t)hh * dh, dh, inv, ps);
                rope_vec(qkv + o + d + (size_t)hh * dh, k + dd + (size_t)hh * dh, dh, inv, ps);
            }
        }
    }
    memset(out, 0, sizeof(float) * tokens * d);
    ts_time_args a = {qkv, q, k, out, key_valid, known, n, enc, ll, heads, dh, d};
    parallel_for((int64_t)rows * heads, threads, ts_time_job, &a);
    free(q);
    free(k);
    free(inv);
    return 0;
}

typedef struct {
    const float *qkv;
    float *out;
    const int32_t *key_valid, *group, *role;
    const int32_t *mstart, *mcount, *mlist;
    int covariates, rows, enc, n, heads, dh, d;
} ts_variate_args;

/* BlockLayout.java:224-243 (role 0 = TARGET, 2 = KNOWN; BlockInput.java:35-37). */
static int ts_variate_allowed(const ts_variate_args *a, int slot, int q, int k) {
    if (a->group[q] != a->group[k]) {
        return 0;
    }
    if (q == k) {
        return 1;
    }
    if (slot < a->enc && !a->key_valid[(size_t)k * a->enc + slot]) {
        return 0;
    }
    if (a->covariates) {
        if (a->role[q] != 0 && a->role[k] == 0) {
            return 0;
        }
        if (a->role[q] == 2 && a->role[k] != 2) {
            return 0;
        }
    }
    return 1;
}

/* CpuTimestral.java:275-312 for one token slot t. */
static void ts_variate_job(void *p, int64_t job) {
    const ts_variate_args *a = (const ts_variate_args *)p;
    int t = (int)job, n = a->n, heads = a->heads, dh = a->dh, d = a->d;
    size_t stride = 3 * (size_t)d;
    double scale = 1.0 / sqrt((double)dh);
    double *pr = (double *)malloc(sizeof(double) * (size_t)(a->rows > 0 ? a->rows : 1));
    for (int i = 0; i < a->rows; i++) {
        const int32_t *m = a->mlist + a->mstart[i];
        int mc = a->mcount[i];
        for (int hh = 0; hh < heads; hh++) {
            size_t qo = ((size_t)i * n + t) * stride + (size_t)hh * dh;
            double max = -INFINITY;
            for (int jj = 0; jj < mc; jj++) {
                int j = m[jj];
                if (!ts_variate_allowed(a, t, i, j)) {
                    pr[jj] = -INFINITY;
                    continue;
                }
                size_t ko = ((size_t)j * n + t) * stride + d + (size_t)hh * dh;
                double dot = 0;
                for (int e = 0; e < dh; e++) {
                    dot += (double)a->qkv[qo + e] * (double)a->qkv[ko + e];
                }
                pr[jj] = dot * scale;
                if (pr[jj] > max) {
                    max = pr[jj];
                }
            }
            double sum = 0;
            for (int jj = 0; jj < mc; jj++) {
                pr[jj] = pr[jj] == -INFINITY ? 0 : exp(pr[jj] - max);
                sum += pr[jj];
            }
            for (int e = 0; e < dh; e++) {
                double acc = 0;
                for (int jj = 0; jj < mc; jj++) {
                    if (pr[jj] != 0) {
                        acc += pr[jj] *
                               (double)a->qkv[((size_t)m[jj] * n + t) * stride + 2 * (size_t)d + (size_t)hh * dh + e];
                    }
                }
                a->out[((size_t)i * n + t) * d + (size_t)hh * dh + e] = (float)(acc / sum);
            }
        }
    }
    free(pr);
}

/* CpuTimestral.java:261-314: attention across the rows of each series, per slot; no RoPE. */
int jco_ts_variate_attention(const float *qkv, float *out, const int32_t *key_valid, const int32_t *group,
                             const int32_t *role, int covariates, int rows, int enc, int n, int heads, int dh, int d,
                             int threads) {
    if (rows < 0 || n < enc || heads < 1 || dh < 1 || d < heads * dh) {
        return -1;
    }
    int32_t *mstart, *mcount, *mlist;
    if (build_members(group, rows, &mstart, &mcount, &mlist) != 0) {
        free(mstart);
        free(mcount);
        free(mlist);
        return -2;
    }
    memset(out, 0, sizeof(float) * (size_t)rows * n * d);
    ts_variate_args a = {qkv, out, key_valid, group, role, mstart, mcount, mlist, covariates, rows, enc, n, heads, dh, d};
    parallel_for(n, threads, ts_variate_job, &a);
    free(mstart);
    free(mcount);
    free(mlist);
    return 0;
}

/* CpuTimestral.java:156-161: att[i] = att[i] * (float) sigmoid(g[i]), sigmoid in double (Ops.java:71-73). */
void jco_ts_gate(float *att, const float *g, int64_t count) {
    for (int64_t i = 0; i < count; i++) {
        att[i] = att[i] * (float)(1.0 / (1.0 + exp(-(double)g[i])));
    }
}

/* ---- Ops.java ----------------------------------------------------------------------------- */

typedef struct {
    const float *x, *w, *b;
    float *y;
    int rows, in, out;
} linear_args;

#define LINEAR_CHUNK 16 /* Ops.java:31: rows per parallel task */

static void linear_job(void *p, int64_t chunk) {
    const linear_args *a = (const linear_args *)p;
    int end = (int)((chunk + 1) * LINEAR_CHUNK < a->rows ? (chunk + 1) * LINEAR_CHUNK : a->rows);
    for (int r = (int)chunk * LINEAR_CHUNK; r < end; r++) {
        const float *xr = a->x + (size_t)r * a->in;
        for (int o = 0; o < a->out; o++) {
            const float *wr = a->w + (size_t)o * a->in;
            double acc = 0;
            for (int i = 0; i < a->in; i++) {
                acc += (double)xr[i] * (double)wr[i];
            }
            a->y[(size_t)r * a->out + o] = (float)(a->b ? acc + (double)a->b[o] : acc);
        }
    }
}

/* Ops.java:33-50: y[r] = W x[r] + b, W is [out, in], double accumulation. */
void jco_linear(const float *x, int rows, const float *w, const float *b, int in, int out, float *y, int threads) {
    linear_args a = {x, w, b, y, rows, in, out};
    parallel_for((rows + LINEAR_CHUNK - 1) / LINEAR_CHUNK, threads, linear_job, &a);
}

/* Ops.java:53-68: x * (float)(1/sqrt(mean(x^2) + eps)) * w per row. */
void jco_rms_norm(const float *x, int rows, int cols, const float *w, float eps, float *y) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * cols;
        double ss = 0;
        for (int c = 0; c < cols; c++) {
            ss += (double)xr[c] * (double)xr[c];
        }
        float inv = (float)(1.0 / sqrt(ss / cols + (double)eps));
        for (int c = 0; c < cols; c++) {
            y[(size_t)r * cols + c] = w ? xr[c] * inv * w[c] : xr[c] * inv;
        }
    }
}

/* Ops.java:79-83 */
void jco_relu(float *x, int64_t count) {
    for (int64_t i = 0; i < count; i++) {
        /* Math.max(x, 0f): NaN stays NaN */
        x[i] = isnan(x[i]) ? x[i] : (x[i] > 0.0f ? x[i] : 0.0f);
    }
}

/* Ops.java:84-88 */
void jco_add(float *acc, const float *x, int64_t count) {
    for (int64_t i = 0; i < count; i++) {
        acc[i] += x[i];
    }
}
