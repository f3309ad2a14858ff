/*
 * oxforge_oracle.c -- CPU restatement of the OxideForge compute-core math.
 *
 * TEST INFRASTRUCTURE ONLY (see oxforge_oracle.h): the parity checker and
 * the timed CPU baseline.  Built with -ffp-contract=off so every f32
 * expression rounds after each operation, like the reference's scalar code.
 */
#include "oxforge_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static int g_threads = 1;

void orc_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }
int orc_get_threads(void) { return g_threads; }

/* ---------------------------------------------------------------- threads */

typedef void (*row_fn)(void *ctx, size_t begin, size_t end);

typedef struct {
    row_fn fn;
    void *ctx;
    size_t begin, end;
} row_job;

static void *row_job_main(void *arg) {
    row_job *job = (row_job *)arg;
    job->fn(job->ctx, job->begin, job->end);
    return NULL;
}

/* Splits [0,n) into contiguous chunks, one per thread. */
static void parallel_rows(size_t n, row_fn fn, void *ctx) {
    int t = g_threads;
    if ((size_t)t > n) t = (int)n;
    if (t <= 1) {
        fn(ctx, 0, n);
        return;
    }
    pthread_t tid[256];
    row_job jobs[256];
    if (t > 256) t = 256;
    size_t chunk = (n + (size_t)t - 1) / (size_t)t;
    int launched = 0;
    for (int i = 0; i < t; i++) {
        size_t b = (size_t)i * chunk, e = b + chunk;
        if (b >= n) break;
        if (e > n) e = n;
        jobs[i].fn = fn;
        jobs[i].ctx = ctx;
        jobs[i].begin = b;
        jobs[i].end = e;
        if (pthread_create(&tid[i], NULL, row_job_main, &jobs[i]) != 0) {
            fn(ctx, b, e); /* run inline if a thread cannot start */
            jobs[i].fn = NULL;
        }
        launched = i + 1;
    }
    for (int i = 0; i < launched; i++)
        if (jobs[i].fn) pthread_join(tid[i], NULL);
}

/* ------------------------------------------------------------------- GEMM */

typedef struct {
    const float *A, *B;
    float *C;
    double *C64;
    size_t M, N, K;
    int ta, tb;
} gemm_ctx;

/* C[i,j] = sum_k opA[i,k] * opB[k,j], f64 accumulate.  The reference kernel
 * (gemm.rs:15-129 strict fp32; gemm.rs:202-373 TF32) overwrites C with the
 * product and takes no alpha/beta (gemm.rs:117-128, 362-372).  Every output
 * sums k = 0 .. K-1 in order; the loops are blocked over GEMM_RB rows and
 * GEMM_CB columns (each B row segment serves GEMM_RB rows from cache), which
 * changes no sum.  Work is split over blocks of GEMM_RB rows. */
#define GEMM_RB ((size_t)8)
#define GEMM_CB ((size_t)256)

static void gemm_rows(void *p, size_t b0, size_t b1) {
    gemm_ctx *g = (gemm_ctx *)p;
    const size_t M = g->M, N = g->N, K = g->K;
    double acc[GEMM_RB][GEMM_CB];
    for (size_t blk = b0; blk < b1; blk++) {
        const size_t i0 = blk * GEMM_RB, ni = i0 + GEMM_RB <= M ? GEMM_RB : M - i0;
        for (size_t j0 = 0; j0 < N; j0 += GEMM_CB) {
            const size_t nj = j0 + GEMM_CB <= N ? GEMM_CB : N - j0;
            for (size_t ii = 0; ii < ni; ii++)
                for (size_t jj = 0; jj < nj; jj++) acc[ii][jj] = 0.0;
            if (!g->tb) {
                for (size_t k = 0; k < K; k++) {
                    const float *brow = g->B + k * N + j0;
                    for (size_t ii = 0; ii < ni; ii++) {
                        const size_t i = i0 + ii;
                        const double a = g->ta ? (double)g->A[k * M + i]
                                               : (double)g->A[i * K + k];
                        for (size_t jj = 0; jj < nj; jj++) acc[ii][jj] += a * (double)brow[jj];
                    }
                }
            } else {
                /* B stored [N,K]: each output is a contiguous dot product. */
                for (size_t ii = 0; ii < ni; ii++) {
                    const size_t i = i0 + ii;
                    for (size_t jj = 0; jj < nj; jj++) {
                        const float *bcol = g->B + (j0 + jj) * K;
                        double s2 = 0.0;
                        for (size_t k = 0; k < K; k++) {
                            const double a = g->ta ? (double)g->A[k * M + i]
                                                   : (double)g->A[i * K + k];
                            s2 += a * (double)bcol[k];
                        }
                        acc[ii][jj] = s2;
                    }
                }
            }
            for (size_t ii = 0; ii < ni; ii++) {
                const size_t i = i0 + ii;
                if (g->C)
                    for (size_t jj = 0; jj < nj; jj++) g->C[i * N + j0 + jj] = (float)acc[ii][jj];
                if (g->C64)
                    for (size_t jj = 0; jj < nj; jj++) g->C64[i * N + j0 + jj] = acc[ii][jj];
            }
        }
    }
}

void orc_gemm(const float *A, const float *B, float *C, size_t M, size_t N,
              size_t K, int trans_a, int trans_b) {
    gemm_ctx g = {A, B, C, NULL, M, N, K, trans_a, trans_b};
    parallel_rows((M + GEMM_RB - 1) / GEMM_RB, gemm_rows, &g);
}

void orc_gemm_f64(const float *A, const float *B, double *C, size_t M,
                  size_t N, size_t K, int trans_a, int trans_b) {
    gemm_ctx g = {A, B, NULL, C, M, N, K, trans_a, trans_b};
    parallel_rows((M + GEMM_RB - 1) / GEMM_RB, gemm_rows, &g);
}

/* -------------------------------------------------------------- transpose */

typedef struct {
    const float *in;
    float *out;
    size_t rows, cols;
} transpose_ctx;

/* Bands of 32 input rows, 32 x 32 blocks within a band (pure data
 * movement: any order gives the same result). */
static void transpose_bands(void *p, size_t b0, size_t b1) {
    transpose_ctx *t = (transpose_ctx *)p;
    for (size_t b = b0; b < b1; b++) {
        const size_t r0 = b * 32, r1 = r0 + 32 < t->rows ? r0 + 32 : t->rows;
        for (size_t c0 = 0; c0 < t->cols; c0 += 32) {
            const size_t c1 = c0 + 32 < t->cols ? c0 + 32 : t->cols;
            for (size_t r = r0; r < r1; r++)
                for (size_t c = c0; c < c1; c++) t->out[c * t->rows + r] = t->in[r * t->cols + c];
        }
    }
}

void orc_transpose(const float *in, float *out, size_t rows, size_t cols) {
    /* layout.rs:29,46-51: out[c * rows + r] = in[r * cols + c]. */
    transpose_ctx t = {in, out, rows, cols};
    parallel_rows((rows + 31) / 32, transpose_bands, &t);
}

/* --------------------------------------------------------------- row ops */

typedef struct {
    float *x;
    const float *a, *b, *g;
    float *out;
    size_t cols;
    float eps;
} row_ctx;

/* row.rs:55-113: m = max_j x_j (identity f32::MIN for inactive lanes);
 * e_j = exp(x_j - m); y_j = e_j / sum(e). */
static void softmax_rows_fn(void *p, size_t r0, size_t r1) {
    row_ctx *c = (row_ctx *)p;
    for (size_t r = r0; r < r1; r++) {
        float *x = c->x + r * c->cols;
        double m = -FLT_MAX;
        for (size_t j = 0; j < c->cols; j++)
            if ((double)x[j] > m) m = (double)x[j];
        double s = 0.0;
        for (size_t j = 0; j < c->cols; j++) s += exp((double)x[j] - m);
        for (size_t j = 0; j < c->cols; j++)
            x[j] = (float)(exp((double)x[j] - m) / s);
    }
}

void orc_softmax_rows(float *x, size_t rows, size_t cols) {
    row_ctx c = {x, NULL, NULL, NULL, NULL, cols, 0.f};
    parallel_rows(rows, softmax_rows_fn, &c);
}

/* row.rs:193-237: s = sum_j p_j g_j; dx_j = p_j (g_j - s). */
static void softmax_bwd_fn(void *p, size_t r0, size_t r1) {
    row_ctx *c = (row_ctx *)p;
    for (size_t r = r0; r < r1; r++) {
        const float *pr = c->a + r * c->cols, *gr = c->b + r * c->cols;
        float *dx = c->out + r * c->cols;
        double s = 0.0;
        for (size_t j = 0; j < c->cols; j++) s += (double)pr[j] * (double)gr[j];
        for (size_t j = 0; j < c->cols; j++)
            dx[j] = (float)((double)pr[j] * ((double)gr[j] - s));
    }
}

void orc_softmax_rows_backward(const float *p, const float *g, float *dx,
                               size_t rows, size_t cols) {
    row_ctx c = {NULL, p, g, NULL, dx, cols, 0.f};
    parallel_rows(rows, softmax_bwd_fn, &c);
}

/* Mean and 1/sqrt(var + eps) of one row, as row.rs:130-170 computes them. */
static void ln_stats(const float *x, size_t n, float eps, double *mean,
                     double *rstd) {
    double s = 0.0;
    for (size_t j = 0; j < n; j++) s += (double)x[j];
    double mu = s / (double)n;
    double v = 0.0;
    for (size_t j = 0; j < n; j++) {
        double d = (double)x[j] - mu;
        v += d * d;
    }
    *mean = mu;
    *rstd = 1.0 / sqrt(v / (double)n + (double)eps);
}

/* row.rs:115-177; extension y = gamma_j * xhat_j + beta_j. */
static void layer_norm_fn(void *p, size_t r0, size_t r1) {
    row_ctx *c = (row_ctx *)p;
    for (size_t r = r0; r < r1; r++) {
        float *x = c->x + r * c->cols;
        double mu, rs;
        ln_stats(x, c->cols, c->eps, &mu, &rs);
        for (size_t j = 0; j < c->cols; j++) {
            double y = ((double)x[j] - mu) * rs;
            if (c->g) y *= (double)c->g[j];
            if (c->b) y += (double)c->b[j];
            x[j] = (float)y;
        }
    }
}

void orc_layer_norm_rows(float *x, const float *gamma, const float *beta,
                         size_t rows, size_t cols, float eps) {
    row_ctx c = {x, NULL, beta, gamma, NULL, cols, eps};
    parallel_rows(rows, layer_norm_fn, &c);
}

/* row.rs:239-347: recompute mu, r, xhat; A = sum g; B = sum g*xhat;
 * dx = r/n * (n*g - A - xhat*B), where g = dy (reference) or dy*gamma. */
static void layer_norm_bwd_fn(void *p, size_t r0, size_t r1) {
    row_ctx *c = (row_ctx *)p;
    const size_t n = c->cols;
    for (size_t r = r0; r < r1; r++) {
        const float *x = c->a + r * n, *dy = c->b + r * n;
        float *dx = c->out + r * n;
        double mu, rs;
        ln_stats(x, n, c->eps, &mu, &rs);
        double A = 0.0, B = 0.0;
        for (size_t j = 0; j < n; j++) {
            double g = (double)dy[j] * (c->g ? (double)c->g[j] : 1.0);
            double xh = ((double)x[j] - mu) * rs;
            A += g;
            B += g * xh;
        }
        for (size_t j = 0; j < n; j++) {
            double g = (double)dy[j] * (c->g ? (double)c->g[j] : 1.0);
            double xh = ((double)x[j] - mu) * rs;
            dx[j] = (float)(rs / (double)n * ((double)n * g - A - xh * B));
        }
    }
}

void orc_layer_norm_backward(const float *x, const float *dy,
                             const float *gamma, float *dx, float *dgamma,
                             float *dbeta, size_t rows, size_t cols,
                             float eps) {
    row_ctx c = {NULL, x, dy, gamma, dx, cols, eps};
    parallel_rows(rows, layer_norm_bwd_fn, &c);
    if (dgamma || dbeta) {
        /* dgamma_j = sum_rows dy * xhat; dbeta_j = sum_rows dy. */
        double *sg = (double *)calloc(cols, sizeof(double));
        double *sb = (double *)calloc(cols, sizeof(double));
        if (!sg || !sb) abort();
        for (size_t r = 0; r < rows; r++) {
            double mu, rs;
            ln_stats(x + r * cols, cols, eps, &mu, &rs);
            for (size_t j = 0; j < cols; j++) {
                double d = (double)dy[r * cols + j];
                sg[j] += d * ((double)x[r * cols + j] - mu) * rs;
                sb[j] += d;
            }
        }
        for (size_t j = 0; j < cols; j++) {
            if (dgamma) dgamma[j] = (float)sg[j];
            if (dbeta) dbeta[j] = (float)sb[j];
        }
        free(sg);
        free(sb);
    }
}

static double rms_of(const float *x, size_t n, float eps) {
    double q = 0.0;
    for (size_t j = 0; j < n; j++) q += (double)x[j] * (double)x[j];
    return sqrt(q / (double)n + (double)eps);
}

/* row.rs:349-396: y = x / sqrt(sum(x^2)/n + eps) -- a division by the
 * root; extension y = gamma_j * (x_j / rms). */
static void rms_norm_fn(void *p, size_t r0, size_t r1) {
    row_ctx *c = (row_ctx *)p;
    for (size_t r = r0; r < r1; r++) {
        float *x = c->x + r * c->cols;
        double rms = rms_of(x, c->cols, c->eps);
        for (size_t j = 0; j < c->cols; j++) {
            double y = (double)x[j] / rms;
            if (c->g) y *= (double)c->g[j];
            x[j] = (float)y;
        }
    }
}

void orc_rms_norm_rows(float *x, const float *gamma, size_t rows, size_t cols,
                       float eps) {
    row_ctx c = {x, NULL, NULL, gamma, NULL, cols, eps};
    parallel_rows(rows, rms_norm_fn, &c);
}

/* row.rs:398-468: q = sum x^2, d = sum x*g; inv = 1/sqrt(q/n + eps);
 * dx = g*inv - x * (d/n * inv^3), with g = dy (reference) or dy*gamma. */
static void rms_norm_bwd_fn(void *p, size_t r0, size_t r1) {
    row_ctx *c = (row_ctx *)p;
    const size_t n = c->cols;
    for (size_t r = r0; r < r1; r++) {
        const float *x = c->a + r * n, *dy = c->b + r * n;
        float *dx = c->out + r * n;
        double inv = 1.0 / rms_of(x, n, c->eps);
        double d = 0.0;
        for (size_t j = 0; j < n; j++)
            d += (double)x[j] * (double)dy[j] * (c->g ? (double)c->g[j] : 1.0);
        double corr = d / (double)n * inv * inv * inv;
        for (size_t j = 0; j < n; j++) {
            double g = (double)dy[j] * (c->g ? (double)c->g[j] : 1.0);
            dx[j] = (float)(g * inv - (double)x[j] * corr);
        }
    }
}

void orc_rms_norm_backward(const float *x, const float *dy, const float *gamma,
                           float *dx, float *dgamma, size_t rows, size_t cols,
                           float eps) {
    row_ctx c = {NULL, x, dy, gamma, dx, cols, eps};
    parallel_rows(rows, rms_norm_bwd_fn, &c);
    if (dgamma) {
        /* dgamma_j = sum_rows dy * x / rms. */
        double *sg = (double *)calloc(cols, sizeof(double));
        if (!sg) abort();
        for (size_t r = 0; r < rows; r++) {
            double inv = 1.0 / rms_of(x + r * cols, cols, eps);
            for (size_t j = 0; j < cols; j++)
                sg[j] += (double)dy[r * cols + j] * (double)x[r * cols + j] * inv;
        }
        for (size_t j = 0; j < cols; j++) dgamma[j] = (float)sg[j];
        free(sg);
    }
}

/* ------------------------------------------------------------ elementwise */

/* apply_binary (elementwise.rs:5-13), one f32 operation. */
static float apply_binary(float l, float r, int op) {
    switch (op) {
    case ORC_ADD: return l + r;
    case ORC_SUB: return l - r;
    case ORC_MUL: return l * r;
    default: return l / r;
    }
}

/* Element-wise ops run over chunks of ELEM_CHUNK elements on the worker
 * threads; each element is computed alone, so the split changes nothing. */
#define ELEM_CHUNK ((size_t)65536)

typedef struct {
    const float *l, *r;
    float *o;
    size_t n;
    int op;
    float p0;
} elem_ctx;

static void binary_chunks(void *p, size_t c0, size_t c1) {
    elem_ctx *e = (elem_ctx *)p;
    const size_t i1 = c1 * ELEM_CHUNK < e->n ? c1 * ELEM_CHUNK : e->n;
    for (size_t i = c0 * ELEM_CHUNK; i < i1; i++) e->o[i] = apply_binary(e->l[i], e->r[i], e->op);
}

void orc_binary(const float *l, const float *r, float *o, size_t n, int op) {
    elem_ctx e = {l, r, o, n, op, 0.f};
    parallel_rows((n + ELEM_CHUNK - 1) / ELEM_CHUNK, binary_chunks, &e);
}

void orc_binary_assign(float *t, const float *r, size_t n, int op) {
    elem_ctx e = {t, r, t, n, op, 0.f};
    parallel_rows((n + ELEM_CHUNK - 1) / ELEM_CHUNK, binary_chunks, &e);
}

/* row.rs:179-191: M[i] = M[i] op row[i mod cols]. */
void orc_binary_assign_by_rows(float *m, const float *row, size_t rows,
                               size_t cols, int op) {
    for (size_t i = 0; i < rows * cols; i++)
        m[i] = apply_binary(m[i], row[i % cols], op);
}

/* Activation constants (linear.rs:22-24), kept as the f32 values Rust uses. */
static const float GELU_SCALE = 0.7978846f;
static const float GELU_CUBIC = 0.044715f;

static float map_one(float x, int op, float p0) {
    double xd = (double)x;
    switch (op) {
    case ORC_MAP_SCALE: return x * p0;
    case ORC_MAP_ADD: return x + p0;
    case ORC_MAP_GELU: { /* linear.rs:30-33 */
        double inner = (double)GELU_SCALE * (xd + (double)GELU_CUBIC * xd * xd * xd);
        return (float)(0.5 * xd * (1.0 + tanh(inner)));
    }
    case ORC_MAP_GELU_D: { /* linear.rs:49-56 */
        double inner = (double)GELU_SCALE * (xd + (double)GELU_CUBIC * xd * xd * xd);
        double t = tanh(inner);
        double dq = (double)GELU_SCALE * 3.0 * (double)GELU_CUBIC;
        double inner_d = (double)GELU_SCALE + dq * xd * xd;
        return (float)(0.5 * (1.0 + t) + 0.5 * xd * (1.0 - t * t) * inner_d);
    }
    case ORC_MAP_RELU: return x > 0.f ? x : 0.f;      /* linear.rs:34-40 */
    case ORC_MAP_RELU_D: return x > 0.f ? 1.f : 0.f;  /* linear.rs:57-63 */
    case ORC_MAP_SILU: return (float)(xd / (1.0 + exp(-xd))); /* linear.rs:41 */
    case ORC_MAP_SILU_D: { /* linear.rs:64-67 */
        double e = exp(-xd);
        return (float)(1.0 / (1.0 + e) + xd * e / ((1.0 + e) * (1.0 + e)));
    }
    case ORC_MAP_EXP_SHIFT: return (float)exp(xd - (double)p0); /* vector.rs:50 */
    case ORC_MAP_HALF_SQ: return 0.5f * x * x;  /* linear.rs:327, f32 as written */
    default: return x;                          /* Identity, linear.rs:29 */
    }
}

static void map_chunks(void *p, size_t c0, size_t c1) {
    elem_ctx *e = (elem_ctx *)p;
    const size_t i1 = c1 * ELEM_CHUNK < e->n ? c1 * ELEM_CHUNK : e->n;
    for (size_t i = c0 * ELEM_CHUNK; i < i1; i++) e->o[i] = map_one(e->o[i], e->op, e->p0);
}

void orc_map(float *x, size_t n, int op, float p0) {
    elem_ctx e = {NULL, NULL, x, n, op, p0};
    parallel_rows((n + ELEM_CHUNK - 1) / ELEM_CHUNK, map_chunks, &e);
}

static void activation_backward_chunks(void *p, size_t c0, size_t c1) {
    elem_ctx *e = (elem_ctx *)p;
    const size_t i1 = c1 * ELEM_CHUNK < e->n ? c1 * ELEM_CHUNK : e->n;
    /* derivative = act'(z) rounded to f32, then gradient * derivative. */
    for (size_t i = c0 * ELEM_CHUNK; i < i1; i++)
        e->o[i] = e->l[i] * map_one(e->r[i], e->op, 0.f);
}

void orc_activation_backward(const float *dy, const float *z, float *g,
                             size_t n, int derivative_op) {
    elem_ctx e = {dy, z, g, n, derivative_op, 0.f};
    parallel_rows((n + ELEM_CHUNK - 1) / ELEM_CHUNK, activation_backward_chunks, &e);
}

/* ------------------------------------------------------------- reductions */

void orc_sum_rows(const float *m, float *out, size_t rows, size_t cols) {
    /* row.rs:16-53: s_r = sum_j M[r, j]. */
    for (size_t r = 0; r < rows; r++) {
        double s = 0.0;
        for (size_t j = 0; j < cols; j++) s += (double)m[r * cols + j];
        out[r] = (float)s;
    }
}

void orc_sum_cols(const float *m, float *out, size_t rows, size_t cols) {
    /* Column sums; the reference computes them as transpose followed by
     * sum_rows (linear.rs:267-272). */
    double *acc = (double *)calloc(cols ? cols : 1, sizeof(double));
    if (!acc) abort();
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < cols; j++) acc[j] += (double)m[r * cols + j];
    for (size_t j = 0; j < cols; j++) out[j] = (float)acc[j];
    free(acc);
}

float orc_reduce_sum(const float *x, size_t n) {
    /* reduction.rs:4-41 with the host loop of span.rs:361-385; an empty span
     * sums to 0 (span.rs:302-304). */
    double s = 0.0;
    for (size_t i = 0; i < n; i++) s += (double)x[i];
    return (float)s;
}

float orc_reduce_max(const float *x, size_t n) {
    /* reduction.rs:93-130; identity f32::MIN, also for an empty span
     * (span.rs:319-321). */
    float m = -FLT_MAX;
    for (size_t i = 0; i < n; i++)
        if (x[i] > m) m = x[i];
    return m;
}

/* ------------------------------------------------------------------ fills */

void orc_fill_seq(float *x, size_t n, int ascending) {
    /* elementwise.rs:23-34: i (Sequence) or len - i (Reserve). */
    for (size_t i = 0; i < n; i++)
        x[i] = ascending ? (float)i : (float)(n - i);
}

void orc_causal_mask(float *m, size_t rows, size_t cols) {
    /* row.rs:5-14: M[r, c] = -inf for c > r. */
    for (size_t r = 0; r < rows; r++)
        for (size_t c = r + 1; c < cols; c++) m[r * cols + c] = -INFINITY;
}

/* common.rs:3-9: x += x << 13; x -= x >> 17; x *= x << 5 (wrapping u32). */
static uint32_t ref_hash(uint32_t x) {
    x += x << 13;
    x -= x >> 17;
    x *= x << 5;
    return x;
}

void orc_fill_random(float *x, size_t n, uint32_t seed) {
    /* elementwise.rs:40-41: (rand as f32) / (u32::MAX as f32). */
    for (size_t i = 0; i < n; i++)
        x[i] = (float)ref_hash(seed + (uint32_t)i) / (float)UINT32_MAX;
}
