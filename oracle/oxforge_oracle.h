/*
 * oxforge_oracle.h -- CPU restatement of the OxideForge compute-core math.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline in bench.py.  Nothing in the product
 * (oxide-forge_amd/) links, loads or calls it; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may.
 *
 * Every function restates the arithmetic of one reference kernel, cited as
 * path:line under /root/reference (MeccBai/oxide-forge).  Conventions:
 *   - matrices are contiguous row-major f32;
 *   - GEMM accumulates in f64 and rounds once to f32;
 *   - row statistics (max/sum/mean/variance/dot) are taken in f64, and the
 *     per-element result is evaluated in f64 and rounded once to f32;
 *   - single-operation elementwise work (binary ops, scale, add_scalar,
 *     by-rows broadcast, transpose, copy) is evaluated in f32 with FMA
 *     contraction disabled, so it is bit-exact by construction.
 *
 * Extensions beyond the reference (kept reducible to it):
 *   - LayerNorm/RMSNorm take optional gamma/beta (NULL = reference path;
 *     gamma=1, beta=0 reproduces the reference formula exactly);
 *   - row kernels accept any cols (the reference asserts cols <= 1024);
 *   - orc_sum_cols is the column sum the reference obtains by
 *     transpose + sum_rows (linear.rs:267-272).
 *
 * Parity pinning of each function is described in the tests that exercise it
 * (tests/test_oracle_pins.py: closed forms, invariants, finite differences,
 * library routines; tests/test_golden.py: known answers from PyTorch float64
 * autograd in tests/golden/).  The reference ships no test data and cannot be
 * built here.
 */
#ifndef OXFORGE_ORACLE_H
#define OXFORGE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* BinaryOp (cuda.rs:3-10): Add, Sub, Mul, Div in #[repr(u8)] order. */
enum { ORC_ADD = 0, ORC_SUB = 1, ORC_MUL = 2, ORC_DIV = 3 };

/* Closures passed to slice_for_each (module.rs:56-64); numbering matches
 * forge_map_op in include/oxforge.h. */
enum {
    ORC_MAP_SCALE = 0,      /* x * p0          matrix.rs:31, span.rs:282   */
    ORC_MAP_ADD = 1,        /* x + p0          matrix.rs:35                */
    ORC_MAP_GELU = 2,       /* tanh GELU       linear.rs:30-33             */
    ORC_MAP_GELU_D = 3,     /* GELU'           linear.rs:49-56             */
    ORC_MAP_RELU = 4,       /* linear.rs:34-40 */
    ORC_MAP_RELU_D = 5,     /* linear.rs:57-63 */
    ORC_MAP_SILU = 6,       /* linear.rs:41    */
    ORC_MAP_SILU_D = 7,     /* linear.rs:64-67 */
    ORC_MAP_EXP_SHIFT = 8,  /* exp(x - p0)     vector.rs:50                */
    ORC_MAP_HALF_SQ = 9,    /* 0.5 * x * x     linear.rs:327               */
    ORC_MAP_IDENTITY = 10   /* x               linear.rs:29                */
};

void orc_set_threads(int threads);
int orc_get_threads(void);

/* C = op(A) * op(B); op(A) is [M,K], op(B) is [K,N].  trans_a: A stored
 * [K,M]; trans_b: B stored [N,K].  f64 accumulate (gemm.rs:15-129 is the
 * strict-fp32 semantic anchor; the TF32 rounding of gemm.rs:202-373 is
 * deliberately not mirrored). */
void orc_gemm(const float *A, const float *B, float *C, size_t M, size_t N,
              size_t K, int trans_a, int trans_b);
/* Same, result kept in f64 (error measurement). */
void orc_gemm_f64(const float *A, const float *B, double *C, size_t M,
                  size_t N, size_t K, int trans_a, int trans_b);

/* out[c*rows + r] = in[r*cols + c]  (layout.rs:29,46-51). */
void orc_transpose(const float *in, float *out, size_t rows, size_t cols);

/* Row softmax in place (row.rs:55-113). */
void orc_softmax_rows(float *x, size_t rows, size_t cols);
/* dx = p * (g - sum(p*g))  (row.rs:193-237). */
void orc_softmax_rows_backward(const float *p, const float *g, float *dx,
                               size_t rows, size_t cols);

/* LayerNorm in place (row.rs:115-177), population variance. */
void orc_layer_norm_rows(float *x, const float *gamma, const float *beta,
                         size_t rows, size_t cols, float eps);
/* LayerNorm backward (row.rs:239-347); dgamma/dbeta optional. */
void orc_layer_norm_backward(const float *x, const float *dy,
                             const float *gamma, float *dx, float *dgamma,
                             float *dbeta, size_t rows, size_t cols,
                             float eps);
/* RMSNorm in place (row.rs:349-396): x / sqrt(sum(x^2)/n + eps). */
void orc_rms_norm_rows(float *x, const float *gamma, size_t rows, size_t cols,
                       float eps);
/* RMSNorm backward (row.rs:398-468). */
void orc_rms_norm_backward(const float *x, const float *dy, const float *gamma,
                           float *dx, float *dgamma, size_t rows, size_t cols,
                           float eps);

/* Elementwise (elementwise.rs:5-79, row.rs:179-191). */
void orc_binary(const float *l, const float *r, float *o, size_t n, int op);
void orc_binary_assign(float *t, const float *r, size_t n, int op);
void orc_binary_assign_by_rows(float *m, const float *row, size_t rows,
                               size_t cols, int op);
void orc_map(float *x, size_t n, int op, float p0);

/* Reductions (row.rs:16-53, reduction.rs:4-130). */
void orc_sum_rows(const float *m, float *out, size_t rows, size_t cols);
void orc_sum_cols(const float *m, float *out, size_t rows, size_t cols);
float orc_reduce_sum(const float *x, size_t n);
float orc_reduce_max(const float *x, size_t n);

/* g = dy * act'(z): Linear::backward's derivative map and multiply
 * (linear.rs:254-265); act is an ORC_MAP_*_D derivative op. */
void orc_activation_backward(const float *dy, const float *z, float *g,
                             size_t n, int derivative_op);

/* slice_set_random (elementwise.rs:36-43) with the hash of common.rs:3-9. */
void orc_fill_random(float *x, size_t n, uint32_t seed);

/* Fills (elementwise.rs:23-34, row.rs:5-14). */
void orc_fill_seq(float *x, size_t n, int ascending);
void orc_causal_mask(float *m, size_t rows, size_t cols);

#ifdef __cplusplus
}
#endif
#endif
