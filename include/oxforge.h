/*
 * oxforge.h -- C ABI of the MI355X-native OxideForge compute core.
 *
 * This is the drop-in boundary that replaces the cuda-oxide context, module
 * and stream routing of the reference (src/cuda.rs, src/cuda/runtime.rs,
 * src/cuda/span.rs and the #[cuda_module] kernel module
 * src/cuda/device/module.rs:6-263).  Host code above it (the C++ classes in
 * oxide-forge_amd/csrc/net, or a Rust shim) keeps the reference's
 * CudaRuntime / Matrix / Vector / executor signatures.
 *
 * Conventions
 *   - Every entry point returns forge_status; nothing aborts inside the
 *     library.  forge_last_error() gives a thread-local detail string.
 *   - Buffers are f32, contiguous, row-major, passed as forge_slice
 *     {ptr,len} by value -- the #[repr(C)] DeviceSliceDescriptor /
 *     DeviceSliceMutDescriptor of span.rs:7-11,45-49.  A slice shorter than
 *     the shape it is used with is FORGE_EINVAL (the reference kernels
 *     silently skip out-of-range indices instead).
 *   - Kernel launches are asynchronous on `stream`; stream == NULL means the
 *     runtime's primary stream (CudaRuntime::stream, runtime.rs:116-118).
 *   - A runtime is not thread-safe; serialise calls on one runtime.
 *   - Device code is loaded from a gfx950 code object with hipModuleLoad and
 *     launched with hipModuleLaunchKernel.
 */
#ifndef OXFORGE_H
#define OXFORGE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum forge_status {
    FORGE_OK = 0,
    FORGE_EINVAL = 1,    /* shape / argument precondition violated       */
    FORGE_ENOMEM = 2,    /* device or host allocation failed             */
    FORGE_EHIP = 3,      /* a HIP runtime call failed                    */
    FORGE_ENOMODULE = 4, /* code object missing or a kernel not found    */
    FORGE_ENODEV = 5,    /* no HIP device / requested device absent      */
    FORGE_EIO = 6        /* a file could not be opened, read or written  */
} forge_status;

typedef struct forge_runtime forge_runtime;
typedef struct forge_stream forge_stream;

/* span.rs:45-49 DeviceSliceMutDescriptor<f32> / span.rs:7-11
 * DeviceSliceDescriptor<f32>; const-ness is by convention of each entry. */
typedef struct forge_slice {
    float *ptr;
    size_t len;
} forge_slice;

/* The same descriptor over u32 elements (DeviceSliceMutDescriptor<u32>, the
 * result buffer of compare_vectors, reduction.rs:132-136). */
typedef struct forge_slice_u32 {
    uint32_t *ptr;
    size_t len;
} forge_slice_u32;

/* BinaryOp, #[repr(u8)] (cuda.rs:3-10). */
typedef enum forge_binary_op {
    FORGE_ADD = 0,
    FORGE_SUB = 1,
    FORGE_MUL = 2,
    FORGE_DIV = 3
} forge_binary_op;

/* The closures the reference passes to slice_for_each (module.rs:56-64),
 * one device functor each.  p0 is the captured scalar where there is one. */
typedef enum forge_map_op {
    FORGE_MAP_SCALE = 0,     /* x * p0           matrix.rs:31, span.rs:282 */
    FORGE_MAP_ADD = 1,       /* x + p0           matrix.rs:35              */
    FORGE_MAP_GELU = 2,      /* Activation::Gelu.forward   linear.rs:30-33 */
    FORGE_MAP_GELU_D = 3,    /* Activation::Gelu.derivative linear.rs:49-56 */
    FORGE_MAP_RELU = 4,      /* linear.rs:34-40 */
    FORGE_MAP_RELU_D = 5,    /* linear.rs:57-63 */
    FORGE_MAP_SILU = 6,      /* linear.rs:41    */
    FORGE_MAP_SILU_D = 7,    /* linear.rs:64-67 */
    FORGE_MAP_EXP_SHIFT = 8, /* exp(x - p0)      vector.rs:50              */
    FORGE_MAP_HALF_SQ = 9,   /* 0.5 * x * x      linear.rs:327             */
    FORGE_MAP_IDENTITY = 10  /* x                linear.rs:29              */
} forge_map_op;

/* Activation applied in a GEMM epilogue (Activation, linear.rs:12-19). */
typedef enum forge_activation {
    FORGE_ACT_IDENTITY = 0,
    FORGE_ACT_GELU = 1,
    FORGE_ACT_RELU = 2,
    FORGE_ACT_SILU = 3
} forge_activation;

/* ------------------------------------------------------------ lifecycle */

/* CudaRuntime::new (runtime.rs:34-45): selects `device`, creates the primary
 * non-blocking stream and loads the code object.  module_path NULL means
 * the code object next to this library (oxforge_kernels.hsaco) or the path
 * in $OXFORGE_KERNELS. */
forge_status forge_runtime_create(int device, const char *module_path,
                                  forge_runtime **out);
/* Drop of CudaRuntime: frees pooled buffers, streams and the module. */
forge_status forge_runtime_destroy(forge_runtime *rt);
/* CudaRuntime::sync (runtime.rs:112-114); stream NULL = primary. */
forge_status forge_sync(forge_runtime *rt, forge_stream *stream);
/* Number of HIP devices visible (0 on a host without a GPU). */
forge_status forge_device_count(int *count);
/* Human-readable status and the last error detail of this thread. */
const char *forge_status_string(forge_status status);
const char *forge_last_error(void);
/* Device properties used by the bench: CU count, LDS bytes per workgroup,
 * peak clock in kHz and the architecture name (e.g. "gfx950"). */
forge_status forge_device_props(forge_runtime *rt, int *cu_count,
                                size_t *lds_bytes, int *clock_khz,
                                char *arch, size_t arch_len);

/* -------------------------------------------------------------- streams */

/* create_extra_streams (runtime.rs:188-192): n new streams, each forked
 * from the primary (they wait for everything queued on it so far). */
forge_status forge_streams_create(forge_runtime *rt, size_t n,
                                  forge_stream **out);
/* fork_streams (runtime.rs:196-200): each stream waits on the primary. */
forge_status forge_streams_fork(forge_runtime *rt, size_t n,
                                forge_stream *const *streams);
/* join_streams (runtime.rs:202-206): the primary waits on each stream. */
forge_status forge_streams_join(forge_runtime *rt, size_t n,
                                forge_stream *const *streams);
/* CudaStream::join(other) as used at linear.rs:126 and matrix.rs:128:
 * `waiter` waits for everything queued on `signaler` (NULL = primary).
 * An event dependency; the host does not block. */
forge_status forge_stream_wait(forge_runtime *rt, forge_stream *waiter,
                               forge_stream *signaler);
forge_status forge_stream_destroy(forge_runtime *rt, forge_stream *stream);
/* Diagnostic (no reference counterpart): the length in floats of the
 * scratch workspace the library holds for `stream` (NULL = primary), which
 * multi-pass kernels (column sums, norm backward partial rows, split-K
 * GEMMs, reductions) grow on first need; 0 if nothing on that stream has
 * needed one.  Lets a test show that an entry point allocated nothing. */
forge_status forge_stream_workspace_floats(forge_runtime *rt, forge_stream *stream,
                                           size_t *floats);

/* --------------------------------------------------------------- events */

/* Device-side timing on a stream.  No reference counterpart: the reference
 * times with host wall clock around runtime.sync() (main.rs:54-65).  Used by
 * the benchmark to time kernels on the stream they are launched on. */
typedef struct forge_event forge_event;
forge_status forge_event_create(forge_runtime *rt, forge_event **out);
forge_status forge_event_record(forge_runtime *rt, forge_stream *stream,
                                forge_event *ev);
/* Milliseconds between two recorded events; waits for `end`. */
forge_status forge_event_elapsed_ms(forge_runtime *rt, forge_event *start,
                                    forge_event *end, float *ms);
forge_status forge_event_destroy(forge_runtime *rt, forge_event *ev);

/* --------------------------------------------------------------- memory */

/* get_uninit_buffer (runtime.rs:47-55): pops an exact-size buffer from the
 * pool or allocates one.  n == 0 yields {NULL, 0}. */
forge_status forge_alloc(forge_runtime *rt, size_t n, forge_slice *out);
/* get_zerod_buffer (runtime.rs:67-71): as forge_alloc, then zero-filled on
 * the primary stream. */
forge_status forge_alloc_zeroed(forge_runtime *rt, size_t n, forge_slice *out);
/* recycle_buffer (runtime.rs:98-110): returns a buffer to the exact-size
 * pool; pending uses must be ordered on the primary stream. */
forge_status forge_recycle(forge_runtime *rt, forge_slice buf);
/* Drop of a DeviceBuffer: releases the memory to the device. */
forge_status forge_free(forge_runtime *rt, forge_slice buf);
/* reserve_buffers (runtime.rs:75-91). */
forge_status forge_reserve(forge_runtime *rt, size_t n, size_t count);
/* Buffers currently held by the pool for size n (for tests). */
forge_status forge_pool_count(forge_runtime *rt, size_t n, size_t *count);

/* get_u32_uninit_buffer (runtime.rs:57-60): a new uninitialised buffer of n
 * u32 values.  Not pooled (the reference allocates it on its stream and
 * frees it on drop); n == 0 yields {NULL, 0}. */
forge_status forge_alloc_u32(forge_runtime *rt, size_t n, forge_slice_u32 *out);
/* Drop of a DeviceBuffer<u32>: waits for the primary stream, then releases
 * the memory. */
forge_status forge_free_u32(forge_runtime *rt, forge_slice_u32 buf);
/* to_host_vec of a DeviceBuffer<u32> (vector.rs:134): device -> host;
 * blocks until done. */
forge_status forge_memcpy_d2h_u32(forge_runtime *rt, uint32_t *dst,
                                  forge_slice_u32 src, size_t n);

/* DeviceBuffer::from_host (matrix.rs:107): host -> device, ordered on the
 * primary stream; returns once the host buffer may be reused. */
forge_status forge_memcpy_h2d(forge_runtime *rt, forge_slice dst,
                              const float *src, size_t n);
/* to_host_vec (matrix.rs:11-13): device -> host; blocks until done. */
forge_status forge_memcpy_d2h(forge_runtime *rt, float *dst, forge_slice src,
                              size_t n);
/* memcpy_dtod_async (runtime.rs:160-167, span.rs:450-457). */
forge_status forge_memcpy_d2d(forge_runtime *rt, forge_stream *stream,
                              forge_slice dst, forge_slice src, size_t n);
/* zero_async (runtime.rs:69): a fill kernel, never hipMemsetAsync, so the
 * call is safe inside a captured graph. */
forge_status forge_fill(forge_runtime *rt, forge_stream *stream,
                        forge_slice x, float value);

/* -------------------------------------------------------------- kernels */

/* matrix_multiply / matrix_multiply_into_on (matrix.rs:113-176, kernel
 * gemm.rs:202-373): C[M,N] = A[M,K] * B[K,N], row-major, C overwritten.
 * True fp32 (v_mfma_f32_16x16x4_f32; v_mfma_f32_32x32x2_f32 in the guarded
 * fallback), not the reference's TF32.  Any M, N, K >= 0 (the reference
 * asserts multiples of 16).  Outputs whose tiles leave three quarters of the
 * CUs idle, with K >= 2048, are computed as K slices summed in slice order
 * (deterministic; the choice depends only on the shape and alignment, the
 * same for this call and forge_gemm_ex_f32). */
forge_status forge_gemm_f32(forge_runtime *rt, forge_stream *stream,
                            forge_slice A, forge_slice B, forge_slice C,
                            size_t M, size_t N, size_t K);

/* Fused GEMM used by the executors (no reference counterpart as one call;
 * it fuses the launch sequence of Linear::affine_on + activate_on,
 * linear.rs:185-230, and of Linear::learn_on, linear.rs:393-415):
 *   op(A) = trans_a ? A^T (A stored [K,M]) : A (stored [M,K])
 *   op(B) = trans_b ? B^T (B stored [N,K]) : B (stored [K,N])
 *   Z = alpha * op(A) op(B)
 *   if bias:     Z = Z + bias[col]           (by-rows add, rows.rs:8-42)
 *   if residual: Z = Z + residual            (binary_assign, matrix.rs:38)
 *   if aux_mul:  Z = Z * aux_mul, or Z * act'(aux_mul) (linear.rs:254-265)
 *   if pre_out:  pre_out = Z
 *   Y = act(Z)
 *   if update:   C = C - update_scale * Y    (SGD, linear.rs:383-384)
 *   else         C = Y
 * Every optional operand is a slice with ptr == NULL when absent.  Each step
 * is one rounded f32 operation, so the result is bit-identical to the
 * reference's separate launches given the same product. */
typedef struct forge_gemm_epilogue {
    float alpha;           /* 1.0f for a plain product                     */
    forge_slice bias;      /* [N] or {NULL,0}                              */
    forge_slice residual;  /* [M,N] or {NULL,0}                            */
    forge_slice aux_mul;   /* [M,N] or {NULL,0}                            */
    forge_slice pre_out;   /* [M,N] or {NULL,0}: stores Z before act       */
    int activation;        /* forge_activation                            */
    int update;            /* 0: C = Y; 1: C = C - update_scale * Y        */
    float update_scale;    /* learning rate for update == 1                */
    int aux_activation;    /* 0: Z = Z * aux_mul; a forge_activation A:
                              Z = Z * A'(aux_mul), the derivative step of
                              Linear::backward (linear.rs:254-265)         */
    /* Row statistics: a parameterless RMSNorm (norm.rs:50-69) of the rows
     * of one product's result folded into the next product.  The divisor of
     * row r is d_r = sqrt(S_r / row_n + row_eps), S_r the sum of the
     * row_parts values row_parts_in[r * row_parts ...] (the row_sumsq_out of
     * the product that formed those rows).  row_div bit 0: Z = Z / d_r right
     * after alpha (op(A) op(B) with A's rows normalised equals the product
     * of the raw rows divided by d_r); bit 1: the residual is divided by d_r
     * before it is added.                                                  */
    forge_slice row_parts_in; /* [M * row_parts] or {NULL,0}               */
    size_t row_parts;
    size_t row_n;
    float row_eps;
    int row_div;
    /* [M * ceil(N / 32)] or {NULL,0}: for each row, the sums of the squares
     * of the stored C values over each 32-column block.                    */
    forge_slice row_sumsq_out;
    /* [N] or {NULL,0}: the column sums of the stored C values (a bias
     * gradient, linear.rs:267-272); col_sums_param ([N] or {NULL,0}) takes
     * param -= col_sums_lr * sum (linear.rs:385-390) in the same pass.  The
     * sums come from per-tile partials written by the product's epilogue and
     * one final pass over them, in an order fixed by the shape.            */
    forge_slice col_sums_out;
    forge_slice col_sums_param;
    float col_sums_lr;
    /* [M] or {NULL,0}: Z = Z - row_sub[r] right after alpha (and the
     * row_div divide).  With alpha = s, row_sub = s * D and aux_mul = P on
     * the product dP = dO V^T this forms the softmax backward
     * dS = P * (dP - D) * s (row.rs:216-236, D_r = sum_j P_rj dP_rj) in the
     * product's epilogue, D coming from forge_*_norm_bwd_sgd_dot.          */
    forge_slice row_sub;
} forge_gemm_epilogue;

forge_status forge_gemm_ex_f32(forge_runtime *rt, forge_stream *stream,
                               int trans_a, int trans_b, forge_slice A,
                               forge_slice B, forge_slice C, size_t M,
                               size_t N, size_t K,
                               const forge_gemm_epilogue *epilogue);

/* The sum of count (1 to 3) products under one fused epilogue:
 *   C = epilogue(sum_z op(A_z) op(B_z)),
 * each A_z [M, K] and B_z [K, N] after op (trans_a / trans_b as in
 * forge_gemm_ex_f32).  It replaces the reference's chain of input-gradient
 * products that accumulate onto one matrix (QkvProjection::backward_self's
 * dX += G_i W_i^T for Q, K and V, attention.rs:104-144): one launch, one
 * read and one write of C instead of one per product.  The result is
 * bit-identical to forge_gemm_ex_f32 on the operands concatenated along K
 * (K' = count K): with an unguarded tile, no K split and no row statistics
 * or column sums in the epilogue it is one launch whose slabs come from
 * each product in turn; otherwise the operands are first copied into that
 * concatenation. */
forge_status forge_gemm_sum_f32(forge_runtime *rt, forge_stream *stream, int trans_a,
                                int trans_b, size_t count, const forge_slice *A,
                                const forge_slice *B, forge_slice C, size_t M, size_t N,
                                size_t K, const forge_gemm_epilogue *epilogue);

/* Tuning entry point (no reference counterpart): forge_gemm_f32 with an
 * explicit plain tile instance: "<BM>x<BN>x<BK>_x" for the unguarded
 * four-wave tiles (128x256x32, 128x128x32, 128x64x32, 64x128x32, 64x64x32),
 * "64x128x32_x8" for the unguarded eight-wave tile, or "64x64x16_2x2_g" for
 * the guarded one.
 * Unguarded tiles require M % BM == N % BN == K % BK == 0, 16-byte aligned
 * operands and K, N <= 2^21; anything else is FORGE_EINVAL.  A suffix
 * "@<n>" (1..16) lets a CU hold at most n of the launch's workgroups (the
 * launch reserves extra LDS); results do not depend on it.  Used by the
 * benchmark's tile sweep. */
forge_status forge_gemm_f32_tile(forge_runtime *rt, forge_stream *stream,
                                 const char *tile_tag, forge_slice A,
                                 forge_slice B, forge_slice C, size_t M,
                                 size_t N, size_t K);

/* Tuning entry point (no reference counterpart): forge_gemm_f32 computed as
 * `splits` K slices (one batched launch) plus a reduction in slice order,
 * with tile "128x128x32_x", "128x64x32_x", "64x128x32_x", "64x64x32_x" or
 * "64x128x32_x8".
 * Requires M % BM == N % BN == K % (splits * BK) == 0, 16-byte aligned
 * operands and 1 <= splits <= 8.  Used by the benchmark's sweep. */
forge_status forge_gemm_f32_split(forge_runtime *rt, forge_stream *stream,
                                  const char *tile_tag, int splits, forge_slice A,
                                  forge_slice B, forge_slice C, size_t M, size_t N,
                                  size_t K);

/* Testing entry point (no reference counterpart): forge_gemm_ex_f32 through
 * the fused-epilogue instance of one named tile ("128x128x32_x",
 * "128x64x32_x", "64x128x32_x", "64x64x32_x", "64x128x32_x8" or
 * "64x64x16_2x2_g"), so every instance the dispatcher can pick is testable
 * at small shapes.  The same
 * shape, alignment and "@<n>" rules as forge_gemm_f32_tile. */
forge_status forge_gemm_ex_f32_tile(forge_runtime *rt, forge_stream *stream,
                                    const char *tile_tag, int trans_a, int trans_b,
                                    forge_slice A, forge_slice B, forge_slice C,
                                    size_t M, size_t N, size_t K,
                                    const forge_gemm_epilogue *epilogue);

/* Diagnostic entry point (no reference counterpart): the name of the kernel
 * that forge_gemm_f32 (fused = 0) or forge_gemm_ex_f32 (fused = 1) launches
 * for a product of this shape and these transposes with 16-byte aligned
 * operands, written NUL-terminated to name (cap bytes; a name that does not
 * fit is FORGE_EINVAL).  A launch that lets a CU hold at most n of its
 * workgroups is reported as "<kernel>@<n>", a product computed as K slices
 * as "<batched slice kernel>/split<N>".  Lets benchmarks and profiles name
 * the kernel they measure. */
forge_status forge_gemm_kernel_name(forge_runtime *rt, int trans_a, int trans_b,
                                    size_t M, size_t N, size_t K, int fused,
                                    char *name, size_t cap);

/* One product of a batch: operands and its own fused epilogue. */
typedef struct forge_gemm_problem {
    forge_slice A, B, C;
    forge_gemm_epilogue epilogue;
} forge_gemm_problem;

/* `count` products of the same shape and transposes in one launch, each as
 * forge_gemm_ex_f32 would compute it (bit-identical; shapes that call splits
 * in K, and products with row statistics or column sums, run one product at
 * a time).  Replaces the three
 * forked streams of the Q/K/V projections (attention.rs:65-94) and of their
 * weight updates (attention.rs:104-144): one launch fills the device without
 * the cross-queue event latency of a fork and join. */
forge_status forge_gemm_batch_f32(forge_runtime *rt, forge_stream *stream,
                                  int trans_a, int trans_b, size_t M, size_t N,
                                  size_t K, size_t count,
                                  const forge_gemm_problem *problems);

/* matrix_transpose (convert.rs:17-63 -> layout.rs:8-55):
 * out[c,r] = in[r,c]; in is [rows,cols]. Bit-exact. */
forge_status forge_transpose_f32(forge_runtime *rt, forge_stream *stream,
                                 forge_slice in, forge_slice out, size_t rows,
                                 size_t cols);

/* Matrix::softmax_rows (norm.rs:8-24 -> row.rs:55-113), in place. */
forge_status forge_softmax_rows(forge_runtime *rt, forge_stream *stream,
                                forge_slice x, size_t rows, size_t cols);
/* softmax_rows_backward (norm.rs:73-101 -> row.rs:193-237):
 * dx = p * (g - sum(p * g)).  dx may not alias p or g. */
forge_status forge_softmax_rows_bwd(forge_runtime *rt, forge_stream *stream,
                                    forge_slice p, forge_slice g,
                                    forge_slice dx, size_t rows, size_t cols);

/* softmax_rows_backward followed by Matrix::scale, fused: the score
 * gradient of attention backward (attention.rs:302-304),
 * dx = (p * (g - sum(p * g))) * scale, two roundings as in the reference. */
forge_status forge_softmax_rows_bwd_scaled(forge_runtime *rt,
                                           forge_stream *stream, forge_slice p,
                                           forge_slice g, forge_slice dx,
                                           size_t rows, size_t cols,
                                           float scale);

/* Matrix::layer_norm (norm.rs:26-48 -> row.rs:115-177), in place.
 * gamma/beta ({NULL,0} = reference path) are the affine extension. */
forge_status forge_layer_norm_rows(forge_runtime *rt, forge_stream *stream,
                                   forge_slice x, forge_slice gamma,
                                   forge_slice beta, size_t rows, size_t cols,
                                   float eps);
/* Matrix::layer_norm with the result written to y (y == x is the in-place
 * call; otherwise y must not overlap x).  Lets a caller that keeps the
 * pre-norm matrix skip the clone the reference makes first
 * (attention.rs:258-281, encoder.rs:114-131). */
forge_status forge_layer_norm_rows_out(forge_runtime *rt, forge_stream *stream,
                                       forge_slice x, forge_slice y,
                                       forge_slice gamma, forge_slice beta,
                                       size_t rows, size_t cols, float eps);
/* layer_norm_backward (norm.rs:103-127 -> row.rs:239-347).  dgamma/dbeta
 * ({NULL,0} to skip) receive column sums over all rows. */
forge_status forge_layer_norm_bwd(forge_runtime *rt, forge_stream *stream,
                                  forge_slice x, forge_slice dy,
                                  forge_slice gamma, forge_slice dx,
                                  forge_slice dgamma, forge_slice dbeta,
                                  size_t rows, size_t cols, float eps);
/* forge_layer_norm_bwd followed by the SGD step of the norm's own
 * parameters, as the training step applies it (the affine extension's
 * gamma/beta take Linear::learn's update, linear.rs:385-390): dx is computed
 * with the gamma given, then gamma -= lr * dgamma and beta -= lr * dbeta
 * (each a rounded product then a rounded difference, bit-identical to
 * forge_layer_norm_bwd then forge_sgd_update) in the final column-sum pass,
 * so the two separate update launches disappear.  gamma and beta (updated in
 * place) and the gradient outputs dgamma/dbeta are each optional. */
forge_status forge_layer_norm_bwd_sgd(forge_runtime *rt, forge_stream *stream,
                                      forge_slice x, forge_slice dy, forge_slice gamma,
                                      forge_slice beta, forge_slice dx,
                                      forge_slice dgamma, forge_slice dbeta,
                                      size_t rows, size_t cols, float eps, float lr);
/* forge_layer_norm_bwd_sgd that also writes, for each row r,
 *   dot[r] = dot_scale * sum_c dx[r, c] * (x[r, c] - sub[r, c]).
 * Used by the attention backward (attention.rs:283-321): with x the
 * attention's pre-norm output P V + X, sub its residual input X and dx the
 * gradient at that output (dO), dot is dot_scale * sum_c dO_rc (P V)_rc =
 * dot_scale * sum_j P_rj dP_rj with dP = dO V^T -- the row term of the
 * softmax backward (row.rs:216-236) from the [S, H] operands instead of the
 * [S, S] ones, so the dP product can form dS in its epilogue
 * (forge_gemm_epilogue row_sub).  dx and the column sums are those of
 * forge_layer_norm_bwd_sgd, bit for bit.  sub [rows, cols] may not overlap
 * dx, nor dot [rows] any matrix operand (FORGE_EINVAL). */
forge_status forge_layer_norm_bwd_sgd_dot(forge_runtime *rt, forge_stream *stream,
                                          forge_slice x, forge_slice dy, forge_slice gamma,
                                          forge_slice beta, forge_slice dx,
                                          forge_slice dgamma, forge_slice dbeta,
                                          forge_slice sub, forge_slice dot, size_t rows,
                                          size_t cols, float eps, float lr, float dot_scale);
/* forge_layer_norm_bwd that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, checks and results (bit-identical) as
 * forge_layer_norm_bwd; the dgamma/dbeta partial rows go to a device scratch
 * array of 2,162,688 floats (8.25 MiB) that each GPU holds until the process
 * ends, instead of the stream's workspace.  Shapes whose partial rows need
 * more are FORGE_EINVAL.  The need grows with the number of partial rows,
 * one per workgroup (16-byte-aligned rows with cols % 4 == 0 and cols <=
 * 2048) or per wave (other rows) of a grid of at most one or two workgroups
 * per CU ($OXFORGE_NORM_BWD_BLOCKS overrides it).  On a device of up to 256
 * CUs (MI355X) without that override, every row count fits up to 2048
 * columns for aligned rows and up to 1024 for others.  The array is shared by every call
 * on one GPU, from every runtime and stream: calls that overlap on one GPU
 * race and must be serialised by the caller.  Nothing in it needs to start
 * at zero (every partial row is written before it is read). */
forge_status forge_layer_norm_bwd_noalloc(forge_runtime *rt, forge_stream *stream,
                                          forge_slice x, forge_slice dy,
                                          forge_slice gamma, forge_slice dx,
                                          forge_slice dgamma, forge_slice dbeta,
                                          size_t rows, size_t cols, float eps);
/* Matrix::rms_norm (norm.rs:50-69 -> row.rs:349-396), in place. */
forge_status forge_rms_norm_rows(forge_runtime *rt, forge_stream *stream,
                                 forge_slice x, forge_slice gamma, size_t rows,
                                 size_t cols, float eps);
/* Matrix::rms_norm with the result written to y (as forge_layer_norm_rows_out). */
forge_status forge_rms_norm_rows_out(forge_runtime *rt, forge_stream *stream,
                                     forge_slice x, forge_slice y, forge_slice gamma,
                                     size_t rows, size_t cols, float eps);
/* rms_norm_backward (norm.rs:129-158 -> row.rs:398-468). */
forge_status forge_rms_norm_bwd(forge_runtime *rt, forge_stream *stream,
                                forge_slice x, forge_slice dy,
                                forge_slice gamma, forge_slice dx,
                                forge_slice dgamma, size_t rows, size_t cols,
                                float eps);
/* forge_rms_norm_bwd followed by gamma -= lr * dgamma in its final
 * column-sum pass (as forge_layer_norm_bwd_sgd). */
forge_status forge_rms_norm_bwd_sgd(forge_runtime *rt, forge_stream *stream,
                                    forge_slice x, forge_slice dy, forge_slice gamma,
                                    forge_slice dx, forge_slice dgamma, size_t rows,
                                    size_t cols, float eps, float lr);
/* forge_rms_norm_bwd_sgd with the row dot of forge_layer_norm_bwd_sgd_dot. */
forge_status forge_rms_norm_bwd_sgd_dot(forge_runtime *rt, forge_stream *stream,
                                        forge_slice x, forge_slice dy, forge_slice gamma,
                                        forge_slice dx, forge_slice dgamma, forge_slice sub,
                                        forge_slice dot, size_t rows, size_t cols, float eps,
                                        float lr, float dot_scale);

/* matrix_binary / vector_binary (matrix.rs:194-219 -> elementwise.rs:45-56):
 * o = l op r over n elements.  Bit-exact. */
forge_status forge_binary(forge_runtime *rt, forge_stream *stream,
                          forge_slice l, forge_slice r, forge_slice o,
                          size_t n, forge_binary_op op);
/* binary_assign (matrix.rs:38-64 -> elementwise.rs:58-68): t = t op r. */
forge_status forge_binary_assign(forge_runtime *rt, forge_stream *stream,
                                 forge_slice t, forge_slice r, size_t n,
                                 forge_binary_op op);
/* binary_assign_by_rows (rows.rs:8-42 -> row.rs:179-191):
 * M[i] = M[i] op row[i mod cols]. */
forge_status forge_binary_assign_by_rows(forge_runtime *rt,
                                         forge_stream *stream, forge_slice m,
                                         forge_slice row, size_t rows,
                                         size_t cols, forge_binary_op op);
/* for_each (span.rs:261-279 -> elementwise.rs:70-79): x = f(x). */
forge_status forge_map(forge_runtime *rt, forge_stream *stream, forge_slice x,
                       size_t n, forge_map_op op, float p0);

/* The SGD step of a bias or norm parameter (linear.rs:385-390: clone the
 * gradient, scale it by lr, subtract) in one pass: param = param - lr * grad,
 * the same two roundings.  Bit-exact. */
forge_status forge_sgd_update(forge_runtime *rt, forge_stream *stream,
                              forge_slice param, forge_slice grad, size_t n,
                              float lr);

/* Linear::backward's derivative step (linear.rs:254-265: clone, map
 * activation.derivative, multiply) in one pass: g = dy * act'(z). */
forge_status forge_activation_backward(forge_runtime *rt, forge_stream *stream,
                                       forge_slice dy, forge_slice z,
                                       forge_slice g, size_t n,
                                       forge_activation activation);

/* matrix_sum_rows (rows.rs:45-88 -> row.rs:16-53): out[r] = sum_j M[r,j]. */
forge_status forge_sum_rows(forge_runtime *rt, forge_stream *stream,
                            forge_slice m, forge_slice out, size_t rows,
                            size_t cols);
/* Column sums, replacing the transpose + sum_rows pair of the bias
 * gradient (linear.rs:267-272): out[c] = sum_r M[r,c]. */
forge_status forge_sum_cols(forge_runtime *rt, forge_stream *stream,
                            forge_slice m, forge_slice out, size_t rows,
                            size_t cols);
/* Column sums of m [rows, cols] and the SGD step of a bias in one pass: the
 * bias gradient of Linear::backward (linear.rs:267-272) and the bias update
 * of Linear::learn (linear.rs:385-390), param -= lr * sum with the same two
 * roundings as forge_sgd_update.  out (the sums) and param are each
 * optional. */
forge_status forge_sum_cols_sgd(forge_runtime *rt, forge_stream *stream, forge_slice m,
                                size_t rows, size_t cols, forge_slice out,
                                forge_slice param, float lr);
/* Vector::sum / Vector::max (span.rs:301-333 -> reduction.rs:4-41,93-130):
 * full reduction of x into out[0] on the device (no host round trip; the
 * caller reads it back when it needs the scalar). */
forge_status forge_reduce_sum(forge_runtime *rt, forge_stream *stream,
                              forge_slice x, size_t n, forge_slice out);
/* DeviceSpan::map_sum (span.rs:144-149, 335-359 -> reduction.rs:43-91):
 * out[0] = sum over i < n of f(x[i]) on the device, f one of the map
 * functors of forge_map (the closures the reference passes); 0 for n == 0. */
forge_status forge_map_sum(forge_runtime *rt, forge_stream *stream, forge_slice x,
                           size_t n, forge_map_op op, float p0, forge_slice out);
forge_status forge_reduce_max(forge_runtime *rt, forge_stream *stream,
                              forge_slice x, size_t n, forge_slice out);

/* slice_set_seq (elementwise.rs:23-34): i (ascending) or n - i. */
forge_status forge_fill_seq(forge_runtime *rt, forge_stream *stream,
                            forge_slice x, size_t n, int ascending);
/* slice_set_random (matrix.rs:283-289 -> elementwise.rs:36-43 with the
 * hash of common.rs:3-9): x[i] = hash(seed + i) / u32::MAX.  Bit-exact. */
forge_status forge_fill_random(forge_runtime *rt, forge_stream *stream,
                               forge_slice x, size_t n, uint32_t seed);
/* Vector::equals (vector.rs:117-136 -> reduction.rs:132-174): out[0] = the
 * number of positions i < n with l[i] != r[i] (0 means equal), counted in
 * integers and stored as the nearest f32 (exact up to 2^24).  Every
 * element is compared (the reference kernel reports block 0 only). */
forge_status forge_compare(forge_runtime *rt, forge_stream *stream,
                           forge_slice l, forge_slice r, size_t n,
                           forge_slice out);
/* forge_compare into the reference's u32 result buffer (vector.rs:121-135,
 * compare_vectors writing DeviceSliceMutDescriptor<u32>): out[0] = the
 * number of positions i < n with l[i] != r[i], exact up to 2^32 - 1 and
 * saturating there (0 means equal). */
forge_status forge_compare_u32(forge_runtime *rt, forge_stream *stream,
                               forge_slice l, forge_slice r, size_t n,
                               forge_slice_u32 out);
/* Matrix::causal_mask (matrix.rs:79-92 -> row.rs:5-14). */
forge_status forge_causal_mask(forge_runtime *rt, forge_stream *stream,
                               forge_slice m, size_t rows, size_t cols);
/* The causal mask of rows first_row .. first_row + rows - 1 of a score
 * matrix, held in m [rows, cols]: M[r, c] = -inf for c > first_row + r (the
 * query-chunked attention masks one chunk of rows at a time). */
forge_status forge_causal_mask_rows(forge_runtime *rt, forge_stream *stream, forge_slice m,
                                    size_t rows, size_t cols, size_t first_row);

#ifdef __cplusplus
}
#endif
#endif
