// oxforge_kernels.hip -- the gfx950 code object loaded by forge_runtime_create
// (hipModuleLoad) and launched by name with hipModuleLaunchKernel.  It plays
// the role of the reference's #[cuda_module] mod kernels
// (src/cuda/device/module.rs:6-263): one extern "C" entry per kernel
// instance; the host picks the instance from the shape and alignment.
#include "common.hpp"
#include "elementwise.hpp"
#include "gemm.hpp"
#include "gemm_x.hpp"
#include "rows.hpp"

using namespace forge;

// ------------------------------------------------------------------- GEMM
// forge_gemm_<ab>_<tile>[_e]
//   ab: n/t for A then B (t = operand stored transposed)
//   tile <BM>x<BN>x<BK>_x: the unguarded four-wave kernel (gemm_x.hpp);
//   tile 64x64x16_2x2_g: the bounds-guarded kernel for any shape and
//   alignment (gemm.hpp); _e: fused epilogue.
// Tiles up to 128 x 128 with 32-wide slabs leave LDS for two workgroups per
// CU; their registers are held to what two waves per SIMD allow.
#define GEMM_X_OCC(BM, BN, BK) ((BM) * (BN) <= 128 * 128 && ((BM) + (BN)) * (BK) <= 256 * 32 ? 2 : 1)
#define GEMM_X_KERNEL(NAME, BM, BN, BK, TA, TB, EPI)                          \
    FORGE_KERNEL void __launch_bounds__(256, GEMM_X_OCC(BM, BN, BK)) NAME(GemmArgs p) { \
        gemm_single_x<BM, BN, BK, TA, TB, EPI>(p);                          \
    }
#define GEMM_GUARDED_KERNEL(NAME, BM, BN, BK, WMW, WNW, TA, TB, EPI)        \
    FORGE_KERNEL void __launch_bounds__(WMW * WNW * 64) NAME(GemmArgs p) {   \
        gemm_single_guarded<BM, BN, BK, WMW, WNW, TA, TB, EPI>(p);           \
    }

// Epilogue instances: the unguarded tiles the dispatcher chooses from (by
// shape, see runtime.cpp choose_gemm) and the guarded fallback.
#define GEMM_FAMILY(AB, TA, TB)                                                      \
    GEMM_X_KERNEL(forge_gemm_##AB##_128x128x32_x_e, 128, 128, 32, TA, TB, true)      \
    GEMM_X_KERNEL(forge_gemm_##AB##_128x64x32_x_e, 128, 64, 32, TA, TB, true)        \
    GEMM_X_KERNEL(forge_gemm_##AB##_64x128x32_x_e, 64, 128, 32, TA, TB, true)        \
    GEMM_X_KERNEL(forge_gemm_##AB##_64x64x32_x_e, 64, 64, 32, TA, TB, true)          \
    GEMM_GUARDED_KERNEL(forge_gemm_##AB##_64x64x16_2x2_g_e, 64, 64, 16, 2, 2, TA, TB, true)

GEMM_FAMILY(nn, false, false)
GEMM_FAMILY(nt, false, true)
GEMM_FAMILY(tn, true, false)
GEMM_FAMILY(tt, true, true)

// Row-statistics instances (forge_gemm_<ab>_<tile>_s): the fused epilogue
// plus the row scales of a folded RMSNorm, the rows' sums of squares and the
// column partial sums (forge_gemm_epilogue row_parts_in, row_sumsq_out,
// col_sums_out).  Separate instances keep the plain fused kernels' code as
// it is: the statistics code in them cost the C5 step about 0.7%.
#define GEMM_X_STATS_KERNEL(NAME, BM, BN, BK, TA, TB)                               \
    FORGE_KERNEL void __launch_bounds__(256, GEMM_X_OCC(BM, BN, BK)) NAME(GemmArgs p) { \
        gemm_single_x<BM, BN, BK, TA, TB, true, 2, 2, true>(p);                     \
    }
#define GEMM_STATS_FAMILY(AB, TA, TB)                                                   \
    GEMM_X_STATS_KERNEL(forge_gemm_##AB##_128x128x32_x_s, 128, 128, 32, TA, TB)        \
    GEMM_X_STATS_KERNEL(forge_gemm_##AB##_128x64x32_x_s, 128, 64, 32, TA, TB)          \
    GEMM_X_STATS_KERNEL(forge_gemm_##AB##_64x128x32_x_s, 64, 128, 32, TA, TB)          \
    GEMM_X_STATS_KERNEL(forge_gemm_##AB##_64x64x32_x_s, 64, 64, 32, TA, TB)
GEMM_STATS_FAMILY(nn, false, false)
GEMM_STATS_FAMILY(nt, false, true)
GEMM_STATS_FAMILY(tn, true, false)
GEMM_STATS_FAMILY(tt, true, true)

// Row-subtrahend instances (forge_gemm_<ab>_<tile>_r): the statistics
// instances plus forge_gemm_epilogue row_sub (the softmax backward formed in
// the dP product).  Separate again, so the _e and _s kernels stay as they
// are (with row_sub in them the C4 forward ran 0.9-1.4 us slower).
#define GEMM_X_ROWSUB_KERNEL(NAME, BM, BN, BK, TA, TB)                              \
    FORGE_KERNEL void __launch_bounds__(256, GEMM_X_OCC(BM, BN, BK)) NAME(GemmArgs p) { \
        gemm_single_x<BM, BN, BK, TA, TB, true, 2, 2, true, true>(p);               \
    }
#define GEMM_ROWSUB_FAMILY(AB, TA, TB)                                                  \
    GEMM_X_ROWSUB_KERNEL(forge_gemm_##AB##_128x128x32_x_r, 128, 128, 32, TA, TB)       \
    GEMM_X_ROWSUB_KERNEL(forge_gemm_##AB##_128x64x32_x_r, 128, 64, 32, TA, TB)         \
    GEMM_X_ROWSUB_KERNEL(forge_gemm_##AB##_64x128x32_x_r, 64, 128, 32, TA, TB)         \
    GEMM_X_ROWSUB_KERNEL(forge_gemm_##AB##_64x64x32_x_r, 64, 64, 32, TA, TB)
GEMM_ROWSUB_FAMILY(nn, false, false)
GEMM_ROWSUB_FAMILY(nt, false, true)
GEMM_ROWSUB_FAMILY(tn, true, false)
GEMM_ROWSUB_FAMILY(tt, true, true)

// K-segment instances (forge_gemm_<ab>_<tile>_k): the fused epilogue over a
// sum of two or three products (forge_gemm_sum_f32), each segment's slabs
// read from its own operands.
#define GEMM_X_SEGK_KERNEL(NAME, BM, BN, BK, TA, TB)                                \
    FORGE_KERNEL void __launch_bounds__(256, GEMM_X_OCC(BM, BN, BK)) NAME(GemmArgs p) { \
        gemm_single_x<BM, BN, BK, TA, TB, true, 2, 2, false, false, true>(p);       \
    }
#define GEMM_SEGK_FAMILY(AB, TA, TB)                                                    \
    GEMM_X_SEGK_KERNEL(forge_gemm_##AB##_128x128x32_x_k, 128, 128, 32, TA, TB)         \
    GEMM_X_SEGK_KERNEL(forge_gemm_##AB##_128x64x32_x_k, 128, 64, 32, TA, TB)           \
    GEMM_X_SEGK_KERNEL(forge_gemm_##AB##_64x128x32_x_k, 64, 128, 32, TA, TB)           \
    GEMM_X_SEGK_KERNEL(forge_gemm_##AB##_64x64x32_x_k, 64, 64, 32, TA, TB)
GEMM_SEGK_FAMILY(nn, false, false)
GEMM_SEGK_FAMILY(nt, false, true)
GEMM_SEGK_FAMILY(tn, true, false)
GEMM_SEGK_FAMILY(tt, true, true)

// Batched instances (forge_gemm_batch_<ab>_<tile>): several same-shape
// products per launch, each with its own operands and epilogue.  They serve
// the Q/K/V projections, forge_gemm_batch_f32 and the K slices of split-K
// products, so every operand layout has them.
#define GEMM_BATCH_KERNEL(NAME, BM, BN, BK, TA, TB)                                    \
    FORGE_KERNEL void __launch_bounds__(256, GEMM_X_OCC(BM, BN, BK)) NAME(GemmBatchArgs b) { \
        gemm_batch_x<BM, BN, BK, TA, TB>(b);                                         \
    }
#define GEMM_BATCH_FAMILY(AB, TA, TB)                                                   \
    GEMM_BATCH_KERNEL(forge_gemm_batch_##AB##_128x128x32_x, 128, 128, 32, TA, TB)      \
    GEMM_BATCH_KERNEL(forge_gemm_batch_##AB##_128x64x32_x, 128, 64, 32, TA, TB)        \
    GEMM_BATCH_KERNEL(forge_gemm_batch_##AB##_64x128x32_x, 64, 128, 32, TA, TB)        \
    GEMM_BATCH_KERNEL(forge_gemm_batch_##AB##_64x64x32_x, 64, 64, 32, TA, TB)
GEMM_BATCH_FAMILY(nn, false, false)
GEMM_BATCH_FAMILY(nt, false, true)
GEMM_BATCH_FAMILY(tn, true, false)
GEMM_BATCH_FAMILY(tt, true, true)

// Split-K: sum of the partial products in split order, then the epilogue.
FORGE_KERNEL void __launch_bounds__(SPLITK_THREADS) forge_gemm_splitk_reduce_v(const float* P,
                                                                            int splits,
                                                                            GemmArgs p) {
    splitk_reduce_body<true>(P, splits, p);
}
FORGE_KERNEL void __launch_bounds__(SPLITK_THREADS) forge_gemm_splitk_reduce_s(const float* P,
                                                                            int splits,
                                                                            GemmArgs p) {
    splitk_reduce_body<false>(P, splits, p);
}

// Eight-wave 64 x 128 tile (4 x 2 waves of 16 x 64): two waves per SIMD
// where a product leaves one tile per CU.
#define GEMM_X8_KERNEL(NAME, TA, TB, EPI)                                           \
    FORGE_KERNEL void __launch_bounds__(512, 1) NAME(GemmArgs p) {                  \
        gemm_single_x<64, 128, 32, TA, TB, EPI, 4, 2>(p);                          \
    }
GEMM_X8_KERNEL(forge_gemm_nn_64x128x32_x8, false, false, false)
GEMM_X8_KERNEL(forge_gemm_nn_64x128x32_x8_e, false, false, true)
GEMM_X8_KERNEL(forge_gemm_nt_64x128x32_x8_e, false, true, true)
GEMM_X8_KERNEL(forge_gemm_tn_64x128x32_x8_e, true, false, true)
GEMM_X8_KERNEL(forge_gemm_tt_64x128x32_x8_e, true, true, true)
#define GEMM_X8_STATS_KERNEL(NAME, TA, TB)                                          \
    FORGE_KERNEL void __launch_bounds__(512, 1) NAME(GemmArgs p) {                  \
        gemm_single_x<64, 128, 32, TA, TB, true, 4, 2, true>(p);                   \
    }
GEMM_X8_STATS_KERNEL(forge_gemm_nn_64x128x32_x8_s, false, false)
GEMM_X8_STATS_KERNEL(forge_gemm_nt_64x128x32_x8_s, false, true)
GEMM_X8_STATS_KERNEL(forge_gemm_tn_64x128x32_x8_s, true, false)
GEMM_X8_STATS_KERNEL(forge_gemm_tt_64x128x32_x8_s, true, true)
#define GEMM_X8_ROWSUB_KERNEL(NAME, TA, TB)                                         \
    FORGE_KERNEL void __launch_bounds__(512, 1) NAME(GemmArgs p) {                  \
        gemm_single_x<64, 128, 32, TA, TB, true, 4, 2, true, true>(p);             \
    }
GEMM_X8_ROWSUB_KERNEL(forge_gemm_nn_64x128x32_x8_r, false, false)
GEMM_X8_ROWSUB_KERNEL(forge_gemm_nt_64x128x32_x8_r, false, true)
GEMM_X8_ROWSUB_KERNEL(forge_gemm_tn_64x128x32_x8_r, true, false)
GEMM_X8_ROWSUB_KERNEL(forge_gemm_tt_64x128x32_x8_r, true, true)
#define GEMM_X8_BATCH_KERNEL(NAME, TA, TB)                                            \
    FORGE_KERNEL void __launch_bounds__(512, 1) NAME(GemmBatchArgs b) {               \
        gemm_batch_x<64, 128, 32, TA, TB, 4, 2>(b);                                 \
    }
GEMM_X8_BATCH_KERNEL(forge_gemm_batch_nn_64x128x32_x8, false, false)
GEMM_X8_BATCH_KERNEL(forge_gemm_batch_nt_64x128x32_x8, false, true)
GEMM_X8_BATCH_KERNEL(forge_gemm_batch_tn_64x128x32_x8, true, false)

// Plain C = A * B instances of forge_gemm_f32 (the headline GEMM).
GEMM_X_KERNEL(forge_gemm_nn_128x256x32_x, 128, 256, 32, false, false, false)
GEMM_X_KERNEL(forge_gemm_nn_128x128x32_x, 128, 128, 32, false, false, false)
GEMM_X_KERNEL(forge_gemm_nn_128x64x32_x, 128, 64, 32, false, false, false)
GEMM_X_KERNEL(forge_gemm_nn_64x128x32_x, 64, 128, 32, false, false, false)
GEMM_X_KERNEL(forge_gemm_nn_64x64x32_x, 64, 64, 32, false, false, false)
GEMM_GUARDED_KERNEL(forge_gemm_nn_64x64x16_2x2_g, 64, 64, 16, 2, 2, false, false, false)

// ------------------------------------------------------------------- rows
#define ROW_KERNEL(NAME, OP, VPT, PARTIALS) \
    FORGE_KERNEL void __launch_bounds__(256) NAME(RowArgs a) { row_kernel_reg<OP, VPT, PARTIALS>(a); }
#define ROW_KERNELS(OPNAME, OP)                                   \
    ROW_KERNEL(forge_row_##OPNAME##_v1, OP, 1, false)             \
    ROW_KERNEL(forge_row_##OPNAME##_v2, OP, 2, false)             \
    ROW_KERNEL(forge_row_##OPNAME##_v4, OP, 4, false)             \
    ROW_KERNEL(forge_row_##OPNAME##_v8, OP, 8, false)             \
    ROW_KERNEL(forge_row_##OPNAME##_v16, OP, 16, false)           \
    FORGE_KERNEL void __launch_bounds__(256) forge_row_##OPNAME##_loop(RowArgs a) { row_kernel_loop<OP>(a); }
// Norm backward instances that also emit per-workgroup dgamma/dbeta
// partials, one workgroup per CU, each wave walking its rows grid-stride:
//   _p:  8 waves; at 1, 2 and 8 float4 per lane the next row is prefetched
//        into registers, at 4 it is not (measured on MI355X, [2048..32768,
//        1024]: 0.5-2% faster without);
//   _p4: 4 waves, no prefetch, for 4 float4 per lane and at least 256 rows
//        per CU ([65536,1024]: LayerNorm backward 133.5 against 135.1 us
//        with 8 waves and 138.5 with 8 waves and prefetch).
// The runtime launches them with WAVES * 64 threads.
#define ROW_PARTIAL_KERNEL(NAME, OP, VPT, W, PF)                                         \
    FORGE_KERNEL void __launch_bounds__(W * 64) NAME(RowArgs a) {                        \
        row_kernel_reg<OP, VPT, true, W, false, PF>(a);                                  \
    }
#define ROW_PARTIAL_KERNELS(OPNAME, OP)                                                  \
    ROW_PARTIAL_KERNEL(forge_row_##OPNAME##_v1_p, OP, 1, ROW_PARTIAL_WAVES, true)        \
    ROW_PARTIAL_KERNEL(forge_row_##OPNAME##_v2_p, OP, 2, ROW_PARTIAL_WAVES, true)        \
    ROW_PARTIAL_KERNEL(forge_row_##OPNAME##_v4_p, OP, 4, ROW_PARTIAL_WAVES, false)       \
    ROW_PARTIAL_KERNEL(forge_row_##OPNAME##_v4_p4, OP, 4, 4, false)                      \
    ROW_PARTIAL_KERNEL(forge_row_##OPNAME##_v8_p, OP, 8, ROW_PARTIAL_WAVES, true)

ROW_KERNELS(softmax, ROW_SOFTMAX)
ROW_KERNELS(layer_norm, ROW_LAYER_NORM)
ROW_KERNELS(rms_norm, ROW_RMS_NORM)
ROW_KERNELS(softmax_bwd, ROW_SOFTMAX_BWD)
ROW_KERNELS(layer_norm_bwd, ROW_LAYER_NORM_BWD)
ROW_KERNELS(rms_norm_bwd, ROW_RMS_NORM_BWD)
ROW_PARTIAL_KERNELS(layer_norm_bwd, ROW_LAYER_NORM_BWD)
ROW_PARTIAL_KERNELS(rms_norm_bwd, ROW_RMS_NORM_BWD)
// _d: the norm backward instances above that also write the row dot
// (RowArgs::dot), without the next-row prefetch.
#define ROW_DOT_KERNEL(NAME, OP, VPT)                                                    \
    FORGE_KERNEL void __launch_bounds__(256) NAME(RowArgs a) {                           \
        row_kernel_reg<OP, VPT, false, ROW_WAVES, true>(a);                              \
    }
#define ROW_PARTIAL_DOT_KERNEL(NAME, OP, VPT, W)                                         \
    FORGE_KERNEL void __launch_bounds__(W * 64) NAME(RowArgs a) {                        \
        row_kernel_reg<OP, VPT, true, W, true, false>(a);                                \
    }
#define ROW_DOT_KERNELS(OPNAME, OP)                                                      \
    ROW_DOT_KERNEL(forge_row_##OPNAME##_v1_d, OP, 1)                                     \
    ROW_DOT_KERNEL(forge_row_##OPNAME##_v2_d, OP, 2)                                     \
    ROW_DOT_KERNEL(forge_row_##OPNAME##_v4_d, OP, 4)                                     \
    ROW_DOT_KERNEL(forge_row_##OPNAME##_v8_d, OP, 8)                                     \
    ROW_DOT_KERNEL(forge_row_##OPNAME##_v16_d, OP, 16)                                   \
    ROW_PARTIAL_DOT_KERNEL(forge_row_##OPNAME##_v1_p_d, OP, 1, ROW_PARTIAL_WAVES)        \
    ROW_PARTIAL_DOT_KERNEL(forge_row_##OPNAME##_v2_p_d, OP, 2, ROW_PARTIAL_WAVES)        \
    ROW_PARTIAL_DOT_KERNEL(forge_row_##OPNAME##_v4_p_d, OP, 4, ROW_PARTIAL_WAVES)        \
    ROW_PARTIAL_DOT_KERNEL(forge_row_##OPNAME##_v4_p4_d, OP, 4, 4)                       \
    ROW_PARTIAL_DOT_KERNEL(forge_row_##OPNAME##_v8_p_d, OP, 8, ROW_PARTIAL_WAVES)
ROW_DOT_KERNELS(layer_norm_bwd, ROW_LAYER_NORM_BWD)
ROW_DOT_KERNELS(rms_norm_bwd, ROW_RMS_NORM_BWD)


// ------------------------------------------------------------ elementwise
#define BINARY_KERNELS(OPNAME, OP)                                                          \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_binary_##OPNAME##_v(              \
        const float* l, const float* r, float* o, long long n) { binary_body<OP, true>(l, r, o, n); } \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_binary_##OPNAME##_s(              \
        const float* l, const float* r, float* o, long long n) { binary_body<OP, false>(l, r, o, n); } \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_binary_assign_##OPNAME##_v(       \
        float* t, const float* r, long long n) { binary_assign_body<OP, true>(t, r, n); }     \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_binary_assign_##OPNAME##_s(       \
        float* t, const float* r, long long n) { binary_assign_body<OP, false>(t, r, n); }    \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_by_rows_##OPNAME##_v(             \
        float* m, const float* row, int rows, int cols) { by_rows_body<OP, true>(m, row, rows, cols); } \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_by_rows_##OPNAME##_s(             \
        float* m, const float* row, int rows, int cols) { by_rows_body<OP, false>(m, row, rows, cols); }

BINARY_KERNELS(add, OP_ADD)
BINARY_KERNELS(sub, OP_SUB)
BINARY_KERNELS(mul, OP_MUL)
BINARY_KERNELS(div, OP_DIV)

#define MAP_KERNELS(OPNAME, OP)                                                     \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_map_##OPNAME##_v(         \
        float* x, long long n, float p0) { map_body<OP, true>(x, n, p0); }          \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_map_##OPNAME##_s(         \
        float* x, long long n, float p0) { map_body<OP, false>(x, n, p0); }

#define MAP_SUM_KERNEL(OPNAME, OP)                                                    \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_map_sum_##OPNAME(              \
        const float* x, long long n, float p0, float* out) {                           \
        reduce_body<OP, false, false>(x, n, p0, out);                                  \
    }                                                                                  \
    FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_map_sum_##OPNAME##_v(          \
        const float* x, long long n, float p0, float* out) {                           \
        reduce_body<OP, false, true>(x, n, p0, out);                                   \
    }
#define MAP_KERNELS_ALL(OPNAME, OP) MAP_KERNELS(OPNAME, OP) MAP_SUM_KERNEL(OPNAME, OP)

MAP_KERNELS_ALL(scale, MAP_SCALE)
MAP_KERNELS_ALL(add, MAP_ADD)
MAP_KERNELS_ALL(gelu, MAP_GELU)
MAP_KERNELS_ALL(gelu_d, MAP_GELU_D)
MAP_KERNELS_ALL(relu, MAP_RELU)
MAP_KERNELS_ALL(relu_d, MAP_RELU_D)
MAP_KERNELS_ALL(silu, MAP_SILU)
MAP_KERNELS_ALL(silu_d, MAP_SILU_D)
MAP_KERNELS_ALL(exp_shift, MAP_EXP_SHIFT)
MAP_KERNELS_ALL(half_sq, MAP_HALF_SQ)
MAP_KERNELS_ALL(identity, MAP_IDENTITY)

FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_fill_v(float* x, long long n, float v) {
    fill_body<true>(x, n, v);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_fill_s(float* x, long long n, float v) {
    fill_body<false>(x, n, v);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_fill_seq(float* x, long long n, int asc) {
    fill_seq_body(x, n, asc);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_fill_random(float* x, long long n,
                                                                  unsigned seed) {
    fill_random_body(x, n, seed);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_act_backward_v(const float* dy, const float* z,
                                                                     float* g, long long n, int act) {
    act_backward_body<true>(dy, z, g, n, act);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_act_backward_s(const float* dy, const float* z,
                                                                     float* g, long long n, int act) {
    act_backward_body<false>(dy, z, g, n, act);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_sgd_v(float* p, const float* g, long long n,
                                                            float lr) {
    sgd_body<true>(p, g, n, lr);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_sgd_s(float* p, const float* g, long long n,
                                                            float lr) {
    sgd_body<false>(p, g, n, lr);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_count_neq(const float* l, const float* r,
                                                                long long n, unsigned* part,
                                                                float* out) {
    count_neq_body(l, r, n, part, out);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_count_final(const unsigned* part, int n,
                                                                  float* out) {
    count_final_body(part, n, out);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_count_neq_u32(const float* l, const float* r,
                                                                    long long n, unsigned* part,
                                                                    unsigned* out) {
    count_neq_body(l, r, n, part, out);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_count_final_u32(const unsigned* part, int n,
                                                                      unsigned* out) {
    count_final_body(part, n, out);
}
FORGE_KERNEL void __launch_bounds__(256) forge_row_rms_parts(const float* part, int parts,
                                                            int rows, int n, float eps, float* d) {
    row_rms_parts_body(part, parts, rows, n, eps, d);
}
FORGE_KERNEL void __launch_bounds__(256) forge_row_sq_parts(const float* m, long long ld, int rows,
                                                           int cols, float* out) {
    row_sq_parts_body(m, ld, rows, cols, out);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_causal_mask(float* m, int rows, int cols,
                                                                  int first_row) {
    causal_mask_body(m, rows, cols, first_row);
}
FORGE_KERNEL void __launch_bounds__(SUMCOL_WAVES * 64) forge_sum_cols_v(const float* m, float* out,
                                                                       int rows, int cols,
                                                                       int rows_per_chunk) {
    sum_cols_body<true>(m, out, rows, cols, rows_per_chunk);
}
FORGE_KERNEL void __launch_bounds__(SUMCOL_WAVES * 64) forge_sum_cols_s(const float* m, float* out,
                                                                       int rows, int cols,
                                                                       int rows_per_chunk) {
    sum_cols_body<false>(m, out, rows, cols, rows_per_chunk);
}
// Column sums, first pass over float4 columns, LOADS loads in flight per lane.
#define SUM_COLS_PART_KERNEL(L)                                                                \
    FORGE_KERNEL void __launch_bounds__(SUMCOL1_THREADS) forge_sum_cols_p##L(                  \
        const float* m, float* part, ColSumOut o, int rows, int cols, int rows_per_chunk) {   \
        sum_cols_part_body<L>(m, part, o, rows, cols, rows_per_chunk);                         \
    }
SUM_COLS_PART_KERNEL(4)
SUM_COLS_PART_KERNEL(8)
SUM_COLS_PART_KERNEL(16)
// Final column-sum passes (ColSumOut: sums to `out`, and optionally the SGD
// step of a parameter vector).  The *2 instances do two independent column
// sums in one launch, blockIdx.y selecting the pair: dgamma and dbeta of the
// LayerNorm backward.
FORGE_KERNEL void __launch_bounds__(SUMCOL_FINAL_WAVES * 64) forge_sum_cols_final(
    const float* m, ColSumOut o, int rows, int cols) {
    sum_cols_final_body(m, o, rows, cols);
}
FORGE_KERNEL void __launch_bounds__(SUMCOL_FINAL_WAVES * 64) forge_sum_cols_final2(
    const float* m0, ColSumOut o0, const float* m1, ColSumOut o1, int rows, int cols) {
    if (blockIdx.y == 0) sum_cols_final_body(m0, o0, rows, cols);
    else sum_cols_final_body(m1, o1, rows, cols);
}
FORGE_KERNEL void __launch_bounds__(SUMCOL_FINAL_V_THREADS) forge_sum_cols_final_v(
    const float* m, ColSumOut o, int rows, int cols) {
    sum_cols_final_v_body(m, o, rows, cols);
}
FORGE_KERNEL void __launch_bounds__(SUMCOL_FINAL_V_THREADS) forge_sum_cols_final2_v(
    const float* m0, ColSumOut o0, const float* m1, ColSumOut o1, int rows, int cols) {
    if (blockIdx.y == 0) sum_cols_final_v_body(m0, o0, rows, cols);
    else sum_cols_final_v_body(m1, o1, rows, cols);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_sum_rows_v(const float* m, float* out, int rows,
                                                                 int cols) {
    sum_rows_body<true>(m, out, rows, cols);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_sum_rows_s(const float* m, float* out, int rows,
                                                                 int cols) {
    sum_rows_body<false>(m, out, rows, cols);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_reduce_sum(const float* x, long long n, float* out) {
    reduce_body<MAP_IDENTITY, false, false>(x, n, 0.0f, out);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_reduce_max(const float* x, long long n, float* out) {
    reduce_body<MAP_IDENTITY, true, false>(x, n, 0.0f, out);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_reduce_sum_v(const float* x, long long n,
                                                                   float* out) {
    reduce_body<MAP_IDENTITY, false, true>(x, n, 0.0f, out);
}
FORGE_KERNEL void __launch_bounds__(EW_THREADS) forge_reduce_max_v(const float* x, long long n,
                                                                   float* out) {
    reduce_body<MAP_IDENTITY, true, true>(x, n, 0.0f, out);
}
FORGE_KERNEL void __launch_bounds__(256) forge_transpose_w(const float* in, float* out, int rows, int cols) {
    transpose_body<256, false>(in, out, rows, cols);
}
FORGE_KERNEL void __launch_bounds__(256) forge_transpose(const float* in, float* out, int rows, int cols) {
    transpose_body<64, false>(in, out, rows, cols);
}
FORGE_KERNEL void __launch_bounds__(256) forge_transpose_g(const float* in, float* out, int rows, int cols) {
    transpose_body<64, true>(in, out, rows, cols);
}
