// gemm.hpp -- fp32 GEMM on CDNA4 matrix cores: the shared GEMM argument
// structs, tile ordering and split-K reduction, and the bounds-guarded
// kernel body that serves shapes or alignments the unguarded four-wave tiles
// (gemm_x.hpp) cannot take: any M, N, K and any alignment.
//
// Replaces matrix_multiply_device (reference gemm.rs:202-373, TF32 mma.sync)
// with true fp32 v_mfma_f32_32x32x2_f32.  Semantics follow the strict-fp32
// kernel gemm.rs:15-129: C = A * B, row-major, C overwritten, f32 accumulate.
//
// Structure of the guarded body
//   - A workgroup computes a BM x BN tile with WARPS_M x WARPS_N waves; each
//     wave owns a (BM/WARPS_M) x (BN/WARPS_N) sub-tile made of 32x32 MFMA
//     blocks whose accumulators live in VGPRs.
//   - K advances in BK slabs.  The next slab is loaded from global memory
//     into registers while the matrix cores work on the current slab in LDS,
//     then stored to the other LDS buffer: one barrier per slab.
//   - An MFMA step consumes k = 2: lanes 0-31 supply k-index 0 and lanes
//     32-63 k-index 1.  Inside each 16-wide k chunk, lane half h supplies
//     k = 16c + 8h + s at step s, so a lane's eight A values (and B values
//     for a transposed B) are contiguous in LDS and load as two ds_read_b128.
//   - LDS tiles keep the orientation of the global tile ("k-contiguous" for
//     A and B^T, "m/n-contiguous" for A^T and B) with a 4-float row pad,
//     which keeps both the b128 row reads and the b32 column reads free of
//     bank conflicts.
//   - Workgroup ids are remapped so that each XCD (workgroups are dealt
//     round-robin over the 8 XCDs) receives a contiguous range of tiles, and
//     tiles are walked in GROUP_M-row bands, so A and B slabs are reused out
//     of each XCD's private L2.
//   - The optional epilogue fuses the Linear launch sequence (bias by rows,
//     residual add, gradient * act'(z), activation, SGD update); each step is
//     one rounded f32 operation, in the reference's order.
#pragma once
#include "common.hpp"

namespace forge {

struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    int M, N, K;
    long long lda, ldb, ldc;  // leading dimensions in elements
    float alpha;
    const float* bias;      // [N] or null
    const float* residual;  // [M, ldc] or null
    const float* aux;       // [M, ldc] or null: Z *= aux (or act'(aux))
    float* pre_out;         // [M, ldc] or null: stores Z before activation
    int act;
    int aux_act;            // 0: Z *= aux; ACT_*: Z *= derivative of that act at aux
    int update;             // 0: C = act(Z); 1: C = C - update_scale * act(Z)
    float update_scale;
    // Row statistics (the RMSNorm of a row folded across a GEMM boundary).
    // The divisor of row r is d_r = sqrt(sum of row_parts values / row_n +
    // row_eps): from row_part [M, row_parts] (partial sums of squares that
    // another product's row_sq wrote), or given directly in row_d [M].
    // row_div bit 0: Z = Z / d_r right after alpha; bit 1: the residual is
    // divided by d_r before it is added.
    const float* row_part;
    const float* row_d;
    int row_parts, row_n;
    float row_eps;
    int row_div;
    // [M, N / 32] or null: the sum of the squares of the stored values over
    // each 32-column block of each row (the unguarded tiles only).
    float* row_sq;
    // [M / TM, N] or null: the column sums of the stored values over each
    // wave's TM rows (the unguarded tiles only; TM = the tile's rows per
    // wave).
    float* col_part;
    // [M] or null: Z = Z - row_sub[r] after alpha and the row_div divide
    // (the softmax backward's row term, folded into the dP product).
    const float* row_sub;
    // K segments (the _k instances): the product is sum_s op(A_s) op(B_s)
    // over K / k_seg segments of k_seg each, A_0 = A, B_0 = B, then A1/B1
    // and A2/B2, every segment with the pitches lda / ldb -- the product of
    // the operands concatenated along K, in the same sum order.
    const float* A1;
    const float* A2;
    const float* B1;
    const float* B2;
    int k_seg;
};
// The host fills the same layout (runtime.cpp GemmArgs).
static_assert(sizeof(GemmArgs) == 216, "kernel argument layout");

constexpr int GEMM_GROUP_M = 8;
constexpr int LDS_PAD = 4;

// Maps hardware workgroup id b of nwg to a logical tile index so that each
// XCD (workgroups are dealt round-robin over the 8 XCDs) receives a
// contiguous range of logical tiles.
__device__ __forceinline__ int xcd_logical(int b, int nwg) {
    const int per_xcd = nwg / 8, rem = nwg % 8;
    const int xcd = b % 8, local = b / 8;
    return xcd < rem ? xcd * (per_xcd + 1) + local
                     : rem * (per_xcd + 1) + (xcd - rem) * per_xcd + local;
}

// Maps a logical tile index to (tile_m, tile_n), walking GEMM_GROUP_M-row
// bands so consecutive tiles share A and B slabs.  Correctness does not
// depend on the order.
__device__ __forceinline__ void gemm_tile_coords(int logical, int num_m, int num_n,
                                                 int& tm, int& tn) {
    const int in_group = GEMM_GROUP_M * num_n;
    const int group = logical / in_group;
    const int first_m = group * GEMM_GROUP_M;
    const int gsize = min(num_m - first_m, GEMM_GROUP_M);
    const int r = logical % in_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

// A batch of GEMMs with the same M and N (and tile instance) in one launch:
// logical tile t belongs to problem t / tiles.  Used for the Q/K/V
// projections and for the K slices of a split-K product.
constexpr int GEMM_BATCH_MAX = 8;
struct GemmBatchArgs {
    GemmArgs p[GEMM_BATCH_MAX];
    int count;  // problems
    int tiles;  // tiles per problem
};

// The fused epilogue on one element z of the product at (row, col), idx =
// row * ldc + col: alpha, row divide, row subtrahend, bias, residual, aux
// multiply (or act'(aux)), pre-activation store, activation, then store or
// SGD update.  Each step is one rounded f32 operation in the reference's
// launch order.
__device__ __forceinline__ void gemm_epilogue_store(const GemmArgs& p, long long idx, int row,
                                                    int col, float z) {
    if (p.alpha != 1.0f) z = p.alpha * z;
    if (p.row_d && (p.row_div & 1)) z = z / p.row_d[row];
    if (p.row_sub) z = z - p.row_sub[row];
    if (p.bias) z = z + p.bias[col];
    if (p.residual) z = z + ((p.row_d && (p.row_div & 2)) ? p.residual[idx] / p.row_d[row]
                                                          : p.residual[idx]);
    if (p.aux) {
        const float m = p.aux_act ? activate_derivative(p.aux_act, p.aux[idx]) : p.aux[idx];
        z = z * m;
    }
    if (p.pre_out) p.pre_out[idx] = z;
    const float y = activate(p.act, z);
    if (p.update) p.C[idx] = p.C[idx] - p.update_scale * y;
    else p.C[idx] = y;
}

template <int ROWS, int COLS, int NT>
struct TileShape {
    static constexpr int F4_PER_ROW = COLS / 4;
    static constexpr int TOTAL = ROWS * F4_PER_ROW;
    static constexpr int PER_THREAD = TOTAL / NT;
    static_assert(TOTAL % NT == 0, "tile must divide evenly over threads");
};

// Loads a ROWS x COLS tile (COLS contiguous in global memory) into registers,
// COLS/4 four-float vectors per row, dealt over NT threads, zero-filling
// outside [vr, vc) with scalar loads (no alignment assumption).  The staging
// registers are the native 4-float vector f4 so they stay in VGPRs.
template <int ROWS, int COLS, int NT>
__device__ __forceinline__ void tile_load_guarded(f4* __restrict__ v,
                                                  const float* __restrict__ g, long long ld,
                                                  int vr, int vc) {
    using S = TileShape<ROWS, COLS, NT>;
#pragma unroll
    for (int i = 0; i < S::PER_THREAD; i++) {
        const int f = threadIdx.x + i * NT;
        const int r = f / S::F4_PER_ROW;
        const int c = (f % S::F4_PER_ROW) * 4;
        const float* q = g + (long long)r * ld + c;
        const bool rok = r < vr;
        v[i].x = (rok && c + 0 < vc) ? q[0] : 0.0f;
        v[i].y = (rok && c + 1 < vc) ? q[1] : 0.0f;
        v[i].z = (rok && c + 2 < vc) ? q[2] : 0.0f;
        v[i].w = (rok && c + 3 < vc) ? q[3] : 0.0f;
    }
}

template <int ROWS, int COLS, int NT>
__device__ __forceinline__ void tile_store(const f4* __restrict__ v,
                                           float* __restrict__ s) {
    using S = TileShape<ROWS, COLS, NT>;
    constexpr int PITCH = COLS + LDS_PAD;
#pragma unroll
    for (int i = 0; i < S::PER_THREAD; i++) {
        const int f = threadIdx.x + i * NT;
        const int r = f / S::F4_PER_ROW;
        const int c = (f % S::F4_PER_ROW) * 4;
        *reinterpret_cast<f4*>(s + r * PITCH + c) = v[i];
    }
}

// Eight operand values of one lane for one 16-wide k chunk.
//   KC layout ([rows][BK+pad], k contiguous): two b128 reads.
//   MC layout ([BK][rows+pad], rows contiguous): eight b32 reads.
template <bool KC, int ROWS, int BK>
__device__ __forceinline__ void load_frag(const float* __restrict__ s, int row,
                                          int chunk, int half, float (&f)[8]) {
    if constexpr (KC) {
        constexpr int PITCH = BK + LDS_PAD;
        const float* p = s + row * PITCH + chunk * 16 + half * 8;
        const f4 a = *reinterpret_cast<const f4*>(p);
        const f4 b = *reinterpret_cast<const f4*>(p + 4);
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
        constexpr int PITCH = ROWS + LDS_PAD;
        const float* p = s + (chunk * 16 + half * 8) * PITCH + row;
#pragma unroll
        for (int k = 0; k < 8; k++) f[k] = p[k * PITCH];
    }
}

template <int BM, int BN, int BK, int WARPS_M, int WARPS_N, bool TA, bool TB, bool EPI>
__device__ __forceinline__ void gemm_body_guarded(const GemmArgs& p, int logical) {
    constexpr int NT = WARPS_M * WARPS_N * 64;
    constexpr int WM = BM / WARPS_M, WN = BN / WARPS_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    static_assert(WM % 32 == 0 && WN % 32 == 0 && BK % 16 == 0, "tile shape");

    // Global tile orientation == LDS orientation.
    // A: !TA -> [BM][BK] (KC)   TA -> [BK][BM] (MC)
    // B: !TB -> [BK][BN] (MC)   TB -> [BN][BK] (KC)
    constexpr int A_ROWS = TA ? BK : BM, A_COLS = TA ? BM : BK;
    constexpr int B_ROWS = TB ? BN : BK, B_COLS = TB ? BK : BN;
    constexpr int A_ELEMS = A_ROWS * (A_COLS + LDS_PAD);
    constexpr int B_ELEMS = B_ROWS * (B_COLS + LDS_PAD);
    __shared__ __attribute__((aligned(16))) float smem[2 * (A_ELEMS + B_ELEMS)];

    const int num_m = (p.M + BM - 1) / BM, num_n = (p.N + BN - 1) / BN;
    int tm, tn;
    gemm_tile_coords(logical, num_m, num_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave / WARPS_N, wn = wave % WARPS_N;
    const int l32 = lane & 31, half = lane >> 5;

    // Global tile origins and the valid extent of each slab (guards only).
    const float* a_base = TA ? p.A + m0 : p.A + (long long)m0 * p.lda;
    const float* b_base = TB ? p.B + (long long)n0 * p.ldb : p.B + n0;
    const long long a_kstride = TA ? (long long)BK * p.lda : BK;
    const long long b_kstride = TB ? BK : (long long)BK * p.ldb;

    f4 ra[TileShape<A_ROWS, A_COLS, NT>::PER_THREAD];
    f4 rb[TileShape<B_ROWS, B_COLS, NT>::PER_THREAD];
    // Valid extents of a slab starting at k0 (used by the guarded loads).
    const int a_vr = TA ? 0 : p.M - m0, a_vc = TA ? p.M - m0 : 0;
    const int b_vr = TB ? p.N - n0 : 0, b_vc = TB ? 0 : p.N - n0;

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int KT = (p.K + BK - 1) / BK;
#define FORGE_LOAD_SLAB(KT_)                                                   \
    do {                                                                       \
        const int kv_ = p.K - (KT_) * BK;                                      \
        tile_load_guarded<A_ROWS, A_COLS, NT>(ra, a_base + (KT_) * a_kstride, p.lda, \
                                              TA ? kv_ : a_vr, TA ? a_vc : kv_);     \
        tile_load_guarded<B_ROWS, B_COLS, NT>(rb, b_base + (KT_) * b_kstride, p.ldb, \
                                              TB ? b_vr : kv_, TB ? kv_ : b_vc);     \
    } while (0)
    if (KT > 0) {
        FORGE_LOAD_SLAB(0);
        tile_store<A_ROWS, A_COLS, NT>(ra, smem);
        tile_store<B_ROWS, B_COLS, NT>(rb, smem + A_ELEMS);
        __syncthreads();
    }

    for (int kt = 0; kt < KT; kt++) {
        const int buf = kt & 1;
        const float* sa = smem + buf * (A_ELEMS + B_ELEMS);
        const float* sb = sa + A_ELEMS;
        if (kt + 1 < KT) FORGE_LOAD_SLAB(kt + 1);

#pragma unroll
        for (int c = 0; c < BK / 16; c++) {
            float af[FM][8], bf[FN][8];
#pragma unroll
            for (int i = 0; i < FM; i++)
                load_frag<!TA, BM, BK>(sa, wm * WM + i * 32 + l32, c, half, af[i]);
#pragma unroll
            for (int j = 0; j < FN; j++)
                load_frag<TB, BN, BK>(sb, wn * WN + j * 32 + l32, c, half, bf[j]);
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
        }

        if (kt + 1 < KT) {
            float* da = smem + (buf ^ 1) * (A_ELEMS + B_ELEMS);
            tile_store<A_ROWS, A_COLS, NT>(ra, da);
            tile_store<B_ROWS, B_COLS, NT>(rb, da + A_ELEMS);
        }
        __syncthreads();
    }
#undef FORGE_LOAD_SLAB

    // Epilogue.  Accumulator register r of a 32x32 block holds
    // row 8*(r/4) + 4*(lane/32) + r%4, column lane%32.
    const int row_base = m0 + wm * WM + 4 * half;
    const int col_base = n0 + wn * WN + l32;
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            v16f& a = acc[i][j];
            const int col = col_base + j * 32;
            // Visits the 16 accumulators of block (i, j) inside the matrix as
            // (r, row, EL(ptr)), EL(ptr) being the element (row, col) of an
            // [M, ldc] operand.
#define FORGE_EPI_EACH(BODY)                                                     \
    _Pragma("unroll") for (int r = 0; r < 16; r++) {                             \
        const int row = row_base + i * 32 + 8 * (r >> 2) + (r & 3);              \
        if (row >= p.M || col >= p.N) continue;                                  \
        const long long idx = (long long)row * p.ldc + col;                      \
        BODY;                                                                    \
    }
#define EL(ptr) (*((ptr) + idx))
            // The same, one element at a time: the scheduler may not
            // interleave the (long) activation code of several elements,
            // which would need registers for all of them at once.
#define FORGE_EPI_EACH_SEQ(BODY) FORGE_EPI_EACH(BODY; __builtin_amdgcn_sched_barrier(0))
            if constexpr (EPI) {
                // Block by block, the fused steps run as separate passes over
                // the block's accumulators, each under one uniform branch:
                // the optional steps neither multiply the unrolled code nor
                // keep more than one block's operands live.  Per element the
                // order (alpha, row divide, row subtrahend, bias, residual,
                // aux, pre_out, activation, store or update) is that of
                // gemm_epilogue_store.
                if (p.alpha != 1.0f) FORGE_EPI_EACH(a[r] = p.alpha * a[r]);
                if (p.row_d && (p.row_div & 1)) {
                    FORGE_EPI_EACH(a[r] = a[r] / p.row_d[row]);
                }
                if (p.row_sub) {
                    FORGE_EPI_EACH(a[r] = a[r] - p.row_sub[row]);
                }
                if (p.bias && col < p.N) {
                    const float b = p.bias[col];
                    FORGE_EPI_EACH(a[r] = a[r] + b);
                }
                if (p.residual) {
                    if (p.row_d && (p.row_div & 2)) {
                        FORGE_EPI_EACH(a[r] = a[r] + EL(p.residual) / p.row_d[row]);
                    } else {
                        FORGE_EPI_EACH(a[r] = a[r] + EL(p.residual));
                    }
                }
                if (p.aux) {
                    switch (p.aux_act) {
                    case ACT_GELU: FORGE_EPI_EACH_SEQ(a[r] = a[r] * gelu_derivative(EL(p.aux))); break;
                    case ACT_RELU: FORGE_EPI_EACH_SEQ(a[r] = a[r] * relu_derivative(EL(p.aux))); break;
                    case ACT_SILU: FORGE_EPI_EACH_SEQ(a[r] = a[r] * silu_derivative(EL(p.aux))); break;
                    default: FORGE_EPI_EACH(a[r] = a[r] * EL(p.aux)); break;
                    }
                }
                if (p.pre_out) FORGE_EPI_EACH(EL(p.pre_out) = a[r]);
                switch (p.act) {
                case ACT_GELU: FORGE_EPI_EACH_SEQ(a[r] = gelu(a[r])); break;
                case ACT_RELU: FORGE_EPI_EACH_SEQ(a[r] = relu(a[r])); break;
                case ACT_SILU: FORGE_EPI_EACH_SEQ(a[r] = silu(a[r])); break;
                default: break;
                }
                if (p.update) {
                    FORGE_EPI_EACH(EL(p.C) = EL(p.C) - p.update_scale * a[r]);
                } else {
                    FORGE_EPI_EACH(EL(p.C) = a[r]);
                }
            } else {
                FORGE_EPI_EACH(EL(p.C) = a[r]);
            }
#undef EL
#undef FORGE_EPI_EACH_SEQ
#undef FORGE_EPI_EACH
        }
    }
}

// One guarded GEMM per launch: grid = tiles.
template <int BM, int BN, int BK, int WARPS_M, int WARPS_N, bool TA, bool TB, bool EPI>
__device__ __forceinline__ void gemm_single_guarded(const GemmArgs& p) {
    gemm_body_guarded<BM, BN, BK, WARPS_M, WARPS_N, TA, TB, EPI>(
        p, xcd_logical(blockIdx.x, gridDim.x));
}

// Sum of the split-K partial products P[s] ([splits][M][N], row pitch N) in
// split order, then the GEMM epilogue of p into p.C (row pitch p.ldc).  The
// order of the sum depends only on the shape, so results are deterministic.
constexpr int SPLITK_THREADS = 256;  // launch size of the reduce kernels
template <bool VEC>
__device__ __forceinline__ void splitk_reduce_body(const float* __restrict__ P, int splits,
                                                   const GemmArgs& p) {
    const long long MN = (long long)p.M * p.N;
    constexpr int W = VEC ? 4 : 1;  // VEC requires N % 4 == 0 and a 16-byte aligned P
    const long long stride = (long long)gridDim.x * SPLITK_THREADS * W;
    // (row, col0) of e, advanced with the grid stride without a 64-bit
    // division per step (which, with the epilogue's operands, would exceed
    // the scalar registers).
    long long e = ((long long)blockIdx.x * SPLITK_THREADS + threadIdx.x) * W;
    int row = (int)(e / p.N), col0 = (int)(e % p.N);
    const int srow = (int)(stride / p.N), scol = (int)(stride % p.N);
    for (; e < MN; e += stride, row += srow, col0 += scol) {
        if (col0 >= p.N) {
            col0 -= p.N;
            row++;
        }
        float z[W];
        if constexpr (VEC) {
            // All slices are loaded before the sum (up to 8 in flight), then
            // added in slice order.
            float4 u[GEMM_BATCH_MAX];
#pragma unroll
            for (int s = 0; s < GEMM_BATCH_MAX; s++)
                if (s < splits) u[s] = load_stream(P + s * MN + e);
            z[0] = u[0].x; z[1] = u[0].y; z[2] = u[0].z; z[3] = u[0].w;
#pragma unroll
            for (int s = 1; s < GEMM_BATCH_MAX; s++) {
                if (s < splits) {
                    z[0] += u[s].x; z[1] += u[s].y; z[2] += u[s].z; z[3] += u[s].w;
                }
            }
        } else {
            z[0] = P[e];
            for (int s = 1; s < splits; s++) z[0] += P[s * MN + e];
        }
#pragma unroll
        for (int w = 0; w < W; w++)
            gemm_epilogue_store(p, (long long)row * p.ldc + col0 + w, row, col0 + w, z[w]);
    }
}

}  // namespace forge
