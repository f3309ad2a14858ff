// gemm.hpp -- fp32 GEMM on CDNA4 matrix cores.
//
// Replaces matrix_multiply_device (reference gemm.rs:202-373, TF32 mma.sync)
// with true fp32 v_mfma_f32_32x32x2_f32.  Semantics follow the strict-fp32
// kernel gemm.rs:15-129: C = A * B, row-major, C overwritten, f32 accumulate.
//
// Structure
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
};

constexpr int GEMM_GROUP_M = 8;
constexpr int LDS_PAD = 4;

// Maps the hardware workgroup id to a (tile_m, tile_n) pair; see the file
// comment.  Correctness does not depend on the dispatch order.
__device__ __forceinline__ void gemm_tile_coords(int num_m, int num_n,
                                                 int& tm, int& tn) {
    const int nwg = num_m * num_n;
    const int b = blockIdx.x;
    const int per_xcd = nwg / 8, rem = nwg % 8;
    const int xcd = b % 8, local = b / 8;
    const int logical = xcd < rem ? xcd * (per_xcd + 1) + local
                                  : rem * (per_xcd + 1) + (xcd - rem) * per_xcd + local;
    const int in_group = GEMM_GROUP_M * num_n;
    const int group = logical / in_group;
    const int first_m = group * GEMM_GROUP_M;
    const int gsize = min(num_m - first_m, GEMM_GROUP_M);
    const int r = logical % in_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

// Loads a ROWS x COLS tile (COLS contiguous in global memory) into registers,
// COLS/4 four-float vectors per row, dealt over NT threads.  GUARD zero-fills
// outside [vr, vc) and uses scalar loads (no alignment assumption).  The
// staging registers are the native 4-float vector f4 so they stay in VGPRs.

template <int ROWS, int COLS, int NT>
struct TileShape {
    static constexpr int F4_PER_ROW = COLS / 4;
    static constexpr int TOTAL = ROWS * F4_PER_ROW;
    static constexpr int PER_THREAD = TOTAL / NT;
    static_assert(TOTAL % NT == 0, "tile must divide evenly over threads");
};

template <int ROWS, int COLS, int NT, bool GUARD>
__device__ __forceinline__ void tile_load(f4* __restrict__ v,
                                          const float* __restrict__ g, long long ld,
                                          int vr, int vc) {
    using S = TileShape<ROWS, COLS, NT>;
#pragma unroll
    for (int i = 0; i < S::PER_THREAD; i++) {
        const int f = threadIdx.x + i * NT;
        const int r = f / S::F4_PER_ROW;
        const int c = (f % S::F4_PER_ROW) * 4;
        const float* q = g + (long long)r * ld + c;
        if constexpr (!GUARD) {
            v[i] = *reinterpret_cast<const f4*>(q);
        } else {
            const bool rok = r < vr;
            v[i].x = (rok && c + 0 < vc) ? q[0] : 0.0f;
            v[i].y = (rok && c + 1 < vc) ? q[1] : 0.0f;
            v[i].z = (rok && c + 2 < vc) ? q[2] : 0.0f;
            v[i].w = (rok && c + 3 < vc) ? q[3] : 0.0f;
        }
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

template <int BM, int BN, int BK, int WARPS_M, int WARPS_N, bool TA, bool TB,
          bool GUARD, bool EPI>
__device__ __forceinline__ void gemm_body(const GemmArgs& p) {
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
    gemm_tile_coords(num_m, num_n, tm, tn);
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
        tile_load<A_ROWS, A_COLS, NT, GUARD>(ra, a_base + (KT_) * a_kstride, p.lda, \
                                             TA ? kv_ : a_vr, TA ? a_vc : kv_);      \
        tile_load<B_ROWS, B_COLS, NT, GUARD>(rb, b_base + (KT_) * b_kstride, p.ldb, \
                                             TB ? b_vr : kv_, TB ? kv_ : b_vc);      \
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
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = n0 + wn * WN + j * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (GUARD && (row >= p.M || col >= p.N)) continue;
                const long long idx = (long long)row * p.ldc + col;
                float z = acc[i][j][r];
                if constexpr (EPI) {
                    if (p.alpha != 1.0f) z = p.alpha * z;
                    if (p.bias) z = z + p.bias[col];
                    if (p.residual) z = z + p.residual[idx];
                    if (p.aux) {
                        const float m = p.aux_act ? activate_derivative(p.aux_act, p.aux[idx])
                                                  : p.aux[idx];
                        z = z * m;
                    }
                    if (p.pre_out) p.pre_out[idx] = z;
                    const float y = activate(p.act, z);
                    if (p.update) p.C[idx] = p.C[idx] - p.update_scale * y;
                    else p.C[idx] = y;
                } else {
                    p.C[idx] = z;
                }
            }
        }
    }
}

}  // namespace forge
