// gemm_x.hpp -- fp32 GEMM on CDNA4 matrix cores, WM x WN wave layout
// (2 x 2, or 4 x 2 for the eight-wave 64x128 tile) with
// v_mfma_f32_16x16x4_f32 and 128-bit LDS operand reads.
//
// Same contract as gemm_body (gemm.hpp): C = A * B row-major, f32 accumulate,
// the same fused epilogue; unguarded (M % BM == N % BN == K % BK == 0,
// 16-byte aligned operands, row pitches up to 2^21 floats).
//
// Structure
//   - A workgroup of WM x WN waves computes a BM x BN tile; each wave owns a
//     (BM/WM) x (BN/WN) sub-tile of FM x FN blocks of 16 x 16, whose
//     accumulators (four floats per lane per block) stay in registers.  The
//     slab loads split evenly over all the waves.  Eight waves keep two
//     waves per SIMD where a CU holds a single workgroup.
//   - One MFMA sums four k values, lane group kq = lane / 16 supplying one.
//     Inside a 16-wide k chunk, sub-step s (0..3) gives lane group kq the
//     value k = 4 kq + s.  (Built with -DFORGE_GEMM_MF=32, wave sub-tiles of
//     32 or more rows and columns use 32 x 32 blocks and
//     v_mfma_f32_32x32x2_f32 instead: two lane groups, 8-wide chunks,
//     k = 4 kh + s, the same slabs and reads otherwise.  It gives the same
//     results to within rounding and ran slower on the 2048-row products and
//     in the transformer layers, so the default build keeps 16 x 16.)
//     A lane's operands for a whole chunk are therefore
//     one 128-bit LDS read per block for an operand that is k-contiguous in
//     LDS (A, or B^T), and one 128-bit read per sub-step for an operand that
//     is m/n-contiguous (B, or A^T).  For the latter the four floats of a
//     read belong to four different blocks: block 4g + e holds rows (or
//     columns) base + 64 g + 4 i + e for MFMA index i.  The epilogue undoes
//     this mapping, and the four columns of a lane become one 128-bit store.
//   - K advances in BK slabs through two LDS stages, loaded straight from
//     global memory into LDS (XDma) one slab ahead.  Slab kt + 1 is waited
//     for, and slab kt + 2 requested, in the middle of slab kt's last chunk.
//   - The main loop issues no vector instructions besides the MFMAs, the
//     LDS operand reads and the slab loads: every address is a precomputed
//     per-lane offset plus scalar registers and immediates.  On gfx950 each
//     other vector instruction between MFMAs costs the matrix pipe about
//     seven cycles (a loop of 128 MFMAs with 32 added VALU instructions
//     runs at 92% of the MFMA rate, with 64 at 89%); scalar instructions
//     cost nothing.
//   - The epilogue goes through LDS: each wave writes its sub-tile there and
//     streams it back as 128-bit rows with the fused steps.
#pragma once
#include "gemm.hpp"

namespace forge {

typedef float v4f __attribute__((ext_vector_type(4)));

template <int F>
struct XVec {
    // Floats per 128/64/32-bit operand read of an m/n-contiguous operand.
    static constexpr int W = F >= 4 ? 4 : F;
    static_assert(F % W == 0, "block count must be a multiple of the read width");
};

// Row (or column) of MFMA index i of block b in a wave sub-tile starting at
// base: k-contiguous operands keep blocks contiguous, m/n-contiguous ones
// interleave them W at a time.
template <bool KC, int F, int MF = 16>
__device__ __forceinline__ int x_index(int base, int b, int i) {
    if constexpr (KC) {
        return base + MF * b + i;
    } else {
        constexpr int W = XVec<F>::W;
        return base + MF * W * (b / W) + W * i + (b % W);
    }
}

// Direct global -> LDS slab loads (global_load_lds_dwordx4): each wave
// instruction fills 1 KiB of LDS, 16 bytes per lane in lane order, from one
// 16-byte piece of the global tile per lane.  A slab is ROWS x COLS floats
// of the global orientation (COLS contiguous); piece q of the LDS slab holds
// row q / P, piece (q % P) ^ swz(row) of that row, P = COLS / 4.  For the
// k-contiguous operand the swizzle makes the 128-bit reads of sixteen
// consecutive rows free of bank conflicts.  The XOR masks were chosen by
// measurement (SQ_LDS_BANK_CONFLICT on gfx950, every read pattern of the
// kernel): row & 7 for 8 pieces per row and row & 15 for 16 are
// conflict-free, while (row & 7) ^ ((row >> 3) & 1), row & 7 with 16 pieces
// and unswizzled rows cost two to four times the read cycles.  The
// m/n-contiguous operand is read contiguously and stored unswizzled.
template <int P, bool SWZ>
__device__ __forceinline__ int x_swz(int row) {
    if constexpr (!SWZ) return 0;
    else if constexpr (P == 8) return row & 7;
    else if constexpr (P == 16) return row & 15;
    else static_assert(P == 8 || P == 16, "k-contiguous slabs are 32 or 64 wide");
    return 0;
}

template <int ROWS, int COLS, bool SWZ, int NW = 4>
struct XSlab {
    static constexpr int P = COLS / 4;
    static constexpr int RPI = 64 / P;          // rows per wave instruction
    static constexpr int INSTR = ROWS * P / 64;  // wave instructions per slab
    static constexpr int PER_WAVE = INSTR / NW;
    static_assert(P <= 64 && 64 % P == 0, "a wave instruction fills whole rows");
    static_assert(INSTR % NW == 0, "slab must split evenly over the waves");
};

// Slab loads of one operand (buffer_load_dwordx4 ... lds).  A lane's byte
// offset from the first row its instruction fills (its row within the
// instruction times the row pitch, plus its swizzled piece) does not depend
// on the slab, so it is computed once (the vector offset); the buffer
// descriptor (the slab's first element), the instruction's row offset (the
// scalar offset) and the LDS destination (M0) are wave-uniform and live in
// scalar registers.  The main loop then spends no vector instructions on
// addresses: each vector instruction between MFMAs costs the matrix pipe
// several cycles, scalar ones do not.  Row pitches up to 2^21 floats keep
// the offsets (at most 256 rows into the slab) below 2^31 bytes; the host
// sends larger ones to the guarded kernel.
template <int ROWS, int COLS, bool SWZ, int NW = 4>
struct XDma {
    using S = XSlab<ROWS, COLS, SWZ, NW>;
    unsigned off[S::PER_WAVE];

    __device__ __forceinline__ void init(long long ld, int wave, int lane) {
#pragma unroll
        for (int i = 0; i < S::PER_WAVE; i++) {
            const int inst = wave * S::PER_WAVE + i;
            const int r = lane / S::P;
            const int piece = (lane % S::P) ^ x_swz<S::P, SWZ>(inst * S::RPI + r);
            off[i] = (unsigned)(r * ld + 4 * piece) * 4u;
        }
    }
    // Slab starting at g (wave-uniform) into LDS at lds (wave-uniform).
    __device__ __forceinline__ void load(float* lds, const float* __restrict__ g, long long ld,
                                         int wave) const {
        // Raw buffer, no range limit below 4 GiB; 0x00020000 is the gfx9
        // word 3 (32-bit data format, no swizzle).
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc((void*)g, (short)0, -1, 0x00020000);
#pragma unroll
        for (int i = 0; i < S::PER_WAVE; i++) {
            const int inst = wave * S::PER_WAVE + i;
            const unsigned row_bytes = (unsigned)(inst * S::RPI) * (unsigned)ld * 4u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsrc, (void __attribute__((address_space(3)))*)(lds + inst * 256), 16, off[i],
                row_bytes, 0, 0);
        }
    }
};

// Operand fragments of one 16-wide k chunk from a slab laid out by XDma:
// frag[b * 4 + s] is block b's value at sub-step s.  The lane's offset (in
// floats, from the start of the LDS array) is precomputed per stage and
// chunk, so each read is one base register plus an immediate.
template <bool KC, int ROWS, int BK, int F, int MF = 16>
struct XFrag {
    static constexpr int KCH = 4 * (64 / MF);  // k values per chunk
    static constexpr int CH = BK / KCH;
    int off[2][CH];

    // stage0: LDS offset of this operand in stage 0; stride: between stages;
    // base: the wave's first row (k-contiguous, a multiple of 16) or column;
    // lr, kg: the lane's row in an MFMA block and its k group.
    __device__ __forceinline__ void init(int stage0, int stride, int base, int lr, int kg) {
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
            for (int c = 0; c < CH; c++) {
                if constexpr (KC) {
                    // Rows base + MF b + lr all have the swizzle of row lr.
                    off[st][c] = stage0 + st * stride + (base + lr) * BK +
                                 4 * ((c * (KCH / 4) + kg) ^ x_swz<BK / 4, true>(lr));
                } else {
                    off[st][c] = stage0 + st * stride + (c * KCH + 4 * kg) * ROWS + base +
                                 XVec<F>::W * lr;
                }
            }
    }
    // stage and chunk are constants once the caller's loops are unrolled.
    __device__ __forceinline__ void load(const float* __restrict__ lds, int stage, int chunk,
                                         float (&frag)[F * 4]) const {
        const float* s = lds + off[stage][chunk];
        if constexpr (KC) {
#pragma unroll
            for (int b = 0; b < F; b++) {
                const f4 v = *reinterpret_cast<const f4*>(s + MF * b * BK);
                frag[b * 4 + 0] = v.x;
                frag[b * 4 + 1] = v.y;
                frag[b * 4 + 2] = v.z;
                frag[b * 4 + 3] = v.w;
            }
        } else {
            constexpr int W = XVec<F>::W;
#pragma unroll
            for (int st = 0; st < 4; st++) {
#pragma unroll
                for (int g = 0; g < F / W; g++) {
                    const float* q = s + st * ROWS + MF * W * g;
                    if constexpr (W == 4) {
                        const f4 v = *reinterpret_cast<const f4*>(q);
                        frag[(4 * g + 0) * 4 + st] = v.x;
                        frag[(4 * g + 1) * 4 + st] = v.y;
                        frag[(4 * g + 2) * 4 + st] = v.z;
                        frag[(4 * g + 3) * 4 + st] = v.w;
                    } else if constexpr (W == 2) {
                        const float2 v = *reinterpret_cast<const float2*>(q);
                        frag[(2 * g + 0) * 4 + st] = v.x;
                        frag[(2 * g + 1) * 4 + st] = v.y;
                    } else {
                        frag[g * 4 + st] = q[0];
                    }
                }
            }
        }
    }
};

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void x_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier after waiting for this wave's slab loads down to N
// outstanding.  __syncthreads() would also wait for the loads of the slab
// after (its release fence waits for every outstanding load into LDS); the
// explicit count keeps that slab in flight.  The empty asm statements stop
// the compiler from moving memory accesses across the barrier.
template <int N>
__device__ __forceinline__ void x_barrier() {
    x_wait_vmcnt<N>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The same after this wave's slab loads and LDS reads have all completed.
__device__ __forceinline__ void x_barrier_all() {
    __builtin_amdgcn_s_waitcnt((0x7 << 4));  // vmcnt(0) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// LDS read instructions per chunk for one operand (x_load_frag_dma).
template <bool KC, int F>
struct XReads {
    static constexpr int N = KC ? F : 4 * (F / XVec<F>::W);
};

// Fused epilogue of one 128-bit group of C at flat index idx, column col:
// the operands (residual, aux, old C, the row subtrahend) are loaded first so
// a batch of groups has its reads in flight together, then per element
// alpha, row divide, row subtrahend, bias, residual, aux (or act'(aux)),
// pre-activation store, activation, and store or SGD update -- the order of
// gemm_epilogue_store, each one rounded f32 operation.
template <bool EPI, bool ROWSUB>
__device__ __forceinline__ void x_epi_load(const GemmArgs& p, long long idx, int row, f4& res,
                                           f4& mul, f4& old, float& sub) {
    res = mul = old = f4{0.0f, 0.0f, 0.0f, 0.0f};
    sub = 0.0f;
    if constexpr (EPI) {
        if (p.residual) res = *reinterpret_cast<const f4*>(p.residual + idx);
        if (p.aux) mul = *reinterpret_cast<const f4*>(p.aux + idx);
        if (p.update) old = *reinterpret_cast<const f4*>(p.C + idx);
        if constexpr (ROWSUB) {
            if (p.row_sub) sub = p.row_sub[row];
        }
    }
}

// The fused steps of NB groups at once.  bias: this lane's four bias values
// (its columns are the same in every group, so they are loaded once per
// tile).  Each choice of step (activation, derivative) is made once for the
// NB groups rather than per element, so the arithmetic of all 4 NB values
// is one straight run of instructions.
template <int NB>
__device__ __forceinline__ void x_epi_apply(int act, float (&y)[4 * NB]) {
    switch (act) {
    case ACT_GELU:
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) y[i] = gelu(y[i]);
        break;
    case ACT_RELU:
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) y[i] = relu(y[i]);
        break;
    case ACT_SILU:
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) y[i] = silu(y[i]);
        break;
    default:
        break;
    }
}

template <int NB>
__device__ __forceinline__ void x_epi_aux(int aux_act, float (&y)[4 * NB],
                                          const float (&m)[4 * NB]) {
    switch (aux_act) {
    case ACT_IDENTITY:
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) y[i] = y[i] * m[i];
        break;
    case ACT_GELU:
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) y[i] = y[i] * gelu_derivative(m[i]);
        break;
    case ACT_RELU:
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) y[i] = y[i] * relu_derivative(m[i]);
        break;
    case ACT_SILU:
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) y[i] = y[i] * silu_derivative(m[i]);
        break;
    default:
#pragma unroll
        for (int i = 0; i < 4 * NB; i++) y[i] = y[i] * activate_derivative(aux_act, m[i]);
        break;
    }
}

// The row statistics of the fused epilogue.  rinv: 1 / d of each group's
// row (formed by the workgroup in LDS from row_part); row: the group's
// global row, for row_sq.
template <int NB>
struct XRowStats {
    float rinv[NB];
    int row[NB];
};

template <bool EPI, int NB, bool STATS = false, bool ROWSUB = false>
__device__ __forceinline__ void x_epi_store(const GemmArgs& p, const f4 (&z)[NB],
                                            const f4 (&res)[NB], const f4 (&mul)[NB],
                                            const f4 (&old)[NB], const float (&sub)[NB], f4 bias,
                                            const long long (&idx)[NB], const XRowStats<NB>& rs,
                                            int lane_col, float (&cs)[4]) {
    float y[4 * NB];
#pragma unroll
    for (int u = 0; u < NB; u++) {
        y[4 * u + 0] = z[u].x; y[4 * u + 1] = z[u].y;
        y[4 * u + 2] = z[u].z; y[4 * u + 3] = z[u].w;
    }
    if constexpr (EPI) {
        if (p.alpha != 1.0f)
#pragma unroll
            for (int i = 0; i < 4 * NB; i++) y[i] = p.alpha * y[i];
        // RMSNorm folded across the boundary: (x / d_r) W = (x W) / d_r,
        // taken as a product with 1 / d_r.
        if constexpr (STATS) {
            if (p.row_part && (p.row_div & 1))
#pragma unroll
                for (int i = 0; i < 4 * NB; i++) y[i] = y[i] * rs.rinv[i / 4];
        }
        // The row subtrahend (the _r instances only).
        if constexpr (ROWSUB) {
            if (p.row_sub)
#pragma unroll
                for (int i = 0; i < 4 * NB; i++) y[i] = y[i] - sub[i / 4];
        }
        if (p.bias)
#pragma unroll
            for (int u = 0; u < NB; u++) {
                y[4 * u + 0] = y[4 * u + 0] + bias.x; y[4 * u + 1] = y[4 * u + 1] + bias.y;
                y[4 * u + 2] = y[4 * u + 2] + bias.z; y[4 * u + 3] = y[4 * u + 3] + bias.w;
            }
        if (p.residual) {
            f4 r[NB];
#pragma unroll
            for (int u = 0; u < NB; u++) r[u] = res[u];
            if constexpr (STATS) {
                if (p.row_part && (p.row_div & 2))
#pragma unroll
                    for (int u = 0; u < NB; u++) {
                        r[u].x = r[u].x * rs.rinv[u]; r[u].y = r[u].y * rs.rinv[u];
                        r[u].z = r[u].z * rs.rinv[u]; r[u].w = r[u].w * rs.rinv[u];
                    }
            }
#pragma unroll
            for (int u = 0; u < NB; u++) {
                y[4 * u + 0] = y[4 * u + 0] + r[u].x; y[4 * u + 1] = y[4 * u + 1] + r[u].y;
                y[4 * u + 2] = y[4 * u + 2] + r[u].z; y[4 * u + 3] = y[4 * u + 3] + r[u].w;
            }
        }
        if (p.aux) {
            float m[4 * NB];
#pragma unroll
            for (int u = 0; u < NB; u++) {
                m[4 * u + 0] = mul[u].x; m[4 * u + 1] = mul[u].y;
                m[4 * u + 2] = mul[u].z; m[4 * u + 3] = mul[u].w;
            }
            x_epi_aux<NB>(p.aux_act, y, m);
        }
        if (p.pre_out)
#pragma unroll
            for (int u = 0; u < NB; u++)
                __builtin_nontemporal_store(f4{y[4 * u], y[4 * u + 1], y[4 * u + 2], y[4 * u + 3]},
                                            reinterpret_cast<f4*>(p.pre_out + idx[u]));
        if (p.act != ACT_IDENTITY) x_epi_apply<NB>(p.act, y);
        if (p.update)
#pragma unroll
            for (int u = 0; u < NB; u++) {
                y[4 * u + 0] = old[u].x - p.update_scale * y[4 * u + 0];
                y[4 * u + 1] = old[u].y - p.update_scale * y[4 * u + 1];
                y[4 * u + 2] = old[u].z - p.update_scale * y[4 * u + 2];
                y[4 * u + 3] = old[u].w - p.update_scale * y[4 * u + 3];
            }
        if (STATS && p.row_sq) {
            // Sum of squares over each 32-column block of the row: the eight
            // lanes of a block (consecutive lanes hold consecutive float4
            // columns of one row) add their four squares, then a xor tree.
            const int parts = p.N >> 5;
#pragma unroll
            for (int u = 0; u < NB; u++) {
                float q = y[4 * u] * y[4 * u];
                q = q + y[4 * u + 1] * y[4 * u + 1];
                q = q + y[4 * u + 2] * y[4 * u + 2];
                q = q + y[4 * u + 3] * y[4 * u + 3];
                q = q + __shfl_xor(q, 1, 64);
                q = q + __shfl_xor(q, 2, 64);
                q = q + __shfl_xor(q, 4, 64);
                if ((threadIdx.x & 7) == 0)
                    p.row_sq[(long long)rs.row[u] * parts + (lane_col >> 5)] = q;
            }
        }
        if (STATS && p.col_part)
#pragma unroll
            for (int u = 0; u < NB; u++) {
                cs[0] = cs[0] + y[4 * u + 0]; cs[1] = cs[1] + y[4 * u + 1];
                cs[2] = cs[2] + y[4 * u + 2]; cs[3] = cs[3] + y[4 * u + 3];
            }
    }
    // Results are stored non-temporally, which measured faster than
    // write-allocating stores: C4 forward 0.5252 -> 0.5234 ms, C5 step
    // 11.530 -> 11.514 ms, the 2048-row products up to 1%, 4096^3 unchanged.
#pragma unroll
    for (int u = 0; u < NB; u++)
        __builtin_nontemporal_store(f4{y[4 * u], y[4 * u + 1], y[4 * u + 2], y[4 * u + 3]},
                                    reinterpret_cast<f4*>(p.C + idx[u]));
}

#ifndef FORGE_GEMM_MF
#define FORGE_GEMM_MF 16
#endif

template <int BM, int BN, int BK, bool TA, bool TB, bool EPI, int WM = 2, int WN = 2,
          bool STATS = false, bool ROWSUB = false, bool SEGK = false>
__device__ __forceinline__ void gemm_body_x(const GemmArgs& p, int logical) {
    static_assert(EPI || !STATS, "row statistics ride on the fused epilogue");
    static_assert(!ROWSUB || STATS, "the row subtrahend rides on the statistics instances");
    constexpr int NW = WM * WN;  // waves: WM x WN sub-tiles of TM x TN
    constexpr int TM = BM / WM, TN = BN / WN;
    // MFMA block: 16 x 16 (v_mfma_f32_16x16x4_f32, four k per instruction,
    // four lane groups) or 32 x 32 (v_mfma_f32_32x32x2_f32, two k, two
    // lane groups).
    constexpr int MF = (FORGE_GEMM_MF == 32 && TM % 32 == 0 && TN % 32 == 0) ? 32 : 16;
    constexpr int FM = TM / MF, FN = TN / MF;
    constexpr int KCH = 4 * (64 / MF);  // k values per chunk (four sub-steps)
    constexpr int CH = BK / KCH;
    constexpr int NACC = MF * MF / 64;  // accumulators per lane per block
    typedef float vacc __attribute__((ext_vector_type(NACC)));
    static_assert(TM % MF == 0 && TN % MF == 0 && BK % KCH == 0, "tile shape");
    constexpr bool A_KC = !TA, B_KC = TB;

    constexpr int A_ROWS = TA ? BK : BM, A_COLS = TA ? BM : BK;
    constexpr int B_ROWS = TB ? BN : BK, B_COLS = TB ? BK : BN;
    constexpr int A_ELEMS = A_ROWS * A_COLS;
    constexpr int B_ELEMS = B_ROWS * B_COLS;
    constexpr int STAGE = A_ELEMS + B_ELEMS;
    using SA = XSlab<A_ROWS, A_COLS, A_KC, NW>;
    using SB = XSlab<B_ROWS, B_COLS, B_KC, NW>;
    constexpr int DMA_PER_STAGE = SA::PER_WAVE + SB::PER_WAVE;
    static_assert(CH % 2 == 0, "slabs hold an even number of 16-wide chunks");
    // The two slab stages, reused by the epilogue for each wave's TM x TN
    // sub-tile of C (row pitch CP).
    constexpr int CP = TN + 4;
    constexpr int EPI_ELEMS = NW * TM * CP;
    constexpr int SMEM = 2 * STAGE > EPI_ELEMS ? 2 * STAGE : EPI_ELEMS;
    // The fused epilogue's row scales (row_part) follow the stages.
    constexpr int ROWD = STATS ? BM : 0;
    static_assert((SMEM + ROWD) * 4 <= 160 * 1024, "LDS budget");
    __shared__ __attribute__((aligned(1024))) float smem_all[SMEM + ROWD];

    const int num_m = p.M / BM, num_n = p.N / BN;
    int tm, tn;
    gemm_tile_coords(logical, num_m, num_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // scalar
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & (MF - 1), kg = lane >> (MF == 16 ? 4 : 5);
    float* const smem = smem_all;

    const int KT = p.K / BK;
    const long long a_kstride = TA ? (long long)BK * p.lda : BK;
    const long long b_kstride = TB ? BK : (long long)BK * p.ldb;
    const float* a_base = TA ? p.A + m0 : p.A + (long long)m0 * p.lda;
    const float* b_base = TB ? p.B + (long long)n0 * p.ldb : p.B + n0;
    // K segments (SEGK): slab k of segment s reads A_s / B_s at k - s * kts.
    // The address is segment 0's plus a delta selected by integer masks, so
    // the main loop stays one branch-free instruction stream (a branch there
    // moves the accumulators out of registers).  Up to three segments; with
    // two, k never reaches 2 * kts.
    const int kts = SEGK ? p.k_seg / BK : KT;
    long long da1 = 0, da2 = 0, db1 = 0, db2 = 0;  // in floats
    if constexpr (SEGK) {
        auto delta = [](const float* seg, const float* base) {
            return (long long)((reinterpret_cast<intptr_t>(seg) -
                                reinterpret_cast<intptr_t>(base)) / (intptr_t)sizeof(float));
        };
        const long long am0 = TA ? m0 : (long long)m0 * p.lda;
        const long long bn0 = TB ? (long long)n0 * p.ldb : n0;
        da1 = delta(p.A1 + am0, a_base) - (long long)kts * a_kstride;
        db1 = delta(p.B1 + bn0, b_base) - (long long)kts * b_kstride;
        if (p.A2) {
            da2 = delta(p.A2 + am0, a_base) - 2LL * kts * a_kstride - da1;
            db2 = delta(p.B2 + bn0, b_base) - 2LL * kts * b_kstride - db1;
        }
    }

    vacc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = (vacc)(0.0f);

    // Fragment origins inside a slab: the wave's first row (KC) or column
    // offset (MC) of its sub-tile.
    const int a_off = wm * TM, b_off = wn * TN;
    float fa[2][FM * 4], fb[2][FN * 4];

    XDma<A_ROWS, A_COLS, A_KC, NW> dma_a;
    XDma<B_ROWS, B_COLS, B_KC, NW> dma_b;
    dma_a.init(p.lda, wave, lane);
    dma_b.init(p.ldb, wave, lane);
    XFrag<A_KC, A_KC ? BK : BM, BK, FM, MF> rd_a;
    XFrag<B_KC, B_KC ? BK : BN, BK, FN, MF> rd_b;
    rd_a.init(0, STAGE, a_off, lr, kg);
    rd_b.init(A_ELEMS, STAGE, b_off, lr, kg);

    auto issue = [&](int k_slab, int stage) {
        float* d = smem + stage * STAGE;
        if constexpr (SEGK) {
            const long long m1 = -(long long)(k_slab >= kts);
            const long long m2 = -(long long)(k_slab >= 2 * kts);
            dma_a.load(d, a_base + k_slab * a_kstride + (da1 & m1) + (da2 & m2), p.lda, wave);
            dma_b.load(d + A_ELEMS, b_base + k_slab * b_kstride + (db1 & m1) + (db2 & m2), p.ldb,
                       wave);
        } else {
            dma_a.load(d, a_base + k_slab * a_kstride, p.lda, wave);
            dma_b.load(d + A_ELEMS, b_base + k_slab * b_kstride, p.ldb, wave);
        }
    };
    auto frags = [&](int stage, int chunk, int slot) {
        rd_a.load(smem_all, stage, chunk, fa[slot]);
        rd_b.load(smem_all, stage, chunk, fb[slot]);
    };
    auto mfmas = [&](int slot, int st0, int st1) {
#pragma unroll
        for (int st = st0; st < st1; st++)
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    if constexpr (MF == 32)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            fa[slot][i * 4 + st], fb[slot][j * 4 + st], acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            fa[slot][i * 4 + st], fb[slot][j * 4 + st], acc[i][j], 0, 0, 0);
                }
    };
    // Instruction counts that the schedule below interleaves.
    constexpr int NMFMA = 4 * FM * FN;  // per chunk
    constexpr int NREAD = XReads<A_KC, FM>::N + XReads<B_KC, FN>::N;  // LDS reads per chunk
    constexpr int NDMA = DMA_PER_STAGE;  // slab loads per stage
    constexpr int MF_PER_READ = NMFMA / 2 / NREAD > 0 ? NMFMA / 2 / NREAD : 1;

    // Row scales of the folded RMSNorm (row_part): thread t < BM sums row
    // m0 + t's row_parts partial sums in index order (float4 loads when
    // row_parts % 4 == 0 and row_part is 16-byte aligned) and stores
    // 1 / sqrt(sum / n + eps) to LDS.  The block completes before the first
    // slab is requested: loads still in flight past it would make the launch
    // wait for all its slab loads before the main loop.
    if constexpr (STATS) {
        if (p.row_part && (int)threadIdx.x < BM) {
            const int parts = p.row_parts;
            const float* row = p.row_part + (long long)(m0 + (int)threadIdx.x) * parts;
            float t = 0.0f;
            if ((parts & 3) == 0 && (reinterpret_cast<uintptr_t>(p.row_part) & 15) == 0) {
                constexpr int RP_MAX = 8;  // float4 loads in flight per round
                const f4* src = reinterpret_cast<const f4*>(row);
                const int rp4 = parts >> 2;
                for (int j0 = 0; j0 < rp4; j0 += RP_MAX) {
                    f4 rp[RP_MAX];
#pragma unroll
                    for (int j = 0; j < RP_MAX; j++)
                        if (j0 + j < rp4) rp[j] = src[j0 + j];
#pragma unroll
                    for (int j = 0; j < RP_MAX; j++)
                        if (j0 + j < rp4) t = ((t + rp[j].x) + rp[j].y + rp[j].z) + rp[j].w;
                }
            } else {
                for (int j = 0; j < parts; j++) t += row[j];
            }
            smem_all[SMEM + threadIdx.x] = 1.0f / sqrtf(t / (float)p.row_n + p.row_eps);
        }
    }

    // Prologue: slabs 0 and 1 in flight, slab 0 waited for (K = 0 reads
    // nothing and stores zeros).
    if (KT > 0) {
        issue(0, 0);
        if (KT > 1) {
            issue(1, 1);
            x_barrier<DMA_PER_STAGE>();
        } else {
            x_barrier<0>();
        }
        frags(0, 0, 0);
    }
    // Slab kt lives in stage kt % 2; the loop handles two slabs per
    // iteration so that every stage (and so every LDS address offset) is a
    // constant.  A slab's last chunk is split: after the first half of its
    // MFMAs every wave has finished reading the stage (the operands are in
    // registers), so after one barrier the next slab's first operands are
    // read and the slab after next is loaded into this stage while the
    // second half of the MFMAs runs.  The loop body is the same instruction
    // stream in every iteration (no branches), which keeps the
    // accumulators in place; a load past the last slab repeats slab KT - 1
    // into the stage that is no longer read.
    constexpr int LAST = (CH - 1) & 1;
    auto early_chunks = [&](int stage) {
#pragma unroll
        for (int c = 0; c + 1 < CH; c++) {
            frags(stage, c + 1, (c + 1) & 1);
            mfmas(c & 1, 0, 4);
#pragma unroll
            for (int r = 0; r < NREAD; r++) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
                __builtin_amdgcn_sched_group_barrier(0x008, MF_PER_READ, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NMFMA - NREAD * MF_PER_READ, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // One slab that has a successor; issue_next: load slab kt + 2 (else no
    // load is left to issue).
    auto body = [&](int kt, int stage, bool issue_next) {
        early_chunks(stage);
        mfmas(LAST, 0, 2);
        __builtin_amdgcn_sched_barrier(0);
        // Slab kt + 1 was loaded one stage ago and is the only load in
        // flight; after the barrier no wave has an LDS read of slab kt
        // outstanding.
        x_barrier_all();
        frags(stage ^ 1, 0, 0);
        if (issue_next) issue(min(kt + 2, KT - 1), stage);
        mfmas(LAST, 2, 4);
#pragma unroll
        for (int r = 0; r < NREAD; r++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        if (issue_next) {
#pragma unroll
            for (int r = 0; r < NDMA; r++) {
                __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // one slab load
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    int kt = 0;
    for (; kt + 2 < KT; kt += 2) {
        body(kt, 0, true);
        body(kt + 1, 1, true);
    }
    // The last one or two slabs.
    if (KT - kt == 2) {
        body(kt, 0, false);
        early_chunks(1);
        mfmas(LAST, 0, 4);
    } else if (KT - kt == 1) {
        early_chunks(0);
        mfmas(LAST, 0, 4);
    }
    // No slab load may still be writing LDS when the workgroup ends.
    x_wait_vmcnt<0>();

    // Epilogue columns of this lane: group q = lane + 64 k of a TN-wide
    // sub-tile row covers columns 4 (q % F4_ROW) onwards, and F4_ROW divides
    // 64, so every group of the lane has the same four columns.  Their bias
    // is loaded here, while the accumulators go through LDS.
    constexpr int F4_ROW = TN / 4;
    static_assert(64 % F4_ROW == 0, "a lane's epilogue columns repeat every group");
    const int row0 = m0 + a_off, col0 = n0 + b_off;
    const int lane_col = col0 + 4 * (lane % F4_ROW);
    f4 bias4 = f4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (EPI) {
        if (p.bias) bias4 = *reinterpret_cast<const f4*>(p.bias + lane_col);
    }

    // Epilogue through LDS.  Each wave writes its accumulators as a plain
    // TM x TN sub-tile into its own LDS region (accumulator r at MFMA row
    // acc_row(r), column lane % MF), then streams the sub-tile
    // back row by row: four consecutive columns per lane, so operands and
    // results move as 128-bit accesses and the fused steps are one compact
    // loop instead of code unrolled over every accumulator.  A wave reads
    // only what it wrote, and LDS executes one wave's accesses in order.
    __syncthreads();  // every wave is done with the slab stages
    float* const cw = smem_all + wave * (TM * CP);
    // MFMA row of accumulator r: 4 kg + r in a 16 x 16 block; in a 32 x 32
    // block, 8 (r / 4) + 4 kg + r % 4.
    auto acc_row = [&](int r) { return MF == 16 ? 4 * kg + r : 8 * (r >> 2) + 4 * kg + (r & 3); };
    if constexpr (!B_KC && XVec<FN>::W == 4) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < NACC; r++) {
                const int rr = x_index<A_KC, FM, MF>(0, i, acc_row(r));
#pragma unroll
                for (int g = 0; g < FN / 4; g++) {
                    const f4 v = {acc[i][4 * g + 0][r], acc[i][4 * g + 1][r],
                                  acc[i][4 * g + 2][r], acc[i][4 * g + 3][r]};
                    *reinterpret_cast<f4*>(cw + rr * CP + 4 * MF * g + 4 * lr) = v;
                }
            }
    } else {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < NACC; r++) {
                const int rr = x_index<A_KC, FM, MF>(0, i, acc_row(r));
#pragma unroll
                for (int j = 0; j < FN; j++)
                    cw[rr * CP + x_index<B_KC, FN, MF>(0, j, lr)] = acc[i][j][r];
            }
    }
    asm volatile("" ::: "memory");
    constexpr int ITER = TM * F4_ROW / 64;  // 128-bit groups per lane
    // Groups whose operands load together.  Eight (every group of a 64 x 128
    // tile at once) raised the four-wave instances from 139-148 to 167-193
    // VGPRs: the C4 forward gained 0.45 us, the C5 step lost 44 us (six ABBA
    // pairs each).
    constexpr int NB = ITER < 4 ? ITER : 4;
    static_assert(ITER % NB == 0, "epilogue batches");
    float cs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
    for (int b0 = 0; b0 < ITER; b0 += NB) {
        // Loads of a batch first, so NB global reads per operand are in
        // flight together.
        f4 z[NB], res[NB], mul[NB], old[NB];
        float sub[NB];
        long long idx[NB];
        XRowStats<NB> rs;
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int q = lane + 64 * (b0 + u);
            const int rr = q / F4_ROW, c4 = q % F4_ROW;
            z[u] = *reinterpret_cast<const f4*>(cw + rr * CP + 4 * c4);
            idx[u] = (long long)(row0 + rr) * p.ldc + lane_col;
            rs.row[u] = row0 + rr;
            rs.rinv[u] = 1.0f;
            if constexpr (STATS) {
                if (p.row_part) rs.rinv[u] = smem_all[SMEM + a_off + rr];
            }
            x_epi_load<EPI, ROWSUB>(p, idx[u], row0 + rr, res[u], mul[u], old[u], sub[u]);
        }
        x_epi_store<EPI, NB, STATS, ROWSUB>(p, z, res, mul, old, sub, bias4, idx, rs, lane_col,
                                            cs);
    }
    if constexpr (STATS) {
        if (p.col_part) {
            // Lanes l, l + F4_ROW, ... hold the same four columns: a xor tree
            // over them, then lanes below F4_ROW store this wave's column sums
            // over its TM rows as partial row tm * WM + wm.
#pragma unroll
            for (int off = F4_ROW; off < 64; off <<= 1)
#pragma unroll
                for (int c = 0; c < 4; c++) cs[c] = cs[c] + __shfl_xor(cs[c], off, 64);
            if (lane < F4_ROW)
                *reinterpret_cast<f4*>(p.col_part + (long long)(tm * WM + wm) * p.N + lane_col) =
                    f4{cs[0], cs[1], cs[2], cs[3]};
        }
    }
}

template <int BM, int BN, int BK, bool TA, bool TB, bool EPI, int WM = 2, int WN = 2,
          bool STATS = false, bool ROWSUB = false, bool SEGK = false>
__device__ __forceinline__ void gemm_single_x(const GemmArgs& p) {
    gemm_body_x<BM, BN, BK, TA, TB, EPI, WM, WN, STATS, ROWSUB, SEGK>(
        p, xcd_logical(blockIdx.x, gridDim.x));
}

template <int BM, int BN, int BK, bool TA, bool TB, int WM = 2, int WN = 2>
__device__ __forceinline__ void gemm_batch_x(const GemmBatchArgs& b) {
    const int logical = xcd_logical(blockIdx.x, gridDim.x);
    const int z = logical / b.tiles;
    gemm_body_x<BM, BN, BK, TA, TB, true, WM, WN>(b.p[z], logical - z * b.tiles);
}

}  // namespace forge
