// rows.hpp -- row-wise kernels: softmax, LayerNorm, RMSNorm (forward and
// backward) and row sums.
//
// The reference runs one 1024-thread block per row with two-level warp-32
// shuffle trees through shared memory and asserts cols <= 1024
// (row.rs:16-468, norm.rs:12,30,54).  Here one 64-lane wavefront owns a row:
//   - register path: the row is held in VGPRs as VPT float4 per lane
//     (cols <= 256*VPT, cols % 4 == 0, 16-byte aligned rows), read once and
//     written once -- the HBM minimum;
//   - looping path: any cols and alignment; the row is streamed from global
//     memory once per reduction pass.
// Reductions are the DPP wave reductions of common.hpp, so there is no LDS
// traffic and no barrier.  Rows are walked grid-stride so the backward
// kernels can keep per-column dgamma/dbeta partials in registers across the
// rows a wave visits; partials are combined per workgroup in LDS and written
// as one row per workgroup, then summed by the column-sum kernel.
#pragma once
#include <float.h>
#include "common.hpp"

namespace forge {

constexpr int ROW_WAVES = 4;          // wavefronts (rows in flight) per workgroup
constexpr int ROW_PARTIAL_WAVES = 8;  // the same for the dgamma/dbeta partial kernels

struct RowArgs {
    const float* x;      // input (forward: in/out when y == x)
    float* y;            // output
    const float* dy;     // upstream gradient (backward)
    const float* gamma;  // [cols] or null
    const float* beta;   // [cols] or null
    float* pgamma;       // [gridDim.x, cols] partial dgamma or null
    float* pbeta;        // [gridDim.x, cols] partial dbeta or null
    int rows, cols;
    float eps;
    float scale;         // softmax backward: dx *= scale (1 = reference kernel)
    int nt_stores;       // 1: non-temporal stores at any size (set by the host)
    int lds_params;      // 1: LayerNorm forward stages gamma/beta in LDS (set by the host)
    // Norm backward row dot (the _d instances and the looping path):
    // dot[r] = dscale * sum_c dx[r, c] * (x[r, c] - dsub[r, c]).  With x the
    // attention output plus its residual input and dsub that input, x - dsub
    // is the attention output O = P V and the dot is the softmax backward's
    // row term sum_j P_rj dP_rj = sum_c dO_rc O_rc (dP = dO V^T).
    const float* dsub;   // [rows, cols] or null
    float* dot;          // [rows] or null
    float dscale;
};

enum RowOp {
    ROW_SOFTMAX = 0,
    ROW_LAYER_NORM = 1,
    ROW_RMS_NORM = 2,
    ROW_SOFTMAX_BWD = 3,
    ROW_LAYER_NORM_BWD = 4,
    ROW_RMS_NORM_BWD = 5
};

__device__ __forceinline__ float sum4(float4 a) { return (a.x + a.y) + (a.z + a.w); }

// exp(x - m) of the softmax as 2^((x - m) * log2 e) on v_exp_f32, with the
// row normalised by one reciprocal and a multiply per element.  Softmax is
// VALU-bound otherwise on gfx950 (a wave64 VALU instruction takes 4 cycles
// and the IEEE expf and divide cost about 25 of them per element).  The
// error against exact arithmetic is below 2e-6 relative for |x - m| < 30 and
// the result is at most 1e-13 below that range; masked -inf entries give 0.
__device__ __forceinline__ float softmax_exp(float x, float m) {
    constexpr float LOG2E = 1.44269504088896341f;
    return __builtin_amdgcn_exp2f((x - m) * LOG2E);
}
__device__ __forceinline__ float max4(float4 a) {
    return fmaxf(fmaxf(a.x, a.y), fmaxf(a.z, a.w));
}

#define F4_APPLY(dst, a, EXPR_X, EXPR_Y, EXPR_Z, EXPR_W) \
    do { dst.x = (EXPR_X); dst.y = (EXPR_Y); dst.z = (EXPR_Z); dst.w = (EXPR_W); } while (0)

// Row `row` into the register arrays of the register path, as loaded:
// every lane loads (past cols it reloads the row's first float4), and
// row_mask then puts the fill values (-FLT_MAX for softmax, 0 otherwise)
// past cols.  The two steps are apart so that a prefetched row is masked
// only when it is used: loads under a lane-mask branch, or a select right
// after them, make the wave wait for the loads at once (and, with loads
// under branches, for every memory operation in flight, its own stores of
// the previous row included).  Streaming loads: the forward kernels
// overwrite the row in place.
template <int OP, int VPT, bool BWD>
__device__ __forceinline__ void row_load(const RowArgs& a, int row, int lane, float4* v,
                                         float4* g) {
    const long long base = (long long)row * a.cols;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const int c = (i * 64 + lane) * 4;
        const long long at = base + (c < a.cols ? c : 0);
        v[i] = load_stream(a.x + at);
        if constexpr (BWD) g[i] = load_stream(a.dy + at);
    }
}

template <int OP, int VPT, bool BWD>
__device__ __forceinline__ void row_mask(const bool* ok, float4* v, float4* g) {
    const float fill = (OP == ROW_SOFTMAX) ? -FLT_MAX : 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        if (!ok[i]) v[i] = make_float4(fill, fill, fill, fill);
        if constexpr (BWD)
            if (!ok[i]) g[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// Register path.  VPT float4 per lane; lane l holds columns
// 4*(64*i + l) .. +3 for i < VPT.  WAVES wavefronts per workgroup, rows
// grid-stride.  The partial-producing backward kernels with at most 8 waves
// walk several rows per wave, so they prefetch the next row's registers
// before reducing the current one.
template <int OP, int VPT, bool PARTIALS, int WAVES = ROW_WAVES, bool DOT = false,
          bool PREFETCH = PARTIALS && WAVES <= 8 && !DOT>
__device__ __forceinline__ void row_kernel_reg(const RowArgs& a) {
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // scalar
    const int cols = a.cols;
    const float n = (float)cols;
    constexpr bool BWD = OP >= ROW_SOFTMAX_BWD;
    constexpr bool USES_GAMMA = OP == ROW_LAYER_NORM || OP == ROW_RMS_NORM ||
                                OP == ROW_LAYER_NORM_BWD || OP == ROW_RMS_NORM_BWD;
    constexpr bool USES_BETA = OP == ROW_LAYER_NORM;
    // gamma/beta are the same for every row: load them once, before the first
    // row's reductions, so their latency is not exposed per row.
    // (not in the 8-float4 partial kernels: with the prefetched row and the
    // column partials, 32 more registers would spill)
    constexpr bool PRELOAD = USES_GAMMA && VPT <= 8 && !(PARTIALS && VPT >= 8);
    float4 gm[PRELOAD ? VPT : 1], bt[(PRELOAD && USES_BETA) ? VPT : 1];
    // RMSNorm forward issues gamma's loads after the first row's (waits are
    // in issue order, and the row's reduction needs only the row): at
    // [4096,1024] 7.17 -> 6.81 us.  LayerNorm forward, which also loads
    // beta, measured slower that way (7.78 -> 8.01 us); it stages both
    // through LDS (below).
    constexpr bool LATE_PRELOAD = PRELOAD && OP == ROW_RMS_NORM;
    auto preload = [&]() {
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const int c = (i * 64 + lane) * 4;
            const bool in = c < cols;
            gm[i] = (a.gamma && in) ? *reinterpret_cast<const float4*>(a.gamma + c)
                                    : make_float4(1.f, 1.f, 1.f, 1.f);
            if constexpr (USES_BETA)
                bt[i] = (a.beta && in) ? *reinterpret_cast<const float4*>(a.beta + c)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    // LayerNorm forward below 64 MiB (the host sets lds_params) stages
    // gamma/beta in LDS once per workgroup instead of loading them per wave
    // (a quarter of the loads): [4096,1024] 8.16 -> 7.88 us, faster in each
    // of twelve paired runs; issuing the first row's loads before the
    // staging was slower (8.52).  At [65536,1024] the staging cost 1.3%
    // (84.5 -> 85.6 us, five paired runs), so larger launches load per wave.
    // The barrier is outside the row loop and lds_params is uniform, so
    // every wave reaches it.
    constexpr bool LDS_PARAMS = PRELOAD && OP == ROW_LAYER_NORM && !PARTIALS;
    if constexpr (LDS_PARAMS) {
        if (a.lds_params) {
            __shared__ float4 sgb[2 * VPT * 64];
            for (int t = threadIdx.x; t < VPT * 64; t += WAVES * 64) {
                const int c = t * 4;
                const bool in = c < cols;
                sgb[t] = (a.gamma && in) ? *reinterpret_cast<const float4*>(a.gamma + c)
                                         : make_float4(1.f, 1.f, 1.f, 1.f);
                sgb[VPT * 64 + t] = (a.beta && in)
                                        ? *reinterpret_cast<const float4*>(a.beta + c)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                gm[i] = sgb[i * 64 + lane];
                bt[i] = sgb[VPT * 64 + i * 64 + lane];
            }
        } else {
            preload();
        }
    } else if constexpr (PRELOAD && !LATE_PRELOAD) {
        preload();
    }
    bool first = true;
    // gamma / beta of float4 column group i (preloaded, or read per use).
    // Read per use, a group past cols reads the row's first group instead,
    // so the load stays in bounds wherever a caller evaluates it.
    auto gamma4 = [&](int i) -> float4 {
        if constexpr (PRELOAD) return gm[i];
        else {
            const int c = (i * 64 + lane) * 4;
            return *reinterpret_cast<const float4*>(a.gamma + (c < cols ? c : 0));
        }
    };
    auto beta4 = [&](int i) -> float4 {
        if constexpr (PRELOAD && USES_BETA) return bt[i];
        else {
            const int c = (i * 64 + lane) * 4;
            return *reinterpret_cast<const float4*>(a.beta + (c < cols ? c : 0));
        }
    };
    static_assert(!PARTIALS || OP == ROW_LAYER_NORM_BWD || OP == ROW_RMS_NORM_BWD,
                  "only the norm backward kernels produce column partials");
    static_assert(!DOT || OP == ROW_LAYER_NORM_BWD || OP == ROW_RMS_NORM_BWD,
                  "only the norm backward kernels produce the row dot");
    // The backward's g = dy * gamma for float4 group i of the current row;
    // past cols (ok false) it is 0 and gamma is not read.  Kept in registers
    // between the two passes where that fits: at 8 float4 per lane the
    // partial kernels would otherwise exceed 256 VGPRs and spill (the
    // LayerNorm backward at [4096,2048] took 38.7 us spilling against
    // 23-28 us recomputing).
    constexpr bool KEEP_G = VPT <= 4;
    auto gdy = [&](int i, float4 dy, bool ok) -> float4 {
        if (!a.gamma) return dy;
        if (!ok) return make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 gm = gamma4(i);
        return make_float4(dy.x * gm.x, dy.y * gm.y, dy.z * gm.z, dy.w * gm.w);
    };

    float4 pg[PARTIALS ? VPT : 1], pb[PARTIALS ? VPT : 1];
    if constexpr (PARTIALS) {
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            pg[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            pb[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }

    // Non-temporal stores from STREAM_NT_MIN on, or at any size when the
    // host asks (RowArgs::nt_stores: the forward kernels).
    const bool nt = a.nt_stores || (long long)a.rows * cols >= STREAM_NT_MIN;
    // Prefetch the next row when a wave walks several rows (the partial
    // kernels, whose grid is capped at one workgroup per CU).  Wider
    // workgroups would not leave the registers for it.
    const int stride = gridDim.x * WAVES;
    int row = blockIdx.x * WAVES + wave;
    float4 nv[PREFETCH ? VPT : 1], ng[(PREFETCH && BWD) ? VPT : 1];
    if (PREFETCH && row < a.rows) row_load<OP, VPT, BWD>(a, row, lane, nv, ng);
    for (; row < a.rows; row += stride) {
        const long long base = (long long)row * cols;
        float4 v[VPT], g[BWD ? VPT : 1], ds[DOT ? VPT : 1];
        bool ok[VPT];
#pragma unroll
        for (int i = 0; i < VPT; i++) ok[i] = (i * 64 + lane) * 4 < cols;
        if constexpr (PREFETCH) {
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                v[i] = nv[i];
                if constexpr (BWD) g[i] = ng[i];
            }
            row_mask<OP, VPT, BWD>(ok, v, g);
            if (row + stride < a.rows) row_load<OP, VPT, BWD>(a, row + stride, lane, nv, ng);
        } else {
            row_load<OP, VPT, BWD>(a, row, lane, v, g);
            if constexpr (DOT) {
                // The row dot's subtrahend, issued behind the row's own loads
                // and first used after the row's first reduction.  DOT
                // instances do not prefetch: at 8 float4 per lane these
                // registers take the prefetch's place.
#pragma unroll
                for (int i = 0; i < VPT; i++) {
                    const int c = (i * 64 + lane) * 4;
                    ds[i] = load_stream(a.dsub + base + (c < cols ? c : 0));
                }
            }
            if constexpr (LATE_PRELOAD) {
                if (first) preload();
                first = false;
            }
            row_mask<OP, VPT, BWD>(ok, v, g);
        }
        float dd = 0.0f;  // DOT: this lane's part of the row dot

        if constexpr (OP == ROW_SOFTMAX) {
            // row.rs:64-112: max, exp(x - max), sum, normalise.
            float m = -FLT_MAX;
#pragma unroll
            for (int i = 0; i < VPT; i++) m = fmaxf(m, max4(v[i]));
            m = wave_max(m);
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                if (ok[i]) {
                    F4_APPLY(v[i], v[i], softmax_exp(v[i].x, m), softmax_exp(v[i].y, m),
                             softmax_exp(v[i].z, m), softmax_exp(v[i].w, m));
                    s += sum4(v[i]);
                }
            }
            const float inv = 1.0f / wave_sum(s);
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                if (ok[i]) {
                    float4 o;
                    F4_APPLY(o, v[i], v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv);
                    store_f4(a.y + base + (i * 64 + lane) * 4, o, nt);
                }
            }
        } else if constexpr (OP == ROW_LAYER_NORM || OP == ROW_LAYER_NORM_BWD) {
            // row.rs:130-170 (forward) and row.rs:260-300 (backward):
            // mean, then population variance of (x - mean), r = 1/sqrt(v+eps).
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; i++) s += sum4(v[i]);
            const float mean = wave_sum(s) / n;
            float q = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                if (ok[i]) {
                    // The row dot's x - dsub, while v still holds x.
                    if constexpr (DOT)
                        F4_APPLY(ds[i], ds[i], v[i].x - ds[i].x, v[i].y - ds[i].y,
                                 v[i].z - ds[i].z, v[i].w - ds[i].w);
                    const float dx0 = v[i].x - mean, dx1 = v[i].y - mean;
                    const float dx2 = v[i].z - mean, dx3 = v[i].w - mean;
                    v[i] = make_float4(dx0, dx1, dx2, dx3);
                    q += (dx0 * dx0 + dx1 * dx1) + (dx2 * dx2 + dx3 * dx3);
                }
            }
            const float rstd = 1.0f / sqrtf(wave_sum(q) / n + a.eps);
            if constexpr (OP == ROW_LAYER_NORM) {
#pragma unroll
                for (int i = 0; i < VPT; i++) {
                    if (!ok[i]) continue;
                    const int c = (i * 64 + lane) * 4;
                    float4 o;
                    F4_APPLY(o, v[i], v[i].x * rstd, v[i].y * rstd, v[i].z * rstd,
                             v[i].w * rstd);
                    if (a.gamma) {
                        const float4 g4 = gamma4(i);
                        F4_APPLY(o, o, o.x * g4.x, o.y * g4.y, o.z * g4.z, o.w * g4.w);
                    }
                    if (a.beta) {
                        const float4 b4 = beta4(i);
                        F4_APPLY(o, o, o.x + b4.x, o.y + b4.y, o.z + b4.z, o.w + b4.w);
                    }
                    store_f4(a.y + base + c, o, nt);
                }
            } else {
                // row.rs:302-346: A = sum g, B = sum g*xhat,
                // dx = r/n * (n*g - A - xhat*B), g = dy (* gamma).  xhat
                // (in place of x - mean) and g are computed once and kept;
                // products and their sums are fused multiply-adds (the
                // backward is otherwise VALU-heavy: 535 vector instructions
                // per 1024-wide row with separate multiplies and adds).
                float4 keep[KEEP_G ? VPT : 1];
                float sa = 0.0f, sb = 0.0f;
#pragma unroll
                for (int i = 0; i < VPT; i++) {
                    const float4 gi = gdy(i, g[i], ok[i]);
                    if constexpr (KEEP_G) keep[i] = gi;
                    F4_APPLY(v[i], v[i], v[i].x * rstd, v[i].y * rstd, v[i].z * rstd,
                             v[i].w * rstd);
                    if (!ok[i]) continue;
                    sa += sum4(gi);
                    sb += fmaf(gi.x, v[i].x, gi.y * v[i].y) + fmaf(gi.z, v[i].z, gi.w * v[i].w);
                }
                sa = wave_sum(sa);
                sb = wave_sum(sb);
                const float scale = rstd / n, nsa = -sa, nsb = -sb;
#pragma unroll
                for (int i = 0; i < VPT; i++) {
                    if (!ok[i]) continue;
                    const int c = (i * 64 + lane) * 4;
                    float4 gi;
                    if constexpr (KEEP_G) gi = keep[i];
                    else gi = gdy(i, g[i], true);
                    float4 o;
                    F4_APPLY(o, v[i], scale * fmaf(v[i].x, nsb, fmaf(n, gi.x, nsa)),
                             scale * fmaf(v[i].y, nsb, fmaf(n, gi.y, nsa)),
                             scale * fmaf(v[i].z, nsb, fmaf(n, gi.z, nsa)),
                             scale * fmaf(v[i].w, nsb, fmaf(n, gi.w, nsa)));
                    store_f4(a.y + base + c, o, nt);
                    if constexpr (DOT)
                        dd += fmaf(o.x, ds[i].x, o.y * ds[i].y) + fmaf(o.z, ds[i].z, o.w * ds[i].w);
                    if constexpr (PARTIALS) {
                        pg[i].x = fmaf(g[i].x, v[i].x, pg[i].x);
                        pg[i].y = fmaf(g[i].y, v[i].y, pg[i].y);
                        pg[i].z = fmaf(g[i].z, v[i].z, pg[i].z);
                        pg[i].w = fmaf(g[i].w, v[i].w, pg[i].w);
                        pb[i].x += g[i].x; pb[i].y += g[i].y;
                        pb[i].z += g[i].z; pb[i].w += g[i].w;
                    }
                }
            }
        } else if constexpr (OP == ROW_RMS_NORM) {
            // row.rs:364-395: y = x / sqrt(sum(x^2)/n + eps).
            float q = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; i++)
                q += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
            const float rms = sqrtf(wave_sum(q) / n + a.eps);
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                if (!ok[i]) continue;
                const int c = (i * 64 + lane) * 4;
                float4 o;
                F4_APPLY(o, v[i], v[i].x / rms, v[i].y / rms, v[i].z / rms, v[i].w / rms);
                if (a.gamma) {
                    const float4 gm = gamma4(i);
                    F4_APPLY(o, o, o.x * gm.x, o.y * gm.y, o.z * gm.z, o.w * gm.w);
                }
                store_f4(a.y + base + c, o, nt);
            }
        } else if constexpr (OP == ROW_SOFTMAX_BWD) {
            // row.rs:216-236: s = sum p*g; dx = p * (g - s).
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; i++)
                s += (v[i].x * g[i].x + v[i].y * g[i].y) + (v[i].z * g[i].z + v[i].w * g[i].w);
            s = wave_sum(s);
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                if (!ok[i]) continue;
                float4 o;
                F4_APPLY(o, v[i], v[i].x * (g[i].x - s), v[i].y * (g[i].y - s),
                         v[i].z * (g[i].z - s), v[i].w * (g[i].w - s));
                if (a.scale != 1.0f)
                    F4_APPLY(o, o, o.x * a.scale, o.y * a.scale, o.z * a.scale, o.w * a.scale);
                store_f4(a.y + base + (i * 64 + lane) * 4, o, nt);
            }
        } else if constexpr (OP == ROW_RMS_NORM_BWD) {
            // row.rs:416-467: inv = 1/sqrt(q/n + eps), c = d/n*inv^3,
            // dx = g*inv - x*c, g = dy (* gamma); g is computed once and
            // kept, products and their sums are fused multiply-adds.
            float4 keep[KEEP_G ? VPT : 1];
            float q = 0.0f, d = 0.0f;
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                const float4 gi = gdy(i, g[i], ok[i]);
                if constexpr (KEEP_G) keep[i] = gi;
                q += fmaf(v[i].x, v[i].x, v[i].y * v[i].y) + fmaf(v[i].z, v[i].z, v[i].w * v[i].w);
                d += fmaf(v[i].x, gi.x, v[i].y * gi.y) + fmaf(v[i].z, gi.z, v[i].w * gi.w);
            }
            q = wave_sum(q);
            d = wave_sum(d);
            const float rms = sqrtf(q / n + a.eps);
            const float inv = 1.0f / rms;
            const float ncorr = -(d / n * inv * inv * inv);
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                if (!ok[i]) continue;
                const int c = (i * 64 + lane) * 4;
                float4 gi;
                if constexpr (KEEP_G) gi = keep[i];
                else gi = gdy(i, g[i], true);
                float4 o;
                F4_APPLY(o, v[i], fmaf(v[i].x, ncorr, gi.x * inv), fmaf(v[i].y, ncorr, gi.y * inv),
                         fmaf(v[i].z, ncorr, gi.z * inv), fmaf(v[i].w, ncorr, gi.w * inv));
                store_f4(a.y + base + c, o, nt);
                if constexpr (DOT) {
                    // v holds x: the row dot's x - dsub, then its products.
                    F4_APPLY(ds[i], ds[i], v[i].x - ds[i].x, v[i].y - ds[i].y, v[i].z - ds[i].z,
                             v[i].w - ds[i].w);
                    dd += fmaf(o.x, ds[i].x, o.y * ds[i].y) + fmaf(o.z, ds[i].z, o.w * ds[i].w);
                }
                if constexpr (PARTIALS) {
                    pg[i].x = fmaf(g[i].x, v[i].x * inv, pg[i].x);
                    pg[i].y = fmaf(g[i].y, v[i].y * inv, pg[i].y);
                    pg[i].z = fmaf(g[i].z, v[i].z * inv, pg[i].z);
                    pg[i].w = fmaf(g[i].w, v[i].w * inv, pg[i].w);
                }
            }
        }
        if constexpr (DOT) {
            dd = wave_sum(dd);
            if (lane == 0) a.dot[row] = a.dscale * dd;
        }
    }

    if constexpr (PARTIALS) {
        // Combine the WAVES waves of this workgroup in LDS (in wave order), then
        // write one partial row per workgroup.
        if (!a.pgamma && !a.pbeta) return;
        extern __shared__ float4 red[];  // [WAVES][cols/4]
        const int c4n = cols / 4;
        for (int pass = 0; pass < 2; pass++) {
            float* dst = pass == 0 ? a.pgamma : a.pbeta;
            if (!dst) continue;  // uniform across the workgroup
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                const int c4 = i * 64 + lane;
                if (c4 < c4n) red[wave * c4n + c4] = pass == 0 ? pg[i] : pb[i];
            }
            __syncthreads();
            for (int c4 = threadIdx.x; c4 < c4n; c4 += WAVES * 64) {
                float4 t = red[c4];
                for (int w = 1; w < WAVES; w++) {
                    const float4 u = red[w * c4n + c4];
                    t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
                }
                reinterpret_cast<float4*>(dst + (long long)blockIdx.x * cols)[c4] = t;
            }
            __syncthreads();
        }
    }
}

// Looping path: any cols and alignment, scalar accesses, one wave per row.
// The norm backward's row dot (RowArgs::dot) is taken here when dot is set.
template <int OP>
__device__ __forceinline__ void row_kernel_loop(const RowArgs& a) {
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int cols = a.cols;
    const float n = (float)cols;
    constexpr bool PARTIALS = (OP == ROW_LAYER_NORM_BWD || OP == ROW_RMS_NORM_BWD);
    // Partials of the looping path are written per wave: row index
    // blockIdx.x * ROW_WAVES + wave of the partial buffer.
    const long long prow = (long long)(blockIdx.x * ROW_WAVES + wave) * cols;
    if constexpr (PARTIALS) {
        for (int c = lane; c < cols; c += 64) {
            if (a.pgamma) a.pgamma[prow + c] = 0.0f;
            if (a.pbeta) a.pbeta[prow + c] = 0.0f;
        }
    }
    for (int row = blockIdx.x * ROW_WAVES + wave; row < a.rows;
         row += gridDim.x * ROW_WAVES) {
        const float* x = a.x + (long long)row * cols;
        float* y = a.y + (long long)row * cols;
        const float* dy = a.dy ? a.dy + (long long)row * cols : nullptr;
        if constexpr (OP == ROW_SOFTMAX) {
            float m = -FLT_MAX;
            for (int c = lane; c < cols; c += 64) m = fmaxf(m, x[c]);
            m = wave_max(m);
            float s = 0.0f;
            for (int c = lane; c < cols; c += 64) s += softmax_exp(x[c], m);
            const float inv = 1.0f / wave_sum(s);
            for (int c = lane; c < cols; c += 64) y[c] = softmax_exp(x[c], m) * inv;
        } else if constexpr (OP == ROW_LAYER_NORM || OP == ROW_LAYER_NORM_BWD) {
            float s = 0.0f;
            for (int c = lane; c < cols; c += 64) s += x[c];
            const float mean = wave_sum(s) / n;
            float q = 0.0f;
            for (int c = lane; c < cols; c += 64) {
                const float d = x[c] - mean;
                q += d * d;
            }
            const float rstd = 1.0f / sqrtf(wave_sum(q) / n + a.eps);
            if constexpr (OP == ROW_LAYER_NORM) {
                for (int c = lane; c < cols; c += 64) {
                    float o = (x[c] - mean) * rstd;
                    if (a.gamma) o = o * a.gamma[c];
                    if (a.beta) o = o + a.beta[c];
                    y[c] = o;
                }
            } else {
                float sa = 0.0f, sb = 0.0f;
                for (int c = lane; c < cols; c += 64) {
                    const float gg = a.gamma ? dy[c] * a.gamma[c] : dy[c];
                    sa += gg;
                    sb += gg * ((x[c] - mean) * rstd);
                }
                sa = wave_sum(sa);
                sb = wave_sum(sb);
                const float scale = rstd / n;
                float dd = 0.0f;
                for (int c = lane; c < cols; c += 64) {
                    const float xh = (x[c] - mean) * rstd;
                    const float gg = a.gamma ? dy[c] * a.gamma[c] : dy[c];
                    const float o = scale * (n * gg - sa - xh * sb);
                    if (a.dot) dd = fmaf(o, x[c] - a.dsub[(long long)row * cols + c], dd);
                    y[c] = o;
                    if (a.pgamma) a.pgamma[prow + c] += dy[c] * xh;
                    if (a.pbeta) a.pbeta[prow + c] += dy[c];
                }
                if (a.dot) {
                    dd = wave_sum(dd);
                    if (lane == 0) a.dot[row] = a.dscale * dd;
                }
            }
        } else if constexpr (OP == ROW_RMS_NORM) {
            float q = 0.0f;
            for (int c = lane; c < cols; c += 64) q += x[c] * x[c];
            const float rms = sqrtf(wave_sum(q) / n + a.eps);
            for (int c = lane; c < cols; c += 64) {
                float o = x[c] / rms;
                if (a.gamma) o = o * a.gamma[c];
                y[c] = o;
            }
        } else if constexpr (OP == ROW_SOFTMAX_BWD) {
            float s = 0.0f;
            for (int c = lane; c < cols; c += 64) s += x[c] * dy[c];
            s = wave_sum(s);
            for (int c = lane; c < cols; c += 64) {
                const float d = x[c] * (dy[c] - s);
                y[c] = a.scale != 1.0f ? d * a.scale : d;
            }
        } else if constexpr (OP == ROW_RMS_NORM_BWD) {
            float q = 0.0f, d = 0.0f;
            for (int c = lane; c < cols; c += 64) {
                const float gg = a.gamma ? dy[c] * a.gamma[c] : dy[c];
                q += x[c] * x[c];
                d += x[c] * gg;
            }
            q = wave_sum(q);
            d = wave_sum(d);
            const float rms = sqrtf(q / n + a.eps);
            const float inv = 1.0f / rms;
            const float corr = d / n * inv * inv * inv;
            float dd = 0.0f;
            for (int c = lane; c < cols; c += 64) {
                const float gg = a.gamma ? dy[c] * a.gamma[c] : dy[c];
                const float o = gg * inv - x[c] * corr;
                if (a.dot) dd = fmaf(o, x[c] - a.dsub[(long long)row * cols + c], dd);
                y[c] = o;
                if (a.pgamma) a.pgamma[prow + c] += dy[c] * (x[c] * inv);
            }
            if (a.dot) {
                dd = wave_sum(dd);
                if (lane == 0) a.dot[row] = a.dscale * dd;
            }
        }
    }
}

}  // namespace forge
