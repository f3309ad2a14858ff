// elementwise.hpp -- bandwidth kernels: binary ops, row broadcast, maps,
// fills, column/row sums, full reductions and the transpose.
//
// The reference launches one thread per element with 1024-thread blocks and
// no vectorisation (runtime.rs:124-130 get_launch_config).  Here every
// streaming kernel is grid-stride over 128-bit (float4) accesses with a
// scalar tail; the VEC=false instances serve unaligned slices.
#pragma once
#include <float.h>
#include "common.hpp"

namespace forge {

// Every kernel here is launched with exactly EW_THREADS threads per
// workgroup, and the bodies use the constant rather than blockDim.x: on
// gfx950 blockDim.x is read from the dispatch packet by a vector memory load
// that every wave waits for before it can form its first address.
constexpr int EW_THREADS = 256;

// The 128-bit streaming loop of the vectorised kernels: one float4 item per
// thread, the host launching enough workgroups to cover every item
// (grid-stride beyond that).  Loads are non-temporal; from STREAM_NT_MIN
// float4 items (64 MiB per operand) the stores are too (store_f4).  Measured on MI355X, in
// place x = s * x at 256 MiB: 6.59 TB/s this way, 5.80 with cached stores,
// 5.51 with four items per thread and at most 8192 workgroups; at 16 MiB
// non-temporal stores cost 4% (6.93 against 6.67 us), so small arrays keep
// cached ones.  f(i, nt) loads item i, computes it and stores it with
// store_f4(.., nt).
template <typename F>
__device__ __forceinline__ void stream_f4(long long n4, F f) {
    const bool nt = n4 >= STREAM_NT_MIN / 4;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    for (long long i = (long long)blockIdx.x * EW_THREADS + threadIdx.x; i < n4; i += stride)
        f(i, nt);
}

// ---------------------------------------------------------------- binary

template <int OP, bool VEC>
__device__ __forceinline__ void binary_body(const float* __restrict__ l,
                                            const float* __restrict__ r,
                                            float* __restrict__ o, long long n) {
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    if constexpr (VEC) {
        const long long n4 = n / 4;
        stream_f4(n4, [&](long long i, bool nt) {
            const float4 a = load_stream(l + 4 * i), b = load_stream(r + 4 * i);
            float4 c;
            c.x = apply_binary<OP>(a.x, b.x);
            c.y = apply_binary<OP>(a.y, b.y);
            c.z = apply_binary<OP>(a.z, b.z);
            c.w = apply_binary<OP>(a.w, b.w);
            // Out of place, the result is stored non-temporally at every
            // size: the C4 forward's position add (8 MiB) made the forward
            // 0.6-1.0 us faster in six paired runs; at 16 MiB the add took
            // 9.91-9.92 against 9.85-9.86 us.
            (void)nt;
            store_f4(o + 4 * i, c, true);
        });
        for (long long i = n4 * 4 + tid; i < n; i += stride)
            o[i] = apply_binary<OP>(l[i], r[i]);
    } else {
        for (long long i = tid; i < n; i += stride) o[i] = apply_binary<OP>(l[i], r[i]);
    }
}

// In-place variant (target aliases the left operand); no __restrict__.
template <int OP, bool VEC>
__device__ __forceinline__ void binary_assign_body(float* t, const float* r,
                                                   long long n) {
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    if constexpr (VEC) {
        const long long n4 = n / 4;
        stream_f4(n4, [&](long long i, bool nt) {
            const float4 a = load_stream(t + 4 * i), b = load_stream(r + 4 * i);
            float4 c;
            c.x = apply_binary<OP>(a.x, b.x);
            c.y = apply_binary<OP>(a.y, b.y);
            c.z = apply_binary<OP>(a.z, b.z);
            c.w = apply_binary<OP>(a.w, b.w);
            store_f4(t + 4 * i, c, nt);
        });
        for (long long i = n4 * 4 + tid; i < n; i += stride)
            t[i] = apply_binary<OP>(t[i], r[i]);
    } else {
        for (long long i = tid; i < n; i += stride) t[i] = apply_binary<OP>(t[i], r[i]);
    }
}

// M[r, c] = M[r, c] op row[c] (row.rs:179-191).  Column tiles on
// blockIdx.x keep the broadcast row in registers; rows are grid-stride on
// blockIdx.y.
template <int OP, bool VEC>
__device__ __forceinline__ void by_rows_body(float* m, const float* __restrict__ row,
                                             int rows, int cols) {
    if constexpr (VEC) {
        const int c4 = blockIdx.x * EW_THREADS + threadIdx.x;
        if (c4 * 4 >= cols) return;
        const float4 b = reinterpret_cast<const float4*>(row)[c4];
        const bool nt = (long long)rows * cols >= STREAM_NT_MIN;
        for (int r = blockIdx.y; r < rows; r += gridDim.y) {
            float* p = m + (long long)r * cols + 4 * c4;
            float4 a = load_stream(p);
            a.x = apply_binary<OP>(a.x, b.x);
            a.y = apply_binary<OP>(a.y, b.y);
            a.z = apply_binary<OP>(a.z, b.z);
            a.w = apply_binary<OP>(a.w, b.w);
            store_f4(p, a, nt);
        }
    } else {
        const int c = blockIdx.x * EW_THREADS + threadIdx.x;
        if (c >= cols) return;
        const float b = row[c];
        for (int r = blockIdx.y; r < rows; r += gridDim.y) {
            float* p = m + (long long)r * cols + c;
            *p = apply_binary<OP>(*p, b);
        }
    }
}

// ------------------------------------------------------------------ maps

enum MapOp {
    MAP_SCALE = 0, MAP_ADD = 1, MAP_GELU = 2, MAP_GELU_D = 3, MAP_RELU = 4,
    MAP_RELU_D = 5, MAP_SILU = 6, MAP_SILU_D = 7, MAP_EXP_SHIFT = 8,
    MAP_HALF_SQ = 9, MAP_IDENTITY = 10
};

template <int OP>
__device__ __forceinline__ float map_one(float x, float p0) {
    if constexpr (OP == MAP_SCALE) return x * p0;
    else if constexpr (OP == MAP_ADD) return x + p0;
    else if constexpr (OP == MAP_GELU) return gelu(x);
    else if constexpr (OP == MAP_GELU_D) return gelu_derivative(x);
    else if constexpr (OP == MAP_RELU) return relu(x);
    else if constexpr (OP == MAP_RELU_D) return relu_derivative(x);
    else if constexpr (OP == MAP_SILU) return silu(x);
    else if constexpr (OP == MAP_SILU_D) return silu_derivative(x);
    else if constexpr (OP == MAP_EXP_SHIFT) return expf(x - p0);
    else if constexpr (OP == MAP_HALF_SQ) return 0.5f * x * x;
    else return x;
}

template <int OP, bool VEC>
__device__ __forceinline__ void map_body(float* x, long long n, float p0) {
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    if constexpr (VEC) {
        const long long n4 = n / 4;
        stream_f4(n4, [&](long long i, bool nt) {
            const float4 a = load_stream(x + 4 * i);
            float4 c;
            c.x = map_one<OP>(a.x, p0);
            c.y = map_one<OP>(a.y, p0);
            c.z = map_one<OP>(a.z, p0);
            c.w = map_one<OP>(a.w, p0);
            store_f4(x + 4 * i, c, nt);
        });
        for (long long i = n4 * 4 + tid; i < n; i += stride) x[i] = map_one<OP>(x[i], p0);
    } else {
        for (long long i = tid; i < n; i += stride) x[i] = map_one<OP>(x[i], p0);
    }
}

// ----------------------------------------------------------------- fills

template <bool VEC>
__device__ __forceinline__ void fill_body(float* x, long long n, float v) {
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    if constexpr (VEC) {
        const long long n4 = n / 4;
        const float4 f = make_float4(v, v, v, v);
        for (long long i = tid; i < n4; i += stride) reinterpret_cast<float4*>(x)[i] = f;
        for (long long i = n4 * 4 + tid; i < n; i += stride) x[i] = v;
    } else {
        for (long long i = tid; i < n; i += stride) x[i] = v;
    }
}

// elementwise.rs:23-34: index as f32 (ascending) or (len - index) as f32.
__device__ __forceinline__ void fill_seq_body(float* x, long long n, int ascending) {
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    for (long long i = tid; i < n; i += stride)
        x[i] = ascending ? (float)(unsigned long long)i
                         : (float)(unsigned long long)(n - i);
}

// slice_set_random (elementwise.rs:36-43) with the hash of common.rs:3-9:
// x += x << 13; x -= x >> 17; x *= x << 5 (wrapping u32), value / u32::MAX.
__device__ __forceinline__ uint32_t forge_hash(uint32_t x) {
    x += x << 13;
    x -= x >> 17;
    x *= x << 5;
    return x;
}

__device__ __forceinline__ void fill_random_body(float* x, long long n, uint32_t seed) {
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    for (long long i = tid; i < n; i += stride)
        x[i] = (float)forge_hash(seed + (uint32_t)i) / (float)4294967295u;
}

// p = p - lr * g: Linear::learn's bias update (linear.rs:385-390: clone the
// gradient, scale it by the learning rate, subtract) in one pass with the
// same two roundings.
template <bool VEC>
__device__ __forceinline__ void sgd_body(float* p, const float* __restrict__ g, long long n,
                                         float lr) {
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    if constexpr (VEC) {
        const long long n4 = n / 4;
        stream_f4(n4, [&](long long i, bool nt) {
            const float4 a = load_stream(p + 4 * i), b = load_stream(g + 4 * i);
            float4 c;
            c.x = a.x - lr * b.x;
            c.y = a.y - lr * b.y;
            c.z = a.z - lr * b.z;
            c.w = a.w - lr * b.w;
            store_f4(p + 4 * i, c, nt);
        });
        for (long long i = n4 * 4 + tid; i < n; i += stride) p[i] = p[i] - lr * g[i];
    } else {
        for (long long i = tid; i < n; i += stride) p[i] = p[i] - lr * g[i];
    }
}

// g = dy * act'(z): Linear::backward's derivative map and multiply
// (linear.rs:254-265) in one pass; same two roundings.
template <bool VEC>
__device__ __forceinline__ void act_backward_body(const float* __restrict__ dy,
                                                  const float* __restrict__ z,
                                                  float* __restrict__ g, long long n, int act) {
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    if constexpr (VEC) {
        const long long n4 = n / 4;
        stream_f4(n4, [&](long long i, bool nt) {
            const float4 a = load_stream(dy + 4 * i), b = load_stream(z + 4 * i);
            float4 c;
            c.x = a.x * activate_derivative(act, b.x);
            c.y = a.y * activate_derivative(act, b.y);
            c.z = a.z * activate_derivative(act, b.z);
            c.w = a.w * activate_derivative(act, b.w);
            store_f4(g + 4 * i, c, nt);
        });
        for (long long i = n4 * 4 + tid; i < n; i += stride)
            g[i] = dy[i] * activate_derivative(act, z[i]);
    } else {
        for (long long i = tid; i < n; i += stride) g[i] = dy[i] * activate_derivative(act, z[i]);
    }
}

// A count as the output type: the f32 nearest to it (exact up to 2^24), or
// the u32 count saturated at 2^32 - 1.
__device__ __forceinline__ void store_count(float* out, unsigned long long t) { out[0] = (float)t; }
__device__ __forceinline__ void store_count(unsigned* out, unsigned long long t) {
    out[0] = t > 0xFFFFFFFFull ? 0xFFFFFFFFu : (unsigned)t;
}

// Count of positions where l != r (compare_vectors, reduction.rs:132-174,
// but over every element; the reference keeps only block 0's count).
// Counts are integers throughout: per-workgroup partials in `part` (u32),
// summed in u64 by count_final_body.  With one workgroup the kernel writes
// the count itself (store_count).
template <typename T>
__device__ __forceinline__ void count_neq_body(const float* __restrict__ l,
                                               const float* __restrict__ r, long long n,
                                               unsigned* __restrict__ part,
                                               T* __restrict__ out) {
    __shared__ unsigned wsum[EW_THREADS / 64];
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    unsigned acc = 0;
    for (long long i = tid; i < n; i += stride) acc += (l[i] == r[i]) ? 0u : 1u;
    acc = wave_sum_u32(acc);
    if (lane_id() == 0) wsum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int w = 0; w < (EW_THREADS >> 6); w++) t += wsum[w];
        if (gridDim.x == 1) store_count(out, t);
        else part[blockIdx.x] = (unsigned)t;
    }
}

// Sum of `n` u32 partial counts in u64, stored by store_count.
template <typename T>
__device__ __forceinline__ void count_final_body(const unsigned* __restrict__ part, int n,
                                                 T* __restrict__ out) {
    __shared__ unsigned long long wsum[EW_THREADS / 64];
    unsigned long long acc = 0;
    for (int i = threadIdx.x; i < n; i += EW_THREADS) acc += part[i];
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
    if (lane_id() == 0) wsum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int w = 0; w < (EW_THREADS >> 6); w++) t += wsum[w];
        store_count(out, t);
    }
}

// row.rs:5-14: M[r, c] = -inf for c > r, where row r of m is row
// first_row + r of the whole score matrix (first_row = 0: the reference).
__device__ __forceinline__ void causal_mask_body(float* m, int rows, int cols, int first_row) {
    for (int r = blockIdx.y; r < rows; r += gridDim.y)
        for (int c = blockIdx.x * EW_THREADS + threadIdx.x; c < cols;
             c += gridDim.x * EW_THREADS)
            if (c > first_row + r) m[(long long)r * cols + c] = -INFINITY;
}

// ------------------------------------------------------------ reductions

// Column sums, first pass: chunk blockIdx.y of rows_per_chunk rows, 4 waves
// taking every 4th row of the chunk.  VEC: a lane owns 4 consecutive columns
// (one float4 load per row, 1 KiB per wave-row) so a workgroup covers 256
// columns; scalar: a lane owns one column, 64 per workgroup.  The 4 wave
// partials are added in LDS in wave order and written to
// out[blockIdx.y * cols + c].  Summation order depends only on the shape.
constexpr int SUMCOL_WAVES = 4;

template <bool VEC>
__device__ __forceinline__ void sum_cols_body(const float* __restrict__ m,
                                              float* __restrict__ out, int rows,
                                              int cols, int rows_per_chunk) {
    __shared__ float4 part[SUMCOL_WAVES][64];
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const int r0 = blockIdx.y * rows_per_chunk;
    const int r1 = min(rows, r0 + rows_per_chunk);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    const int c = VEC ? (blockIdx.x * 64 + lane) * 4 : blockIdx.x * 64 + lane;
    if (c < cols) {
        int r = r0 + wave;
#pragma unroll 4
        for (; r < r1; r += SUMCOL_WAVES) {
            const float* p = m + (long long)r * cols + c;
            if constexpr (VEC) {
                const float4 v = *reinterpret_cast<const float4*>(p);
                acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
            } else {
                acc.x += *p;
            }
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && c < cols) {
        float4 t = part[0][lane];
        for (int w = 1; w < SUMCOL_WAVES; w++) {
            const float4 u = part[w][lane];
            t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
        }
        float* o = out + (long long)blockIdx.y * cols + c;
        if constexpr (VEC) *reinterpret_cast<float4*>(o) = t;
        else *o = t.x;
    }
}

// The final passes write the column sums to `out` (when not null) and,
// when `param` is not null, apply the SGD step of that parameter vector in
// the same pass: param -= lr * sum with the two roundings of the reference's
// clone-scale-subtract (linear.rs:385-390).
struct ColSumOut {
    float* out;
    float* param;
    float lr;
};

__device__ __forceinline__ void colsum_store(const ColSumOut& o, int c, float v) {
    if (o.out) o.out[c] = v;
    if (o.param) o.param[c] = o.param[c] - o.lr * v;
}

__device__ __forceinline__ void colsum_store4(const ColSumOut& o, int c, float4 v) {
    if (o.out) *reinterpret_cast<float4*>(o.out + c) = v;
    if (o.param) {
        float4 p = *reinterpret_cast<const float4*>(o.param + c);
        p.x = p.x - o.lr * v.x;
        p.y = p.y - o.lr * v.y;
        p.z = p.z - o.lr * v.z;
        p.w = p.w - o.lr * v.w;
        *reinterpret_cast<float4*>(o.param + c) = p;
    }
}

// Column sums, final pass over a short matrix (the first pass's partial
// rows, or any matrix of few rows): 16 waves per workgroup each take every
// 16th row of 64 columns, then add in LDS in wave order.
constexpr int SUMCOL_FINAL_WAVES = 16;

__device__ __forceinline__ void sum_cols_final_body(const float* __restrict__ m,
                                                    const ColSumOut& o, int rows, int cols) {
    __shared__ float part[SUMCOL_FINAL_WAVES][64];
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    float acc = 0.0f;
    if (c < cols) {
#pragma unroll 8
        for (int r = wave; r < rows; r += SUMCOL_FINAL_WAVES) acc += m[(long long)r * cols + c];
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && c < cols) {
        float t = part[0][lane];
        for (int w = 1; w < SUMCOL_FINAL_WAVES; w++) t += part[w][lane];
        colsum_store(o, c, t);
    }
}

// The same final pass for 16-byte aligned float4 columns.  A workgroup of
// 256 threads owns 16 columns (four float4 groups q); thread t = 4 s + q
// sums rows s, s + 64, s + 128, ... of group q with four rows' loads in
// flight, then the 64 row-slot sums of each group are added in LDS by a
// fixed tree.  The order depends only on the shape.  With the short
// matrices this pass sees (the first pass's or the norm backward's partial
// rows, at most a few hundred) a launch is mostly load latency: one round
// of loads per 256 rows on 4 x more workgroups than the scalar pass.
constexpr int SUMCOL_FINAL_V_THREADS = 256;
constexpr int SUMCOL_FINAL_V_COLS = 16;

__device__ __forceinline__ void sum_cols_final_v_body(const float* __restrict__ m,
                                                      const ColSumOut& o, int rows, int cols) {
    constexpr int SLOTS = SUMCOL_FINAL_V_THREADS / 4;
    __shared__ float4 part[SLOTS][4];
    const int q = threadIdx.x & 3, s = threadIdx.x >> 2;
    const int c = blockIdx.x * SUMCOL_FINAL_V_COLS + 4 * q;
    const bool in = c < cols;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (in) {
        const float* p = m + c;
        int r = s;
        for (; r + 3 * SLOTS < rows; r += 4 * SLOTS) {
            float4 u[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                u[j] = *reinterpret_cast<const float4*>(p + (long long)(r + j * SLOTS) * cols);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc.x += u[j].x; acc.y += u[j].y; acc.z += u[j].z; acc.w += u[j].w;
            }
        }
        for (; r < rows; r += SLOTS) {
            const float4 u = *reinterpret_cast<const float4*>(p + (long long)r * cols);
            acc.x += u.x; acc.y += u.y; acc.z += u.z; acc.w += u.w;
        }
    }
    part[s][q] = acc;
    __syncthreads();
#pragma unroll
    for (int st = SLOTS / 2; st > 0; st >>= 1) {
        if (s < st) {
            const float4 u = part[s + st][q];
            float4 t = part[s][q];
            t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
            part[s][q] = t;
        }
        __syncthreads();
    }
    if (s == 0 && in) colsum_store4(o, c, part[0][q]);
}

// Column sums, first pass over 16-byte aligned float4 columns.  Workgroup
// (x, y) owns the 64 columns 64 x .. 64 x + 63 of the rows of chunk y:
// thread t = 16 s + q sums the float4 column group q of rows s, s + 16,
// s + 32, ... of the chunk in order (one chain per row slot s; LOADS loads
// in flight per batch of 16 LOADS rows), then the 16 slots add by a halving
// tree in LDS (slot s + st into s for st = 8, 4, 2, 1).  With one chunk
// that is the result (stored with the SGD step, as the final passes do);
// otherwise it is the chunk's partial row part[y, :], for
// forge_sum_cols_final_v.  The order depends only on the shape.
//
// A one-launch form, in which the last workgroup of each column group to
// finish adds the partial rows, needs every workgroup to release its
// partial row at agent scope first; on gfx950 that release writes back the
// XCD's L2, and the launch took 25-43 us at [4096,1024] against 7.7 us for
// the two launches, so the partial rows go through a kernel boundary.  A
// one-launch form without partial rows, each workgroup owning a strip of 4,
// 8 or 16 columns over every row (about 256 strips), took 12.0-16.4 us at
// [4096,1024] and 15.3-20.5 us at [4096,2048] against 7.4 and 9.9 us: its
// lanes read 16-64 bytes per row, and those narrow strided requests cost
// more than the boundary.
constexpr int SUMCOL1_THREADS = 256;
constexpr int SUMCOL1_COLS = 64;
constexpr int SUMCOL1_SLOTS = SUMCOL1_THREADS / (SUMCOL1_COLS / 4);

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

template <int LOADS>
__device__ __forceinline__ void sum_cols_part_body(const float* __restrict__ m,
                                                   float* __restrict__ part,
                                                   const ColSumOut& o, int rows, int cols,
                                                   int rows_per_chunk) {
    __shared__ float4 red[SUMCOL1_SLOTS][SUMCOL1_COLS / 4];
    const int q = threadIdx.x & 15, s = threadIdx.x >> 4;
    const int c = blockIdx.x * SUMCOL1_COLS + 4 * q;
    const bool in = c < cols;
    const int r0 = blockIdx.y * rows_per_chunk;
    const int r1 = min(rows, r0 + rows_per_chunk);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (in) {
        for (int b = r0 + s; b < r1; b += SUMCOL1_SLOTS * LOADS) {
            float4 v[LOADS];
#pragma unroll
            for (int j = 0; j < LOADS; j++) {
                const int r = b + j * SUMCOL1_SLOTS;
                v[j] = r < r1 ? load_stream(m + (long long)r * cols + c)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < LOADS; j++) acc = add4(acc, v[j]);
        }
    }
    red[s][q] = acc;
    __syncthreads();
#pragma unroll
    for (int st = SUMCOL1_SLOTS / 2; st > 0; st >>= 1) {
        if (s < st) red[s][q] = add4(red[s][q], red[s + st][q]);
        __syncthreads();
    }
    if (s != 0 || !in) return;
    if (gridDim.y == 1) colsum_store4(o, c, red[0][q]);
    else *reinterpret_cast<float4*>(part + (long long)blockIdx.y * cols + c) = red[0][q];
}

// Row statistics of the GEMM epilogue where the product's own kernel does
// not form them (the bounds-guarded and split-K paths).
// d[r] = sqrt(sum of part[r, 0..parts) / n + eps), the partials added in
// index order: the divisor the unguarded tiles form in their prologue.
__device__ __forceinline__ void row_rms_parts_body(const float* __restrict__ part, int parts,
                                                   int rows, int n, float eps,
                                                   float* __restrict__ d) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float* p = part + (long long)r * parts;
    float t = 0.0f;
    for (int j = 0; j < parts; j++) t += p[j];
    d[r] = sqrtf(t / (float)n + eps);
}

// out[r, b] = sum over the columns 32 b .. 32 b + 31 (< cols) of row r of
// m [rows, ld] of the squares, in column order: row_sumsq_out from C.
__device__ __forceinline__ void row_sq_parts_body(const float* __restrict__ m, long long ld,
                                                  int rows, int cols, float* __restrict__ out) {
    const int parts = (cols + 31) / 32;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * parts) return;
    const int r = (int)(i / parts), b = (int)(i % parts);
    const float* p = m + (long long)r * ld + 32 * b;
    const int e = min(32, cols - 32 * b);
    float q = 0.0f;
    for (int c = 0; c < e; c++) q += p[c] * p[c];
    out[i] = q;
}

// Row sums: one wave per row (row.rs:16-53).
template <bool VEC>
__device__ __forceinline__ void sum_rows_body(const float* __restrict__ m,
                                              float* __restrict__ out, int rows,
                                              int cols) {
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    constexpr int waves = EW_THREADS >> 6;
    for (int r = blockIdx.x * waves + wave; r < rows; r += gridDim.x * waves) {
        const float* p = m + (long long)r * cols;
        float s = 0.0f;
        // Unrolled so that four loads per lane are in flight; the sum is
        // still taken in column order.
        if constexpr (VEC) {
#pragma unroll 4
            for (int c4 = lane; c4 < cols / 4; c4 += 64) {
                const float4 a = load_stream(p + 4 * c4);
                s += (a.x + a.y) + (a.z + a.w);
            }
        } else {
#pragma unroll 4
            for (int c = lane; c < cols; c += 64) s += p[c];
        }
        s = wave_sum(s);
        if (lane == 0) out[r] = s;
    }
}

// Block-level reduction to one value per workgroup (partials), grid-stride:
// the sum (reduction.rs:4-41), the max with identity -FLT_MAX
// (reduction.rs:93-130), or the sum of a map functor's values
// (slice_map_sum, reduction.rs:43-91).  With VEC (x 16-byte aligned) each
// lane keeps RED_UNROLL float4 loads in flight per step, one per grid
// stride, with one accumulator each (a lane's four floats fold in x, y, z,
// w order); the accumulators fold in order, then the wave and the
// workgroup.  Without VEC, one float per step.  The order depends only on n
// and the grid, so results are deterministic.
constexpr int RED_UNROLL = 4;

template <int OP, bool IS_MAX>
__device__ __forceinline__ float red_fold(float acc, float v, float p0) {
    if constexpr (IS_MAX) return fmaxf(acc, v);
    else return acc + map_one<OP>(v, p0);
}

template <int OP, bool IS_MAX, bool VEC>
__device__ __forceinline__ void reduce_body(const float* __restrict__ x, long long n, float p0,
                                            float* __restrict__ out) {
    __shared__ float part[EW_THREADS / 64];
    const long long tid = (long long)blockIdx.x * EW_THREADS + threadIdx.x;
    const long long stride = (long long)gridDim.x * EW_THREADS;
    constexpr float ident = IS_MAX ? -FLT_MAX : 0.0f;
    float acc = ident;
    if constexpr (VEC) {
        const long long n4 = n / 4;
        float a[RED_UNROLL];
#pragma unroll
        for (int u = 0; u < RED_UNROLL; u++) a[u] = ident;
        long long i = tid;
        // Steps whose RED_UNROLL loads are all in range: loads first, then
        // the folds.
        for (; i + (RED_UNROLL - 1) * stride < n4; i += RED_UNROLL * stride) {
            float4 v[RED_UNROLL];
#pragma unroll
            for (int u = 0; u < RED_UNROLL; u++) v[u] = load_stream(x + 4 * (i + u * stride));
#pragma unroll
            for (int u = 0; u < RED_UNROLL; u++) {
                a[u] = red_fold<OP, IS_MAX>(a[u], v[u].x, p0);
                a[u] = red_fold<OP, IS_MAX>(a[u], v[u].y, p0);
                a[u] = red_fold<OP, IS_MAX>(a[u], v[u].z, p0);
                a[u] = red_fold<OP, IS_MAX>(a[u], v[u].w, p0);
            }
        }
        for (; i < n4; i += stride) {
            const float4 v = load_stream(x + 4 * i);
            a[0] = red_fold<OP, IS_MAX>(a[0], v.x, p0);
            a[0] = red_fold<OP, IS_MAX>(a[0], v.y, p0);
            a[0] = red_fold<OP, IS_MAX>(a[0], v.z, p0);
            a[0] = red_fold<OP, IS_MAX>(a[0], v.w, p0);
        }
        for (long long j = n4 * 4 + tid; j < n; j += stride) a[0] = red_fold<OP, IS_MAX>(a[0], x[j], p0);
        acc = a[0];
#pragma unroll
        for (int u = 1; u < RED_UNROLL; u++) acc = IS_MAX ? fmaxf(acc, a[u]) : acc + a[u];
    } else {
        for (long long i = tid; i < n; i += stride) acc = red_fold<OP, IS_MAX>(acc, x[i], p0);
    }
    acc = IS_MAX ? wave_max(acc) : wave_sum(acc);
    const int wave = threadIdx.x >> 6;
    if (lane_id() == 0) part[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = part[0];
        for (int w = 1; w < (EW_THREADS >> 6); w++)
            t = IS_MAX ? fmaxf(t, part[w]) : t + part[w];
        out[blockIdx.x] = t;
    }
}

// ------------------------------------------------------------- transpose

// out[c, r] = in[r, c] for in [rows, cols] (layout.rs:8-55).  A workgroup of
// 256 threads moves one 64 x TC tile through LDS (pitch TC + 1).  Each wave
// load instruction covers 4 input rows x 16 float4, and each wave store covers
// 4 output rows x 16 float4, so with the odd pitch both the scalar LDS stores
// and the column reads that assemble each float4 store are bank-conflict
// free.  TC = 256 (1 KiB contiguous per input row) is the unguarded path when
// cols allows it: wider input rows per tile keep HBM busier than 64x64 tiles
// (about 5.2 against 4.8 TB/s at [8192, 4096]); TC = 64 serves every other
// shape, GUARD for edges and unaligned views.
constexpr int TR_ROWS = 64;
// Transposes from TR_NT_MIN floats (16 MiB) on store non-temporally: at
// [8192, 4096] 39.9-40.0 us against 51.1-51.3 us with cached stores (and
// 42.7-43.0 us with non-temporal loads instead, 49.9-50.5 us with both), in
// three rounds on one device.  Smaller ones keep cached stores.
constexpr long long TR_NT_MIN = 4ll << 20;

template <int TC, bool GUARD>
__device__ __forceinline__ void transpose_body(const float* __restrict__ in,
                                               float* __restrict__ out, int rows,
                                               int cols) {
    static_assert(TC % 64 == 0 && (!GUARD || TC == 64), "tile width");
    constexpr int P = TC + 1, Q = TC / 64;
    __shared__ float tile[TR_ROWS * P];
    const int t = threadIdx.x;  // 256 threads
    const int tiles_c = (cols + TC - 1) / TC;
    const int tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
    const int r0 = tr * TR_ROWS, c0 = tc * TC;
    const int sub = t & 15;  // float4 slot inside 64 columns
    const int rr = t >> 4;   // 0..15
    const bool nt = (long long)rows * cols >= TR_NT_MIN;
    float4 v[4 * Q];
#pragma unroll
    for (int i = 0; i < 4 * Q; i++) {
        const int lr = rr + 16 * (i / Q), lc = 64 * (i % Q) + 4 * sub;
        const int r = r0 + lr, c = c0 + lc;
        if constexpr (!GUARD) {
            v[i] = *reinterpret_cast<const float4*>(in + (long long)r * cols + c);
        } else {
            const float* p = in + (long long)r * cols + c;
            const bool ok = r < rows;
            v[i].x = (ok && c + 0 < cols) ? p[0] : 0.0f;
            v[i].y = (ok && c + 1 < cols) ? p[1] : 0.0f;
            v[i].z = (ok && c + 2 < cols) ? p[2] : 0.0f;
            v[i].w = (ok && c + 3 < cols) ? p[3] : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < 4 * Q; i++) {
        const int lr = rr + 16 * (i / Q), lc = 64 * (i % Q) + 4 * sub;
        float* s = tile + lr * P + lc;
        s[0] = v[i].x; s[1] = v[i].y; s[2] = v[i].z; s[3] = v[i].w;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4 * Q; i++) {
        const int lc = rr + 16 * i;  // input column = output row
        const int lr = sub * 4;      // first of four input rows
        float4 w;
        w.x = tile[(lr + 0) * P + lc];
        w.y = tile[(lr + 1) * P + lc];
        w.z = tile[(lr + 2) * P + lc];
        w.w = tile[(lr + 3) * P + lc];
        const int orow = c0 + lc, ocol = r0 + lr;
        if constexpr (!GUARD) {
            store_f4(out + (long long)orow * rows + ocol, w, nt);
        } else if (orow < cols) {
            float* p = out + (long long)orow * rows + ocol;
            if (ocol + 0 < rows) p[0] = w.x;
            if (ocol + 1 < rows) p[1] = w.y;
            if (ocol + 2 < rows) p[2] = w.z;
            if (ocol + 3 < rows) p[3] = w.w;
        }
    }
}

}  // namespace forge
