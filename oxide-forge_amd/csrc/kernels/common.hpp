// common.hpp -- shared device helpers for the gfx950 (CDNA4) kernels.
//
// Wavefronts are 64 lanes.  Cross-lane reductions use DPP row operations
// (quad_perm, row_half_mirror, row_mirror) to reduce inside each 16-lane row,
// then v_readlane to combine the four rows into a wave-uniform scalar.  Every
// lane of a row ends with the same bits (float addition and fmax are
// commutative, and each step pairs the same two partial values), so the
// result is deterministic and identical in every lane.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define FORGE_KERNEL extern "C" __global__

namespace forge {

typedef float v16f __attribute__((ext_vector_type(16)));

// DPP control words (GFX9 encoding).
constexpr int DPP_QUAD_1032 = 0xB1;      // quad_perm:[1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;      // quad_perm:[2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over the 64 lanes; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = v + dpp_mov<DPP_QUAD_1032>(v);
    v = v + dpp_mov<DPP_QUAD_2301>(v);
    v = v + dpp_mov<DPP_ROW_HALF_MIRROR>(v);
    v = v + dpp_mov<DPP_ROW_MIRROR>(v);
    return (readlane(v, 0) + readlane(v, 16)) +
           (readlane(v, 32) + readlane(v, 48));
}

// Integer sum over the 64 lanes (wraps modulo 2^32); wave-uniform.
__device__ __forceinline__ unsigned wave_sum_u32(unsigned v) {
    v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, DPP_QUAD_1032, 0xF, 0xF, false);
    v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, DPP_QUAD_2301, 0xF, 0xF, false);
    v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, DPP_ROW_HALF_MIRROR, 0xF, 0xF, false);
    v += (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, DPP_ROW_MIRROR, 0xF, 0xF, false);
    return ((unsigned)__builtin_amdgcn_readlane((int)v, 0) + (unsigned)__builtin_amdgcn_readlane((int)v, 16)) +
           ((unsigned)__builtin_amdgcn_readlane((int)v, 32) + (unsigned)__builtin_amdgcn_readlane((int)v, 48));
}

// Max over the 64 lanes; the result is wave-uniform.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<DPP_QUAD_1032>(v));
    v = fmaxf(v, dpp_mov<DPP_QUAD_2301>(v));
    v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
    return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)),
                 fmaxf(readlane(v, 32), readlane(v, 48)));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Native 4-float vector (stays in VGPRs; the nontemporal builtins take it).
typedef float f4 __attribute__((ext_vector_type(4)));

// Streaming 128-bit load with the nontemporal hint, for data a kernel reads
// once.  On MI355X a store to a line that an ordinary load has just cached is
// markedly slower than a store to an uncached line: an in-place x = x * s
// over 16 MiB takes 8.1 us with ordinary loads and 6.6 us with nontemporal
// ones (out of place: 7.2 us and 7.1 us).  Every in-place streaming and row
// kernel therefore reads its operands with this load.
__device__ __forceinline__ float4 load_stream(const float* p) {
    const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// Outputs of at least STREAM_NT_MIN floats (64 MiB) are stored
// non-temporally: they do not fit the 256 MiB MALL beside their inputs, and
// write-allocating them there costs bandwidth (6.59 against 5.80 TB/s for an
// in-place float4 scale of 256 MiB on MI355X).  Smaller ones keep cached
// stores (at 16 MiB non-temporal ones are 4% slower for that scale), except
// where a kernel measured faster without (the GEMM epilogue, the softmax and
// RMSNorm forward).
constexpr long long STREAM_NT_MIN = 16ll << 20;

__device__ __forceinline__ void store_f4(float* p, float4 v, bool nt) {
    if (nt)
        __builtin_nontemporal_store(f4{v.x, v.y, v.z, v.w}, reinterpret_cast<f4*>(p));
    else
        *reinterpret_cast<float4*>(p) = v;
}

// BinaryOp (cuda.rs:3-10) applied as one rounded f32 operation
// (elementwise.rs:5-13).
enum BinOp { OP_ADD = 0, OP_SUB = 1, OP_MUL = 2, OP_DIV = 3 };

template <int OP>
__device__ __forceinline__ float apply_binary(float l, float r) {
    if constexpr (OP == OP_ADD) return l + r;
    else if constexpr (OP == OP_SUB) return l - r;
    else if constexpr (OP == OP_MUL) return l * r;
    else return l / r;
}

// Activation (linear.rs:21-70).  The expression order follows the reference
// so that, with contraction disabled, only tanhf/expf rounding differs.
constexpr float GELU_SCALE = 0.7978846f;
constexpr float GELU_CUBIC = 0.044715f;
constexpr float GELU_DERIVATIVE_QUADRATIC = GELU_SCALE * 3.0f * GELU_CUBIC;

enum Act { ACT_IDENTITY = 0, ACT_GELU = 1, ACT_RELU = 2, ACT_SILU = 3 };

// GELU in the tanh form of linear.rs:26-43, 0.5 x (1 + tanh(u)) with
// u = GELU_SCALE (x + GELU_CUBIC x^3), evaluated through the identity
// 0.5 (1 + tanh(u)) = s = 1 / (1 + exp(-2u)) = 1 / (1 + 2^t),
// t = -2 log2(e) u = x (GELU_T1 + GELU_T3 x^2): the hardware base-2
// exponential (v_exp_f32) and reciprocal instead of tanhf.  The two
// constants fold -2 log2(e) into the reference's f32 constants (computed in
// double, rounded once), so the exponent takes four operations instead of
// seven; the activation epilogue of the GEMM is several times cheaper than
// with tanhf, and the identity avoids tanh's cancellation in 1 + tanh(u) for
// negative u.  The error of 2^t grows with |t|, but where it matters 2^t is
// large and the result x / (1 + 2^t) is tiny: within 2e-6 (relative, plus
// 2e-6 absolute) of the f64 formula over x ~ N(0, 2) and at the extremes
// (x = +-inf give the reference's inf and NaN).
constexpr float GELU_T1 = -2.302208185195923f;   // -2 log2(e) GELU_SCALE
constexpr float GELU_T3 = -0.10294323414564133f; // GELU_T1 GELU_CUBIC

__device__ __forceinline__ float gelu_exp2_arg(float x) {
    return x * (GELU_T1 + GELU_T3 * (x * x));
}

__device__ __forceinline__ float gelu(float x) {
    const float e = __builtin_amdgcn_exp2f(gelu_exp2_arg(x));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// d/dx of the above: 0.5 (1 + t) + 0.5 x (1 - t^2) u' with t = tanh(u)
// becomes s + 2 x s (1 - s) u', and 1 - s = e s (1 where e overflows).
__device__ __forceinline__ float gelu_derivative(float x) {
    const float e = __builtin_amdgcn_exp2f(gelu_exp2_arg(x));
    const float s = __builtin_amdgcn_rcpf(1.0f + e);
    const float one_minus_s = __builtin_isinf(e) ? 1.0f : e * s;
    const float inner_derivative = GELU_SCALE + GELU_DERIVATIVE_QUADRATIC * x * x;
    return s + 2.0f * x * s * one_minus_s * inner_derivative;
}

__device__ __forceinline__ float relu(float x) { return x > 0.0f ? x : 0.0f; }
__device__ __forceinline__ float relu_derivative(float x) {
    return x > 0.0f ? 1.0f : 0.0f;
}
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float silu_derivative(float x) {
    float e = expf(-x);
    return 1.0f / (1.0f + e) + x * e / ((1.0f + e) * (1.0f + e));
}

__device__ __forceinline__ float activate(int act, float x) {
    switch (act) {
    case ACT_GELU: return gelu(x);
    case ACT_RELU: return relu(x);
    case ACT_SILU: return silu(x);
    default: return x;
    }
}

__device__ __forceinline__ float activate_derivative(int act, float x) {
    switch (act) {
    case ACT_GELU: return gelu_derivative(x);
    case ACT_RELU: return relu_derivative(x);
    case ACT_SILU: return silu_derivative(x);
    default: return 1.0f;
    }
}

}  // namespace forge
