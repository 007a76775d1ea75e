// Device-side scalar functions shared by the kernels: e^x, GELU and SiLU as
// the reference's CPU path computes them (core/src/cpu/kernels/rowwise.rs:31-113),
// so every tier uses the same published methods: Cephes' expf polynomial
// and Numerical Recipes' erfcc fit, with the exponent's -x^2/2 carried as
// an exact two-float sum. Wave64 reductions too.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "kernels.h"

namespace rocm {

// A launch's extent on the device: the rows and packed tokens of its span,
// from the run's dimensions (scalar loads, made uniform) or as given.
struct Live {
    int row0, rows, tok0, tokens, max_len, seq;
};
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ Live live_of(const Span &s) {
    if (!s.dims) return Live{s.row0, s.rows, s.tok0, s.tokens, s.max_len, s.seq};
    const RunDims *d = s.dims;
    if (s.part < 0)
        return Live{0, uniform(d->batch), 0, uniform(d->tokens), uniform(d->max_len), uniform(d->seq)};
    const PartDims *p = &d->part[s.part];
    return Live{uniform(p->row0), uniform(p->rows), uniform(p->tok0), uniform(p->tokens), uniform(p->max_len),
                uniform(d->seq)};
}

__device__ __forceinline__ float dev_exp(float x) {
    const float lo = -80.0f;
    const float c = fminf(fmaxf(x, lo), 88.0f);
    const float n = floorf(__fadd_rn(__fmul_rn(c, 1.44269504088896340736f), 0.5f));
    float r = __fsub_rn(c, __fmul_rn(n, 0.693359375f));
    r = __fsub_rn(r, __fmul_rn(n, -2.12194440e-4f));
    const float r2 = __fmul_rn(r, r);
    float p = __fadd_rn(__fmul_rn(1.9875691e-4f, r), 1.3982e-3f);
    p = __fadd_rn(__fmul_rn(p, r), 8.3334519073e-3f);
    p = __fadd_rn(__fmul_rn(p, r), 4.1665795894e-2f);
    p = __fadd_rn(__fmul_rn(p, r), 1.6666665459e-1f);
    p = __fadd_rn(__fmul_rn(p, r), 0.5f);
    const float e = __fadd_rn(__fadd_rn(__fmul_rn(p, r2), r), 1.0f);
    const uint32_t n_int = __float_as_uint(__fadd_rn(n, 12582912.0f)) - 0x4b400000u;
    const float scale = __uint_as_float((n_int + 127u) << 23);
    return x < lo ? 0.0f : __fmul_rn(e, scale);
}

__device__ __forceinline__ float dev_gelu(float x) {
    const float xc = fminf(fmaxf(x, -16.0f), 16.0f);
    const float z = __fmul_rn(fabsf(xc), 0.70710678118654752440f);
    const float t = __frcp_rn(__fadd_rn(1.0f, __fmul_rn(0.5f, z)));
    float p = 0.17087277f;
    p = __fadd_rn(-0.8221522f, __fmul_rn(t, p));
    p = __fadd_rn(1.48851587f, __fmul_rn(t, p));
    p = __fadd_rn(-1.13520398f, __fmul_rn(t, p));
    p = __fadd_rn(0.27886807f, __fmul_rn(t, p));
    p = __fadd_rn(-0.18628806f, __fmul_rn(t, p));
    p = __fadd_rn(0.09678418f, __fmul_rn(t, p));
    p = __fadd_rn(0.37409196f, __fmul_rn(t, p));
    p = __fadd_rn(1.00002368f, __fmul_rn(t, p));
    p = __fadd_rn(-1.26551223f, __fmul_rn(t, p));
    // -xc^2 / 2 = hi + lo exactly (Dekker's product by an FMA), and hi + p = a + e.
    const float sq = __fmul_rn(xc, xc);
    const float sq_lo = __fmaf_rn(xc, xc, -sq);
    const float hi = -0.5f * sq, lo = -0.5f * sq_lo;
    const float a = __fadd_rn(hi, p);
    const float bb = __fsub_rn(a, hi);
    const float err = __fadd_rn(__fsub_rn(hi, __fsub_rn(a, bb)), __fsub_rn(p, bb));
    const float r = __fmul_rn(t, __fmul_rn(dev_exp(a), __fadd_rn(1.0f, __fadd_rn(err, lo))));
    return __fmul_rn(__fmul_rn(0.5f, x), x >= 0.0f ? __fsub_rn(2.0f, r) : r);
}

// GELU for the 16-bit tiers, whose outputs keep 8 to 11 bits: GELU's tanh
// form, 0.5 x (1 + tanh(u)), u = sqrt(2 / pi) (x + 0.044715 x^3), the form
// the reference's CUDA backend gives an F16 output in its FASTEST tier
// (core/cuda/kernels.cu:163-173, docs/cuda.md:668-676). With
// 0.5 (1 + tanh(u)) = 1 / (1 + e^{-2u}) it is x / (1 + 2^{-2u log2 e}):
// two multiplies and a multiply-add for the exponent, the hardware's exp2
// and reciprocal, one add and one multiply, against the erf form's twenty.
// Within 4.7e-4 of erf's GELU absolutely (at x = 2.7, a quarter of an F16
// ulp there); at -inf the exponential is +inf and the value is -0, at +inf
// it is x.
__device__ __forceinline__ float dev_gelu_fast(float x) {
    constexpr float k = -2.0f * 0.79788456080286535588f * 1.44269504088896340736f;   // -2 sqrt(2/pi) log2 e
    const float e = __builtin_amdgcn_exp2f(x * fmaf(0.044715f * k, x * x, k));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float dev_silu(float x) {
    return __fdiv_rn(x, __fadd_rn(1.0f, dev_exp(-x)));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) { return (__bf16)v; }

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(__bf16 v) { return (float)v; }

}  // namespace rocm
