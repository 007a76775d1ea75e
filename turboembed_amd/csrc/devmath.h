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

namespace rocm {

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

// GELU for the 16-bit tiers, whose outputs keep 8 to 11 bits: erf by
// Abramowitz and Stegun's formula 7.1.26 (absolute error under 1.5e-7), on
// the hardware's exp2 and reciprocal: a dozen instructions against the
// erfcc fit's fifty.
__device__ __forceinline__ float dev_gelu_fast(float x) {
    const float z = fabsf(x) * 0.70710678118654752440f;
    const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));
    float p = fmaf(1.061405429f, t, -1.453152027f);
    p = fmaf(p, t, 1.421413741f);
    p = fmaf(p, t, -0.284496736f);
    p = fmaf(p, t, 0.254829592f);
    p *= t;
    // erfc(z) = p e^{-z^2}, e^{-z^2} = 2^{-z^2 log2 e}; gelu(x) = x/2 (2 - erfc)
    // for x >= 0 and x/2 erfc(|z|) below, with no cancellation.
    const float r = p * __builtin_amdgcn_exp2f(-z * z * 1.44269504088896340736f);
    return 0.5f * x * (x >= 0.0f ? 2.0f - r : r);
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
