// Row arithmetic shared by the row kernels and the GEMM's LayerNorm
// epilogue: a 32-lane half-wave holds one row of `hidden` columns, lane hl
// taking 8 consecutive columns 8 (hl + 32 g) .. + 7 of each group g of 256.
// Both the separate add + LayerNorm and the one fused into a product's
// epilogue go through these functions, so one row gives the same bits
// whichever kernel norms it.
#pragma once

#include "devmath.h"

namespace rocm {

typedef float float4_t __attribute__((ext_vector_type(4)));

// Eight consecutive columns at p, as F32.
template <typename H> __device__ __forceinline__ void load8(const H *p, float (&v)[8]) {
    typedef H h8 __attribute__((ext_vector_type(8)));
    const h8 q = *(const h8 *)p;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = to_f32(q[k]);
}
__device__ __forceinline__ void load8(const float *p, float (&v)[8]) {
    const float4_t a = *(const float4_t *)p, b = *(const float4_t *)(p + 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = a[k], v[4 + k] = b[k];
}
template <typename H> __device__ __forceinline__ void store8(H *p, const float (&v)[8]) {
    typedef H h8 __attribute__((ext_vector_type(8)));
    h8 q;
#pragma unroll
    for (int k = 0; k < 8; ++k) q[k] = from_f32<H>(v[k]);
    *(h8 *)p = q;
}
__device__ __forceinline__ void store8(float *p, const float (&v)[8]) {
    *(float4_t *)p = float4_t{v[0], v[1], v[2], v[3]};
    *(float4_t *)(p + 4) = float4_t{v[4], v[5], v[6], v[7]};
}

// The sum over a 32-lane half of the wave.
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// A half-wave row's norm weight and bias (0 where absent), 8 columns a lane
// in each group of 256.
template <int G>
__device__ __forceinline__ void load_wb8(const float *__restrict__ w, const float *__restrict__ b, int hidden, int hl,
                                         float (&wv)[G][8], float (&bv)[G][8]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 8 * (hl + 32 * g);
#pragma unroll
        for (int k = 0; k < 8; ++k) wv[g][k] = bv[g][k] = 0.0f;
        if (c >= hidden) continue;
        load8(w + c, wv[g]);
        if (b) load8(b + c, bv[g]);
    }
}

// A half-wave row's mean and 1 / sqrt(var + eps), the biased variance
// about the mean (two passes over registers), both summed in F32.
template <int G>
__device__ __forceinline__ void ln_pair_stats(const float (&v)[G][8], int hidden, int hl, float eps, float &mean,
                                              float &inv) {
    float s = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 8; k += 2) s += v[g][k] + v[g][k + 1];
    mean = half_sum(s) / (float)hidden;
    float q = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (8 * (hl + 32 * g) < hidden)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float c = v[g][k] - mean;
                q = fmaf(c, c, q);
            }
    inv = 1.0f / sqrtf(half_sum(q) / (float)hidden + eps);
}

// One normalized value, (v - mean) * inv, then times w plus b in one
// rounding: the same operations whichever kernel calls it.
__device__ __forceinline__ float ln_out(float v, float mean, float inv, float w, float b) {
#pragma clang fp contract(off)
    return fmaf((v - mean) * inv, w, b);
}

// A half-wave row normalized, (v - mean) / sqrt(var + eps) * w + b.
template <int G>
__device__ __forceinline__ void ln_pair_apply(float (&v)[G][8], int hidden, int hl, const float (&wv)[G][8],
                                              const float (&bv)[G][8], float eps) {
    float mean, inv;
    ln_pair_stats<G>(v, hidden, hl, eps, mean, inv);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 8; ++k) v[g][k] = ln_out(v[g][k], mean, inv, wv[g][k], bv[g][k]);
}

// A row's int8 codes (symmetric, scale = max |r| / 127 over the row) from
// its normalized values as rounded to H, 8 columns a lane as above, into
// qr (the row's first code) and *scale (written by lane 0 of the half).
template <int G, typename H>
__device__ __forceinline__ void quant_pair_row(const float (&v)[G][8], int hidden, int hl, int8_t *qr, float *scale) {
    float r[G][8], mx = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            r[g][k] = 8 * (hl + 32 * g) < hidden ? to_f32(from_f32<H>(v[g][k])) : 0.0f;
            mx = fmaxf(mx, fabsf(r[g][k]));
        }
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float iv = mx > 0.0f ? 127.0f / mx : 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 8 * (hl + 32 * g);
        if (c >= hidden) continue;
        uint32_t w[2] = {0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int code = (int)fminf(fmaxf(rintf(r[g][k] * iv), -127.0f), 127.0f);
            w[k >> 2] |= (uint32_t)(uint8_t)(int8_t)code << (8 * (k & 3));
        }
        *(uint2 *)(qr + c) = uint2{w[0], w[1]};
    }
    if (hl == 0) *scale = mx / 127.0f;
}

}  // namespace rocm
