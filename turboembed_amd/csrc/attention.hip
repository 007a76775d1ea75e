// Softmax attention within each packed row and head: ctx = softmax(Q K^T /
// sqrt(d) + mask) V over the row's live keys (reference
// core/src/cpu/kernels/attend.rs:84-322). Masked keys, and keys outside a
// sliding window, score minus infinity; a query whose keys are all masked
// gets a zero context (attend.rs:216-224).
//
// Q, K and V are head-major, [3][heads][tcap][d], so one head's keys of one
// row are contiguous rows of d values.
#include "kernels.h"
#include "devmath.h"

namespace rocm {

// The scalar path: one workgroup of 64 lanes per (64-query block, head, row),
// a lane per query, the keys staged through LDS 64 at a time, an online
// softmax in F32 with Cephes' exp. Every tier's reference path.
template <typename T, int D>
__global__ void __launch_bounds__(64) attention_simple_kernel(const T *__restrict__ qkv, int tcap, int heads,
                                                              Packing p, const int32_t *__restrict__ mask, int seq,
                                                              int window, T *__restrict__ ctx) {
    const int r = blockIdx.z, head = blockIdx.y, q0 = blockIdx.x * 64;
    const int len = p.len[r];
    if (q0 >= len) return;
    const int start = p.start[r];
    const int lane = threadIdx.x, i = q0 + lane;
    const T *Q = qkv + ((size_t)head * tcap + start) * D;
    const T *K = qkv + ((size_t)(heads + head) * tcap + start) * D;
    const T *V = qkv + ((size_t)(2 * heads + head) * tcap + start) * D;
    const int32_t *mk = mask + (size_t)r * seq;
    constexpr int KC = D <= 64 ? 64 : 32;   // keys staged a step
    __shared__ float ks[KC][D + 1], vs[KC][D + 1];
    __shared__ float live[KC];
    float q[D], acc[D];
    const float scale = 1.0f / sqrtf((float)D);
#pragma unroll
    for (int c = 0; c < D; ++c) {
        q[c] = i < len ? to_f32(Q[(size_t)i * D + c]) : 0.0f;
        acc[c] = 0.0f;
    }
    float mx = -INFINITY, l = 0.0f;
    for (int j0 = 0; j0 < len; j0 += KC) {
        __syncthreads();
        for (int x = lane; x < KC * D; x += 64) {
            const int j = x / D, c = x % D;
            const bool in = j0 + j < len;
            ks[j][c] = in ? to_f32(K[(size_t)(j0 + j) * D + c]) : 0.0f;
            vs[j][c] = in ? to_f32(V[(size_t)(j0 + j) * D + c]) : 0.0f;
        }
        if (lane < KC) live[lane] = (j0 + lane < len && mk[j0 + lane] != 0) ? 1.0f : 0.0f;
        __syncthreads();
        const int nj = min(KC, len - j0);
        for (int j = 0; j < nj; ++j) {
            const int key = j0 + j;
            if (live[j] == 0.0f) continue;
            if (window < INT32_MAX && (key + window < i || key > i + window)) continue;
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < D; ++c) s = fmaf(q[c], ks[j][c], s);
            s *= scale;
            if (s > mx) {
                const float f = mx == -INFINITY ? 0.0f : dev_exp(mx - s);
                l *= f;
#pragma unroll
                for (int c = 0; c < D; ++c) acc[c] *= f;
                mx = s;
            }
            const float pj = dev_exp(s - mx);
            l += pj;
#pragma unroll
            for (int c = 0; c < D; ++c) acc[c] = fmaf(pj, vs[j][c], acc[c]);
        }
    }
    if (i >= len) return;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    T *out = ctx + (size_t)(start + i) * heads * D + head * D;
#pragma unroll
    for (int c = 0; c < D; ++c) out[c] = from_f32<T>(acc[c] * inv);
}

template <typename T>
static hipError_t attention_t(hipStream_t s, const void *qkv, int tcap, int heads, int d, const Packing &p,
                              const int32_t *mask, int seq, int batch, int max_len, int window, void *ctx) {
    const dim3 grid((max_len + 63) / 64, heads, batch);
#define ATT_CASE(D)                                                                                             \
    case D:                                                                                                     \
        hipLaunchKernelGGL((attention_simple_kernel<T, D>), grid, dim3(64), 0, s, (const T *)qkv, tcap, heads, p, \
                           mask, seq, window, (T *)ctx);                                                        \
        break;
    switch (d) {
        ATT_CASE(8)
        ATT_CASE(16)
        ATT_CASE(32)
        ATT_CASE(64)
        ATT_CASE(128)
    default: return hipErrorInvalidValue;
    }
#undef ATT_CASE
    return hipGetLastError();
}

hipError_t attention(hipStream_t s, Dt dt, const void *qkv, int tcap, int heads, int d, const Packing &p,
                     const int32_t *mask, int seq, int batch, int max_len, int window, void *ctx) {
    if (max_len <= 0) return hipSuccess;
    switch (dt) {
    case Dt::F16: return attention_t<_Float16>(s, qkv, tcap, heads, d, p, mask, seq, batch, max_len, window, ctx);
    case Dt::BF16: return attention_t<__bf16>(s, qkv, tcap, heads, d, p, mask, seq, batch, max_len, window, ctx);
    default: return attention_t<float>(s, qkv, tcap, heads, d, p, mask, seq, batch, max_len, window, ctx);
    }
}

}  // namespace rocm
