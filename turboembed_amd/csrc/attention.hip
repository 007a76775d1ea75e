// Softmax attention within each packed row and head: ctx = softmax(Q K^T /
// sqrt(d) + mask) V over the row's live keys (reference
// core/src/cpu/kernels/attend.rs:84-322). Masked keys, and keys outside a
// sliding window, score minus infinity; a query whose keys are all masked
// gets a zero context (attend.rs:216-224).
//
// Q and K are head-major, [heads][tcap][d], so one head's keys of one row
// are contiguous rows of d values; V follows transposed, [heads][d][tcap], so
// one head's values of a run of keys are contiguous in each column.
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
    const T *Vt = qkv + (size_t)2 * heads * tcap * D + (size_t)head * D * tcap + start;
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
            vs[j][c] = in ? to_f32(Vt[(size_t)c * tcap + j0 + j]) : 0.0f;
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


// ---- The matrix-core path (F16 and BF16 operands, F32 softmax and sums) ----------
//
// One workgroup of 4 waves per (128-query block, head, row); each wave owns
// 32 queries. Keys go 64 at a time through LDS: K as stored, and V already
// transposed by the QKV epilogue, both loaded as 16-byte vectors.
//
// Scores are computed transposed, S^T = K Q^T on v_mfma_f32_32x32x16, so that
// each lane holds one query (its column, lane % 32) and 16 of the 32 keys of
// a sub-block, the other 16 in the lane 32 away. The online softmax then
// needs one cross-lane step per block (the max with lane ^ 32), and each
// query's running max and sum are a lane's own scalars. The context is also
// computed transposed, O^T += V^T P^T: P^T is the B operand straight from the
// score registers (converted to the operand type), and O^T keeps a query per
// lane, so rescaling by exp(m_old - m_new) is a per-lane multiply.
//
// Key order inside a 32-key sub-block: MFMA row m of the scores reads key
// swap23(m) (bits 2 and 3 of m exchanged). Score register r of a lane in
// half h then holds key 16 (r / 8) + 8 h + r % 8, so registers 0..7 and
// 8..15 are each 8 consecutive keys: exactly the 8 k-slots the lane feeds
// the P^T V^T product per 16-key step, matching 16-byte reads of V^T rows.
// Softmax runs in base 2 on v_exp_f32. A query with no live key in reach
// gets a zero context.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));

template <typename T> struct AttnMma;
template <> struct AttnMma<_Float16> {
    typedef half8_t frag;
    static __device__ __forceinline__ floatx16_t run(frag a, frag b, floatx16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct AttnMma<__bf16> {
    typedef bf16x8_t frag;
    static __device__ __forceinline__ floatx16_t run(frag a, frag b, floatx16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

__device__ __forceinline__ int swap23(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

template <typename T, int D>
__global__ void __launch_bounds__(256) attention_mfma_kernel(const T *__restrict__ qkv, int tcap, int heads,
                                                             Packing p, const int32_t *__restrict__ mask, int seq,
                                                             int window, T *__restrict__ ctx) {
    constexpr int QB = 128, KB = 64;
    constexpr int KS = D + 8;     // LDS row of K, padded by 16 bytes
    constexpr int VS = KB + 8;    // LDS row of V^T
    typedef typename AttnMma<T>::frag frag;
    typedef uint32_t vec4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) T ks[KB * KS];
    __shared__ __attribute__((aligned(16))) T vts[D * VS];
    __shared__ float live[KB];

    const int r = blockIdx.z, head = blockIdx.y, q0 = blockIdx.x * QB;
    const int len = p.len[r];
    if (q0 >= len) return;
    const int start = p.start[r];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5, ql = lane & 31;
    const int query = q0 + wave * 32 + ql;
    const T *Q = qkv + ((size_t)head * tcap + start) * D;
    const T *K = qkv + ((size_t)(heads + head) * tcap + start) * D;
    const T *Vt = qkv + (size_t)2 * heads * tcap * D + (size_t)head * D * tcap + start;
    const int32_t *mk = mask + (size_t)r * seq;

    // This lane's query as the B operand of S^T, d/16 fragments of 8.
    frag qf[D / 16];
    {
        const T *qrow = Q + (size_t)min(query, len - 1) * D + h * 8;
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
            const vec4 v = *(const vec4 *)(qrow + s * 16);
            qf[s] = *(const frag *)&v;
        }
    }
    // log2(e) / sqrt(d): scores go straight to base 2.
    const float scale = 1.4426950408889634f / sqrtf((float)D);
    floatx16_t o[D / 32];
#pragma unroll
    for (int t = 0; t < D / 32; ++t) o[t] = floatx16_t{};
    float m_run = -INFINITY, l_run = 0.0f;

    int k_lo = 0, k_hi = len;
    if (window < INT32_MAX) {
        k_lo = max(0, q0 - window) / KB * KB;
        k_hi = min(len, q0 + QB + window);
    }
    for (int kb = k_lo; kb < k_hi; kb += KB) {
        __syncthreads();
        // K rows kb .. kb + 63: 64 x D as 16-byte vectors; rows past len are 0.
#pragma unroll
        for (int i = 0; i < KB * D / 8 / 256; ++i) {
            const int v = tid + 256 * i, row = v / (D / 8), c = (v % (D / 8)) * 8;
            vec4 x = vec4{0, 0, 0, 0};
            if (kb + row < len) x = *(const vec4 *)(K + (size_t)(kb + row) * D + c);
            *(vec4 *)&ks[row * KS + c] = x;
        }
        // V^T columns kb .. kb + 63 of each of the D rows.
#pragma unroll
        for (int i = 0; i < KB * D / 8 / 256; ++i) {
            const int v = tid + 256 * i, c = v / (KB / 8), j = (v % (KB / 8)) * 8;
            const T *src = Vt + (size_t)c * tcap + kb + j;
            vec4 x;
            if (kb + j + 8 <= len) {
                x = *(const vec4 *)src;
            } else {
                T tmp[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) tmp[e] = kb + j + e < len ? src[e] : from_f32<T>(0.0f);
                x = *(const vec4 *)tmp;
            }
            *(vec4 *)&vts[c * VS + j] = x;
        }
        if (tid < KB) live[tid] = (kb + tid < len && mk[kb + tid] != 0) ? 1.0f : 0.0f;
        __syncthreads();

        floatx16_t sc[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            floatx16_t a = floatx16_t{};
            const T *krow = &ks[(sub * 32 + swap23(ql)) * KS + h * 8];
#pragma unroll
            for (int s = 0; s < D / 16; ++s) a = AttnMma<T>::run(*(const frag *)(krow + s * 16), qf[s], a);
            sc[sub] = a;
        }
        // Scale, mask, and the block's max for this query.
        float mx = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const int j = sub * 32 + 16 * (rr >> 3) + 8 * h + (rr & 7);
                const int key = kb + j;
                bool ok = live[j] != 0.0f;
                if (window < INT32_MAX) ok = ok && key + window >= query && key <= query + window;
                const float v = ok ? sc[sub][rr] * scale : -INFINITY;
                sc[sub][rr] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // Every lane runs the same instructions below (the matrix cores take
        // the whole wave): a query with nothing live in reach yet adds zeros
        // and keeps its state.
        const float m_new = fmaxf(m_run, mx);
        const bool none = m_new == -INFINITY;
        const float m_use = none ? 0.0f : m_new;
        const float alpha = m_run == -INFINITY ? (none ? 1.0f : 0.0f) : __builtin_amdgcn_exp2f(m_run - m_use);
        float rs = 0.0f;
        typename AttnMma<T>::frag pf[2][2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int step = 0; step < 2; ++step) {
                T pv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = sc[sub][step * 8 + e];
                    const float pe = x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(x - m_use);
                    rs += pe;
                    pv[e] = from_f32<T>(pe);
                }
                pf[sub][step] = *(const frag *)pv;
            }
        l_run = l_run * alpha + rs;
        m_run = m_new;
#pragma unroll
        for (int t = 0; t < D / 32; ++t) o[t] *= alpha;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int step = 0; step < 2; ++step)
#pragma unroll
                for (int t = 0; t < D / 32; ++t) {
                    const frag vf = *(const frag *)&vts[(32 * t + ql) * VS + sub * 32 + step * 16 + h * 8];
                    o[t] = AttnMma<T>::run(vf, pf[sub][step], o[t]);
                }
    }
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    if (query >= len) return;
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    T *out = ctx + (size_t)(start + query) * heads * D + head * D;
#pragma unroll
    for (int t = 0; t < D / 32; ++t)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            const int c = 32 * t + 8 * (rr >> 2) + 4 * h + (rr & 3);
            out[c] = from_f32<T>(o[t][rr] * inv);
        }
}

template <typename T>
static hipError_t attention_mfma_t(hipStream_t s, const void *qkv, int tcap, int heads, int d, const Packing &p,
                                   const int32_t *mask, int seq, int batch, int max_len, int window, void *ctx) {
    const dim3 grid((max_len + 127) / 128, heads, batch);
    switch (d) {
    case 32:
        hipLaunchKernelGGL((attention_mfma_kernel<T, 32>), grid, dim3(256), 0, s, (const T *)qkv, tcap, heads, p, mask,
                           seq, window, (T *)ctx);
        break;
    case 64:
        hipLaunchKernelGGL((attention_mfma_kernel<T, 64>), grid, dim3(256), 0, s, (const T *)qkv, tcap, heads, p, mask,
                           seq, window, (T *)ctx);
        break;
    case 128:
        hipLaunchKernelGGL((attention_mfma_kernel<T, 128>), grid, dim3(256), 0, s, (const T *)qkv, tcap, heads, p,
                           mask, seq, window, (T *)ctx);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t attention(hipStream_t s, Dt dt, const void *qkv, int tcap, int heads, int d, const Packing &p,
                     const int32_t *mask, int seq, int batch, int max_len, int window, void *ctx, bool simple) {
    if (max_len <= 0) return hipSuccess;
    const bool mfma = (d == 32 || d == 64 || d == 128) && !simple;
    switch (dt) {
    case Dt::F16:
        return mfma ? attention_mfma_t<_Float16>(s, qkv, tcap, heads, d, p, mask, seq, batch, max_len, window, ctx)
                    : attention_t<_Float16>(s, qkv, tcap, heads, d, p, mask, seq, batch, max_len, window, ctx);
    case Dt::BF16:
        return mfma ? attention_mfma_t<__bf16>(s, qkv, tcap, heads, d, p, mask, seq, batch, max_len, window, ctx)
                    : attention_t<__bf16>(s, qkv, tcap, heads, d, p, mask, seq, batch, max_len, window, ctx);
    default: return attention_t<float>(s, qkv, tcap, heads, d, p, mask, seq, batch, max_len, window, ctx);
    }
}

}  // namespace rocm
