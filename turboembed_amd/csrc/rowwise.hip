// Row-wise kernels of the encoder: packing, embedding + LayerNorm, LayerNorm,
// pooling (rows and ranges) with the cut and L2, and weight narrowing.
// All are HBM-bound; each reads its input once, coalesced, with wave64
// shuffle reductions and no atomics on floats.
#include <algorithm>
#include <mutex>

#include "kernels.h"
#include "launch.h"
#include "devmath.h"
#include "rowmath.h"

namespace rocm {

// ---- Packing ------------------------------------------------------------------
//
// One workgroup. Each row's packed length is its last live column + 1
// (reference core/src/cpu/encoder/mod.rs:395-405; core/cuda/kernels.cu:290-381):
// integer maxima, then an exclusive scan in row order. Integer work only,
// so the result is exact.
__global__ void __launch_bounds__(1024) pack_rows_kernel(const int32_t *__restrict__ mask,
                                                         const RunDims *__restrict__ dims, Packing p) {
    extern __shared__ int32_t lens[];
    const int batch = uniform(dims->batch), seq = uniform(dims->seq);
    // Each wave takes whole rows: every lane's last live column among its
    // strided ones, then the wave's maximum (no atomics on a few shared words).
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    // (Rows of a multiple of 4 columns are read 16 bytes a lane, 256 columns
    // a wave a step; a wave's four rows at a time, their reads issued
    // together.)
    typedef int int4_t __attribute__((ext_vector_type(4)));
    constexpr int RW = 4;
    for (int r0 = wave; r0 < batch; r0 += RW * waves) {
        int last[RW];
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            const int r = r0 + j * waves;
            last[j] = 0;
            if (r >= batch) continue;
            const int32_t *row = mask + (size_t)r * seq;
            if ((seq & 3) == 0) {
#pragma unroll 4
                for (int c = 4 * lane; c < seq; c += 256) {
                    const int4_t v = *(const int4_t *)(row + c);
                    last[j] = v[3] ? c + 4 : v[2] ? c + 3 : v[1] ? c + 2 : v[0] ? c + 1 : last[j];
                }
            } else {
                for (int c = lane; c < seq; c += 64)
                    if (row[c] != 0) last[j] = c + 1;
            }
        }
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            int l = last[j];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) l = max(l, __shfl_xor(l, o, 64));
            const int r = r0 + j * waves;
            if (lane == 0 && r < batch) lens[r] = l;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int t = 0;
        for (int r = 0; r < batch; ++r) {
            const int l = lens[r];
            p.start[r] = t;
            p.len[r] = l;
            t += l;
        }
        p.tokens[0] = t;
    }
}

// Each packed token's place, a thread per column of the rows (grid-strided):
// a column under its row's length is token start + column.
__global__ void __launch_bounds__(256) place_tokens_kernel(const RunDims *__restrict__ dims, Packing p) {
    const int batch = uniform(dims->batch), seq = uniform(dims->seq), n = batch * seq;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const int r = i / seq, c = i - r * seq;
        if (c < p.len[r]) {
            const int at = p.start[r] + c;
            p.at[at] = i;
            p.row[at] = r;
            p.pos[at] = c;
        }
    }
}

hipError_t pack_rows(hipStream_t s, const int32_t *mask, const RunDims *dims, int max_batch, int max_seq, Packing p) {
    enqueue(pack_rows_kernel, dim3(1), dim3(1024), max_batch * sizeof(int32_t), s, mask, dims, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t blocks = std::min<size_t>(((size_t)max_batch * max_seq + 255) / 256, 1024);
    enqueue(place_tokens_kernel, dim3(blocks), dim3(256), 0, s, dims, p);
    return hipGetLastError();
}

// ---- LayerNorm over one token per wave ------------------------------------------
//
// Each lane holds G groups of 4 consecutive columns of the row, columns
// 4 (lane + 64 g) .. + 3, read and written as 16-byte (F32) or 8-byte
// (16-bit) vectors (hidden is a multiple of 8). The mean and the biased
// variance are summed in F32 across the wave, the variance about the mean
// (two passes over registers).
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void load4(const float *p, float (&v)[4]) {
    const float4_t q = *(const float4_t *)p;
    v[0] = q[0], v[1] = q[1], v[2] = q[2], v[3] = q[3];
}
template <typename H> __device__ __forceinline__ void load4(const H *p, float (&v)[4]) {
    typedef H h4 __attribute__((ext_vector_type(4)));
    const h4 q = *(const h4 *)p;
    v[0] = to_f32(q[0]), v[1] = to_f32(q[1]), v[2] = to_f32(q[2]), v[3] = to_f32(q[3]);
}
__device__ __forceinline__ void store4(float *p, const float (&v)[4]) { *(float4_t *)p = float4_t{v[0], v[1], v[2], v[3]}; }
template <typename H> __device__ __forceinline__ void store4(H *p, const float (&v)[4]) {
    typedef H h4 __attribute__((ext_vector_type(4)));
    *(h4 *)p = h4{from_f32<H>(v[0]), from_f32<H>(v[1]), from_f32<H>(v[2]), from_f32<H>(v[3])};
}

// A lane's columns of a LayerNorm's weight and bias (bias 0 where absent).
template <int G>
__device__ __forceinline__ void load_wb(const float *__restrict__ w, const float *__restrict__ b, int hidden,
                                        float (&wv)[G][4], float (&bv)[G][4]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 4 * (lane + 64 * g);
#pragma unroll
        for (int k = 0; k < 4; ++k) wv[g][k] = bv[g][k] = 0.0f;
        if (c >= hidden) continue;
        load4(w + c, wv[g]);
        if (b) load4(b + c, bv[g]);
    }
}

// A wave's row normalized: (v - mean) / sqrt(var + eps) * w + b, the mean
// and variance over the row's `hidden` columns.
template <int G>
__device__ __forceinline__ void ln_apply(float (&v)[G][4], int hidden, const float (&wv)[G][4],
                                         const float (&bv)[G][4], float eps) {
    const int lane = threadIdx.x & 63;
    float s = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (4 * (lane + 64 * g) < hidden) s += (v[g][0] + v[g][1]) + (v[g][2] + v[g][3]);
    const float mean = wave_sum(s) / (float)hidden;
    float q = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (4 * (lane + 64 * g) < hidden)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float c = v[g][k] - mean;
                q = fmaf(c, c, q);
            }
    const float var = wave_sum(q) / (float)hidden;
    const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (4 * (lane + 64 * g) >= hidden) continue;
#pragma unroll
        for (int k = 0; k < 4; ++k) v[g][k] = (v[g][k] - mean) * inv * wv[g][k] + bv[g][k];
    }
}

template <int G>
__device__ __forceinline__ void ln_wave(float (&v)[G][4], int hidden, const float *__restrict__ w,
                                        const float *__restrict__ b, float eps) {
    float wv[G][4], bv[G][4];
    load_wb<G>(w, b, hidden, wv, bv);
    ln_apply<G>(v, hidden, wv, bv, eps);
}

template <int G, typename H>
__device__ __forceinline__ void store_row(const float (&v)[G][4], int hidden, float *xf, H *xh) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 4 * (lane + 64 * g);
        if (c < hidden) {
            if (xf) store4(xf + c, v[g]);
            if (xh) store4(xh + c, v[g]);
        }
    }
}

// The row's int8 codes and scale from its values as rounded to H (what a
// 16-bit output holds), as quantize_rows makes them: scale = max |v| / 127,
// code = clamp(rint(v * 127 / max), -127, 127).
template <int G, typename H>
__device__ __forceinline__ void quant_row(const float (&v)[G][4], int hidden, int8_t *q, float *scale) {
    const int lane = threadIdx.x & 63;
    float r[G][4], mx = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            r[g][k] = 4 * (lane + 64 * g) < hidden ? to_f32(from_f32<H>(v[g][k])) : 0.0f;
            mx = fmaxf(mx, fabsf(r[g][k]));
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 4 * (lane + 64 * g);
        if (c >= hidden) continue;
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int code = (int)fminf(fmaxf(rintf(r[g][k] * inv), -127.0f), 127.0f);
            w |= (uint32_t)(uint8_t)(int8_t)code << (8 * k);
        }
        *(uint32_t *)(q + c) = w;
    }
    if (lane == 0) *scale = mx / 127.0f;
}

template <int G, typename H>
__global__ void __launch_bounds__(256) embed_ln_kernel(Span sp, int hidden, const int32_t *__restrict__ ids,
                                                       const int32_t *__restrict__ types, Packing p,
                                                       int offset, const float *__restrict__ word,
                                                       const float *__restrict__ pos, const float *__restrict__ type,
                                                       const float *__restrict__ ln_w, const float *__restrict__ ln_b,
                                                       float eps, float *__restrict__ x, H *__restrict__ xh,
                                                       const int32_t *__restrict__ zero_mask, QuantOut qo) {
    const Live lv = live_of(sp);
    const int local = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (local >= lv.tokens) return;
    const int t = lv.tok0 + local;
    const int lane = threadIdx.x & 63;
    const int at = p.at[t];
    const int id = ids[at];
    const int ty = types ? types[at] : 0;
    const float *wr = word + (size_t)id * hidden;
    const float *pr = pos ? pos + (size_t)(p.pos[t] + offset) * hidden : nullptr;
    const float *tr = type ? type + (size_t)ty * hidden : nullptr;
    float v[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 4 * (lane + 64 * g);
        if (c < hidden) {
            load4(wr + c, v[g]);
            float a[4];
            if (pr) {
                load4(pr + c, a);
#pragma unroll
                for (int k = 0; k < 4; ++k) v[g][k] = v[g][k] + a[k];
            }
            if (tr) {
                load4(tr + c, a);
#pragma unroll
                for (int k = 0; k < 4; ++k) v[g][k] = v[g][k] + a[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[g][k] = 0.0f;
        }
    }
    ln_wave<G>(v, hidden, ln_w, ln_b, eps);
    // DeBERTa: a masked token is zero after the embedding.
    if (zero_mask && zero_mask[at] == 0)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < 4; ++k) v[g][k] = 0.0f;
    store_row<G, H>(v, hidden, x ? x + (size_t)t * hidden : nullptr, xh ? xh + (size_t)t * hidden : nullptr);
    if (qo.q) quant_row<G, H>(v, hidden, qo.q + (size_t)lv.tok0 * qo.tok_stride + (size_t)local * hidden, qo.scale + t);
}

template <int G, typename H>
__global__ void __launch_bounds__(256) layer_norm_kernel(Span sp, int hidden, const float *__restrict__ in,
                                                         const float *__restrict__ ln_w,
                                                         const float *__restrict__ ln_b, float eps, float *out_f32,
                                                         H *__restrict__ out_h) {
    const Live lv = live_of(sp);
    const int local = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (local >= lv.tokens) return;
    const int t = lv.tok0 + local;
    const int lane = threadIdx.x & 63;
    const float *row = in + (size_t)t * hidden;
    float v[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 4 * (lane + 64 * g);
        if (c < hidden) load4(row + c, v[g]);
        else
#pragma unroll
            for (int k = 0; k < 4; ++k) v[g][k] = 0.0f;
    }
    ln_wave<G>(v, hidden, ln_w, ln_b, eps);
    store_row<G, H>(v, hidden, out_f32 ? out_f32 + (size_t)t * hidden : nullptr,
                    out_h ? out_h + (size_t)t * hidden : nullptr);
}

// The residual add and a LayerNorm in one pass (a wave a token): v = x + y,
// then x = LN(v) (post-norm) or x = v (pre-norm), and out_h = LN(v). One
// read of x and of the product, one write of x and of the operand copy.
template <int G, typename Y, typename H, bool RES_H>
__global__ void __launch_bounds__(256) add_layer_norm_kernel(Span sp, int hidden, float *__restrict__ x,
                                                             const Y *__restrict__ y, const float *__restrict__ ln_w,
                                                             const float *__restrict__ ln_b, float eps, int pre_norm,
                                                             int keep_f32, H *__restrict__ out_h, QuantOut qo) {
    const Live lv = live_of(sp);
    const int local = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (local >= lv.tokens) return;
    const int t = lv.tok0 + local;
    const int lane = threadIdx.x & 63;
    float *row = x + (size_t)t * hidden;
    const Y *yr = y + (size_t)t * hidden;
    H *hr = out_h ? out_h + (size_t)t * hidden : nullptr;
    // The norm's weight and bias first: their reads overlap the row's.
    float wv[G][4], bv[G][4];
    load_wb<G>(ln_w, ln_b, hidden, wv, bv);
    float v[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 4 * (lane + 64 * g);
        if (c < hidden) {
            float a[4];
            // The residual: x, or (RES_H) the 16-bit rows the last norm wrote.
            if constexpr (RES_H) load4(hr + c, v[g]);
            else load4(row + c, v[g]);
            load4(yr + c, a);
#pragma unroll
            for (int k = 0; k < 4; ++k) v[g][k] = v[g][k] + a[k];
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[g][k] = 0.0f;
        }
    }
    if (pre_norm) store_row<G, H>(v, hidden, row, nullptr);
    ln_apply<G>(v, hidden, wv, bv, eps);
    store_row<G, H>(v, hidden, pre_norm || !keep_f32 ? nullptr : row, hr);
    if (qo.q) quant_row<G, H>(v, hidden, qo.q + (size_t)lv.tok0 * qo.tok_stride + (size_t)local * hidden, qo.scale + t);
}

// add_layer_norm_kernel's work two rows a wave at a time: each 32-lane half
// takes R rows in turn, 8 consecutive columns a lane in each group of 256
// (16-byte reads and writes of 16-bit rows, where a wave a row moves 8 bytes
// a lane), with the norm's weight and bias read once for them (both halves
// read the same words). Every row's loads go out before the first row's
// sums. Hidden a multiple of 8. WAVES sets the block (64 WAVES threads),
// its launch bound and the rows it takes (2 R a wave): a block launched
// wider than its bound is refused by the runtime at launch, and rows
// numbered for another width would be skipped or taken twice, so the
// launcher derives both from this one parameter (pair_blocks).
template <int WAVES, int R> static dim3 pair_blocks(int tokens) {
    static_assert(WAVES >= 1 && WAVES <= 16 && R >= 1, "1 to 16 waves a block");
    constexpr int ROWS = 2 * WAVES * R;   // rows a block
    return dim3((tokens + ROWS - 1) / ROWS);
}

template <int G, typename Y, typename H, bool RES_H, int R, int WAVES>
__global__ void __launch_bounds__(64 * WAVES)
add_ln_pair_kernel(Span sp, int hidden, float *__restrict__ x, const Y *__restrict__ y, const float *__restrict__ ln_w,
                   const float *__restrict__ ln_b, float eps, int pre_norm, int keep_f32, H *__restrict__ out_h,
                   QuantOut qo) {
    const Live lv = live_of(sp);
    // This half's first row (it takes R consecutive rows).
    const int local0 = ((blockIdx.x * WAVES + (threadIdx.x >> 6)) * 2 + ((threadIdx.x >> 5) & 1)) * R;
    // (A half's lanes all share its rows; the sums stay within the half.)
    if (local0 >= lv.tokens) return;
    const int hl = threadIdx.x & 31;
    float wv[G][8], bv[G][8];
    load_wb8<G>(ln_w, ln_b, hidden, hl, wv, bv);
    float v[R][G][8];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int t = lv.tok0 + min(local0 + i, lv.tokens - 1);
        const float *row = x + (size_t)t * hidden;
        const Y *yr = y + (size_t)t * hidden;
        const H *hr = out_h + (size_t)t * hidden;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int c = 8 * (hl + 32 * g);
            if (c < hidden) {
                float a[8];
                if constexpr (RES_H) load8(hr + c, v[i][g]);
                else load8(row + c, v[i][g]);
                load8(yr + c, a);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[i][g][k] = v[i][g][k] + a[k];
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) v[i][g][k] = 0.0f;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int local = local0 + i;
        if (local >= lv.tokens) break;
        const int t = lv.tok0 + local;
        float *row = x + (size_t)t * hidden;
        H *hr = out_h ? out_h + (size_t)t * hidden : nullptr;
        if (pre_norm)
#pragma unroll
            for (int g = 0; g < G; ++g)
                if (8 * (hl + 32 * g) < hidden) store8(row + 8 * (hl + 32 * g), v[i][g]);
        ln_pair_apply<G>(v[i], hidden, hl, wv, bv, eps);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int c = 8 * (hl + 32 * g);
            if (c >= hidden) continue;
            if (!pre_norm && keep_f32) store8(row + c, v[i][g]);
            if (hr) store8(hr + c, v[i][g]);
        }
        // The row's int8 codes from its values as rounded to H, as quant_row.
        if (qo.q)
            quant_pair_row<G, H>(v[i], hidden, hl, qo.q + (size_t)lv.tok0 * qo.tok_stride + (size_t)local * hidden,
                                 qo.scale + t);
    }
}

// Rows a half-wave takes (2: BERT-base 0.9% faster a step than 1, with
// the weight reads halved; 4 is 2.5% slower, its registers halving the
// waves a SIMD), and waves a block (4: two-wave blocks were 13% slower).
constexpr int LN_ROWS = 2, LN_WAVES = 4;

template <typename H, int G, typename Y>
static hipError_t add_ln_v(hipStream_t s, const Span &sp, int tokens, int hidden, float *x, const void *y,
                           const float *ln_w, const float *ln_b, float eps, int pre_norm, void *out_h,
                           const QuantOut &qo, bool res_h, bool keep_f32) {
    // Two rows a wave on the 16-bit residual (measured: BERT-base's norms 6%
    // faster; on F32 rows, ModernBERT's, 2% slower). Other runs keep one
    // layout for all their norms: a layer read's final norm (layer_norm)
    // must give the bits of the fused one.
    if constexpr (sizeof(Y) == 2 && sizeof(H) == 2) {
        if (res_h && hidden % 8 == 0) {
            enqueue((add_ln_pair_kernel<G, Y, H, true, LN_ROWS, LN_WAVES>),
                    (pair_blocks<LN_WAVES, LN_ROWS>(tokens)), dim3(64 * LN_WAVES), 0, s,
                    sp, hidden, x, (const Y *)y, ln_w, ln_b, eps, pre_norm, (int)keep_f32, (H *)out_h, qo);
            return hipGetLastError();
        }
    }
    if (res_h && sizeof(H) == 2)
        enqueue((add_layer_norm_kernel<G, Y, H, sizeof(H) == 2>), dim3((tokens + 3) / 4), dim3(256), 0, s,
                sp, hidden, x, (const Y *)y, ln_w, ln_b, eps, pre_norm, (int)keep_f32, (H *)out_h, qo);
    else
        enqueue((add_layer_norm_kernel<G, Y, H, false>), dim3((tokens + 3) / 4), dim3(256), 0, s, sp,
                hidden, x, (const Y *)y, ln_w, ln_b, eps, pre_norm, (int)keep_f32, (H *)out_h, qo);
    return hipGetLastError();
}

template <typename H, int G>
static hipError_t add_ln_y(hipStream_t s, const Span &sp, int tokens, int hidden, float *x, const void *y, Dt ydt,
                           const float *ln_w, const float *ln_b, float eps, int pre_norm, void *out_h,
                           const QuantOut &qo, bool res_h, bool keep_f32) {
    switch (ydt) {
    case Dt::F16:
        return add_ln_v<H, G, _Float16>(s, sp, tokens, hidden, x, y, ln_w, ln_b, eps, pre_norm, out_h, qo, res_h,
                                        keep_f32);
    case Dt::BF16:
        return add_ln_v<H, G, __bf16>(s, sp, tokens, hidden, x, y, ln_w, ln_b, eps, pre_norm, out_h, qo, res_h,
                                      keep_f32);
    case Dt::F32:
        return add_ln_v<H, G, float>(s, sp, tokens, hidden, x, y, ln_w, ln_b, eps, pre_norm, out_h, qo, res_h,
                                     keep_f32);
    default: return hipErrorInvalidValue;
    }
}

// embed_ln_kernel's work for a 16-bit residual (no F32 rows, no codes) two
// tokens a wave: each 32-lane half takes a token, 8 consecutive columns a
// lane in each group of 256 (twice the tokens' dependent id and row reads in
// flight a wave), the norm's weight and bias read once for both.
template <int G, typename H, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) embed_ln_pair_kernel(Span sp, int hidden, const int32_t *__restrict__ ids,
                                                            const int32_t *__restrict__ types, Packing p, int offset,
                                                            const float *__restrict__ word,
                                                            const float *__restrict__ pos,
                                                            const float *__restrict__ type,
                                                            const float *__restrict__ ln_w,
                                                            const float *__restrict__ ln_b, float eps,
                                                            H *__restrict__ xh, const int32_t *__restrict__ zero_mask) {
    const Live lv = live_of(sp);
    const int local = (blockIdx.x * WAVES + (threadIdx.x >> 6)) * 2 + ((threadIdx.x >> 5) & 1);
    // (A half's lanes all share its token; the sums stay within the half.)
    if (local >= lv.tokens) return;
    const int t = lv.tok0 + local, hl = threadIdx.x & 31;
    const int at = p.at[t];
    const int id = ids[at];
    const int ty = types ? types[at] : 0;
    const float *wr = word + (size_t)id * hidden;
    const float *pr = pos ? pos + (size_t)(p.pos[t] + offset) * hidden : nullptr;
    const float *tr = type ? type + (size_t)ty * hidden : nullptr;
    float wv[G][8], bv[G][8];
    load_wb8<G>(ln_w, ln_b, hidden, hl, wv, bv);
    float v[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 8 * (hl + 32 * g);
        if (c < hidden) {
            load8(wr + c, v[g]);
            float a[8];
            if (pr) {
                load8(pr + c, a);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[g][k] = v[g][k] + a[k];
            }
            if (tr) {
                load8(tr + c, a);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[g][k] = v[g][k] + a[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[g][k] = 0.0f;
        }
    }
    ln_pair_apply<G>(v, hidden, hl, wv, bv, eps);
    // DeBERTa: a masked token is zero after the embedding.
    if (zero_mask && zero_mask[at] == 0)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < 8; ++k) v[g][k] = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c = 8 * (hl + 32 * g);
        if (c < hidden) store8(xh + (size_t)t * hidden + c, v[g]);
    }
}

template <typename H, int G>
static hipError_t embed_ln_v(hipStream_t s, const Span &sp, int tokens, int hidden, const int32_t *ids,
                             const int32_t *types, const Packing &p, int offset, const float *word, const float *pos,
                             const float *type, const float *ln_w, const float *ln_b, float eps, float *x, void *xh,
                             const int32_t *zero_mask, const QuantOut &qo) {
    if constexpr (sizeof(H) == 2) {
        if (!x && xh && !qo.q && hidden % 8 == 0) {
            enqueue((embed_ln_pair_kernel<G, H, LN_WAVES>), (pair_blocks<LN_WAVES, 1>(tokens)),
                    dim3(64 * LN_WAVES), 0, s, sp, hidden, ids,
                    types, p, offset, word, pos, type, ln_w, ln_b, eps, (H *)xh, zero_mask);
            return hipGetLastError();
        }
    }
    enqueue((embed_ln_kernel<G, H>), dim3((tokens + 3) / 4), dim3(256), 0, s, sp, hidden, ids, types, p,
            offset, word, pos, type, ln_w, ln_b, eps, x, (H *)xh, zero_mask, qo);
    return hipGetLastError();
}

template <typename H, int G>
static hipError_t ln_v(hipStream_t s, const Span &sp, int tokens, int hidden, const float *in, const float *ln_w,
                       const float *ln_b, float eps, float *out_f32, void *out_h) {
    enqueue((layer_norm_kernel<G, H>), dim3((tokens + 3) / 4), dim3(256), 0, s, sp, hidden, in, ln_w,
            ln_b, eps, out_f32, (H *)out_h);
    return hipGetLastError();
}

// The groups of 4 columns a lane holds, G = ceil(hidden / 256), up to
// hidden 2048; hidden a multiple of 4 (the model's is of 8).
#define ROWWISE_DISPATCH(FN, ...)                                                              \
    {                                                                                          \
        if (hidden % 4 != 0) return hipErrorInvalidValue;                                      \
        const int g = (hidden + 255) / 256;                                                    \
        if (g <= 1) return FN<H, 1>(__VA_ARGS__);                                              \
        if (g <= 2) return FN<H, 2>(__VA_ARGS__);                                              \
        if (g <= 3) return FN<H, 3>(__VA_ARGS__);                                              \
        if (g <= 4) return FN<H, 4>(__VA_ARGS__);                                              \
        if (g <= 6) return FN<H, 6>(__VA_ARGS__);                                              \
        if (g <= 8) return FN<H, 8>(__VA_ARGS__);                                              \
        return hipErrorInvalidValue;                                                           \
    }

template <typename H>
static hipError_t embed_ln_t(hipStream_t s, const Span &sp, int tokens, int hidden, const int32_t *ids,
                             const int32_t *types, const Packing &p, int offset, const float *word, const float *pos,
                             const float *type, const float *ln_w, const float *ln_b, float eps, float *x, void *xh,
                             const int32_t *zero_mask, const QuantOut &qo) {
    ROWWISE_DISPATCH(embed_ln_v, s, sp, tokens, hidden, ids, types, p, offset, word, pos, type, ln_w, ln_b, eps, x, xh,
                     zero_mask, qo)
}

template <typename H>
static hipError_t ln_t(hipStream_t s, const Span &sp, int tokens, int hidden, const float *in, const float *ln_w,
                       const float *ln_b, float eps, float *out_f32, void *out_h) {
    ROWWISE_DISPATCH(ln_v, s, sp, tokens, hidden, in, ln_w, ln_b, eps, out_f32, out_h)
}

template <typename H>
static hipError_t add_ln_t(hipStream_t s, const Span &sp, int tokens, int hidden, float *x, const void *y, Dt ydt,
                           const float *ln_w, const float *ln_b, float eps, int pre_norm, void *out_h,
                           const QuantOut &qo, bool res_h, bool keep_f32) {
    ROWWISE_DISPATCH(add_ln_y, s, sp, tokens, hidden, x, y, ydt, ln_w, ln_b, eps, pre_norm, out_h, qo, res_h, keep_f32)
}

hipError_t embed_ln(hipStream_t s, const Span &sp, int max_tokens, int hidden, const int32_t *ids,
                    const int32_t *types, const Packing &p, int position_offset, const float *word, const float *pos,
                    const float *type, const float *ln_w, const float *ln_b, float eps, float *x, void *xh, Dt dt,
                    const int32_t *zero_mask, const QuantOut &qo) {
    if (max_tokens <= 0) return hipSuccess;
    if (qo.q && (dt != Dt::F16 || !xh || hidden % 4 != 0)) return hipErrorInvalidValue;
    switch (dt) {
    case Dt::F16:
        return embed_ln_t<_Float16>(s, sp, max_tokens, hidden, ids, types, p, position_offset, word, pos, type, ln_w,
                                    ln_b, eps, x, xh, zero_mask, qo);
    case Dt::BF16:
        return embed_ln_t<__bf16>(s, sp, max_tokens, hidden, ids, types, p, position_offset, word, pos, type, ln_w,
                                  ln_b, eps, x, xh, zero_mask, qo);
    default:
        return embed_ln_t<float>(s, sp, max_tokens, hidden, ids, types, p, position_offset, word, pos, type, ln_w,
                                 ln_b, eps, x, xh, zero_mask, qo);
    }
}

hipError_t add_layer_norm(hipStream_t s, const Span &sp, int max_tokens, int hidden, float *x, const void *y, Dt ydt,
                          const float *ln_w, const float *ln_b, float eps, int pre_norm, void *out_h, Dt dt,
                          const QuantOut &qo, bool res_h, bool keep_f32) {
    if (max_tokens <= 0) return hipSuccess;
    if (qo.q && (dt != Dt::F16 || !out_h || hidden % 4 != 0)) return hipErrorInvalidValue;
    // A 16-bit residual is a post-norm's, read from and written to out_h.
    if (res_h && (dt == Dt::F32 || !out_h || pre_norm)) return hipErrorInvalidValue;
    if (!keep_f32 && !res_h) return hipErrorInvalidValue;
    switch (dt) {
    case Dt::F16:
        return add_ln_t<_Float16>(s, sp, max_tokens, hidden, x, y, ydt, ln_w, ln_b, eps, pre_norm, out_h, qo, res_h,
                                  keep_f32);
    case Dt::BF16:
        return add_ln_t<__bf16>(s, sp, max_tokens, hidden, x, y, ydt, ln_w, ln_b, eps, pre_norm, out_h, qo, res_h,
                                keep_f32);
    default:
        return add_ln_t<float>(s, sp, max_tokens, hidden, x, y, ydt, ln_w, ln_b, eps, pre_norm, out_h, qo, res_h,
                               keep_f32);
    }
}

hipError_t layer_norm(hipStream_t s, const Span &sp, int max_tokens, int hidden, const float *in, const float *ln_w,
                      const float *ln_b, float eps, float *out_f32, void *out_h, Dt dt) {
    if (max_tokens <= 0) return hipSuccess;
    switch (dt) {
    case Dt::F16: return ln_t<_Float16>(s, sp, max_tokens, hidden, in, ln_w, ln_b, eps, out_f32, out_h);
    case Dt::BF16: return ln_t<__bf16>(s, sp, max_tokens, hidden, in, ln_w, ln_b, eps, out_f32, out_h);
    default: return ln_t<float>(s, sp, max_tokens, hidden, in, ln_w, ln_b, eps, out_f32, out_h);
    }
}

// ---- Pooling ----------------------------------------------------------------------
//
// One workgroup per output vector. Mode 0 pools row i as `pooling` says;
// mode 1 pools range i, (row, start, end) in `ranges`. A mean is the F32 sum
// of the live tokens' states in column order, times one over their count
// (reference core/src/cpu/encoder/mod.rs:443-468); a row's mean is the range
// (row, 0, len) through the same code, so a whole-row range gives the row's
// vector bit for bit. The cut to output_dim comes before the L2 norm, summed
// in F64 and floored at 1e-12 (mod.rs:470-482).
//
// HEAD: range i's mean over all hidden values goes through the span head
// instead, out[i, o] = bias[o] + sum_c w[o, c] * mean[c] with the products
// and sums in F64, rounded to F32 once (include/turbo/turbo_backend.h:418-422;
// the core's host head, core/src/qa/session.rs:268-276, sums the same terms).
constexpr int POOL_THREADS = 256;

// Item i's tokens: a row's live extent (mode 0) or a range within it.
__device__ __forceinline__ void pool_span(int i, int mode, const Packing &p, const uint32_t *__restrict__ ranges, int &r,
                                          int &c0, int &c1) {
    if (mode == 0) {
        r = i;
        c0 = 0;
        c1 = p.len[r];
    } else {
        r = (int)ranges[3 * i];
        c0 = (int)ranges[3 * i + 1];
        c1 = min((int)ranges[3 * i + 2], p.len[r]);
    }
}

// The run's pooling as its dimensions give it: item count and mode (ranges
// when count > 0, else the rows), the pooling of a row, the output width, L2
// and the span head.
struct PoolRun {
    int items, mode, pooling, od, l2, head;
};
__device__ __forceinline__ PoolRun pool_run(const RunDims *__restrict__ d, int hidden) {
    const int count = uniform(d->count), head = uniform(d->head);
    return PoolRun{count ? count : uniform(d->batch), count ? 1 : 0, uniform(d->pooling),
                   head ? hidden : uniform(d->output_dim), uniform(d->l2), head};
}

// Work item w = (item i, chunk k), over a grid-stride loop: the F32 sum, in
// token order, of chunk k of item i's tokens (its live ones, when the item
// has any live token; else all of them), and how many it summed. Tokens are
// read 8 at a time (their loads in flight together), and added in order. A
// row's CLS or LAST vector needs no sums.
__global__ void __launch_bounds__(POOL_THREADS) pool_part_kernel(const RunDims *__restrict__ dims,
                                                                 const float *__restrict__ x, int hidden, Packing p,
                                                                 const int32_t *__restrict__ mask,
                                                                 const uint32_t *__restrict__ ranges,
                                                                 float *__restrict__ part, int32_t *__restrict__ cnt,
                                                                 int chunks) {
    const PoolRun pr = pool_run(dims, hidden);
    if (pr.mode == 0 && pr.pooling != 1) return;
    const int seq = uniform(dims->seq), od = pr.od;
    for (int w = blockIdx.x; w < pr.items * chunks; w += gridDim.x) {
        const int i = w / chunks, k = w % chunks;
        int r, c0, c1;
        pool_span(i, pr.mode, p, ranges, r, c0, c1);
        const int cs = c0 + k * POOL_CHUNK;
        if (cs >= c1) continue;   // past the item: the finish reads only its own chunks
        const int ce = min(cs + POOL_CHUNK, c1), start = p.start[r];
        const int32_t *mk = mask + (size_t)r * seq;
        int any = 0;
        for (int q = c0 + (int)threadIdx.x; q < c1 && !any; q += POOL_THREADS) any = mk[q] != 0;
        const bool live_only = __syncthreads_or(any) != 0;
        constexpr int MAXV = 8;
        float acc[MAXV];
#pragma unroll
        for (int v = 0; v < MAXV; ++v) acc[v] = 0.0f;
        int n = 0;
        for (int q0 = cs; q0 < ce; q0 += 8) {
            bool use[8];
            float val[8][MAXV];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int q = q0 + j;
                use[j] = q < ce && (!live_only || mk[q] != 0);
                const float *row = x + (size_t)(start + (use[j] ? q : cs)) * hidden;
#pragma unroll
                for (int v = 0; v < MAXV; ++v) {
                    const int c = threadIdx.x + POOL_THREADS * v;
                    val[j][v] = (use[j] && c < od) ? row[c] : 0.0f;
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (!use[j]) continue;
#pragma unroll
                for (int v = 0; v < MAXV; ++v) acc[v] = __fadd_rn(acc[v], val[j][v]);
                ++n;
            }
        }
        float *dst = part + ((size_t)i * chunks + k) * od;
#pragma unroll
        for (int v = 0; v < MAXV; ++v) {
            const int c = threadIdx.x + POOL_THREADS * v;
            if (c < od) dst[c] = acc[v];
        }
        if (threadIdx.x == 0) cnt[(size_t)i * chunks + k] = n;
    }
}

// Item i over a grid-stride loop: its vector from the chunk sums (or its
// CLS or LAST row), then the cut and L2, or the span head.
__global__ void __launch_bounds__(POOL_THREADS) pool_kernel(const RunDims *__restrict__ dims,
                                                            const float *__restrict__ x, int hidden, Packing p,
                                                            const uint32_t *__restrict__ ranges,
                                                            float *__restrict__ out, const float *__restrict__ hw,
                                                            const float *__restrict__ hb, int hout,
                                                            const float *__restrict__ sums,
                                                            const int32_t *__restrict__ cnt, int chunks) {
    __shared__ double part[POOL_THREADS / 64];
    __shared__ double hpart[HEAD_MAX][POOL_THREADS / 64];
    const PoolRun pr = pool_run(dims, hidden);
    const int od = pr.od;
    constexpr int MAXV = 8;   // output_dim up to 2048
    for (int i = blockIdx.x; i < pr.items; i += gridDim.x) {
        int r, c0, c1;
        pool_span(i, pr.mode, p, ranges, r, c0, c1);
        const int start = p.start[r];
        float acc[MAXV];
#pragma unroll
        for (int v = 0; v < MAXV; ++v) acc[v] = 0.0f;
        if (pr.mode == 0 && pr.pooling != 1) {
            const int tok = pr.pooling == 2 ? start : start + p.len[r] - 1;   // CLS: column 0; LAST: last live
#pragma unroll
            for (int v = 0; v < MAXV; ++v) {
                const int c = threadIdx.x + POOL_THREADS * v;
                if (c < od) acc[v] = x[(size_t)tok * hidden + c];
            }
        } else {
            // The chunks' sums in chunk order (one chunk: its sum exactly).
            const int nch = (c1 - c0 + POOL_CHUNK - 1) / POOL_CHUNK;
            int n = 0;
            for (int k = 0; k < nch; ++k) {
                const float *src = sums + ((size_t)i * chunks + k) * od;
#pragma unroll
                for (int v = 0; v < MAXV; ++v) {
                    const int c = threadIdx.x + POOL_THREADS * v;
                    if (c < od) acc[v] = __fadd_rn(acc[v], src[c]);
                }
                n += cnt[(size_t)i * chunks + k];
            }
            const float inv = __fdiv_rn(1.0f, (float)n);
#pragma unroll
            for (int v = 0; v < MAXV; ++v) acc[v] = __fmul_rn(acc[v], inv);
        }
        if (pr.head) {
            // od is hidden here: every value of the mean meets the head.
            for (int o = 0; o < hout; ++o) {
                double t = 0.0;
#pragma unroll
                for (int v = 0; v < MAXV; ++v) {
                    const int c = threadIdx.x + POOL_THREADS * v;
                    if (c < od) t = fma((double)hw[(size_t)o * hidden + c], (double)acc[v], t);
                }
                t = wave_sum(t);
                if ((threadIdx.x & 63) == 0) hpart[o][threadIdx.x >> 6] = t;
            }
            __syncthreads();
            if ((int)threadIdx.x < hout) {
                double tot = (double)hb[threadIdx.x];
#pragma unroll
                for (int w = 0; w < POOL_THREADS / 64; ++w) tot += hpart[threadIdx.x][w];
                out[(size_t)i * hout + threadIdx.x] = (float)tot;
            }
            __syncthreads();   // hpart is read before the next item writes it
            continue;
        }
        if (pr.l2) {
            double s = 0.0;
#pragma unroll
            for (int v = 0; v < MAXV; ++v) {
                const int c = threadIdx.x + POOL_THREADS * v;
                if (c < od) s += (double)acc[v] * (double)acc[v];
            }
            s = wave_sum(s);
            if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
            __syncthreads();
            double tot = 0.0;
#pragma unroll
            for (int w = 0; w < POOL_THREADS / 64; ++w) tot += part[w];
            __syncthreads();   // part is read before the next item writes it
            const double norm = fmax(sqrt(tot), 1e-12);
            const float inv = (float)(1.0 / norm);
#pragma unroll
            for (int v = 0; v < MAXV; ++v) acc[v] = __fmul_rn(acc[v], inv);
        }
#pragma unroll
        for (int v = 0; v < MAXV; ++v) {
            const int c = threadIdx.x + POOL_THREADS * v;
            if (c < od) out[(size_t)i * od + c] = acc[v];
        }
    }
}

// Workgroups a pooling launch takes at most: items beyond them loop.
constexpr int POOL_GRID = 2048;

hipError_t pool(hipStream_t s, const RunDims *dims, int max_items, const float *x, int hidden, const Packing &p,
                const int32_t *mask, const uint32_t *ranges, const PoolScratch &ps, float *out, const float *hw,
                const float *hb, int hout) {
    if (hidden > 8 * POOL_THREADS || hout < 0 || hout > HEAD_MAX) return hipErrorInvalidValue;
    if (max_items <= 0) return hipSuccess;
    if (!ps.part || !ps.cnt || ps.chunks <= 0) return hipErrorInvalidValue;
    const int part_blocks = (int)std::min<long>((long)max_items * ps.chunks, POOL_GRID);
    enqueue(pool_part_kernel, dim3(part_blocks), dim3(POOL_THREADS), 0, s, dims, x, hidden, p, mask, ranges,
            ps.part, ps.cnt, ps.chunks);
    enqueue(pool_kernel, dim3(std::min(max_items, POOL_GRID)), dim3(POOL_THREADS), 0, s, dims, x, hidden, p,
            ranges, out, hw, hb, hout, ps.part, ps.cnt, ps.chunks);
    return hipGetLastError();
}

// ---- Symmetric int8 rows -------------------------------------------------------------
//
// One wave per row: the row's absolute maximum by a wave reduction, scale =
// max / 127, q = round-to-nearest-even(x * (127 / max)) within [-127, 127].
template <typename S>
__global__ void __launch_bounds__(256) quantize_rows_kernel(const S *__restrict__ src, int rows, int cols, int ld,
                                                            int8_t *__restrict__ dst, float *__restrict__ scale) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const S *row = src + (size_t)r * ld;
    float mx = 0.0f;
    for (int c = lane; c < cols; c += 64) mx = fmaxf(mx, fabsf(to_f32(row[c])));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
    int8_t *out = dst + (size_t)r * cols;
    for (int c = lane; c < cols; c += 64) {
        const float q = rintf(to_f32(row[c]) * inv);
        out[c] = (int8_t)fminf(fmaxf(q, -127.0f), 127.0f);
    }
    if (lane == 0) scale[r] = mx / 127.0f;
}

// The same rows, 8 consecutive columns a lane per step (16-byte loads of
// F16, 8-byte stores of the codes), a row's values held in registers between
// its maximum and its codes: cols a multiple of 8 up to 8 * 64 * QMAXK.
constexpr int QMAXK = 8;
template <typename S>
__global__ void __launch_bounds__(256) quantize_rows8_kernel(const S *__restrict__ src, int rows, int cols, int ld,
                                                             int8_t *__restrict__ dst, float *__restrict__ scale) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const S *row = src + (size_t)r * ld;
    float v[QMAXK][8];
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < QMAXK; ++k) {
        const int c = 8 * (lane + 64 * k);
        if (c < cols) {
            float a[4], b[4];
            load4(row + c, a);
            load4(row + c + 4, b);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[k][q] = a[q];
                v[k][4 + q] = b[q];
                mx = fmaxf(mx, fmaxf(fabsf(a[q]), fabsf(b[q])));
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
    int8_t *out = dst + (size_t)r * cols;
#pragma unroll
    for (int k = 0; k < QMAXK; ++k) {
        const int c = 8 * (lane + 64 * k);
        if (c < cols) {
            uint32_t w[2] = {0, 0};
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int code = (int)fminf(fmaxf(rintf(v[k][q] * inv), -127.0f), 127.0f);
                w[q >> 2] |= (uint32_t)(uint8_t)(int8_t)code << (8 * (q & 3));
            }
            *(uint2 *)(out + c) = make_uint2(w[0], w[1]);
        }
    }
    if (lane == 0) scale[r] = mx / 127.0f;
}

hipError_t quantize_rows(hipStream_t s, const void *src, Dt src_dt, int rows, int cols, int ld, int8_t *dst,
                         float *scale) {
    if (rows <= 0) return hipSuccess;
    const dim3 grid((rows + 3) / 4);
    if (cols % 8 == 0 && ld % 8 == 0 && cols <= 8 * 64 * QMAXK && (src_dt == Dt::F32 || src_dt == Dt::F16)) {
        if (src_dt == Dt::F32)
            enqueue(quantize_rows8_kernel<float>, grid, dim3(256), 0, s, (const float *)src, rows, cols, ld,
                    dst, scale);
        else
            enqueue(quantize_rows8_kernel<_Float16>, grid, dim3(256), 0, s, (const _Float16 *)src, rows,
                    cols, ld, dst, scale);
        return hipGetLastError();
    }
    if (src_dt == Dt::F32)
        enqueue(quantize_rows_kernel<float>, grid, dim3(256), 0, s, (const float *)src, rows, cols, ld, dst,
                scale);
    else if (src_dt == Dt::F16)
        enqueue(quantize_rows_kernel<_Float16>, grid, dim3(256), 0, s, (const _Float16 *)src, rows, cols,
                ld, dst, scale);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// A span's rows: src row t at src + t * ld, dst row t at dst + tok0 *
// dst_tok + (t - tok0) * cols (bytes), scale t at scale + t.
template <typename S>
__global__ void __launch_bounds__(256) quantize_span_kernel(Span sp, const S *__restrict__ src, int cols, int ld,
                                                            int8_t *__restrict__ dst, int dst_tok,
                                                            float *__restrict__ scale) {
    const Live lv = live_of(sp);
    const int local = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (local >= lv.tokens) return;
    const int t = lv.tok0 + local, lane = threadIdx.x & 63;
    const S *row = src + (size_t)t * ld;
    float v[QMAXK][8];
    float mx = 0.0f;
    // (Eight values a lane a step: one 16-byte load of F16, two of F32;
    // every step's loads go out before the first maximum.)
#pragma unroll
    for (int k = 0; k < QMAXK; ++k) {
        const int c = 8 * (lane + 64 * k);
        if (c < cols) load8(row + c, v[k]);
    }
#pragma unroll
    for (int k = 0; k < QMAXK; ++k) {
        const int c = 8 * (lane + 64 * k);
        if (c < cols)
#pragma unroll
            for (int q = 0; q < 8; ++q) mx = fmaxf(mx, fabsf(v[k][q]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
    int8_t *out = dst + (size_t)lv.tok0 * dst_tok + (size_t)local * cols;
#pragma unroll
    for (int k = 0; k < QMAXK; ++k) {
        const int c = 8 * (lane + 64 * k);
        if (c < cols) {
            uint32_t w[2] = {0, 0};
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int code = (int)fminf(fmaxf(rintf(v[k][q] * inv), -127.0f), 127.0f);
                w[q >> 2] |= (uint32_t)(uint8_t)(int8_t)code << (8 * (q & 3));
            }
            *(uint2 *)(out + c) = make_uint2(w[0], w[1]);
        }
    }
    if (lane == 0) scale[t] = mx / 127.0f;
}

hipError_t quantize_span(hipStream_t s, const Span &sp, int max_rows, const void *src, Dt src_dt, int cols, int ld,
                         int8_t *dst, int dst_tok, float *scale) {
    if (max_rows <= 0) return hipSuccess;
    // The codes of a row are the ones quantize_rows makes (same arithmetic).
    if (cols % 8 != 0 || ld % 8 != 0 || cols > 8 * 64 * QMAXK || (src_dt != Dt::F32 && src_dt != Dt::F16))
        return hipErrorInvalidValue;
    const dim3 grid((max_rows + 3) / 4);
    if (src_dt == Dt::F32)
        enqueue(quantize_span_kernel<float>, grid, dim3(256), 0, s, sp, (const float *)src, cols, ld, dst,
                dst_tok, scale);
    else
        enqueue(quantize_span_kernel<_Float16>, grid, dim3(256), 0, s, sp, (const _Float16 *)src, cols, ld,
                dst, dst_tok, scale);
    return hipGetLastError();
}

// ---- Uniform fill (measurement operands) ---------------------------------------------
//
// Each value from a 32-bit integer hash of its index and the seed (the
// "lowbias32" mixer: xorshift-multiply rounds), top 24 bits to [-amp, amp).
__global__ void __launch_bounds__(256) fill_uniform_kernel(float *__restrict__ dst, size_t n, float amp,
                                                           uint32_t seed) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        uint32_t h = (uint32_t)i * 0x9e3779b9u ^ (uint32_t)(i >> 32) ^ seed * 0x85ebca6bu;
        h ^= h >> 16;
        h *= 0x7feb352du;
        h ^= h >> 15;
        h *= 0x846ca68bu;
        h ^= h >> 16;
        dst[i] = amp * ((float)(h >> 8) * (2.0f / 16777216.0f) - 1.0f);
    }
}

hipError_t fill_uniform(hipStream_t s, float *dst, size_t n, float amp, uint32_t seed) {
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
    enqueue(fill_uniform_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, n, amp, seed);
    return hipGetLastError();
}

// ---- Vector codes (int8 and ubinary) ----------------------------------------------------
//
// int8: a thread a value, IEEE F32 subtraction, division and floor as the
// reference computes them on the host (core/src/quantize.rs:60-70); a NaN
// lands in the bottom bucket there, and does here (fmaxf/fminf drop NaN).
// ubinary: a thread an output byte, its eight values' signs.
__global__ void __launch_bounds__(256) int8_codes_kernel(const float *__restrict__ x, int rows, int dim,
                                                         const float *__restrict__ ranges, uint8_t *__restrict__ out) {
    const size_t n = (size_t)rows * dim;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const int d = (int)(i % dim);
        const float lo = ranges[d], hi = ranges[dim + d];
        float step = __fdiv_rn(__fsub_rn(hi, lo), 255.0f);
        if (step == 0.0f) step = 1.0f;
        const float q = fminf(fmaxf(floorf(__fdiv_rn(__fsub_rn(x[i], lo), step)), 0.0f), 255.0f);
        out[i] = (uint8_t)(int8_t)((int)q - 128);
    }
}

__global__ void __launch_bounds__(256) ubinary_codes_kernel(const float *__restrict__ x, int rows, int dim,
                                                            uint8_t *__restrict__ out) {
    const int per = (dim + 7) / 8;
    const size_t n = (size_t)rows * per;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const int r = (int)(i / per), b = (int)(i % per);
        const float *row = x + (size_t)r * dim;
        uint32_t byte = 0;
        for (int k = 0; k < 8; ++k) {
            const int d = 8 * b + k;
            if (d < dim && row[d] > 0.0f) byte |= 0x80u >> k;
        }
        out[i] = (uint8_t)byte;
    }
}

hipError_t quantize_codes(hipStream_t s, const float *x, int rows, int dim, int mode, const float *ranges,
                          uint8_t *out) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    const size_t n = mode == 2 ? (size_t)rows * dim : (size_t)rows * ((dim + 7) / 8);
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 65536);
    if (mode == 2)
        enqueue(int8_codes_kernel, dim3(blocks), dim3(256), 0, s, x, rows, dim, ranges, out);
    else if (mode == 3)
        enqueue(ubinary_codes_kernel, dim3(blocks), dim3(256), 0, s, x, rows, dim, out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// ---- A fixed staging area for callers that cannot allocate ------------------------------
//
// buffer_quantize stages its codes in device memory it allocates per call;
// its no-allocation variant stages them (and the int8 ranges) here instead:
// one file-scope array a GPU, held until the process ends. On the host the
// array's name stands for a host-side stand-in, not a device address, so its
// address on each device is looked up once, with that device current, and
// kept; host code passes that address to kernels and copies, never the name.
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

hipError_t static_scratch(int device, void **ptr) {
    static std::mutex lock;
    static void *addr[MAX_DEVICES] = {};
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(lock);
    if (!addr[device]) {
        int current = -1;
        hipError_t e = hipGetDevice(&current);
        if (e != hipSuccess) return e;
        if (current != device) return hipErrorInvalidDevice;
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[device] = p;
    }
    *ptr = addr[device];
    return hipSuccess;
}

// ---- Plain copy (the traffic counters' reference) ---------------------------------------

__global__ void __launch_bounds__(256) copy_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

hipError_t copy_bytes(hipStream_t s, const void *src, void *dst, size_t bytes) {
    if (bytes % 16 != 0) return hipErrorInvalidValue;
    const size_t n = bytes / 16;
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 256 * 32);
    enqueue(copy_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (const uint4 *)src, (uint4 *)dst, n);
    return hipGetLastError();
}

__global__ void __launch_bounds__(256) copy_rows_kernel(Span sp, const uint4 *__restrict__ src,
                                                        uint4 *__restrict__ dst, int row_vecs) {
    const Live lv = live_of(sp);
    const size_t n = (size_t)lv.tokens * row_vecs, base = (size_t)lv.tok0 * row_vecs;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[base + i] = src[base + i];
}

hipError_t copy_rows(hipStream_t s, const Span &sp, int max_tokens, const void *src, void *dst, size_t row_bytes) {
    if (row_bytes % 16 != 0) return hipErrorInvalidValue;
    const size_t n = (size_t)max_tokens * (row_bytes / 16);
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 256 * 32);
    enqueue(copy_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, sp, (const uint4 *)src, (uint4 *)dst,
            (int)(row_bytes / 16));
    return hipGetLastError();
}

// ---- Weight narrowing ------------------------------------------------------------------

template <typename H>
__global__ void narrow_kernel(const float *__restrict__ src, H *__restrict__ dst, size_t n, int32_t *overflow) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float v = src[i];
        const H h = from_f32<H>(v);
        if (overflow && isinf(to_f32(h)) && !isinf(v)) *overflow = 1;
        dst[i] = h;
    }
}

hipError_t narrow(hipStream_t s, const float *src, void *dst, size_t n, Dt dt, int32_t *overflow) {
    const int blocks = (int)std::min<size_t>((n + 255) / 256, 65536);
    if (n == 0) return hipSuccess;
    if (dt == Dt::F16)
        enqueue(narrow_kernel<_Float16>, dim3(blocks), dim3(256), 0, s, src, (_Float16 *)dst, n, overflow);
    else if (dt == Dt::BF16)
        enqueue(narrow_kernel<__bf16>, dim3(blocks), dim3(256), 0, s, src, (__bf16 *)dst, n, overflow);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace rocm
