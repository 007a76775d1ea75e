// Launchers of the rocm backend's gfx950 kernels. Every launcher enqueues on
// the given stream and returns the launch's error; none allocates or syncs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rocm {

// The arithmetic type of a session's GEMM operands and activations. I8 is
// GEMM operands alone: int8 weights (per output channel) and activations (per
// token), int32 sums; its activations are F16.
enum class Dt : int { F32 = 0, F16 = 1, BF16 = 2, I8 = 3 };

inline size_t dt_bytes(Dt d) { return d == Dt::F32 ? 4 : d == Dt::I8 ? 1 : 2; }

// Where each packed token of a run sits, written on the device by pack_rows
// (reference core/src/cpu/encoder/mod.rs:379-424; core/cuda/kernels.h:56-77).
// A row's tokens are its columns 0 .. len - 1 (len = last live column + 1),
// one after another, rows in order.
struct Packing {
    int32_t *start;     // [max_batch] first packed token of each row
    int32_t *len;       // [max_batch] packed tokens of each row
    int32_t *at;        // [tcap] r * seq + p of each packed token
    int32_t *row;       // [tcap] the row of each packed token
    int32_t *tokens;    // [1] packed tokens of the run
};

hipError_t pack_rows(hipStream_t s, const int32_t *mask, int batch, int seq, Packing p);

// Int8 operand rows a LayerNorm can write beside its 16-bit output (the next
// product's operand): the codes of each row's values as rounded to the 16-bit
// type, with its scale, exactly as quantize_rows makes them from that output.
struct QuantOut {
    int8_t *q = nullptr;   // [tokens][hidden]
    float *scale = nullptr;   // [tokens]
};

// x[t] = LN(word[id] + pos[p + offset] + type[ty]) (BERT, RoBERTa), or, with
// pos NULL, LN(word[id] (+ type[ty] when type is not NULL)) (rotary
// families); ln_b NULL is no bias. Writes x (F32) and, when xh is not NULL,
// its copy in `dt`. With zero_mask (the rows' mask, DeBERTa-v2), a token
// whose mask is 0 is zero instead.
hipError_t embed_ln(hipStream_t s, int tokens, int hidden, const int32_t *ids, const int32_t *types,
                    const Packing &p, int seq, int position_offset, const float *word, const float *pos,
                    const float *type, const float *ln_w, const float *ln_b, float eps, float *x, void *xh, Dt dt,
                    const int32_t *zero_mask = nullptr, const QuantOut &qo = QuantOut());

// DeBERTa-v2's disentangled attention over qkv (as attention reads it) into
// ctx: for each live query i and live key j of a row, the score
// (q_i . k_j + q_i . pos_k[b] + k_j . pos_q[b]) / sqrt(3 d), b =
// buckets[i - j + positions - 1]; pos is the layer's [2 position_buckets][2 H]
// F32 shared-key projections of the relative rows, query then key. A masked
// query (mask 0 before the row's last live token) attends uniformly to every
// position through it.
hipError_t deberta_attention(hipStream_t s, Dt dt, const void *qkv, int tcap, int heads, int d, const Packing &p,
                             const int32_t *mask, int seq, int batch, int max_len, const float *pos,
                             const int32_t *buckets, int positions, void *ctx);

// out = LN(in) row by row over `tokens` rows of `hidden`; out_f32 and out_h
// (in `dt`) may each be NULL, and out_f32 may be in (in place). ln_b NULL is
// no bias.
hipError_t layer_norm(hipStream_t s, int tokens, int hidden, const float *in, const float *ln_w, const float *ln_b,
                      float eps, float *out_f32, void *out_h, Dt dt);

// The residual add and a LayerNorm in one pass, row by row: v = x + y (y in
// ydt: F32, F16 or BF16). Post-norm (pre_norm 0): x = LN(v), and out_h =
// LN(v) in `dt` when not NULL. Pre-norm (pre_norm 1): x = v, and out_h =
// LN(v) in `dt` (out_h F32 on the F32 tier). ln_b NULL is no bias.
hipError_t add_layer_norm(hipStream_t s, int tokens, int hidden, float *x, const void *y, Dt ydt, const float *ln_w,
                          const float *ln_b, float eps, int pre_norm, void *out_h, Dt dt,
                          const QuantOut &qo = QuantOut());

// What a GEMM does with each output once its sum is done.
enum class Epi : int {
    Plain = 0,     // outf[m, n] = acc + bias (F32 out; kernel tests)
    Qkv = 1,       // head-major [3][heads][tcap][d] in the operand type: acc + bias
    Gelu = 2,      // out[m, n] = gelu(acc + bias) in the operand type
    Residual = 3,  // x[m, n] += acc + bias (F32)
    QkvRope = 4,   // as Qkv, Q and K rotated by their tokens' positions (pair-adjacent columns)
    Gated = 5,     // out[m, n / 2] = act(acc_n + b_n) * (acc_{n+1} + b_{n+1}) in the operand type
    Bias = 6,      // out[m, n] = acc + bias, in the operand type or (out_f32) F32: a product the next kernel adds
};

struct EpiArgs {
    Epi kind = Epi::Plain;
    const float *bias = nullptr;   // [n] or NULL
    void *out = nullptr;           // Plain (F32), Qkv, Gelu, Gated: the output
    int ldo = 0;                   // row stride of out (elements)
    float *x = nullptr;            // Residual: [m, ldo] F32
    int tcap = 0, heads = 0, d = 0, hidden = 0;   // Qkv scatter
    int tok0 = 0;                  // Qkv, QkvRope: the packed token of row 0 of A (of at, and of the scatter)
    const float *cos = nullptr, *sin = nullptr;   // QkvRope: [positions][d / 2]
    const int32_t *at = nullptr;   // QkvRope: each token's r * seq + p
    int seq = 0;
    int silu = 0;                  // Gated: SiLU instead of GELU
    int out_f32 = 0;               // Bias: F32 outputs (else the operand type; F16 for int8 operands)
    // I8 operands: output (m, n) is the int32 sum times a_scale[m] * w_scale[n].
    const float *a_scale = nullptr, *w_scale = nullptr;
};

// C[m, n] = sum_k A[m, k] W[n, k] over m < M (rows of A, ld lda), n < N, k < K,
// operands in `dt`, F32 accumulation on MFMA, then the epilogue. `tile`
// picks the block shape (0 = the launcher's choice for the shape).
hipError_t gemm(hipStream_t s, Dt dt, int M, int N, int K, const void *A, int lda, const void *W,
                const EpiArgs &e, int tile = 0);
int gemm_tiles();   // how many block shapes `tile` may name (1..n)
// A block shape's name in a choices string ("auto" for 0, the launcher's
// rule), and the shape a name (or a bare number) spells, -1 for none.
const char *gemm_tile_name(int tile);
int gemm_tile_by_name(const char *s, size_t n);
// The block shapes worth timing for products of this operand type and
// shape (K, lda and the epilogue decide which kernels take them) into out:
// how many.
int gemm_candidates(Dt dt, int K, int lda, const EpiArgs &e, int *out, int cap);
// A test hook standing in for a device that cannot launch one block shape:
// the shape a name spells (NULL or "" for none) fails to launch from now on.
// False for a name that spells no shape. gemm_made_to_fail says whether a
// shape is the one.
bool gemm_fail_variant(const char *name);
bool gemm_made_to_fail(int tile);

// Softmax attention within each row and head over Q and K ([heads][tcap][d]
// each) and V transposed ([heads][d][tcap]), in `dt`, one after another in
// qkv, into ctx [tokens, heads * d] in `dt`. window: keys within `window` of
// the query (|i - j| <= window), or INT32_MAX. F16 and BF16 run on the matrix
// cores unless `simple`; F32 runs the scalar path.
hipError_t attention(hipStream_t s, Dt dt, const void *qkv, int tcap, int heads, int d, const Packing &p,
                     const int32_t *mask, int seq, int batch, int max_len, int window, void *ctx,
                     bool simple = false);

// A mean's tokens are summed in chunks of POOL_CHUNK, each chunk in token
// order by its own workgroup, then the chunks' sums in chunk order: `part`
// holds [count][chunks][output_dim] F32 sums and `cnt` [count][chunks]
// token counts, chunks >= ceil(seq / POOL_CHUNK).
constexpr int POOL_CHUNK = 256;
struct PoolScratch {
    float *part = nullptr;
    int32_t *cnt = nullptr;
    int chunks = 0;
};

// One vector per row (mode 0: MEAN/CLS/LAST as pooling says) or per range
// (mode 1: the mean over the range's live tokens), cut to output_dim, L2
// normalized when l2, into out [count, output_dim] F32.
hipError_t pool(hipStream_t s, const float *x, int hidden, const Packing &p, const int32_t *mask, int seq,
                int count, const uint32_t *ranges, int pooling, int output_dim, int l2, const PoolScratch &ps,
                float *out);

// The MFMA rate probe: `blocks` workgroups of 4 waves, each wave 8 chains of
// 32x32x16 F16 products for `iters` rounds, fixed or random operands; out
// takes 256 floats, clk the shader and real-time (100 MHz) counts of one wave.
hipError_t mfma_probe(hipStream_t s, int blocks, int iters, int random, float *out, unsigned long long *clk);

// The span head's outputs at most (2 for start and end).
constexpr int HEAD_MAX = 16;

// Range i's mean over all `hidden` values (as pool's mode 1) through a linear
// head, w [hout, hidden] and b [hout] F32, its sums in F64: out [count, hout].
hipError_t pool_head(hipStream_t s, const float *x, int hidden, const Packing &p, const int32_t *mask, int seq,
                     int count, const uint32_t *ranges, const float *hw, const float *hb, int hout,
                     const PoolScratch &ps, float *out);

// Symmetric int8 rows: for each of `rows` rows of `cols` values (row stride
// ld, F32 or F16 per src_dt), scale = max |x| / 127 and q = round(x / scale)
// (q = 0 and scale 0 for a zero row), into dst [rows][cols] and scale [rows].
// Per output channel for weights, per token for activations.
hipError_t quantize_rows(hipStream_t s, const void *src, Dt src_dt, int rows, int cols, int ld, int8_t *dst,
                         float *scale);

// Vector codes of rows x dim F32 values (reference core/src/quantize.rs:48-80,
// sentence-transformers' quantize_embeddings layout): mode 2 (int8) with
// ranges [2][dim] (minimums, then maximums) on the device, a byte a value,
// clamp(floor((x - min) / step), 0, 255) - 128 with step = (max - min) / 255
// or 1 where that is 0, every step in F32; mode 3 (ubinary) the sign bits
// x > 0, eight to a byte, the first value in the top bit, a last byte padded
// with 0 bits. Into out (rows * dim or rows * ((dim + 7) / 8) bytes).
hipError_t quantize_codes(hipStream_t s, const float *x, int rows, int dim, int mode, const float *ranges,
                          uint8_t *out);

// The fixed staging area of the no-allocation buffer_quantize: a device
// array of STATIC_SCRATCH_BYTES on each GPU, alive until the process ends.
// static_scratch gives its address on `device`, which must be the current
// device (looked up once a device, then kept). Every caller on one GPU shares
// it: calls that overlap on one GPU race.
constexpr size_t STATIC_SCRATCH_BYTES = (size_t)16 << 20;
constexpr int MAX_DEVICES = 64;
hipError_t static_scratch(int device, void **ptr);

// dst = src over `bytes` (a multiple of 16), 16-byte vectors, one pass.
hipError_t copy_bytes(hipStream_t s, const void *src, void *dst, size_t bytes);

// n values uniform in [-amp, amp) from a counter hash of (seed, index).
hipError_t fill_uniform(hipStream_t s, float *dst, size_t n, float amp, uint32_t seed);

// F32 -> F16 (round to nearest even) or BF16 copies of weights; `overflow`
// (device int, may be NULL) is set to 1 when an F16 value overflows.
hipError_t narrow(hipStream_t s, const float *src, void *dst, size_t n, Dt dt, int32_t *overflow);

}  // namespace rocm
