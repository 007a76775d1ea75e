// Launchers of the rocm backend's gfx950 kernels. Every launcher enqueues on
// the given stream and returns the launch's error; none allocates or syncs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rocm {

// The timing hook of every launch. A timed run sets `stop` (and `start`)
// before a launcher and clears them after it: the first kernel the launcher
// enqueues on this thread takes the start event and each takes the stop
// event, bound to the kernels' own dispatch packets, so the pair spans the
// kernels' execution with no marker packet between launches. `bound` says
// that a kernel took them.
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
    bool bound = false;
};
LaunchTiming &launch_timing();

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
    int32_t *pos;       // [tcap] the column p of each packed token (its position in its row)
    int32_t *tokens;    // [1] packed tokens of the run
};

// The dimensions of a run, written by the host beside the rows and read on
// the device by every kernel of the run, so one captured graph serves every
// batch of a token bin: grids are sized for the bin's bounds, and a
// workgroup past the run's own extent leaves at once. A split run's parts
// each have their rows, packed tokens and longest row (an unused part has
// none). Options the pooling reads are here too.
constexpr int MAX_PARTS = 4;
struct PartDims {
    int32_t row0, rows, tok0, tokens, max_len, pad[3];
};
struct RunDims {
    int32_t batch, seq, tokens, max_len;    // rows, their stride, packed tokens, longest row
    int32_t count, pooling, output_dim, l2; // ranges (0: one vector a row), pooling, width, L2 normalize
    int32_t head, pad[7];                   // 1: ranges through the span head
    PartDims part[MAX_PARTS];
};

// The rows and packed tokens one launch works on: part `part` of the run
// whose dimensions `dims` points to (-1: the whole run), read on the device;
// or, with dims NULL, the values given here (kernel tests and the tuner).
struct Span {
    const RunDims *dims = nullptr;
    int part = -1;
    int row0 = 0, rows = 0, tok0 = 0, tokens = 0, max_len = 0, seq = 0;
};
inline Span span_of(const RunDims *dims, int part) {
    Span s;
    s.dims = dims;
    s.part = part;
    return s;
}
inline Span span_tokens(int tokens) {
    Span s;
    s.tokens = tokens;
    return s;
}

// Packs the run's rows (batch and seq from the dimensions; batch at most
// max_batch).
hipError_t pack_rows(hipStream_t s, const int32_t *mask, const RunDims *dims, int max_batch, int max_seq,
                     Packing p);

// Int8 operand rows a LayerNorm can write beside its 16-bit output (the next
// product's operand): the codes of each row's values as rounded to the 16-bit
// type, with its scale, exactly as quantize_rows makes them from that output.
struct QuantOut {
    int8_t *q = nullptr;   // [tokens][hidden] from token 0 of the run...
    float *scale = nullptr;   // [tokens]
    int tok_stride = 0;    // ...a part's rows starting tok0 * tok_stride bytes in
};

// x[t] = LN(word[id] + pos[p + offset] + type[ty]) (BERT, RoBERTa), or, with
// pos NULL, LN(word[id] (+ type[ty] when type is not NULL)) (rotary
// families); ln_b NULL is no bias. Writes x (F32) and, when xh is not NULL,
// its copy in `dt`. With zero_mask (the rows' mask, DeBERTa-v2), a token
// whose mask is 0 is zero instead.
// Over the whole run's tokens (span part -1); max_tokens bounds the grid.
hipError_t embed_ln(hipStream_t s, const Span &sp, int max_tokens, int hidden, const int32_t *ids,
                    const int32_t *types, const Packing &p, int position_offset, const float *word, const float *pos,
                    const float *type, const float *ln_w, const float *ln_b, float eps, float *x, void *xh, Dt dt,
                    const int32_t *zero_mask = nullptr, const QuantOut &qo = QuantOut());

// DeBERTa-v2's disentangled attention over qkv (as attention reads it) into
// ctx: for each live query i and live key j of a row, the score
// (q_i . k_j + q_i . pos_k[b] + k_j . pos_q[b]) / sqrt(3 d), b =
// buckets[i - j + positions - 1]; pos is the layer's [2 position_buckets][2 H]
// F32 shared-key projections of the relative rows, query then key. A masked
// query (mask 0 before the row's last live token) attends uniformly to every
// position through it.
// The span's rows; max_rows and max_len bound the grid and the LDS. With
// pos_t (F16 and BF16, d = 64: the same table in the operand type) on the
// matrix cores; the caller passes it only where no 63 consecutive distances
// span more than 64 relative rows.
hipError_t deberta_attention(hipStream_t s, Dt dt, const void *qkv, int tcap, int heads, int d, const Packing &p,
                             const int32_t *mask, const Span &sp, int max_rows, int max_len, const float *pos,
                             const int32_t *buckets, int positions, const void *pos_t, void *ctx);

// out = LN(in) row by row over `tokens` rows of `hidden`; out_f32 and out_h
// (in `dt`) may each be NULL, and out_f32 may be in (in place). ln_b NULL is
// no bias.
// Row pointers are the run's token 0; the span's tokens are normed.
hipError_t layer_norm(hipStream_t s, const Span &sp, int max_tokens, int hidden, const float *in, const float *ln_w,
                      const float *ln_b, float eps, float *out_f32, void *out_h, Dt dt);

// The residual add and a LayerNorm in one pass, row by row: v = x + y (y in
// ydt: F32, F16 or BF16). Post-norm (pre_norm 0): x = LN(v), and out_h =
// LN(v) in `dt` when not NULL. Pre-norm (pre_norm 1): x = v, and out_h =
// LN(v) in `dt` (out_h F32 on the F32 tier). ln_b NULL is no bias.
// A post-norm on 16-bit rows may carry its residual in them (res_h): v =
// out_h + y, and x = LN(v) only with keep_f32 (out_h = LN(v) always).
// Over the span's tokens; x, y and out_h point at the run's token 0.
hipError_t add_layer_norm(hipStream_t s, const Span &sp, int max_tokens, int hidden, float *x, const void *y, Dt ydt,
                          const float *ln_w, const float *ln_b, float eps, int pre_norm, void *out_h, Dt dt,
                          const QuantOut &qo = QuantOut(), bool res_h = false, bool keep_f32 = true);

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
    int tok0 = 0;                  // set on the device: the packed token of row 0 of A (of at, and of the scatter)
    const float *cos = nullptr, *sin = nullptr;   // QkvRope: [positions][d / 2]
    const int32_t *pos = nullptr;  // QkvRope: each packed token's position in its row
    int silu = 0;                  // Gated: SiLU instead of GELU
    int out_f32 = 0;               // Bias: F32 outputs (else the operand type; F16 for int8 operands)
    int out_bf16 = 0;              // Bias on F16 operands: BF16 outputs (F32's range at half its bytes)
    // I8 operands: output (m, n) is the int32 sum times a_scale[m] * w_scale[n].
    const float *a_scale = nullptr, *w_scale = nullptr;
    // Split K (Bias products): the F32 slices' workspace and its capacity.
    float *ws = nullptr;
    size_t ws_floats = 0;
};

// C[m, n] = sum_k A[m, k] W[n, k] over the span's tokens m (rows of A, ld
// lda), n < N, k < K, operands in `dt`, F32 accumulation on MFMA, then the
// epilogue. A, a row-major output and the int8 activation scales point at
// the run's token 0; the span's rows start tok0 * a_tok rows of A in (a_tok
// 0: lda) and tok0 rows of the output in; max_m bounds the grid. `tile`
// picks the block shape (0 = the launcher's choice for max_m).
hipError_t gemm(hipStream_t s, Dt dt, const Span &sp, int max_m, int N, int K, const void *A, int lda, int a_tok,
                const void *W, const EpiArgs &e, int tile = 0);
// The same with explicit rows M from token 0 (kernel tests and the tuner).
inline hipError_t gemm(hipStream_t s, Dt dt, int M, int N, int K, const void *A, int lda, const void *W,
                       const EpiArgs &e, int tile = 0) {
    return gemm(s, dt, span_tokens(M), M, N, K, A, lda, 0, W, e, tile);
}
int gemm_tiles();   // how many block shapes `tile` may name (1..n)
// A block shape's name in a choices string ("auto" for 0, the launcher's
// rule), and the shape a name (or a bare number) spells, -1 for none.
const char *gemm_tile_name(int tile);
int gemm_tile_by_name(const char *s, size_t n);
// The block shapes worth timing for products of this operand type and
// shape (K, lda and the epilogue decide which kernels take them) into out:
// how many.
int gemm_candidates(Dt dt, int K, int lda, const EpiArgs &e, int *out, int cap);
// The 256 x 384 block shape (8 waves of 128 x 96): a split run's products' shape.
constexpr int WIDE_TILE = 15;
// A post-norm product of N = hidden with the residual add and the LayerNorm
// in its epilogue (whole-row tiles): y = A W^T + bias rounded to the operand
// type, v = out_h + y, out_h = LN(v) (and x = LN(v) in F32 with keep_f32),
// each row with the bits add_layer_norm gives it after the plain product.
// Rows point at the run's token 0; the span's tokens are taken.
struct LnArgs {
    const float *bias = nullptr;   // [hidden] the product's bias, or NULL
    float *x = nullptr;            // [tokens][hidden] F32 rows (written with keep_f32)
    void *out_h = nullptr;         // [tokens][hidden] 16-bit rows: the residual, then LN(v)
    const float *ln_w = nullptr, *ln_b = nullptr;   // ln_b NULL: no bias
    float eps = 0;
    int res_h = 1;                 // the residual is carried in out_h (the one form taken)
    int keep_f32 = 0;
};
// The whole-row block shape (128 x 768, 8 waves of 128 x 96).
constexpr int LN_TILE = 17;
// Split K on the staged kernel (Bias products with EpiArgs.ws): 128 x 128
// tiles over 4 slices of K, 64 x 64 over 2. The workspace takes slices x
// M x N floats.
constexpr int SPLITK_TILE_4 = 18, SPLITK_TILE_2 = 19, SPLITK_MAX = 4;
bool gemm_splitk_tile(int tile);
bool gemm_ln_tile(int tile);
// Whether the fused kernel takes a product of this operand type, hidden size,
// inner size and operand stride on a session whose residual is in the
// 16-bit rows (res_h).
bool gemm_ln_takes(Dt dt, int hidden, int K, int lda, bool res_h);
hipError_t gemm_ln(hipStream_t s, Dt dt, const Span &sp, int max_m, int hidden, int K, const void *A, int lda,
                   int a_tok, const void *W, const LnArgs &e, int tile = 0);
// A test hook standing in for a device that cannot launch one block shape:
// the shape a name spells (NULL or "" for none) fails to launch from now on.
// False for a name that spells no shape. gemm_made_to_fail says whether a
// shape is the one.
bool gemm_fail_variant(const char *name);
bool gemm_made_to_fail(int tile);

// Softmax attention within each row and head over Q and K ([heads][tcap][d]
// each) and V transposed ([heads][d][tcap]), in `dt`, one after another in
// qkv, into ctx [tokens, heads * d] in `dt`. window: keys within `window` of
// the query (|i - j| <= window), or INT32_MAX. F16 and BF16 heads of 64 run
// on the matrix cores (path 0: 256-query workgroups; 2: 128-query ones)
// unless path is 1; F32 runs the scalar path.
// The span's rows; max_rows and max_len bound the grid.
hipError_t attention(hipStream_t s, Dt dt, const void *qkv, int tcap, int heads, int d, const Packing &p,
                     const int32_t *mask, const Span &sp, int max_rows, int max_len, int window, void *ctx,
                     int path = 0);

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

// The run's vectors, as its dimensions say: one a row (count 0: MEAN, CLS
// or LAST as pooling says) or one a range (the mean over the range's live
// tokens), cut to output_dim, L2 normalized when l2, into out
// [items, output_dim] F32; with head set, each range's mean over all
// `hidden` values through the span head (hw [hout, hidden], hb [hout] F32,
// F64 sums) into out [count, hout]. max_items bounds the grid.
hipError_t pool(hipStream_t s, const RunDims *dims, int max_items, const float *x, int hidden, const Packing &p,
                const int32_t *mask, const uint32_t *ranges, const PoolScratch &ps, float *out,
                const float *hw = nullptr, const float *hb = nullptr, int hout = 0);

// The MFMA rate probe: `blocks` workgroups of 4 waves, each wave 8 chains of
// 32x32x16 F16 products for `iters` rounds, fixed or random operands; out
// takes 256 floats, clk the shader and real-time (100 MHz) counts of one wave.
hipError_t mfma_probe(hipStream_t s, int blocks, int iters, int random, float *out, unsigned long long *clk);

// The span head's outputs at most (2 for start and end).
constexpr int HEAD_MAX = 16;


// Symmetric int8 rows: for each of `rows` rows of `cols` values (row stride
// ld, F32 or F16 per src_dt), scale = max |x| / 127 and q = round(x / scale)
// (q = 0 and scale 0 for a zero row), into dst [rows][cols] and scale [rows].
// Per output channel for weights, per token for activations.
hipError_t quantize_rows(hipStream_t s, const void *src, Dt src_dt, int rows, int cols, int ld, int8_t *dst,
                         float *scale);
// The same over a span's tokens: src, dst and scale point at the run's token
// 0; the span's rows start tok0 * ld values of src, tok0 * dst_tok bytes of
// dst (rows of cols bytes from there) and tok0 scales in. max_rows bounds
// the grid.
hipError_t quantize_span(hipStream_t s, const Span &sp, int max_rows, const void *src, Dt src_dt, int cols, int ld,
                         int8_t *dst, int dst_tok, float *scale);

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
// dst = src over the span's tokens, rows of row_bytes (a multiple of 16)
// from the run's token 0; max_tokens bounds the grid.
hipError_t copy_rows(hipStream_t s, const Span &sp, int max_tokens, const void *src, void *dst, size_t row_bytes);

// n values uniform in [-amp, amp) from a counter hash of (seed, index).
hipError_t fill_uniform(hipStream_t s, float *dst, size_t n, float amp, uint32_t seed);

// F32 -> F16 (round to nearest even) or BF16 copies of weights; `overflow`
// (device int, may be NULL) is set to 1 when an F16 value overflows.
hipError_t narrow(hipStream_t s, const float *src, void *dst, size_t n, Dt dt, int32_t *overflow);

}  // namespace rocm
