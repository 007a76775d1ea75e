/* The oracle: a CPU restatement of TurboEmbed's CPU encoder (the reference's
 * core/src/cpu/), used only as the checker of the rocm backend's results and
 * as the CPU baseline the benchmark times beside it. It is test
 * infrastructure: no product code links, loads or calls it.
 *
 * It takes the same seam structs a backend does (turbo_backend_model,
 * turbo_backend_embed_rows, turbo_token_range), so a test hands the same
 * description to the oracle and to the backend.
 */
#ifndef TURBO_ORACLE_H
#define TURBO_ORACLE_H

#include "turbo/turbo_seam.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One run: rows (and, when count > 0, ranges pooled by the mean) through the
 * encoder `m` describes, into out: [batch, output_dim] or [count, output_dim]
 * F32. `hidden`, when not NULL, receives the final hidden states of the
 * packed tokens, [tokens, hidden] F32 (room for batch * seq rows).
 * With rows->head 1 on a range write to a model with a span head (m->head,
 * m->head_out), out is [count, head_out]: each range's mean over all hidden
 * values, not normalized, through the head, its sums in F64 from the bias
 * (reference core/src/qa/session.rs:268-276). With rows->taps T > 1 on a
 * range write, out is [T, count, output_dim]: block k the ranges pooled
 * after layer L - T + k + 1 of L (a ModernBERT's through final_norm), the
 * last block the final layer's; with rows->tap_alone 1 it is the first of
 * those alone, [count, output_dim], the model cut after that layer
 * (core/src/cpu/encoder/mod.rs:292-373).
 * `threads` 0 is one per processor. Returns TURBO_OK or a status; `why`
 * (may be NULL) receives a message of up to why_len bytes. */
int32_t oracle_encode(const turbo_backend_model *m, const turbo_backend_embed_rows *rows,
                      const turbo_token_range *ranges, uint32_t count, uint32_t threads,
                      float *out, float *hidden, char *why, uint32_t why_len);

/* The packing alone (reference core/src/cpu/encoder/mod.rs:379-424): for each
 * row its first packed token and its packed length, and for each packed
 * token its place r * seq + p in the rows. Returns the packed tokens. */
uint32_t oracle_pack(const int32_t *mask, uint32_t batch, uint32_t seq, uint32_t row_stride,
                     const turbo_token_range *ranges, uint32_t count,
                     uint32_t *start, uint32_t *len, uint32_t *at);

/* The scalar functions the encoder uses, for their own tests. */
// Vector codes as the reference core makes them on the host
// (core/src/quantize.rs:48-80): mode 2 int8 with ranges [2][dim], mode 3
// ubinary. out holds rows * dim or rows * ((dim + 7) / 8) bytes.
void  oracle_quantize(const float *x, uint32_t rows, uint32_t dim, uint32_t mode, const float *ranges, uint8_t *out);
float oracle_exp(float x);
// Seconds the last oracle_encode spent on its rows (the weights' layout excluded).
double oracle_last_encode_seconds(void);
/* A limit on the gated MLP's product act(gate) * up, 0 for none (the
 * default, the CPU path's F32): an F16 tier stores that product saturated at
 * 65504, and is checked against the oracle with this limit set. */
void  oracle_set_gated_limit(float limit);
/* Worker threads pin themselves to the process's CPUs, one each (for a
 * timed CPU baseline), when on is not 0. */
void  oracle_set_pinning(int32_t on);
/* DeBERTa-v2's relative row of a signed distance (core/src/deberta/math.rs:30-40). */
uint32_t oracle_deberta_bucket(int64_t distance, uint32_t buckets, uint32_t maximum);
float oracle_gelu(float x);
float oracle_silu(float x);
void  oracle_layer_norm(float *y, const float *w, const float *b, uint32_t n, float eps);

#ifdef __cplusplus
}
#endif

#endif
