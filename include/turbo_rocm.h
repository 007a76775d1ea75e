/* SPDX-License-Identifier: Apache-2.0
 *
 * The rocm backend's C ABI: libturbo_rocm.so.
 *
 * The drop-in boundary is one symbol, the backend's function table, which
 * the TurboEmbed core lists beside its other backends. Everything else here
 * is the host-side checking the core does before it calls a backend (so a
 * harness without the Rust core checks rows as the core does) and hooks for
 * tests and measurement, which the core never calls.
 */
#ifndef TURBO_ROCM_H
#define TURBO_ROCM_H

#include "turbo/turbo_seam.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The backend's table, name "rocm". Replaces, for AMD gfx950 GPUs, the
 * reference's turbo_cuda_backend (core/cuda/backend.cpp:3776-3809), and is
 * linked into the core's LINKED list the same way
 * (core/src/backend/mod.rs:338-360, extern static as core/src/cuda.rs:8-17).
 * Every function follows include/turbo/turbo_backend.h:455-627. */
extern const turbo_backend turbo_rocm_backend;

/* The numeric class of BF16 operands with F32 sums: this backend's BF16 tier.
 * The reference defines classes 1, 2, 4 and 8 (turbo_backend.h:226-229); this
 * is the next free bit, which the core's NUMERICS_ALLOWED table
 * (core/src/tuning.rs:32-41) needs for a BF16-stored model. */
#define TURBO_ROCM_NUMERIC_BF16_F32ACC 16u

/* The numeric class of int8 operands with int32 sums, dequantized in F32: a
 * symmetric scale per weight row (output channel) and per token, this
 * backend's I8 tier. It runs for a model whose turbo_backend_model.compute_dtype
 * is TURBO_DTYPE_I8, at MODEL and FASTEST; the reference's only I8 encoder is
 * a compiled Hailo graph (core/hailo/backend.cpp:441-443, 510). */
#define TURBO_ROCM_NUMERIC_I8_I32ACC 32u

/* ---- The core's checks of a write (core/src/session/tokens.rs:274-384) ----
 *
 * turbo_rocm_check_tokens: the rows' shape within max_batch x max_seq, each id
 * under vocab, each type under types (types may be NULL), each mask entry 0
 * or 1 with a 1 in every row, and, when max_tokens is not 0, each row's
 * length through its last live token at most max_tokens. row_stride 0 is seq.
 * Returns TURBO_OK or the status the core returns, with its message. */
int32_t turbo_rocm_check_tokens(uint32_t batch, uint32_t seq, uint32_t row_stride, const int32_t *ids,
                                const int32_t *mask, const int32_t *types, uint32_t max_batch, uint32_t max_seq,
                                uint32_t vocab, uint32_t token_types, uint32_t max_tokens, turbo_error *err);

/* turbo_rocm_check_ranges: count ranges of the rows above (the core's
 * check_ranges, core/src/session/tokens.rs:274-306, for a backend that does
 * not compute mask-0 columns): count 1 to max_ranges, each row under batch,
 * start under end, end at most seq, and a live token inside. */
int32_t turbo_rocm_check_ranges(uint32_t batch, uint32_t seq, uint32_t row_stride, const int32_t *mask,
                                const turbo_token_range *ranges, uint32_t count, uint32_t max_ranges,
                                turbo_error *err);

/* ---- The rerank caller (core/src/tokenizer/pair.rs:27-99,
 * core/src/session/rerank.rs:47-219) ----
 *
 * turbo_rocm_pair_windows: a query and a passage, as token ids, into the
 * encoder windows of the pair template [start] query [end] passage [end]
 * (RoBERTa, roberta != 0: [start] query [end] [end] passage [end], one
 * segment): the query cut to query_tokens on the right, the passage covered
 * by windows of max_tokens - specials - query tokens, stride apart (0:
 * disjoint). Each window is a row of max_tokens ids and types (BERT: type 1
 * from the passage on) padded with id 0, and its length. Writes up to
 * capacity windows and *windows = their number; TURBO_E_CAPACITY when more
 * are needed. Errors as the reference's: field 2 max_tokens, 1 query_tokens,
 * 3 stride. */
int32_t turbo_rocm_pair_windows(const int32_t *query, uint32_t query_len, const int32_t *passage, uint32_t passage_len,
                                int32_t start_id, int32_t end_id, uint32_t roberta, uint32_t query_tokens,
                                uint32_t max_tokens, uint32_t stride, int32_t *ids, int32_t *types, uint32_t *lengths,
                                uint32_t capacity, uint32_t *windows, turbo_error *err);

/* turbo_rocm_rerank_scores: the sequence classification head over n CLS
 * states [n, hidden] F32 (core/src/session/rerank.rs:166-191): the pooler
 * (dense [hidden, hidden] + bias, tanh; skipped when pooler_weight is NULL)
 * and the one-logit classifier, each summed in F64 from its bias and rounded
 * to F32. A non-finite state or logit is TURBO_E_INTERNAL. */
int32_t turbo_rocm_rerank_scores(const float *states, uint32_t n, uint32_t hidden, const float *pooler_weight,
                                 const float *pooler_bias, const float *classifier_weight, float classifier_bias,
                                 float *scores, turbo_error *err);

/* turbo_rocm_rerank_run: the windows of `pairs` pairs ([windows, seq] ids and
 * types, each window's length, and the pair it belongs to) through a
 * TURBO_TASK_RERANK session of this backend, max_batch windows a run, as
 * CLS rows at full width with no normalization, then the head above; each
 * pair's score is the largest of its windows' (core/src/session/rerank.rs:
 * 111-219). pairs may not exceed the session's max_batch. */
int32_t turbo_rocm_rerank_run(void *session, const int32_t *ids, const int32_t *types, const uint32_t *lengths,
                              uint32_t windows, uint32_t seq, const uint32_t *owner, uint32_t pairs,
                              const float *pooler_weight, const float *pooler_bias, const float *classifier_weight,
                              float classifier_bias, float *scores, turbo_error *err);

/* turbo_rocm_buffer_quantize_static: this backend's buffer_quantize entry
 * without an allocation. It has no counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The same codes, byte
 * for byte, as buffer_quantize, staged in a fixed device area of 16 MiB a GPU
 * (allocated once with the library, held until the process ends) instead of
 * memory allocated per call: the codes, then on a 256-byte boundary the int8
 * ranges ([2, dim] F32), must fit it, or the call fails with
 * TURBO_E_INVALID_ARGUMENT before any device work. It calls no allocating
 * routine. Every context on a GPU shares that GPU's area; a lock per GPU,
 * held through the call, serializes calls from any thread and context. run,
 * when not NULL, gets the int8 ranges' bytes in h2d_bytes and the device
 * allocations the call made (none) in device_allocs. */
int32_t turbo_rocm_buffer_quantize_static(void *buffer, uint32_t quantization, const float *int8_ranges, uint32_t rows,
                                          uint32_t dim, turbo_backend_run *run, turbo_error *err);

/* ---- Test and measurement hooks (no counterpart in the reference's seam; the
 * reference's CUDA backend keeps similar ones, core/src/cuda.rs:177-499) ---- */

/* Makes the GEMM block shape `name` (as a choices string spells it, e.g.
 * "256x256"; NULL or "" for none) fail to launch from now on, in place of a
 * device that cannot take it: the launcher's rule picks another shape, the
 * tuner skips it, a cached choice naming it is not taken, and a session that
 * forces it is refused with TURBO_E_UNSUPPORTED (the reference's
 * turbo_cuda_fail_variant, core/src/cuda.rs:461-469,
 * core/cuda/backend.cpp:2430-2440, 3006-3010). Process-wide. */
int32_t turbo_rocm_fail_variant(const char *name, turbo_error *err);

/* The last run's packing, read back from the device: each row's first packed
 * token and length ([batch] each), each packed token's r * seq + p ([tokens]),
 * and the packed token count. */
int32_t turbo_rocm_session_packing(void *session, int32_t *start, int32_t *len, int32_t *at, uint32_t *tokens,
                                   turbo_error *err);

/* The last run's final hidden states, [tokens, hidden] F32. */
int32_t turbo_rocm_session_hidden(void *session, float *out, uint64_t floats, turbo_error *err);

/* The backend's heap allocations so far: every malloc-family and operator
 * new call its own code has made (counted as they happen), in the process
 * and on the calling thread. A run's turbo_backend_run.host_allocs is the
 * change of the thread's count across it. Either pointer may be NULL. */
int32_t turbo_rocm_host_allocs(uint64_t *process, uint64_t *thread, turbo_error *err);

/* Times every kernel of the session's later runs with HIP events, each
 * launch's pair bound to its kernels' own dispatch packets (the first
 * kernel's start, the last one's end: no marker packet between launches) on
 * the stream it runs on (a split run's parts side by side, as the run
 * executes them; timed runs launch their kernels directly rather than
 * replay a graph, and take a replay's time); turbo_rocm_session_times then writes
 * "<kernel> <ms> <launches>" lines: the milliseconds summed over the last
 * run's launches of that kernel, and how many there were;
 * turbo_rocm_session_intervals writes "<kernel> <start> <end>" a launch, in
 * ms from the run's start, in launch order. */
int32_t turbo_rocm_session_timing(void *session, uint32_t on, turbo_error *err);
int32_t turbo_rocm_session_times(void *session, char *out, uint32_t len, turbo_error *err);
int32_t turbo_rocm_session_intervals(void *session, char *out, uint32_t len, turbo_error *err);

/* Runs the last written rows `runs` more times, back to back on the
 * context's stream, then waits: the rows stay resident on the device, so
 * this is the device's throughput on them, for measurement. */
int32_t turbo_rocm_session_replay(void *session, uint32_t runs, turbo_error *err);

/* How many graphs the session has captured (one per bin of packed tokens, at
 * session_open) and how many runs replayed one since. */
int32_t turbo_rocm_session_graphs(void *session, uint64_t *captured, uint64_t *launched, turbo_error *err);

/* The session's kernel choices, as TURBO_ROCM_CHOICES takes them. */
int32_t turbo_rocm_session_choices(void *session, char *out, uint32_t len, turbo_error *err);

/* One GEMM, out [M, N] = A [M, K] W [N, K]^T + bias (bias may be NULL), with
 * the operands narrowed on the device to dtype (TURBO_DTYPE_F32, F16 or
 * BF16) or quantized to int8 rows (TURBO_DTYPE_I8: a symmetric scale per row
 * of A and of W, int32 sums, dequantized in F32), and block shape `tile`
 * (0 = the default choice). Allocates its own device memory; for kernel tests. */
int32_t turbo_rocm_gemm_check(uint32_t ordinal, uint32_t dtype, uint32_t M, uint32_t N, uint32_t K, const float *A,
                              const float *W, const float *bias, float *out, uint32_t tile, turbo_error *err);

/* The average milliseconds of `iters` back-to-back launches of the GEMM
 * [M, K] x [N, K]^T with the residual epilogue, block shape `tile`, on
 * device-resident uniform random operands of dtype; for tuning sweeps. */
int32_t turbo_rocm_gemm_time(uint32_t ordinal, uint32_t dtype, uint32_t M, uint32_t N, uint32_t K, uint32_t tile,
                             uint32_t iters, float *ms, turbo_error *err);

/* A plain device copy of `bytes` (a multiple of 16) from one buffer to
 * another, `iters` times, on device `ordinal`: the average milliseconds of
 * a launch into *ms. A measurement hook with no counterpart
 * in the reference: its launches read and write exactly `bytes`, so the
 * profiler's traffic counters can be scaled by what they read for it. */
int32_t turbo_rocm_copy_probe(uint32_t ordinal, uint64_t bytes, uint32_t iters, float *ms, turbo_error *err);

/* The matrix cores' sustained rate: every compute unit's 4 waves issue 8
 * independent chains of 32x32x16 F16 products for iters rounds, with fixed
 * operands, or with random ones changing every product (random 1), as a
 * GEMM's do; *tflops is the rate, *mhz the shader clock under that load. A
 * measurement hook with no counterpart in the reference: the ceiling a
 * GEMM's data lets the chip sustain, beside the published peak. */
int32_t turbo_rocm_mfma_probe(uint32_t ordinal, uint32_t random, uint32_t iters, float *tflops, float *mhz,
                              turbo_error *err);

#ifdef __cplusplus
}
#endif

#endif /* TURBO_ROCM_H */
