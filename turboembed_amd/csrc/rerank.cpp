// The rerank caller of the encoder, on the host: pair windows over token ids,
// the runs that encode them through the backend's table, and the sequence
// classification head. Restates the reference core's caller side
// (core/src/tokenizer/pair.rs:27-99, core/src/session/rerank.rs:111-219),
// which the encoder path serves with CLS rows at full width, unnormalized.
#include <cmath>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "turbo_rocm.h"
#include "session.h"

using namespace rocm;

namespace {

// One window's class-head logit (core/src/session/rerank.rs:166-191): the
// pooler's dense rows summed in F64 from the bias, tanh, rounded to F32;
// then the classifier's one row the same way. Without a pooler the
// classifier reads the CLS state itself.
float head_logit(const float *x, uint32_t hidden, const float *pooler_w, const float *pooler_b, const float *cls_w,
                 float cls_b, std::vector<float> &pooled) {
    const float *in = x;
    if (pooler_w) {
        pooled.resize(hidden);
        for (uint32_t o = 0; o < hidden; ++o) {
            const float *w = pooler_w + (size_t)o * hidden;
            double sum = pooler_b ? (double)pooler_b[o] : 0.0;
            for (uint32_t k = 0; k < hidden; ++k) sum += (double)w[k] * (double)x[k];
            pooled[o] = (float)std::tanh(sum);
        }
        in = pooled.data();
    }
    double sum = (double)cls_b;
    for (uint32_t k = 0; k < hidden; ++k) sum += (double)cls_w[k] * (double)in[k];
    return (float)sum;
}

}  // namespace

extern "C" {

int32_t turbo_rocm_pair_windows(const int32_t *query, uint32_t query_len, const int32_t *passage, uint32_t passage_len,
                                int32_t start_id, int32_t end_id, uint32_t roberta, uint32_t query_tokens,
                                uint32_t max_tokens, uint32_t stride, int32_t *ids, int32_t *types, uint32_t *lengths,
                                uint32_t capacity, uint32_t *windows, turbo_error *err) {
    return guarded(err, [&] {
        const uint32_t specials = roberta ? 4 : 3;
        if (max_tokens <= specials + 1)
            fail(TURBO_E_INVALID_ARGUMENT, "pair max_tokens must leave content space within max_seq", 2);
        if (query_tokens >= max_tokens - specials)
            fail(TURBO_E_INVALID_ARGUMENT, "pair query_tokens must leave a passage token", 1);
        if ((query_len && !query) || (passage_len && !passage) || !windows)
            fail(TURBO_E_INVALID_ARGUMENT, "pair windows: NULL ids");
        // The query is cut on the right; the passage is covered by windows
        // of `room` tokens, `step` apart (disjoint for stride 0).
        const uint32_t q = std::min(query_len, query_tokens);
        const uint32_t room = max_tokens - specials - q;
        const uint32_t step = stride == 0 ? room : stride;
        if (step == 0 || step > room)
            fail(TURBO_E_INVALID_ARGUMENT, "pair stride must be within passage capacity", 3);
        uint32_t n = 0;
        for (uint32_t start = 0;; start += step) {
            const uint32_t end = std::min<uint64_t>((uint64_t)start + room, passage_len);
            if (n < capacity) {
                int32_t *row = ids + (size_t)n * max_tokens;
                int32_t *ty = types + (size_t)n * max_tokens;
                uint32_t at = 0;
                row[at++] = start_id;
                for (uint32_t i = 0; i < q; ++i) row[at++] = query[i];
                row[at++] = end_id;
                if (roberta) row[at++] = end_id;
                const uint32_t boundary = at;
                for (uint32_t i = start; i < end; ++i) row[at++] = passage[i];
                row[at++] = end_id;
                // BERT's template marks the passage and its end token type 1;
                // RoBERTa's has one segment.
                for (uint32_t i = 0; i < at; ++i) ty[i] = (!roberta && i >= boundary) ? 1 : 0;
                for (uint32_t i = at; i < max_tokens; ++i) {
                    row[i] = 0;
                    ty[i] = 0;
                }
                lengths[n] = at;
            }
            ++n;
            if (end == passage_len) break;
        }
        *windows = n;
        if (n > capacity)
            fail(TURBO_E_CAPACITY, "pair windows: " + std::to_string(n) + " over capacity " + std::to_string(capacity));
        return TURBO_OK;
    });
}

int32_t turbo_rocm_rerank_scores(const float *states, uint32_t n, uint32_t hidden, const float *pooler_weight,
                                 const float *pooler_bias, const float *classifier_weight, float classifier_bias,
                                 float *scores, turbo_error *err) {
    return guarded(err, [&] {
        if (!states || !classifier_weight || !scores || hidden == 0)
            fail(TURBO_E_INVALID_ARGUMENT, "rerank head: NULL tensors or zero width");
        std::vector<float> pooled;
        for (uint32_t i = 0; i < n; ++i) {
            const float *x = states + (size_t)i * hidden;
            for (uint32_t k = 0; k < hidden; ++k)
                if (!std::isfinite(x[k])) fail(TURBO_E_INTERNAL, "non-finite rerank encoder output");
            const float v = head_logit(x, hidden, pooler_weight, pooler_bias, classifier_weight, classifier_bias, pooled);
            if (!std::isfinite(v)) fail(TURBO_E_INTERNAL, "rerank relevance overflows F32");
            scores[i] = v;
        }
        return TURBO_OK;
    });
}

int32_t turbo_rocm_rerank_run(void *session, const int32_t *ids, const int32_t *types, const uint32_t *lengths,
                              uint32_t windows, uint32_t seq, const uint32_t *owner, uint32_t pairs,
                              const float *pooler_weight, const float *pooler_bias, const float *classifier_weight,
                              float classifier_bias, float *scores, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        if (!s || !ids || !types || !lengths || !owner || !scores || windows == 0 || pairs == 0 || seq == 0)
            fail(TURBO_E_INVALID_ARGUMENT, "rerank run: NULL arguments or zero counts");
        if (s->task != TURBO_TASK_RERANK) fail(TURBO_E_UNSUPPORTED_TASK, "model task is not rerank");
        if (pairs > s->max_batch) fail(TURBO_E_CAPACITY, "pair count exceeds max_batch");
        if (seq > s->max_seq) fail(TURBO_E_CAPACITY, "rerank run: windows wider than the session's max_seq");
        const uint32_t H = s->model->hidden;
        for (uint32_t w = 0; w < windows; ++w)
            if (owner[w] >= pairs || lengths[w] == 0 || lengths[w] > seq)
                fail(TURBO_E_INVALID_ARGUMENT, "rerank run: window " + std::to_string(w));
        for (uint32_t p = 0; p < pairs; ++p) scores[p] = -std::numeric_limits<float>::infinity();
        std::vector<int32_t> mask((size_t)std::min(windows, s->max_batch) * seq);
        std::vector<float> states, logits;
        // Windows in runs of max_batch, each row's CLS state read back and
        // scored; a pair's score is its best window's.
        for (uint32_t start = 0; start < windows; start += s->max_batch) {
            const uint32_t n = std::min(windows - start, s->max_batch);
            for (uint32_t r = 0; r < n; ++r)
                for (uint32_t c = 0; c < seq; ++c) mask[(size_t)r * seq + c] = c < lengths[start + r] ? 1 : 0;
            turbo_backend_embed_rows rows{};
            rows.struct_size = sizeof rows;
            rows.batch = n;
            rows.seq = seq;
            rows.row_stride = seq;
            rows.ids = ids + (size_t)start * seq;
            rows.mask = mask.data();
            rows.types = types + (size_t)start * seq;
            rows.pooling = TURBO_POOLING_CLS;
            rows.normalize = TURBO_NORMALIZE_NONE;
            rows.output_dim = H;
            int32_t rc = turbo_rocm_backend.embed_write(session, &rows, err);
            if (rc != TURBO_OK) return rc;
            turbo_backend_run run{};
            run.struct_size = sizeof run;
            rc = turbo_rocm_backend.session_run(session, &run, err);
            if (rc != TURBO_OK) return rc;
            states.resize((size_t)n * H);
            rc = turbo_rocm_backend.buffer_read(run.output, states.data(), states.size() * 4, err);
            if (rc != TURBO_OK) return rc;
            logits.resize(n);
            rc = turbo_rocm_rerank_scores(states.data(), n, H, pooler_weight, pooler_bias, classifier_weight,
                                          classifier_bias, logits.data(), err);
            if (rc != TURBO_OK) return rc;
            for (uint32_t r = 0; r < n; ++r) {
                float &sc = scores[owner[start + r]];
                sc = std::max(sc, logits[r]);
            }
        }
        return TURBO_OK;
    });
}

}  // extern "C"
