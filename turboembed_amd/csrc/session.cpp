// Models and sessions of the rocm backend: weights on the device, the
// session's memory, rows written, and the run's kernels.
//
// A run's kernels, in order (the reference's CPU run, core/src/cpu/encoder/
// mod.rs:309-374 and rotary/mod.rs:88-175, and the CUDA graph,
// core/cuda/backend.cpp:2020-2361):
//   pack_rows -> embed_ln -> per layer { QKV GEMM (+bias, head-major; RoPE on
//   the rotary families) -> attention -> out GEMM (+bias, residual into x) ->
//   LayerNorm -> FFN-in GEMM (+bias, GELU; or the gated product) -> FFN-out
//   GEMM (+bias, residual) -> LayerNorm } -> pool (+cut, +L2).
// ModernBERT is pre-norm: the norms come before the products they feed and
// final_norm follows the last layer.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "session.h"
#include "turbo_rocm.h"

namespace rocm {

// ---- Weights ---------------------------------------------------------------------

namespace {

float half_bits_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else {
            float f = std::ldexp((float)m, -24);
            std::memcpy(&u, &f, 4);
            u |= s;
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Assembles every tensor the kernels read, in F32, into one host image laid
// out as the device copy will be; each piece starts on a 256-byte boundary.
struct Image {
    std::vector<float> data;
    size_t add(size_t n) {
        const size_t at = (data.size() + 63) / 64 * 64;
        data.resize(at + n, 0.0f);
        return at;
    }
};

const turbo_backend_tensor &tensor_at(const turbo_backend_model *d, uint32_t i) { return d->tensors[i]; }

// Widen tensor i to F32 into dst (n floats), checking its size.
void widen(const turbo_backend_model *d, uint32_t i, size_t n, float *dst, const char *what) {
    const turbo_backend_tensor &t = tensor_at(d, i);
    const size_t el = d->dtype == TURBO_DTYPE_F32 ? 4 : 2;
    if (!t.data || t.bytes != n * el)
        fail(TURBO_E_INVALID_ARGUMENT, std::string("rocm: tensor ") + std::to_string(i) + " (" +
                                           (t.name ? t.name : what) + ") holds " + std::to_string(t.bytes) +
                                           " bytes, not " + std::to_string(n * el));
    if (d->dtype == TURBO_DTYPE_F32) {
        std::memcpy(dst, t.data, n * 4);
        return;
    }
    const uint16_t *src = static_cast<const uint16_t *>(t.data);
    if (d->dtype == TURBO_DTYPE_F16) {
        for (size_t k = 0; k < n; ++k) dst[k] = half_bits_to_float(src[k]);
    } else {
        for (size_t k = 0; k < n; ++k) {
            const uint32_t u = (uint32_t)src[k] << 16;
            std::memcpy(&dst[k], &u, 4);
        }
    }
}

}  // namespace

// DeBERTa-v2's relative row of a signed distance (reference
// core/src/deberta/math.rs:30-40, transformers' make_log_bucket_position):
// within half the buckets the distance itself; beyond,
// ceil(ln(|d| / mid) / ln((max - 1) / mid) * (mid - 1)) + mid with F32
// logarithms, signed; offset by the buckets and clamped to the table.
static uint32_t deberta_bucket(int64_t distance, uint32_t buckets, uint32_t maximum) {
    const int64_t mid = buckets / 2, mag0 = distance < 0 ? -distance : distance;
    int64_t mag = mag0;
    if (mag0 > mid) {
        const float a = std::log((float)mag0 / (float)mid), c = std::log((float)(maximum - 1) / (float)mid);
        mag = (int64_t)std::ceil(a / c * (float)(mid - 1)) + mid;
    }
    const int64_t v = (distance < 0 ? -mag : mag) + buckets;
    return (uint32_t)std::min<int64_t>(std::max<int64_t>(v, 0), 2 * (int64_t)buckets - 1);
}

Model *model_load(Context *c, const turbo_backend_model *d) {
    if (d->struct_size < offsetof(turbo_backend_model, tensors) + sizeof(void *))
        fail(TURBO_E_INVALID_STRUCT_SIZE, "rocm: turbo_backend_model of " + std::to_string(d->struct_size) + " bytes");
    const bool deberta = d->family == TURBO_FAMILY_DEBERTA_V2;
    const bool bert = d->family == TURBO_FAMILY_BERT || d->family == TURBO_FAMILY_ROBERTA || deberta;
    const bool modern = d->family == TURBO_FAMILY_MODERNBERT, nomic = d->family == TURBO_FAMILY_NOMIC_BERT;
    if (!bert && !modern && !nomic)
        fail(TURBO_E_UNSUPPORTED, "rocm: family " + std::to_string(d->family) +
                                      ": the rocm backend runs BERT, RoBERTa, DeBERTa-v2, ModernBERT and nomic-bert "
                                      "encoders");
    if (d->format != TURBO_FORMAT_SAFETENSORS) fail(TURBO_E_UNSUPPORTED, "rocm: only raw weights (safetensors) load");
    if (d->dtype != TURBO_DTYPE_F32 && d->dtype != TURBO_DTYPE_F16 && d->dtype != TURBO_DTYPE_BF16)
        fail(TURBO_E_UNSUPPORTED, "rocm: weights of dtype " + std::to_string(d->dtype));
    if (d->lookahead != 0) fail(TURBO_E_UNSUPPORTED, "rocm: a banded (lookahead) model");
    if (d->heads == 0 || d->hidden % d->heads != 0) fail(TURBO_E_INVALID_ARGUMENT, "rocm: hidden is not heads * d");
    const uint32_t H = d->hidden, dh = H / d->heads, I = d->intermediate;
    if (dh != 8 && dh != 16 && dh != 32 && dh != 64 && dh != 128)
        fail(TURBO_E_UNSUPPORTED, "rocm: head width " + std::to_string(dh) + " (8, 16, 32, 64 or 128)");
    if (H % 8 != 0 || I % 8 != 0 || H > 2048)
        fail(TURBO_E_UNSUPPORTED, "rocm: hidden " + std::to_string(H) + " and intermediate " + std::to_string(I) +
                                      " must be multiples of 8, hidden at most 2048");
    // A span head (TASK_EXTRACTIVE_QA): [head_out, hidden] and [head_out]
    // F32, applied to a headed range write's means (turbo_backend.h:332-337).
    const bool headed = d->struct_size >= offsetof(turbo_backend_model, head_out) + 4 && d->head && d->head_out;
    if (headed) {
        if (d->head_out > HEAD_MAX || d->head_out > H)
            fail(TURBO_E_UNSUPPORTED, "rocm: a head of " + std::to_string(d->head_out) + " outputs (at most " +
                                          std::to_string(HEAD_MAX) + ")");
        const turbo_backend_tensor &w = d->head[0], &b = d->head[1];
        if (!w.data || !b.data || w.dtype != TURBO_DTYPE_F32 || b.dtype != TURBO_DTYPE_F32 ||
            w.bytes != (uint64_t)d->head_out * H * 4 || b.bytes != (uint64_t)d->head_out * 4)
            fail(TURBO_E_INVALID_ARGUMENT, "rocm: the head is [" + std::to_string(d->head_out) + ", " +
                                               std::to_string(H) + "] and [" + std::to_string(d->head_out) + "] F32");
    }

    // compute_dtype I8 on raw weights: the manifest asks for int8 GEMMs
    // (per-channel weights, per-token activations), as a compiled I8 graph
    // fixes them for the reference's Hailo backend (core/hailo/backend.cpp:441-443).
    const uint32_t fixed = d->struct_size >= offsetof(turbo_backend_model, compute_dtype) + 4 ? d->compute_dtype : 0;
    if (fixed != 0 && fixed != TURBO_DTYPE_I8 && fixed != TURBO_DTYPE_F32 && fixed != TURBO_DTYPE_F16 &&
        fixed != TURBO_DTYPE_BF16)
        fail(TURBO_E_UNSUPPORTED, "rocm: compute_dtype " + std::to_string(fixed));

    auto m = std::make_unique<Model>();
    m->ctx = c;
    m->int8 = fixed == TURBO_DTYPE_I8;
    m->family = d->family;
    m->dtype = d->dtype;
    m->layers = d->layers;
    m->hidden = H;
    m->heads = d->heads;
    m->inter = I;
    m->vocab = d->vocab_size;
    m->positions = d->max_positions;
    m->types = d->token_types;
    m->position_offset = d->position_offset;
    m->eps = (float)d->layer_norm_eps;
    m->rotary = modern || nomic;
    m->modern = modern;

    Image img;
    struct Off {
        size_t word = 0, pos = SIZE_MAX, type = SIZE_MAX, emb_w = 0, emb_b = SIZE_MAX, final_w = SIZE_MAX,
               rope = SIZE_MAX;
    } off;
    struct LOff {
        size_t wqkv, bqkv = SIZE_MAX, wo, bo = SIZE_MAX, ln1_w = SIZE_MAX, ln1_b = SIZE_MAX, w1, b1 = SIZE_MAX, w2,
                     b2 = SIZE_MAX, ln2_w, ln2_b = SIZE_MAX;
        size_t n_in;
    };
    std::vector<LOff> loff(d->layers);
    auto put = [&](uint32_t i, size_t n, const char *what) {
        const size_t at = img.add(n);
        widen(d, i, n, &img.data[at], what);
        return at;
    };
    std::vector<float> reln;   // DeBERTa-v2: the normalized relative rows
    uint32_t rel_buckets = 0, rel_max = 0;
    if (bert) {
        const uint32_t emb = deberta ? TURBO_DEBERTA_EMBEDDING_TENSORS : TURBO_BERT_EMBEDDING_TENSORS;
        if (d->tensor_count != emb + d->layers * TURBO_BERT_LAYER_TENSORS)
            fail(TURBO_E_INVALID_ARGUMENT, "rocm: tensor_count " + std::to_string(d->tensor_count));
        if (deberta) {
            if (d->struct_size < offsetof(turbo_backend_model, max_relative_positions) + 4 ||
                d->position_buckets < 2 || d->max_relative_positions < 2 || d->token_types > 1)
                fail(TURBO_E_INVALID_ARGUMENT, "rocm: a DeBERTa-v2 model has position_buckets and "
                                               "max_relative_positions of 2 or more, and no token types");
            rel_buckets = d->position_buckets;
            rel_max = d->max_relative_positions;
            off.word = put(TURBO_DEBERTA_WORD_EMBEDDINGS, (size_t)d->vocab_size * H, "word");
            off.emb_w = put(TURBO_DEBERTA_EMBEDDINGS_LN_WEIGHT, H, "ln");
            off.emb_b = put(TURBO_DEBERTA_EMBEDDINGS_LN_BIAS, H, "ln");
            // The relative rows through their own LayerNorm, in F64 (reference
            // core/src/deberta/weights.rs:91-92, math.rs:9-27).
            const size_t rows = (size_t)2 * rel_buckets;
            reln.resize(rows * H);
            std::vector<float> w(H), bb(H);
            widen(d, TURBO_DEBERTA_RELATIVE_EMBEDDINGS, rows * H, reln.data(), "relative");
            widen(d, TURBO_DEBERTA_RELATIVE_LN_WEIGHT, H, w.data(), "relative ln");
            widen(d, TURBO_DEBERTA_RELATIVE_LN_BIAS, H, bb.data(), "relative ln");
            for (size_t r = 0; r < rows; ++r) {
                float *y = &reln[r * H];
                double sum = 0.0, var = 0.0;
                for (uint32_t i = 0; i < H; ++i) sum += (double)y[i];
                const double mean = sum / H;
                for (uint32_t i = 0; i < H; ++i) var += ((double)y[i] - mean) * ((double)y[i] - mean);
                const double scale = 1.0 / std::sqrt(var / H + d->layer_norm_eps);
                for (uint32_t i = 0; i < H; ++i) y[i] = (float)(((double)y[i] - mean) * scale * w[i] + bb[i]);
            }
        } else {
            off.word = put(TURBO_BERT_WORD_EMBEDDINGS, (size_t)d->vocab_size * H, "word");
            off.pos = put(TURBO_BERT_POSITION_EMBEDDINGS, (size_t)d->max_positions * H, "position");
            off.type = put(TURBO_BERT_TOKEN_TYPE_EMBEDDINGS, (size_t)std::max(1u, d->token_types) * H, "type");
            off.emb_w = put(TURBO_BERT_EMBEDDINGS_LN_WEIGHT, H, "ln");
            off.emb_b = put(TURBO_BERT_EMBEDDINGS_LN_BIAS, H, "ln");
        }
        for (uint32_t l = 0; l < d->layers; ++l) {
            const uint32_t b = emb + l * TURBO_BERT_LAYER_TENSORS;
            LOff &o = loff[l];
            // Q, K and V back to back: one [3H, H] product.
            o.wqkv = img.add((size_t)3 * H * H);
            widen(d, b + TURBO_BERT_Q_WEIGHT, (size_t)H * H, &img.data[o.wqkv], "q");
            widen(d, b + TURBO_BERT_K_WEIGHT, (size_t)H * H, &img.data[o.wqkv + (size_t)H * H], "k");
            widen(d, b + TURBO_BERT_V_WEIGHT, (size_t)H * H, &img.data[o.wqkv + (size_t)2 * H * H], "v");
            o.bqkv = img.add((size_t)3 * H);
            widen(d, b + TURBO_BERT_Q_BIAS, H, &img.data[o.bqkv], "q bias");
            widen(d, b + TURBO_BERT_K_BIAS, H, &img.data[o.bqkv + H], "k bias");
            widen(d, b + TURBO_BERT_V_BIAS, H, &img.data[o.bqkv + 2 * H], "v bias");
            o.wo = put(b + TURBO_BERT_ATTN_OUT_WEIGHT, (size_t)H * H, "out");
            o.bo = put(b + TURBO_BERT_ATTN_OUT_BIAS, H, "out bias");
            o.ln1_w = put(b + TURBO_BERT_ATTN_LN_WEIGHT, H, "attn ln");
            o.ln1_b = put(b + TURBO_BERT_ATTN_LN_BIAS, H, "attn ln");
            o.w1 = put(b + TURBO_BERT_FFN_IN_WEIGHT, (size_t)I * H, "ffn in");
            o.b1 = put(b + TURBO_BERT_FFN_IN_BIAS, I, "ffn in bias");
            o.w2 = put(b + TURBO_BERT_FFN_OUT_WEIGHT, (size_t)H * I, "ffn out");
            o.b2 = put(b + TURBO_BERT_FFN_OUT_BIAS, H, "ffn out bias");
            o.ln2_w = put(b + TURBO_BERT_FFN_LN_WEIGHT, H, "ffn ln");
            o.ln2_b = put(b + TURBO_BERT_FFN_LN_BIAS, H, "ffn ln");
            o.n_in = I;
        }
    } else {
        if (d->struct_size < offsetof(turbo_backend_model, global_every) + 4)
            fail(TURBO_E_INVALID_STRUCT_SIZE, "rocm: a rotary model needs the rotary fields");
        if (d->mlp != TURBO_MLP_GATED || dh % 2 || d->rope_pairs * 2 != dh || !d->rope_table)
            fail(TURBO_E_INVALID_ARGUMENT, "rocm: a rotary model has a gated MLP and a rope table of d/2 pairs");
        const uint32_t emb = modern ? TURBO_MODERNBERT_EMBEDDING_TENSORS : TURBO_NOMIC_EMBEDDING_TENSORS;
        const uint32_t per = modern ? TURBO_MODERNBERT_LAYER_TENSORS : TURBO_NOMIC_LAYER_TENSORS;
        if (d->tensor_count != emb + d->layers * per)
            fail(TURBO_E_INVALID_ARGUMENT, "rocm: tensor_count " + std::to_string(d->tensor_count));
        m->silu = d->activation == TURBO_ACTIVATION_SILU;
        m->window = d->attention_window / 2;
        m->global_every = d->global_every;
        m->pairs = d->rope_pairs;
        if (modern) {
            off.word = put(TURBO_MODERNBERT_WORD_EMBEDDINGS, (size_t)d->vocab_size * H, "word");
            off.emb_w = put(TURBO_MODERNBERT_EMBEDDINGS_LN_WEIGHT, H, "ln");
            off.final_w = put(TURBO_MODERNBERT_FINAL_NORM_WEIGHT, H, "final norm");
        } else {
            off.word = put(TURBO_NOMIC_WORD_EMBEDDINGS, (size_t)d->vocab_size * H, "word");
            off.type = put(TURBO_NOMIC_TOKEN_TYPE_EMBEDDINGS, (size_t)std::max(1u, d->token_types) * H, "type");
            off.emb_w = put(TURBO_NOMIC_EMBEDDINGS_LN_WEIGHT, H, "ln");
            off.emb_b = put(TURBO_NOMIC_EMBEDDINGS_LN_BIAS, H, "ln");
        }
        const size_t rope_n = (size_t)4 * d->max_positions * d->rope_pairs;
        off.rope = img.add(rope_n);
        std::memcpy(&img.data[off.rope], d->rope_table, rope_n * 4);
        std::vector<float> tmp;
        for (uint32_t l = 0; l < d->layers; ++l) {
            const uint32_t b = emb + l * per;
            LOff &o = loff[l];
            // Q and K rows pair-adjacent per head, (c, c + d/2), V as stored
            // (reference core/src/cpu/kernels/pairs.rs:146-161): the RoPE
            // epilogue then finds each pair in neighbouring columns.
            tmp.resize((size_t)3 * H * H);
            widen(d, b + (modern ? TURBO_MODERNBERT_QKV_WEIGHT : TURBO_NOMIC_QKV_WEIGHT), tmp.size(), tmp.data(),
                  "qkv");
            o.wqkv = img.add(tmp.size());
            size_t row = 0;
            for (uint32_t third = 0; third < 2; ++third)
                for (uint32_t head = 0; head < H; head += dh)
                    for (uint32_t cc = 0; cc < dh / 2; ++cc)
                        for (uint32_t src : {third * H + head + cc, third * H + head + cc + dh / 2})
                            std::memcpy(&img.data[o.wqkv + (row++) * H], &tmp[(size_t)src * H], H * 4);
            std::memcpy(&img.data[o.wqkv + row * H], &tmp[(size_t)2 * H * H], (size_t)H * H * 4);
            o.wo = put(b + (modern ? TURBO_MODERNBERT_ATTN_OUT_WEIGHT : TURBO_NOMIC_ATTN_OUT_WEIGHT), (size_t)H * H,
                       "out");
            // Gate row j then up row j (pairs.rs:163-166).
            std::vector<float> gate((size_t)I * H), up((size_t)I * H);
            if (modern) {
                tmp.resize((size_t)2 * I * H);
                widen(d, b + TURBO_MODERNBERT_FFN_IN_WEIGHT, tmp.size(), tmp.data(), "ffn in");
                std::copy(tmp.begin(), tmp.begin() + (size_t)I * H, gate.begin());
                std::copy(tmp.begin() + (size_t)I * H, tmp.end(), up.begin());
            } else {
                widen(d, b + TURBO_NOMIC_FFN_GATE_WEIGHT, gate.size(), gate.data(), "ffn gate");
                widen(d, b + TURBO_NOMIC_FFN_UP_WEIGHT, up.size(), up.data(), "ffn up");
            }
            o.w1 = img.add((size_t)2 * I * H);
            for (uint32_t j = 0; j < I; ++j) {
                std::memcpy(&img.data[o.w1 + (size_t)(2 * j) * H], &gate[(size_t)j * H], H * 4);
                std::memcpy(&img.data[o.w1 + (size_t)(2 * j + 1) * H], &up[(size_t)j * H], H * 4);
            }
            o.w2 = put(b + (modern ? TURBO_MODERNBERT_FFN_OUT_WEIGHT : TURBO_NOMIC_FFN_OUT_WEIGHT), (size_t)H * I,
                       "ffn out");
            if (modern) {
                if (l > 0) o.ln1_w = put(b + TURBO_MODERNBERT_ATTN_LN_WEIGHT, H, "attn norm");
                o.ln2_w = put(b + TURBO_MODERNBERT_FFN_LN_WEIGHT, H, "mlp norm");
            } else {
                o.ln1_w = put(b + TURBO_NOMIC_ATTN_LN_WEIGHT, H, "norm1");
                o.ln1_b = put(b + TURBO_NOMIC_ATTN_LN_BIAS, H, "norm1");
                o.ln2_w = put(b + TURBO_NOMIC_FFN_LN_WEIGHT, H, "norm2");
                o.ln2_b = put(b + TURBO_NOMIC_FFN_LN_BIAS, H, "norm2");
            }
            o.n_in = (size_t)2 * I;
        }
    }

    size_t head_w = SIZE_MAX, head_b = SIZE_MAX;
    if (headed) {
        head_w = img.add((size_t)d->head_out * H);
        std::memcpy(&img.data[head_w], d->head[0].data, (size_t)d->head_out * H * 4);
        head_b = img.add(d->head_out);
        std::memcpy(&img.data[head_b], d->head[1].data, (size_t)d->head_out * 4);
        m->head_out = d->head_out;
    }

    OnDevice on(c->ordinal);
    m->f32.reset(dev_alloc(img.data.size() * 4, "model weights"));
    check(hipMemcpy(m->f32.get(), img.data.data(), img.data.size() * 4, hipMemcpyHostToDevice), "model weights");
    const float *base = static_cast<const float *>(m->f32.get());
    auto at = [&](size_t o) -> const float * { return o == SIZE_MAX ? nullptr : base + o; };
    m->word = at(off.word);
    m->pos = at(off.pos);
    m->type = at(off.type);
    m->emb_w = at(off.emb_w);
    m->emb_b = at(off.emb_b);
    m->final_w = at(off.final_w);
    m->rope = at(off.rope);
    m->head_w = at(head_w);
    m->head_b = at(head_b);
    for (const LOff &o : loff) {
        Model::Layer L{};
        L.wqkv = at(o.wqkv);
        L.bqkv = at(o.bqkv);
        L.wo = at(o.wo);
        L.bo = at(o.bo);
        L.ln1_w = at(o.ln1_w);
        L.ln1_b = at(o.ln1_b);
        L.w1 = at(o.w1);
        L.b1 = at(o.b1);
        L.w2 = at(o.w2);
        L.b2 = at(o.b2);
        L.ln2_w = at(o.ln2_w);
        L.ln2_b = at(o.ln2_b);
        L.n_qkv = (size_t)3 * H;
        L.n_in = o.n_in;
        m->ls.push_back(L);
    }
    if (deberta) {
        // Each layer's query and key projections of the normalized relative
        // rows (shared keys): the first 2 H rows of its QKV product and bias,
        // one F32 product a layer on the device; and the relative row of each
        // distance a session can reach.
        m->deberta = true;
        const size_t rows = (size_t)2 * rel_buckets;
        DevPtr rel(dev_alloc(rows * H * 4, "relative rows"));
        check(hipMemcpy(rel.get(), reln.data(), rows * H * 4, hipMemcpyHostToDevice), "relative rows");
        m->rel_pos.reset(dev_alloc((size_t)d->layers * rows * 2 * H * 4, "relative projections"));
        float *pos = static_cast<float *>(m->rel_pos.get());
        for (uint32_t l = 0; l < d->layers; ++l) {
            EpiArgs e;
            e.kind = Epi::Plain;
            e.bias = m->ls[l].bqkv;
            e.out = pos + (size_t)l * rows * 2 * H;
            e.ldo = (int)(2 * H);
            check(gemm(nullptr, Dt::F32, (int)rows, (int)(2 * H), (int)H, rel.get(), (int)H, m->ls[l].wqkv, e, 0),
                  "relative projections");
            m->ls[l].pos_qk = pos + (size_t)l * rows * 2 * H;
        }
        std::vector<int32_t> table((size_t)2 * m->positions - 1);
        for (int64_t dist = -(int64_t)m->positions + 1; dist < (int64_t)m->positions; ++dist)
            table[(size_t)(dist + m->positions - 1)] = (int32_t)deberta_bucket(dist, rel_buckets, rel_max);
        m->rel_rows = rows;
        m->rel_tiles = true;
        for (size_t i = 0; i + 1 < table.size(); ++i)
            m->rel_tiles = m->rel_tiles && (table[i + 1] - table[i] == 0 || table[i + 1] - table[i] == 1);
        m->rel_table.reset(dev_alloc(table.size() * 4, "relative buckets"));
        check(hipMemcpy(m->rel_table.get(), table.data(), table.size() * 4, hipMemcpyHostToDevice), "relative buckets");
        check(hipDeviceSynchronize(), "relative projections");
    }
    // The F32 weights serve the F32 tier as they are.
    for (const Model::Layer &L : m->ls) m->gemm_w[(int)Dt::F32].push_back({L.wqkv, L.wo, L.w1, L.w2});
    return m.release();
}

// The GEMM weights narrowed to `dt`, made on the first session that needs
// them and kept with the model (reference turbo.h: one resident copy per
// compute dtype, shared by the model's sessions).
std::vector<LayerWeights> &Model::weights_in(Dt dt) {
    std::lock_guard<std::mutex> g(lock);
    auto &w = gemm_w[(int)dt];
    if (!w.empty()) return w;
    const size_t H = hidden;
    size_t total = 0;
    for (const Layer &L : ls) total += L.n_qkv * H + H * H + L.n_in * H + H * inter;
    OnDevice on(ctx->ordinal);
    if (dt == Dt::I8) {
        // Symmetric per-output-channel int8: each weight row's scale is its
        // largest magnitude over 127.
        size_t rows = 0;
        for (const Layer &L : ls) rows += L.n_qkv + H + L.n_in + H;
        narrowed[(int)dt].reset(dev_alloc(total + rows * 4 + 256, "int8 weights"));
        int8_t *q = static_cast<int8_t *>(narrowed[(int)dt].get());
        float *sc = reinterpret_cast<float *>(q + ((total + 255) & ~(size_t)255));
        std::vector<LayerWeights> out;
        auto one = [&](const float *src, size_t n, size_t k, const float **scale) {
            check(quantize_rows(ctx->stream, src, Dt::F32, (int)n, (int)k, (int)k, q, sc), "quantizing weights");
            const void *at = q;
            *scale = sc;
            q += n * k;
            sc += n;
            return at;
        };
        for (const Layer &L : ls) {
            LayerWeights lw;
            lw.qkv = one(L.wqkv, L.n_qkv, H, &lw.s_qkv);
            lw.out = one(L.wo, H, H, &lw.s_out);
            lw.ffn_in = one(L.w1, L.n_in, H, &lw.s_ffn_in);
            lw.ffn_out = one(L.w2, H, inter, &lw.s_ffn_out);
            out.push_back(lw);
        }
        check(hipStreamSynchronize(ctx->stream), "quantizing weights");
        w = std::move(out);
        return w;
    }
    narrowed[(int)dt].reset(dev_alloc(total * 2 + 256, "narrowed weights"));
    char *p = static_cast<char *>(narrowed[(int)dt].get());
    int32_t *flag = reinterpret_cast<int32_t *>(p + total * 2);
    check(hipMemsetAsync(flag, 0, 4, ctx->stream), "narrowing weights");
    std::vector<LayerWeights> out;
    size_t at = 0;
    auto one = [&](const float *src, size_t n) {
        void *dst = p + at * 2;
        check(narrow(ctx->stream, src, dst, n, dt, flag), "narrowing weights");
        at += n;
        return (const void *)dst;
    };
    for (const Layer &L : ls) {
        LayerWeights lw;
        lw.qkv = one(L.wqkv, L.n_qkv * H);
        lw.out = one(L.wo, H * H);
        lw.ffn_in = one(L.w1, L.n_in * H);
        lw.ffn_out = one(L.w2, H * inter);
        out.push_back(lw);
    }
    int32_t over = 0;
    check(hipMemcpyAsync(&over, flag, 4, hipMemcpyDeviceToHost, ctx->stream), "narrowing weights");
    check(hipStreamSynchronize(ctx->stream), "narrowing weights");
    if (dt == Dt::F16 && over) f16_overflow = true;
    w = std::move(out);
    return w;
}

// DeBERTa-v2's relative projections narrowed to `dt` (F16 or BF16), made on
// the first session that needs them and kept with the model; null where a
// value passes F16's range (those sessions keep the F32 table's scalar path).
const void *Model::rel_pos_in(Dt dt) {
    std::lock_guard<std::mutex> g(lock);
    DevPtr &p = rel_narrowed[(int)dt];
    if (p) return rel_overflow[(int)dt] ? nullptr : p.get();
    const size_t n = (size_t)layers * rel_rows * 2 * hidden;
    OnDevice on(ctx->ordinal);
    p.reset(dev_alloc(n * 2 + 256, "narrowed relative projections"));
    int32_t *flag = reinterpret_cast<int32_t *>(static_cast<char *>(p.get()) + ((n * 2 + 255) & ~(size_t)255));
    check(hipMemsetAsync(flag, 0, 4, ctx->stream), "narrowing relative projections");
    check(narrow(ctx->stream, static_cast<const float *>(rel_pos.get()), p.get(), n, dt, flag),
          "narrowing relative projections");
    int32_t over = 0;
    check(hipMemcpyAsync(&over, flag, 4, hipMemcpyDeviceToHost, ctx->stream), "narrowing relative projections");
    check(hipStreamSynchronize(ctx->stream), "narrowing relative projections");
    rel_overflow[(int)dt] = over != 0;
    return rel_overflow[(int)dt] ? nullptr : p.get();
}

void model_release(Model *m) {
    if (!m) return;
    {
        OnDevice on(m->ctx->ordinal);
        (void)hipStreamSynchronize(m->ctx->stream);
        for (auto &n : m->narrowed) n.reset();
        m->f32.reset();
    }
    delete m;
}

// ---- Sessions -----------------------------------------------------------------------

namespace {

// The numeric class a dtype's GEMMs compute in. BF16 and I8 have none in
// the reference's header; this backend's are the next free bits.
uint32_t numeric_of(Dt dt) {
    switch (dt) {
    case Dt::F16: return TURBO_NUMERIC_F16_F32ACC;
    case Dt::BF16: return TURBO_ROCM_NUMERIC_BF16_F32ACC;
    case Dt::I8: return TURBO_ROCM_NUMERIC_I8_I32ACC;
    default: return TURBO_NUMERIC_F32_FMA;
    }
}

uint32_t dtype_of(Dt dt) {
    switch (dt) {
    case Dt::I8: return TURBO_DTYPE_I8;
    case Dt::F16: return TURBO_DTYPE_F16;
    case Dt::BF16: return TURBO_DTYPE_BF16;
    default: return TURBO_DTYPE_F32;
    }
}

// Whether a session's attention can take the matrix-core path: 16-bit
// activations and 64-wide heads.
bool mfma_attention(Dt act, uint32_t head_width) { return act != Dt::F32 && head_width == 64; }

}  // namespace

static void split_defaults(Session &s);
static bool ln_fusable(const Session &s, int g);

// Split K takes the out and FFN-out products (N the hidden size) of the
// bins whose runs do not split into parts and hold at most SPLITK_ROWS
// packed tokens, off the int8 tier: launches of a few row tiles.
constexpr uint32_t SPLITK_ROWS = 4096;
static uint32_t parts_of_bin(const Session &s, int b);
static bool splitk_fits(const Session &s, int b, int g) {
    return (g == G_OUT || g == G_FFN2) && s.dt != Dt::I8 && parts_of_bin(s, b) == 1 &&
           bin_tokens(b, (uint64_t)s.max_batch * s.max_seq) <= SPLITK_ROWS;
}

// The ints between the rows' ids, mask and types planes: max_batch x
// max_seq, rounded up to a multiple of 4.
static size_t plane_ints(const Session &s) { return ((size_t)s.max_batch * s.max_seq + 3) / 4 * 4; }

Session *session_open(Model *m, const turbo_backend_session_desc *desc, turbo_backend_tuning *tuning) {
    if (desc->task != TURBO_TASK_EMBED && desc->task != TURBO_TASK_RERANK)
        fail(TURBO_E_UNSUPPORTED_TASK, "rocm: task " + std::to_string(desc->task));
    if (desc->cpu_threads != 0)
        fail(TURBO_E_UNSUPPORTED_OPTION, "rocm: cpu_threads applies to a CPU device alone", 6);
    if (desc->max_batch == 0 || desc->max_seq == 0) fail(TURBO_E_INVALID_SHAPE, "rocm: max_batch and max_seq");
    // The packing kernel keeps a length per row in LDS.
    if (desc->max_batch > 16384) fail(TURBO_E_UNSUPPORTED, "rocm: max_batch above 16384");
    // Every position a row can reach has a table row (BERT's positions from
    // position_offset; a rotary model's cos/sin table).
    const uint64_t reach = (uint64_t)desc->max_seq + (m->rotary ? 0 : m->position_offset);
    if (reach > m->positions)
        fail(TURBO_E_INVALID_ARGUMENT, "rocm: max_seq " + std::to_string(desc->max_seq) + " reaches past the model's " +
                                           std::to_string(m->positions) + " positions");
    Dt dt;
    switch (desc->precision) {
    case TURBO_PRECISION_EXACT: dt = Dt::F32; break;
    case TURBO_PRECISION_MODEL:
        dt = m->dtype == TURBO_DTYPE_F16 ? Dt::F16 : m->dtype == TURBO_DTYPE_BF16 ? Dt::BF16 : Dt::F32;
        break;
    case TURBO_PRECISION_FASTEST: dt = m->dtype == TURBO_DTYPE_BF16 ? Dt::BF16 : Dt::F16; break;
    default: fail(TURBO_E_INVALID_ENUM, "rocm: precision " + std::to_string(desc->precision), 3);
    }
    if (m->int8 && desc->precision != TURBO_PRECISION_EXACT) {
        // The int8 kernel reads whole 64-byte rows of both operands.
        if (m->hidden % 64 != 0 || m->inter % 64 != 0)
            fail(TURBO_E_UNSUPPORTED, "rocm: int8 GEMMs need hidden and intermediate sizes in multiples of 64");
        dt = Dt::I8;
    }
    // The open's launches (weights narrowed on first need, the tuner's runs,
    // the graphs' capture) take the context's streams from its other
    // sessions' runs until it returns: a launch of theirs would land in a
    // capture.
    std::lock_guard<std::recursive_mutex> on_ctx(m->ctx->lock);
    auto s = std::make_unique<Session>();
    s->model = m;
    s->ctx = m->ctx;
    s->task = desc->task;
    s->max_batch = desc->max_batch;
    s->max_seq = desc->max_seq;
    s->max_ranges = desc->struct_size >= offsetof(turbo_backend_session_desc, max_ranges) + 4 && desc->max_ranges
                        ? desc->max_ranges
                        : desc->max_batch;
    s->precision = desc->precision;
    if (dt != Dt::F32) {
        s->w = &m->weights_in(dt);
        // A GEMM weight past F16's range computes in F32 (as the reference's
        // CUDA backend does, core/cuda/backend.cpp:1168-1225).
        if (dt == Dt::F16 && m->f16_overflow) dt = Dt::F32;
    }
    if (dt == Dt::F32) s->w = &m->weights_in(Dt::F32);
    s->dt = dt;
    s->act = dt == Dt::I8 ? Dt::F16 : dt;
    if (m->deberta && m->rel_tiles && s->act != Dt::F32 && m->hidden / m->heads == 64)
        s->rel_pos_t = m->rel_pos_in(s->act);
    s->compute_dtype = dtype_of(dt);
    if (tuning && tuning->struct_size >= offsetof(turbo_backend_tuning, numerics_used) + 4) {
        if (tuning->numerics_allowed && !(tuning->numerics_allowed & numeric_of(dt)))
            fail(TURBO_E_UNSUPPORTED_OPTION,
                 "rocm: the precision's numeric classes do not include this backend's " +
                     std::to_string(numeric_of(dt)),
                 3);
    }
    // Kernel choices: the rule's, then a cached string (ON and RETUNE), then
    // what TURBO_ROCM_CHOICES forces (every mode).
    const uint32_t mode = tuning && tuning->struct_size >= offsetof(turbo_backend_tuning, mode) + 4 ? tuning->mode
                                                                                                     : TURBO_AUTOTUNE_OFF;
    const bool tuned_mode = mode == TURBO_AUTOTUNE_ON || mode == TURBO_AUTOTUNE_RETUNE;
    if (const char *g = std::getenv("TURBO_ROCM_SPLIT"))
        s->split_parts = (uint32_t)std::min<long>(std::max<long>(std::strtol(g, nullptr, 10), 1), Session::MAX_PARTS);
    Choices &kc = s->kc;
    kc.bins = bins_for((uint64_t)desc->max_batch * desc->max_seq);
    // DeBERTa-v2's matrix-core form needs its relative projections in the
    // operand type: a model whose projections pass F16's range (or whose
    // buckets the form's tiles cannot hold) runs the scalar form, and its
    // choices say so.
    const bool mfma_attn = mfma_attention(s->act, m->hidden / m->heads) && !(m->deberta && !s->rel_pos_t);
    for (int b = 0; b < kc.bins; ++b) kc.bin[b].attn = mfma_attn ? ATTN_MFMA : ATTN_SIMPLE;
    split_defaults(*s);
    bool cached = false;
    if (tuned_mode && tuning->cached && *tuning->cached) {
        std::string why;
        Choices c = kc;
        // A cached choice of a block shape that cannot launch here is not taken.
        bool launchable = true;
        if (parse_choices(tuning->cached, &c, false, &why)) {
            for (int b = 0; b < c.bins; ++b)
                for (int g = 0; g < G_COUNT; ++g) {
                    if (gemm_made_to_fail(c.bin[b].tile[g])) {
                        launchable = false;
                        why = std::string(BIN_NAME[b]) + ":" + GEMM_NAME[g] + "=" + gemm_tile_name(c.bin[b].tile[g]) +
                              " cannot launch on this device";
                    } else if ((gemm_ln_tile(c.bin[b].tile[g]) && !ln_fusable(*s, g)) ||
                               (gemm_splitk_tile(c.bin[b].tile[g]) && !splitk_fits(*s, b, g))) {
                        launchable = false;
                        why = std::string(BIN_NAME[b]) + ":" + GEMM_NAME[g] + "=" + gemm_tile_name(c.bin[b].tile[g]) +
                              " does not take this product";
                    }
                }
        }
        if (launchable && why.empty()) {
            kc = c;
            cached = true;
            m->ctx->say(LOG_DEBUG, "rocm: kernels from the cache: " + std::string(tuning->cached));
        } else {
            m->ctx->say(LOG_DEBUG, "rocm: the cached kernels are not taken (" + why + "): " + tuning->cached);
        }
    }
    if (const char *env = std::getenv("TURBO_ROCM_CHOICES")) {
        std::string why;
        if (!parse_choices(env, &kc, true, &why))
            fail(TURBO_E_INVALID_ARGUMENT, "rocm: TURBO_ROCM_CHOICES " + std::string(env) + ": " + why);
    }
    // A forced block shape that cannot launch on this device refuses the
    // session (reference core/cuda/backend.cpp:3006-3010).
    for (int b = 0; b < kc.bins; ++b)
        for (int g = 0; g < G_COUNT; ++g)
            if (kc.bin[b].tile_forced[g] && gemm_made_to_fail(kc.bin[b].tile[g]))
                fail(TURBO_E_UNSUPPORTED, std::string("rocm: ") + BIN_NAME[b] + ":" + GEMM_NAME[g] + "=" +
                                              gemm_tile_name(kc.bin[b].tile[g]) +
                                              ": the GEMM kernel cannot launch on this device");
    // The whole-row shape carries the add + LayerNorm after an out or
    // FFN-out product of a session whose residual is in 16-bit rows: forced
    // on another product or session, it is refused.
    for (int b = 0; b < kc.bins; ++b)
        for (int g = 0; g < G_COUNT; ++g)
            if (gemm_ln_tile(kc.bin[b].tile[g]) && !ln_fusable(*s, g))
                fail(TURBO_E_UNSUPPORTED_OPTION, std::string("rocm: ") + BIN_NAME[b] + ":" + GEMM_NAME[g] + "=" +
                                                     gemm_tile_name(kc.bin[b].tile[g]) +
                                                     ": the LayerNorm-fused shape takes the out and FFN-out products "
                                                     "of F16 post-norm sessions of hidden 768 alone");
    for (int b = 0; b < kc.bins; ++b)
        for (int g = 0; g < G_COUNT; ++g)
            if (gemm_splitk_tile(kc.bin[b].tile[g]) && !splitk_fits(*s, b, g))
                fail(TURBO_E_UNSUPPORTED_OPTION, std::string("rocm: ") + BIN_NAME[b] + ":" + GEMM_NAME[g] + "=" +
                                                     gemm_tile_name(kc.bin[b].tile[g]) +
                                                     ": split K takes the out and FFN-out products of bins of at "
                                                     "most 4096 tokens whose runs do not split, off the int8 tier");
    // The scalar path is the only one some sessions have.
    for (int b = 0; b < kc.bins; ++b)
        if (!mfma_attn) kc.bin[b].attn = ATTN_SIMPLE;
    const bool measure = ((mode == TURBO_AUTOTUNE_ON && !cached) || mode == TURBO_AUTOTUNE_RETUNE) && !all_forced(kc);
    if (const char *g = std::getenv("TURBO_ROCM_GRAPHS")) s->graphs = std::strcmp(g, "0") != 0;

    const size_t H = m->hidden, I = m->inter, B = s->max_batch, S = s->max_seq;
    s->tcap = B * S;
    const size_t el = dt_bytes(s->act);
    OnDevice on(m->ctx->ordinal);
    auto alloc = [&](size_t bytes, const char *what) {
        s->owned.emplace_back(dev_alloc(bytes, what));
        return s->owned.back().get();
    };
    // Rows, the run's dimensions and the ranges in one allocation, in the
    // staging buffer's order: the ids, mask and types planes, then (on a
    // 64-byte boundary) the dimensions, the ranges right after them.
    // (Each plane starts on 16 bytes: the packing kernel reads a row's mask
    // 16 bytes a lane when the run's seq is a multiple of 4.)
    const size_t plane = plane_ints(*s);
    const size_t dims_at = (3 * plane + 15) / 16 * 16;
    s->staging_ints = dims_at + sizeof(RunDims) / 4 + 3 * (size_t)s->max_ranges;
    int32_t *rows = static_cast<int32_t *>(alloc(s->staging_ints * 4, "session rows"));
    s->ids = rows;
    s->mask = rows + plane;
    s->types = rows + 2 * plane;
    s->dims_dev = reinterpret_cast<RunDims *>(rows + dims_at);
    s->ranges = reinterpret_cast<uint32_t *>(s->dims_dev + 1);
    check(hipMemset(s->dims_dev, 0, sizeof(RunDims)), "session rows");
    s->row_lens.assign(B, 0);
    int32_t *pk = static_cast<int32_t *>(alloc((2 * B + 3 * s->tcap + 64) * 4, "session packing"));
    s->pk.start = pk;
    s->pk.len = pk + B;
    s->pk.at = pk + 2 * B;
    s->pk.row = pk + 2 * B + s->tcap;
    s->pk.pos = pk + 2 * B + 2 * s->tcap;
    s->pk.tokens = pk + 2 * B + 3 * s->tcap;
    s->x = static_cast<float *>(alloc(s->tcap * H * 4, "session states"));
    s->xh = alloc(s->tcap * H * 4, "session states");
    // Q, K and V, plus a 256-byte tail: the attention kernel's 16-byte loads
    // of V^T may run a few elements past a row. Zeroed once, so every value
    // it can read is finite.
    s->qkv = alloc(3 * s->tcap * H * el + 256, "session qkv");
    check(hipMemset(s->qkv, 0, 3 * s->tcap * H * el + 256), "session qkv");
    s->ctxb = alloc(s->tcap * H * el, "session context");
    s->ffn = alloc(s->tcap * I * el, "session ffn");
    // The out and FFN-out products go to y and are added to x by the
    // LayerNorm that follows: in the operand type on 16-bit post-norm
    // sessions (the reference's CUDA backend adds an F16 product,
    // core/cuda/kernels.cu:466-509; a BF16 product rounds at 2^-9 of itself,
    // and the sum and its norm stay F32); in BF16 on the 16-bit rotary
    // families, whose gated FFN sums can pass F16's 65504 (the reference
    // takes them in F32 for that, core/cuda/backend.cpp:2319-2324; BF16 has
    // F32's range at half its bytes); in F32 on the F32 tier. A rotary
    // family's y also holds a layer read's F32 final norm, so it keeps 4
    // bytes an element.
    s->ydt = s->act == Dt::F32 ? Dt::F32 : m->rotary ? Dt::BF16 : s->act;
    s->y = alloc(s->tcap * H * (m->rotary ? 4 : dt_bytes(s->ydt)), "session products");
    // Split K's slices: SPLITK_MAX of the small bins' largest out or FFN-out
    // product (rows x hidden F32).
    if (dt != Dt::I8) {
        s->splitk_floats = (size_t)SPLITK_MAX * std::min<size_t>(s->tcap, SPLITK_ROWS) * H;
        s->splitk_ws = static_cast<float *>(alloc(s->splitk_floats * 4, "session split-K slices"));
    }
    if (dt == Dt::I8) {
        s->aq = static_cast<int8_t *>(alloc(s->tcap * std::max(H, I), "session int8 operand"));
        s->ascale = static_cast<float *>(alloc(s->tcap * 4, "session int8 scales"));
    }
    const size_t outs = std::max<size_t>(B, s->max_ranges);
    s->out = static_cast<float *>(alloc(outs * H * 4, "session output"));
    s->pool_scratch.chunks = (int)((S + POOL_CHUNK - 1) / POOL_CHUNK);
    s->pool_scratch.part = static_cast<float *>(alloc(outs * s->pool_scratch.chunks * H * 4, "session pooling"));
    s->pool_scratch.cnt = static_cast<int32_t *>(alloc(outs * s->pool_scratch.chunks * 4, "session pooling"));
    s->output.ctx = m->ctx;
    s->output.placement = TURBO_PLACE_DEVICE;
    s->output.dev = s->out;
    s->output.bytes = outs * H * 4;
    s->output.owned = false;
    check(hipHostMalloc((void **)&s->staging, s->staging_ints * 4, hipHostMallocDefault), "session staging");
    counted_device_alloc();   // page-locked memory is the driver's
    s->dims_host = reinterpret_cast<RunDims *>(s->staging + dims_at);

    const auto t0 = std::chrono::steady_clock::now();
    std::string timings;
    bool measured = false;
    if (measure) {
        measured = tune(*s, tuning->budget_ms, &timings);
        // The tuner's products leave Q, K and V holding its values: zero
        // them again, so every value attention can read stays finite.
        check(hipMemsetAsync(s->qkv, 0, 3 * s->tcap * H * el + 256, m->ctx->stream), "session qkv");
        check(hipStreamSynchronize(m->ctx->stream), "session qkv");
    }
    s->choices = format_choices(kc);
    // Each bin's graph, with the bin's choices (after the tuner's timing).
    capture_graphs(*s);
    if (tuning) {
        const uint32_t k = forced_knobs(kc);
        tuning->tuned = all_forced(kc) ? TURBO_TUNED_FORCED
                        : measured     ? TURBO_TUNED_MEASURED
                        : cached       ? TURBO_TUNED_CACHE
                        : k            ? TURBO_TUNED_FORCED
                                       : TURBO_TUNED_DEFAULT;
        tuning->tune_ms = (uint32_t)std::chrono::duration_cast<std::chrono::milliseconds>(
                              std::chrono::steady_clock::now() - t0)
                              .count();
        std::snprintf(tuning->choices, sizeof tuning->choices, "%s", s->choices.c_str());
        if (tuning->timings && tuning->timings_len) {
            // What fits, cut at a line's end.
            std::string t = timings;
            if (t.size() + 1 > tuning->timings_len) {
                t.resize(tuning->timings_len - 1);
                const size_t nl = t.rfind('\n');
                t.resize(nl == std::string::npos ? 0 : nl + 1);
            }
            std::memcpy(tuning->timings, t.c_str(), t.size() + 1);
        }
        if (tuning->struct_size >= offsetof(turbo_backend_tuning, numerics_used) + 4)
            tuning->numerics_used = tuning->numerics_allowed;
    }
    return s.release();
}

void session_release(Session *s) {
    if (!s) return;
    {
        OnDevice on(s->ctx->ordinal);
        (void)hipStreamSynchronize(s->ctx->stream);
        if (s->staging) (void)hipHostFree(s->staging);
        for (hipGraphExec_t g : s->graph)
            if (g) (void)hipGraphExecDestroy(g);
        for (hipEvent_t e : s->ev) (void)hipEventDestroy(e);
        if (s->ev0) (void)hipEventDestroy(s->ev0);
        s->owned.clear();
    }
    delete s;
}

// Runs of more than this many packed tokens split their rows over the
// context's streams: the bins above it (le16k, gt16k) capture their graphs
// with parts, the ones at or below it without.
constexpr uint32_t SPLIT_MIN_TOKENS = 4096;

// The parts a bin's runs take at most.
static uint32_t parts_of_bin(const Session &s, int b) {
    const bool splits = b > 0 && (uint32_t)BIN_EDGE[b - 1] >= SPLIT_MIN_TOKENS;
    return splits && s.split_parts > 1 && s.max_batch >= 2 ? std::min(s.split_parts, s.max_batch) : 1;
}

// The rule's choice in a bin whose runs split into parts: the 256 x 384
// block shape on every product that can take it. The parts run the same
// kernels side by side, and shapes fastest alone lose there: a 256 x 384
// product at N = 768 fills half the compute units and the other part's the
// rest. Measured on MI355X, a batch with it on all four products against
// the shapes the tuner finds fastest alone: BERT-base 64 x 512 8.05 ms
// against 8.23-8.35, ModernBERT 16 x 2048-8192 45.4-45.6 ms against
// 45.4-46.6 (timing whole runs in the tuner could not tell them apart
// reliably: its short bursts run at clocks a sustained run does not).
static void split_defaults(Session &s) {
    const Model &m = *s.model;
    for (int b = 0; b < s.kc.bins; ++b) {
        if (parts_of_bin(s, b) < 2) continue;
        BinChoice &bc = s.kc.bin[b];
        for (int g = 0; g < G_COUNT; ++g) {
            if (bc.tile_forced[g] || gemm_made_to_fail(WIDE_TILE)) continue;
            EpiArgs e;
            e.kind = g == G_QKV ? Epi::Qkv : Epi::Bias;
            e.hidden = (int)m.hidden;
            const int K = g == G_FFN2 ? (int)m.inter : (int)m.hidden;
            int cand[16];
            const int n = gemm_candidates(s.dt, K, K, e, cand, 16);
            if (std::find(cand, cand + n, WIDE_TILE) != cand + n) bc.tile[g] = WIDE_TILE;
        }
    }
}

void session_write(Session *s, const turbo_backend_embed_rows *r, const turbo_token_range *ranges, uint32_t count) {
    if (r->batch == 0 || r->seq == 0) fail(TURBO_E_INVALID_SHAPE, "rocm: batch and seq may not be 0");
    if (r->batch > s->max_batch || r->seq > s->max_seq)
        fail(TURBO_E_CAPACITY, "rocm: " + std::to_string(r->batch) + " rows of " + std::to_string(r->seq) +
                                   " over the session's " + std::to_string(s->max_batch) + " of " +
                                   std::to_string(s->max_seq));
    // Layer reads (turbo_backend.h:423-435): ranges from each of the last
    // taps layers, or with tap_alone the first of them alone.
    const bool has_taps = r->struct_size >= offsetof(turbo_backend_embed_rows, tap_alone) + 4;
    const uint32_t taps = has_taps && r->taps > 1 ? r->taps : 1;
    const bool alone = has_taps && r->tap_alone != 0;
    if (has_taps && r->tap_alone > 1)
        fail(TURBO_E_INVALID_ARGUMENT, "rocm: tap_alone " + std::to_string(r->tap_alone) + " (0 or 1)", 10);
    if (taps > 1) {
        if (count == 0) fail(TURBO_E_INVALID_ARGUMENT, "rocm: layer reads pool ranges", 9);
        if (taps > s->model->layers)
            fail(TURBO_E_INVALID_ARGUMENT, "rocm: layers " + std::to_string(taps) + ": the model has 1 to " +
                                               std::to_string(s->model->layers) + " to read", 9);
        if (r->head) fail(TURBO_E_UNSUPPORTED_OPTION, "rocm: the span head reads the final layer", 9);
        if (!alone && (uint64_t)taps * count > s->max_ranges)
            fail(TURBO_E_CAPACITY, "rocm: " + std::to_string(count) + " ranges from " + std::to_string(taps) +
                                       " layers over max_ranges " + std::to_string(s->max_ranges));
    } else if (alone) {
        fail(TURBO_E_INVALID_ARGUMENT, "rocm: tap_alone with one layer read", 10);
    }
    // A headed write (turbo_backend.h:418-422): ranges on a model with a
    // span head, rows [count, head_out], normalize NONE.
    const bool head = r->struct_size >= offsetof(turbo_backend_embed_rows, head) + 4 && r->head;
    if (head) {
        if (!s->model->head_out) fail(TURBO_E_INVALID_ARGUMENT, "rocm: a head write to a model loaded without one");
        if (count == 0) fail(TURBO_E_INVALID_ARGUMENT, "rocm: a head write pools ranges");
        if (r->normalize != TURBO_NORMALIZE_NONE)
            fail(TURBO_E_UNSUPPORTED_OPTION, "rocm: the span head's logits are not normalized", 4);
        if (r->output_dim != s->model->head_out)
            fail(TURBO_E_UNSUPPORTED_OPTION, "rocm: output_dim " + std::to_string(r->output_dim) +
                                                 ": a head write's rows are the head's " +
                                                 std::to_string(s->model->head_out) + " logits", 6);
    } else if (r->output_dim == 0 || r->output_dim > s->model->hidden) {
        fail(TURBO_E_INVALID_ARGUMENT, "rocm: output_dim " + std::to_string(r->output_dim));
    }
    if (count > s->max_ranges) fail(TURBO_E_CAPACITY, "rocm: " + std::to_string(count) + " ranges over max_ranges");
    const uint32_t B = r->batch, S = r->seq, stride = r->row_stride ? r->row_stride : r->seq;
    if (stride < S) fail(TURBO_E_INVALID_SHAPE, "rocm: row_stride under seq");
    // Rows are packed with no stride, in the session's planes of B x S.
    std::lock_guard<std::recursive_mutex> g(s->ctx->lock);
    OnDevice on(s->ctx->ordinal);
    // The staging buffer may still feed the last write's copy.
    check(hipStreamSynchronize(s->ctx->stream), "embed_write");
    const size_t plane = plane_ints(*s);
    int32_t *ids = s->staging, *mask = ids + plane, *types = mask + plane;
    uint32_t *rg = reinterpret_cast<uint32_t *>(s->dims_host + 1);
    uint32_t tokens = 0, max_len = 0;
    uint32_t *lens = s->row_lens.data();   // each row's packed length (sized at session_open)
    const Model &m = *s->model;
    const int32_t ntypes = (int32_t)std::max(1u, m.types);
    for (uint32_t row = 0; row < B; ++row) {
        const size_t src = (size_t)row * stride, dst = (size_t)row * S;
        std::memcpy(ids + dst, r->ids + src, S * 4);
        std::memcpy(mask + dst, r->mask + src, S * 4);
        if (r->types) std::memcpy(types + dst, r->types + src, S * 4);
        else std::memset(types + dst, 0, S * 4);
        // The core has checked these; the device reads tables by them, so
        // they are held to their ranges here too.
        for (uint32_t p = 0; p < S; ++p)
            if (ids[dst + p] < 0 || (uint32_t)ids[dst + p] >= m.vocab || types[dst + p] < 0 ||
                types[dst + p] >= ntypes)
                fail(TURBO_E_INVALID_ARGUMENT, "rocm: row " + std::to_string(row) + " column " + std::to_string(p) +
                                                   ": an id or type outside the model's");
        uint32_t len = 0;
        for (uint32_t p = S; p > 0; --p)
            if (mask[dst + p - 1] != 0) {
                len = p;
                break;
            }
        if (len == 0) fail(TURBO_E_INVALID_ARGUMENT, "rocm: row " + std::to_string(row) + " has no live token");
        lens[row] = len;
        tokens += len;
        max_len = std::max(max_len, len);
    }
    for (uint32_t i = 0; i < count; ++i) {
        const turbo_token_range &g2 = ranges[i];
        if (g2.row >= B || g2.start >= g2.end || g2.end > S)
            fail(TURBO_E_INVALID_ARGUMENT, "rocm: ranges[" + std::to_string(i) + "]");
        rg[3 * i] = g2.row;
        rg[3 * i + 1] = g2.start;
        rg[3 * i + 2] = g2.end;
    }
    // Split the rows into parts of about equal packed tokens (rows in
    // order: part i ends at the first row where the tokens reach i + 1
    // parts' share), on runs of the bins that split; not when ranges are
    // read from layers before the last (each read pools every row). A run
    // takes its bin's parts (or one row a part when it has fewer rows), so
    // each part stays within a share of the bin plus one row: the bounds its
    // graph's grids were sized for.
    uint32_t parts = 1;
    if (B >= 2 && tokens > SPLIT_MIN_TOKENS && (alone || taps == 1)) parts = std::min(s->split_parts, B);
    parts = std::max(parts, 1u);
    uint32_t part_row[MAX_PARTS + 1], part_tok[MAX_PARTS + 1], part_len[MAX_PARTS];
    {
        uint32_t row = 0, t = 0;
        for (uint32_t i = 0; i < parts; ++i) {
            part_row[i] = row;
            part_tok[i] = t;
            part_len[i] = 0;
            const uint64_t share = (uint64_t)tokens * (i + 1) / parts;
            // At least one row a part, and one left for each part after it.
            do {
                part_len[i] = std::max(part_len[i], lens[row]);
                t += lens[row++];
            } while (row < B - (parts - 1 - i) && (i + 1 == parts || t < share));
        }
        part_row[parts] = row;
        part_tok[parts] = t;
    }
    // The run's dimensions, beside the ranges: what every kernel of the run
    // reads on the device. A part past the run's is empty.
    RunDims &d = *s->dims_host;
    std::memset(&d, 0, sizeof d);
    d.batch = (int32_t)B;
    d.seq = (int32_t)S;
    d.tokens = (int32_t)tokens;
    d.max_len = (int32_t)max_len;
    d.count = (int32_t)count;
    d.pooling = (int32_t)r->pooling;
    d.output_dim = (int32_t)r->output_dim;
    d.l2 = r->normalize == TURBO_NORMALIZE_L2 ? 1 : 0;
    d.head = head ? 1 : 0;
    for (uint32_t i = 0; i < MAX_PARTS; ++i) {
        PartDims &pd = d.part[i];
        if (i < parts) {
            pd.row0 = (int32_t)part_row[i];
            pd.rows = (int32_t)(part_row[i + 1] - part_row[i]);
            pd.tok0 = (int32_t)part_tok[i];
            pd.tokens = (int32_t)(part_tok[i + 1] - part_tok[i]);
            pd.max_len = (int32_t)part_len[i];
        } else {
            pd.row0 = (int32_t)B;
            pd.tok0 = (int32_t)tokens;
        }
    }
    // Planes are B*S long here but the device keeps them max_batch*max_seq
    // apart: three copies, then the dimensions and the ranges in one; rows
    // that fill the planes go in one copy with them (the staging buffer and
    // the device hold the same layout).
    const size_t n = (size_t)B * S * 4, tail = sizeof(RunDims) + (size_t)count * 12;
    if ((size_t)B * S == plane) {
        const size_t at = (size_t)(reinterpret_cast<char *>(s->dims_host) - reinterpret_cast<char *>(s->staging));
        check(hipMemcpyAsync(s->ids, s->staging, at + tail, hipMemcpyHostToDevice, s->ctx->stream), "embed_write");
    } else {
        check(hipMemcpyAsync(s->ids, ids, n, hipMemcpyHostToDevice, s->ctx->stream), "embed_write");
        check(hipMemcpyAsync(s->mask, mask, n, hipMemcpyHostToDevice, s->ctx->stream), "embed_write");
        check(hipMemcpyAsync(s->types, types, n, hipMemcpyHostToDevice, s->ctx->stream), "embed_write");
        check(hipMemcpyAsync(s->dims_dev, s->dims_host, tail, hipMemcpyHostToDevice, s->ctx->stream), "embed_write");
    }
    s->h2d = 3 * n + tail;
    s->batch = B;
    s->seq = S;
    s->pooling = r->pooling;
    s->normalize = r->normalize;
    s->output_dim = r->output_dim;
    s->head = head;
    s->taps = taps;
    s->tap_alone = alone;
    s->parts = parts;
    std::copy(part_row, part_row + parts + 1, s->part_row);
    std::copy(part_tok, part_tok + parts + 1, s->part_tok);
    std::copy(part_len, part_len + parts, s->part_len);
    s->count = count;
    s->tokens = tokens;
    s->max_len = max_len;
    s->has_types = r->types != nullptr;
    s->written = true;
}

// Records, when the session times its runs, an event on the first stream as
// the run starts and an event pair around each launch on the launch's own
// stream, so a launch's interval is measured as the run executes it (a split
// run's parts side by side).
// The pair of a launch is bound to its kernels' dispatch packets (the
// launch hook of the launchers): the start event to the first kernel's start,
// the stop event to the last kernel's end, so the timed run executes as an
// untimed one does, with no marker packet between its launches. A launch that
// enqueued no kernel gets a marker pair of no length.
LaunchTiming &launch_timing() {
    static thread_local LaunchTiming t;
    return t;
}

struct Timer {
    Session &s;
    explicit Timer(Session &ss) : s(ss) {
        s.ev_used = 0;
        if (s.timing && s.ev0) (void)hipEventRecord(s.ev0, s.ctx->stream);
    }
    ~Timer() { launch_timing() = LaunchTiming{}; }
    void begin(const char *name, hipStream_t st) {
        (void)st;
        if (!s.timing || s.ev_used + 2 > s.ev.size()) return;
        s.ev_name[s.ev_used / 2] = name;
        launch_timing() = LaunchTiming{s.ev[s.ev_used], s.ev[s.ev_used + 1], false};
    }
    void end(hipStream_t st) {
        if (!s.timing || s.ev_used + 2 > s.ev.size()) return;
        if (!launch_timing().bound) {
            (void)hipEventRecord(s.ev[s.ev_used], st);
            (void)hipEventRecord(s.ev[s.ev_used + 1], st);
        }
        launch_timing() = LaunchTiming{};
        s.ev_used += 2;
    }
};

// One of a layer's four products: its output columns N, inner size K,
// operand rows A, weights and epilogue, as the run launches it.
struct LayerGemm {
    int N = 0, K = 0;
    const void *A = nullptr, *W = nullptr;
    const float *wscale = nullptr;
    EpiArgs e;
};

// The operand the QKV and FFN-in products read: x itself on the F32 tier
// (post-norm), else the narrowed copy or the pre-norm rows in xh.
static const void *layer_input(const Session &s) {
    const Model &m = *s.model;
    return s.act == Dt::F32 && !m.modern ? (const void *)s.x : s.xh;
}

// Product g of layer l, its operand and outputs at the run's token 0 (a
// launch's span moves them to its own first token on the device).
static LayerGemm layer_gemm(Session &s, uint32_t l, GemmSlot g) {
    Model &m = *s.model;
    const Model::Layer &L = m.ls[l];
    const LayerWeights &W = (*s.w)[l];
    const int H = (int)m.hidden, I = (int)m.inter, dh = H / (int)m.heads;
    LayerGemm r;
    switch (g) {
    case G_QKV:
        r.N = (int)L.n_qkv;
        r.K = H;
        r.A = layer_input(s);
        r.W = W.qkv;
        r.wscale = W.s_qkv;
        r.e.bias = L.bqkv;
        r.e.out = s.qkv;
        r.e.tcap = (int)s.tcap;
        r.e.heads = (int)m.heads;
        r.e.d = dh;
        r.e.hidden = H;
        if (m.rotary) {
            const bool global = m.global_every == 0 || l % m.global_every == 0;
            const size_t half = (size_t)m.positions * m.pairs;
            r.e.kind = Epi::QkvRope;
            r.e.cos = m.rope + (global ? 0 : 2 * half);
            r.e.sin = r.e.cos + half;
            r.e.pos = s.pk.pos;
        } else {
            r.e.kind = Epi::Qkv;
        }
        break;
    case G_OUT:
    case G_FFN2:
        // The residual's product alone: the add + LayerNorm after it adds it to x.
        r.N = H;
        r.K = g == G_OUT ? H : I;
        r.A = g == G_OUT ? s.ctxb : s.ffn;
        r.W = g == G_OUT ? W.out : W.ffn_out;
        r.wscale = g == G_OUT ? W.s_out : W.s_ffn_out;
        r.e.kind = Epi::Bias;
        r.e.bias = g == G_OUT ? L.bo : L.b2;
        r.e.out = s.y;
        r.e.ldo = H;
        r.e.out_f32 = s.ydt == Dt::F32 ? 1 : 0;
        r.e.out_bf16 = s.ydt == Dt::BF16 && s.act == Dt::F16 ? 1 : 0;
        r.e.ws = s.splitk_ws;
        r.e.ws_floats = s.splitk_floats;
        break;
    default:
        r.N = (int)L.n_in;
        r.K = H;
        r.A = layer_input(s);
        r.W = W.ffn_in;
        r.wscale = W.s_ffn_in;
        r.e.out = s.ffn;
        r.e.ldo = I;
        r.e.bias = L.b1;
        r.e.kind = m.rotary ? Epi::Gated : Epi::Gelu;
        r.e.silu = m.silu ? 1 : 0;
        break;
    }
    return r;
}

// How large a run's launches are: every grid covers the largest run of the
// bin (whose kernel choices they take), so the launches of a bin are the same
// whether captured into its graph or launched directly, and give the same
// bits. A part's tokens are at most a share of the bin's plus one row (its
// last row crosses the share) plus one (the share's rounding).
struct Bounds {
    int bin = 0;
    uint32_t tokens = 0, rows = 0, max_len = 0, parts = 1, part_tokens = 0, items = 0;
};

static Bounds bounds_of(const Session &s, int b, uint32_t parts) {
    Bounds o;
    o.bin = b;
    o.tokens = bin_tokens(b, s.tcap);
    o.rows = std::min<uint32_t>(s.max_batch, o.tokens);
    o.max_len = std::min<uint32_t>(s.max_seq, o.tokens);
    o.parts = std::max(parts, 1u);
    const uint32_t bp = o.parts;
    o.part_tokens = bp == 1 ? o.tokens : std::min(o.tokens, (o.tokens + bp - 1) / bp + 1 + o.max_len);
    o.items = std::max(o.rows, s.max_ranges);
    return o;
}

// Post-norm F16 sessions carry the residual stream between a layer's norms
// in the 16-bit GEMM operand rows (xh) alone: each add + LayerNorm reads 2
// bytes of residual and writes 2 an element, where F32 rows would take 4
// and 4 more (the products read the 16-bit rows either way; the sum x + y
// is now taken from them too). The F32 rows are written where they are
// read: after the last layer, and after a layer whose ranges are read.
// BF16 keeps F32 rows (8 bits of mantissa would carry the residual too
// coarsely), as do pre-norm models, whose residual no norm bounds.
static bool residual_in_operand(const Session &s) { return s.act == Dt::F16 && !s.model->modern; }

// Whether product g (out or FFN-out) can take its residual add and
// LayerNorm in its epilogue (the whole-row shapes): post-norm F16
// sessions carrying the residual in the 16-bit rows, at a hidden size the
// kernel is built for.
static bool ln_fusable(const Session &s, int g) {
    const Model &m = *s.model;
    if (g != G_OUT && g != G_FFN2) return false;
    const int K = g == G_OUT ? (int)m.hidden : (int)m.inter;
    return s.dt == Dt::F16 && residual_in_operand(s) && gemm_ln_takes(s.dt, (int)m.hidden, K, K, true);
}

// The layers over part `part` of the run's rows, on stream st: every
// product, norm and attention launch reads that part's rows and tokens from
// the run's dimensions. Layer reads pool their ranges as they pass.
// The layers a run takes: every one, or through the one read alone (a
// model cut after it); the tuner's runs the first few alone.
static uint32_t layers_of_run(const Session &s) {
    const Model &m = *s.model;
    uint32_t nl = s.tap_alone ? m.layers + 1 - s.taps : m.layers;
    if (s.layers_limit) nl = std::min(nl, s.layers_limit);
    return nl;
}

static void run_layers(Session &s, hipStream_t st, int part, const Bounds &bd, Timer &tm, uint32_t l0, uint32_t l1) {
    Model &m = *s.model;
    const int H = (int)m.hidden, I = (int)m.inter, heads = (int)m.heads, dh = H / heads;
    const Dt dt = s.act;   // activations; the GEMMs take s.dt
    const bool f32 = dt == Dt::F32, i8 = s.dt == Dt::I8;
    const BinChoice &bc = s.kc.bin[bd.bin];
    const Span sp = span_of(s.dims_dev, part), whole = span_of(s.dims_dev, -1);
    const int T = (int)bd.part_tokens;   // the grids' rows
    auto run = [&](const char *name, hipError_t e) { check(e, name); };
#define LAUNCH(NAME, CALL)  \
    do {                    \
        tm.begin(NAME, st); \
        run(NAME, CALL);    \
        tm.end(st);         \
    } while (0)
    // One GEMM of the layer. On the I8 tier its operand rows are quantized
    // first (per token; each part's rows at its own tokens of the operand
    // buffer, whose rows are max(H, I) wide), and the epilogue takes both scales.
    static const char *const NAMES[G_COUNT] = {"gemm_qkv", "gemm_out", "gemm_ffn_in", "gemm_ffn_out"};
    // On the I8 tier the LayerNorms that make the QKV and FFN-in operands
    // write their int8 rows too (the codes quantize_rows would make of their
    // 16-bit output); the product that follows then skips its quantize.
    const int qrow = std::max(H, I);
    QuantOut qo;
    if (i8) {
        qo.q = s.aq;
        qo.scale = s.ascale;
        qo.tok_stride = qrow;
    }
    // (The int8 rows of a layer's first operand are the previous layer's
    // last norm's.)
    bool aq_ready = i8 && l0 > 0;
    auto mm = [&](uint32_t l, GemmSlot g) {
        LayerGemm lg = layer_gemm(s, l, g);
        const void *A = lg.A;
        int a_tok = 0;
        if (i8) {
            if (!(aq_ready && (g == G_QKV || g == G_FFN1)))
                LAUNCH("quantize", quantize_span(st, sp, T, A, Dt::F16, lg.K, lg.K, s.aq, qrow, s.ascale));
            aq_ready = false;
            lg.e.a_scale = s.ascale;
            lg.e.w_scale = lg.wscale;
            A = s.aq;
            a_tok = qrow;
        }
        LAUNCH(NAMES[g], gemm(st, s.dt, sp, T, lg.N, lg.K, A, lg.K, a_tok, lg.W, lg.e, bc.tile[g]));
    };
    // The out or FFN-out product of layer l with its residual add and the
    // norm (w, b) in its epilogue, when the bin's choice for it is the
    // whole-row shape: whether it ran so. (F16 post-norm sessions alone,
    // whose residual is carried in xh; no int8 rows follow.)
    auto mm_ln = [&](uint32_t l, GemmSlot g, const float *w, const float *b, bool keep_f32) {
        if (!gemm_ln_tile(bc.tile[g]) || !ln_fusable(s, g)) return false;
        const LayerGemm lg = layer_gemm(s, l, g);
        LnArgs ln;
        ln.bias = lg.e.bias;
        ln.x = s.x;
        ln.out_h = s.xh;
        ln.ln_w = w;
        ln.ln_b = b;
        ln.eps = m.eps;
        ln.res_h = 1;
        ln.keep_f32 = keep_f32 ? 1 : 0;
        LAUNCH(g == G_OUT ? "gemm_out_ln" : "gemm_ffn_out_ln",
               gemm_ln(st, s.dt, sp, T, H, lg.K, lg.A, lg.K, 0, lg.W, ln, bc.tile[g]));
        return true;
    };
    // The GEMM operand copy of x after an add + LayerNorm: xh, or on the F32
    // tier x itself (post-norm) or xh as F32 (pre-norm).
    void *norm_out = f32 && !m.modern ? nullptr : s.xh;
    const bool res_h = residual_in_operand(s);
    // Layers run: every one, or through the one read alone (a model cut
    // after it). Ranges are pooled after each of the last `reads` layers run
    // into block k of the output, [reads, count, output_dim], the final
    // layer's last (reference core/src/cpu/encoder/mod.rs:292-373); a run
    // with reads before the last is never split. A ModernBERT read is
    // final_norm(x), the scale the final states are on
    // (core/src/cpu/encoder/rotary/mod.rs:84-86, 161-168), normed into y,
    // which is free between a layer's last add and the next layer's out product.
    const uint32_t nl = layers_of_run(s);
    const uint32_t reads = s.tap_alone ? 1 : s.taps;
    const int od = (int)s.output_dim;
    for (uint32_t l = l0; l < std::min(l1, nl); ++l) {
        const Model::Layer &L = m.ls[l];
        int window = INT32_MAX;
        if (m.rotary) {
            const bool global = m.global_every == 0 || l % m.global_every == 0;
            if (!global) window = (int)m.window;
        }
        mm(l, G_QKV);
        if (m.deberta)
            LAUNCH("attention", deberta_attention(st, dt, s.qkv, (int)s.tcap, heads, dh, s.pk, s.mask, sp,
                                                  (int)bd.rows, (int)bd.max_len, L.pos_qk,
                                                  static_cast<const int32_t *>(m.rel_table.get()), (int)m.positions,
                                                  s.rel_pos_t && bc.attn != ATTN_SIMPLE
                                                      ? static_cast<const char *>(s.rel_pos_t) +
                                                            (size_t)l * m.rel_rows * 2 * H * dt_bytes(dt)
                                                      : nullptr,
                                                  s.ctxb));
        else
            LAUNCH("attention", attention(st, dt, s.qkv, (int)s.tcap, heads, dh, s.pk, s.mask, sp, (int)bd.rows,
                                          (int)bd.max_len, window, s.ctxb, bc.attn));
        // Post-norm: x = LN1(x + y), in the product's epilogue on the
        // whole-row shape. Pre-norm: x += y, xh = LN_mlp(x).
        if (!mm_ln(l, G_OUT, L.ln1_w, L.ln1_b, !res_h)) {
            mm(l, G_OUT);
            if (m.modern)
                LAUNCH("add_layer_norm",
                       add_layer_norm(st, sp, T, H, s.x, s.y, s.ydt, L.ln2_w, nullptr, m.eps, 1, norm_out, dt, qo));
            else
                LAUNCH("add_layer_norm", add_layer_norm(st, sp, T, H, s.x, s.y, s.ydt, L.ln1_w, L.ln1_b, m.eps, 0,
                                                        norm_out, dt, qo, res_h, !res_h));
        }
        aq_ready = i8;
        mm(l, G_FFN1);
        // Post-norm: x = LN2(x + y). Pre-norm: x += y and the next layer's
        // attention norm into xh, or after the last layer x = LN_final(x + y).
        const QuantOut next = l + 1 < nl ? qo : QuantOut();
        // A 16-bit residual writes the F32 rows where they are read: after
        // the last layer, and after a layer whose ranges are read.
        const bool keep_f32 = !res_h || l + 1 == nl || (reads > 1 && l + reads >= nl);
        if (!mm_ln(l, G_FFN2, L.ln2_w, L.ln2_b, keep_f32)) {
            mm(l, G_FFN2);
            if (!m.modern)
                LAUNCH("add_layer_norm", add_layer_norm(st, sp, T, H, s.x, s.y, s.ydt, L.ln2_w, L.ln2_b, m.eps, 0,
                                                        norm_out, dt, next, res_h, keep_f32));
            else if (l + 1 < nl)
                LAUNCH("add_layer_norm", add_layer_norm(st, sp, T, H, s.x, s.y, s.ydt, m.ls[l + 1].ln1_w, nullptr,
                                                        m.eps, 1, norm_out, dt, next));
            else
                LAUNCH("add_layer_norm",
                       add_layer_norm(st, sp, T, H, s.x, s.y, s.ydt, m.final_w, nullptr, m.eps, 0, nullptr, dt));
        }
        aq_ready = i8 && l + 1 < nl;
        if (reads > 1 && l + 1 < nl && l + reads >= nl) {
            const float *src = s.x;
            if (m.modern) {
                LAUNCH("layer_norm", layer_norm(st, whole, (int)bd.tokens, H, s.x, m.final_w, nullptr, m.eps,
                                                (float *)s.y, nullptr, Dt::F32));
                src = (const float *)s.y;
            }
            float *block = s.out + (size_t)(l + reads - nl) * s.count * od;
            LAUNCH("pool", pool(st, s.dims_dev, (int)bd.items, src, H, s.pk, s.mask, s.ranges, s.pool_scratch, block));
        }
    }
#undef LAUNCH
}

// A run's launches on the context's streams: the whole run's embedding,
// each part's layers (forked onto the side streams and joined back), the
// pooling.
static void encode(Session &s, const Bounds &bd) {
    Model &m = *s.model;
    Context &c = *s.ctx;
    hipStream_t st = c.stream;
    const int H = (int)m.hidden;
    const Dt dt = s.act;
    const bool f32 = dt == Dt::F32;
    const Span whole = span_of(s.dims_dev, -1);
    Timer tm(s);
    auto run = [&](const char *name, hipError_t e) { check(e, name); };
#define LAUNCH(NAME, CALL)  \
    do {                    \
        tm.begin(NAME, st); \
        run(NAME, CALL);    \
        tm.end(st);         \
    } while (0)
    LAUNCH("pack_rows", pack_rows(st, s.mask, s.dims_dev, (int)s.max_batch, (int)s.max_seq, s.pk));
    // (A 16-bit residual starts in xh alone.)
    LAUNCH("embed_ln", embed_ln(st, whole, (int)bd.tokens, H, s.ids, s.types, s.pk, (int)m.position_offset, m.word,
                                m.pos, m.type, m.emb_w, m.emb_b, m.eps, residual_in_operand(s) ? nullptr : s.x,
                                f32 ? nullptr : s.xh, dt,
                                m.deberta ? s.mask : nullptr));
    // ModernBERT's first layer reads the embeddings' rows as they are (no
    // attention norm); on the F32 tier xh is the pre-norm rows' F32 copy.
    if (m.modern && f32) LAUNCH("copy", copy_rows(st, whole, (int)bd.tokens, s.x, s.xh, (size_t)H * 4));
    // A split run: the rows' parts run their layers on the context's
    // streams, forked here and joined before the pooling, so one part's
    // memory-bound and latency-bound launches overlap another's products.
    // (Launched directly, the parts' layers go out in turn, a layer of each
    // part at a time, so every stream has work from the start.)
    const uint32_t nl = layers_of_run(s);
    if (bd.parts > 1) {
        check(hipEventRecord(c.fork, st), "forking the run");
        for (uint32_t i = 1; i < bd.parts; ++i) check(hipStreamWaitEvent(c.side[i - 1], c.fork, 0), "forking the run");
        for (uint32_t l = 0; l < nl; ++l)
            for (uint32_t i = 0; i < bd.parts; ++i) run_layers(s, i == 0 ? st : c.side[i - 1], (int)i, bd, tm, l, l + 1);
        for (uint32_t i = 1; i < bd.parts; ++i) {
            check(hipEventRecord(c.join[i - 1], c.side[i - 1]), "joining the run");
            check(hipStreamWaitEvent(st, c.join[i - 1], 0), "joining the run");
        }
    } else {
        run_layers(s, st, 0, bd, tm, 0, nl);
    }
    const uint32_t reads = s.tap_alone ? 1 : s.taps;
    LAUNCH("pool", pool(st, s.dims_dev, (int)bd.items, s.x, H, s.pk, s.mask, s.ranges, s.pool_scratch,
                        s.out + (size_t)(reads - 1) * s.count * s.output_dim, m.head_w, m.head_b, (int)m.head_out));
#undef LAUNCH
}

// Captures bin b's graph: its launches with the bin's bounds and choices,
// forked over the parts its runs may take.
static void capture_bin(Session &s, int b) {
    hipStream_t st = s.ctx->stream;
    s.bin_parts[b] = parts_of_bin(s, b);
    // Capture sees no rows: the run's options that change which kernels
    // launch (layer reads) take no graph, so the capture is a plain run's.
    const uint32_t taps = s.taps, count = s.count, od = s.output_dim;
    const bool alone = s.tap_alone;
    s.taps = 1;
    s.tap_alone = false;
    s.count = 0;
    s.output_dim = s.model->hidden;
    struct Restore {
        Session &s;
        uint32_t taps, count, od;
        bool alone;
        ~Restore() {
            s.taps = taps;
            s.tap_alone = alone;
            s.count = count;
            s.output_dim = od;
        }
    } restore{s, taps, count, od, alone};
    check(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capturing a bin's graph");
    hipGraph_t g = nullptr;
    try {
        encode(s, bounds_of(s, b, s.bin_parts[b]));
    } catch (...) {
        (void)hipStreamEndCapture(st, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    check(hipStreamEndCapture(st, &g), "capturing a bin's graph");
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    check(e, "instantiating a bin's graph");
    s.graph[b] = exec;
    ++s.captures;
}

void capture_graphs(Session &s) {
    if (!s.graphs) return;
    for (int b = 0; b < s.kc.bins; ++b) capture_bin(s, b);
}

void launch_run(Session &s) {
    const int b = bin_of(s.tokens, s.kc.bins);
    if (s.graphs && !s.timing && s.taps == 1 && !s.tap_alone && s.graph[b]) {
        // The written parts fit the bin's graph by the split rule; checked
        // anyway (a graph past its bounds would drop tokens), and a run that
        // did not fit would launch its kernels directly.
        const Bounds gb = bounds_of(s, b, s.bin_parts[b]);
        bool fits = s.parts <= gb.parts;
        for (uint32_t i = 0; i < s.parts; ++i)
            fits = fits && s.part_tok[i + 1] - s.part_tok[i] <= gb.part_tokens && s.part_len[i] <= gb.max_len &&
                   s.part_row[i + 1] - s.part_row[i] <= gb.rows;
        if (fits) {
            check(hipGraphLaunch(s.graph[b], s.ctx->stream), "launching the run's graph");
            ++s.graph_launches;
            return;
        }
    }
    encode(s, bounds_of(s, b, s.parts));
}

// Rows for the tuner's runs of bin b: the bin's token count (its upper edge,
// or the session's capacity) as rows of max_seq tokens, the last one
// shorter, ids spread over the vocabulary, types 0, one vector a row.
static void write_tuner_rows(Session &s, int b) {
    const Model &m = *s.model;
    const uint32_t T = bin_tokens(b, s.tcap), S = s.max_seq;
    const uint32_t rows = std::min<uint32_t>(s.max_batch, (T + S - 1) / S);
    std::vector<int32_t> ids((size_t)rows * S), mask((size_t)rows * S, 0);
    for (size_t i = 0; i < ids.size(); ++i) ids[i] = (int32_t)((i * 7919 + 1000) % m.vocab);
    for (uint32_t r = 0; r < rows; ++r) {
        const uint32_t len = std::min(S, T - std::min(T, r * S));
        for (uint32_t p = 0; p < std::max(len, 1u); ++p) mask[(size_t)r * S + p] = 1;
    }
    turbo_backend_embed_rows d{};
    d.struct_size = sizeof d;
    d.batch = rows;
    d.seq = S;
    d.ids = ids.data();
    d.mask = mask.data();
    d.pooling = TURBO_POOLING_CLS;
    d.normalize = TURBO_NORMALIZE_NONE;
    d.output_dim = m.hidden;
    session_write(&s, &d, nullptr, 0);
}

// Bin b's run through its first `layers` layers with the bin's current
// choices, captured as a graph (its parts forked as a run's are) and
// replayed back to back for about target_ms: milliseconds a replay.
static float time_layers(Session &s, int b, uint32_t layers, float target_ms, hipEvent_t e0, hipEvent_t e1) {
    hipStream_t st = s.ctx->stream;
    s.layers_limit = layers;
    struct Reset {
        Session &s;
        ~Reset() { s.layers_limit = 0; }
    } reset{s};
    check(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "the tuner's graph");
    hipGraph_t g = nullptr;
    try {
        encode(s, bounds_of(s, b, parts_of_bin(s, b)));
    } catch (...) {
        (void)hipStreamEndCapture(st, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    check(hipStreamEndCapture(st, &g), "the tuner's graph");
    hipGraphExec_t exec = nullptr;
    const hipError_t ie = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    check(ie, "the tuner's graph");
    struct Drop {
        hipGraphExec_t e;
        ~Drop() { (void)hipGraphExecDestroy(e); }
    } drop{exec};
    // Two replays to warm up, timed for the count that fills target_ms.
    check(hipEventRecord(e0, st), "the tuner's events");
    for (int i = 0; i < 2; ++i) check(hipGraphLaunch(exec, st), "the tuner's run");
    check(hipEventRecord(e1, st), "the tuner's events");
    check(hipEventSynchronize(e1), "the tuner's run");
    float ms = 0;
    check(hipEventElapsedTime(&ms, e0, e1), "the tuner's events");
    const int n = std::min(64, std::max(4, (int)(target_ms / std::max(ms / 2, 1e-3f))));
    check(hipEventRecord(e0, st), "the tuner's events");
    for (int i = 0; i < n; ++i) check(hipGraphLaunch(exec, st), "the tuner's run");
    check(hipEventRecord(e1, st), "the tuner's events");
    check(hipEventSynchronize(e1), "the tuner's run");
    check(hipEventElapsedTime(&ms, e0, e1), "the tuner's events");
    return ms / n;
}

// The tuner (the counterpart of the reference's, core/cuda/backend.cpp:
// 2419-2880, core/cuda/autotune.h:21-41): for each bin, largest first, the
// knobs in turn -- each product's block shape (with, for the out and FFN-out
// products of a session that can fuse it, the whole-row shape carrying the
// add + LayerNorm) and the attention path -- each candidate timed as the
// bin's run through its first layer (the first global and local layers of a
// windowed model) on rows of the bin's token count, as the run launches it:
// split into its parts on the context's streams, captured and replayed back
// to back for a few milliseconds (sustained: short bursts run at clocks a
// sustained run does not). The incumbent (the rule's choice, or the cached
// one) is timed again at each knob; a candidate replaces it when it is 2%
// faster. Forced knobs and shapes that cannot launch are not timed. Lines
// <bin>/<knob>/<variant>=<ms a layer's run>. Stops at the budget. Returns
// whether anything was timed.
bool tune(Session &s, uint32_t budget_ms, std::string *timings) {
    using Clock = std::chrono::steady_clock;
    const Clock::time_point deadline = Clock::now() + std::chrono::milliseconds(budget_ms);
    constexpr float MARGIN = 0.98f;
    Model &m = *s.model;
    const uint32_t layers = m.window && m.global_every > 1 ? std::min(m.layers, m.global_every) : 1;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    check(hipEventCreate(&e0), "the tuner's events");
    struct Events {
        hipEvent_t a, b;
        ~Events() {
            if (a) (void)hipEventDestroy(a);
            if (b) (void)hipEventDestroy(b);
        }
    } guard{e0, nullptr};
    check(hipEventCreate(&e1), "the tuner's events");
    guard.b = e1;
    const bool mfma_attn = mfma_attention(s.act, m.hidden / m.heads);
    bool any = false;
    char line[160];
    for (int b = s.kc.bins - 1; b >= 0 && Clock::now() < deadline; --b) {
        const uint32_t P = parts_of_bin(s, b);
        write_tuner_rows(s, b);
        const float target = P > 1 ? 6.0f : 2.0f;
        BinChoice &bc = s.kc.bin[b];
        auto timed = [&](const char *knob, const char *variant) {
            const float ms = time_layers(s, b, layers, target, e0, e1);
            std::snprintf(line, sizeof line, "%s/%s/%s=%.4f\n", BIN_NAME[b], knob, variant, ms);
            *timings += line;
            any = true;
            return ms;
        };
        // The clock settles under the bin's load before the first timing.
        (void)time_layers(s, b, layers, 10.0f, e0, e1);
        for (int g = 0; g < G_COUNT && Clock::now() < deadline; ++g) {
            if (bc.tile_forced[g]) continue;
            const LayerGemm lg = layer_gemm(s, 0, (GemmSlot)g);
            int cand[20];
            int n = gemm_candidates(s.dt, lg.K, lg.K, lg.e, cand, 16);   // (room for 3 more below)
            // Split bins: the large shapes alone (each part's product fills
            // about half the chip beside the other part's).
            if (P > 1) {
                int k = 0;
                for (int i = 0; i < n; ++i)
                    if (cand[i] == WIDE_TILE || cand[i] == 7 || cand[i] == 13 || cand[i] == 16) cand[k++] = cand[i];
                n = k;
            }
            if (ln_fusable(s, g)) cand[n++] = LN_TILE;
            if (splitk_fits(s, b, g)) {
                cand[n++] = SPLITK_TILE_4;
                cand[n++] = SPLITK_TILE_2;
            }
            const int incumbent = bc.tile[g];
            float best = timed(GEMM_NAME[g], gemm_tile_name(incumbent));
            int pick = incumbent;
            const float bar = best;
            for (int i = 0; i < n && Clock::now() < deadline; ++i) {
                if (cand[i] == incumbent || gemm_made_to_fail(cand[i])) continue;
                bc.tile[g] = cand[i];
                float ms = 0;
                try {
                    ms = timed(GEMM_NAME[g], gemm_tile_name(cand[i]));
                } catch (...) {
                    bc.tile[g] = incumbent;
                    throw;
                }
                bc.tile[g] = incumbent;
                if (ms < best) {
                    best = ms;
                    pick = cand[i];
                }
            }
            if (pick != incumbent && best <= MARGIN * bar) bc.tile[g] = pick;
        }
        if (mfma_attn && !bc.attn_forced && !m.deberta && Clock::now() < deadline) {
            const int incumbent = bc.attn;
            const float bar = timed("attn", ATTN_NAME[incumbent]);
            const int other = incumbent == ATTN_MFMA ? ATTN_MFMA128 : ATTN_MFMA;
            bc.attn = other;
            float ms = 0;
            try {
                ms = timed("attn", ATTN_NAME[other]);
            } catch (...) {
                bc.attn = incumbent;
                throw;
            }
            bc.attn = ms <= MARGIN * bar ? other : incumbent;
        }
    }
    s.written = false;
    s.ctx->say(LOG_DEBUG, "rocm: tuned kernels: " + format_choices(s.kc));
    return any;
}

void session_run(Session *s, turbo_backend_run *out) {
    if (!s->written) fail(TURBO_E_INVALID_STATE, "rocm: the session has no rows written since its last run");
    s->written = false;
    const uint64_t dev0 = device_allocs_on_thread(), host0 = host_allocs_on_thread();
    {
        std::lock_guard<std::recursive_mutex> g(s->ctx->lock);
        OnDevice on(s->ctx->ordinal);
        try {
            launch_run(*s);
        } catch (...) {
            (void)hipStreamSynchronize(s->ctx->stream);
            throw;
        }
        check(hipStreamSynchronize(s->ctx->stream), "the run");
    }
    const uint32_t n_out = s->count ? s->count * (s->tap_alone ? 1 : s->taps) : s->batch;
    s->output.bytes = (uint64_t)n_out * s->output_dim * 4;
    out->placement = TURBO_PLACE_DEVICE;
    out->output = &s->output;
    out->host = nullptr;
    out->h2d_bytes = s->h2d;
    out->d2h_bytes = 0;
    out->host_allocs = host_allocs_on_thread() - host0;
    out->device_allocs = device_allocs_on_thread() - dev0;
    uint32_t *st = out->stage;
    st[TURBO_EMBED_STAGE_UPLOAD] = TURBO_STAGE_DEVICE;
    st[TURBO_EMBED_STAGE_LOOKUP] = TURBO_STAGE_DEVICE;
    st[TURBO_EMBED_STAGE_ENCODE] = TURBO_STAGE_DEVICE;
    st[TURBO_EMBED_STAGE_POOL] = TURBO_STAGE_DEVICE;
    st[TURBO_EMBED_STAGE_NORMALIZE] = s->normalize == TURBO_NORMALIZE_L2 ? TURBO_STAGE_FUSED : TURBO_STAGE_UNUSED;
    st[TURBO_EMBED_STAGE_DOWNLOAD] = TURBO_STAGE_UNUSED;
}

}  // namespace rocm

// ---- Test and measurement hooks ----------------------------------------------------------

using namespace rocm;

extern "C" {

int32_t turbo_rocm_host_allocs(uint64_t *process, uint64_t *thread, turbo_error *err) {
    return guarded(err, [&] {
        if (process) *process = host_allocs.load();
        if (thread) *thread = host_allocs_on_thread();
        return TURBO_OK;
    });
}

int32_t turbo_rocm_fail_variant(const char *name, turbo_error *err) {
    return guarded(err, [&] {
        if (!gemm_fail_variant(name))
            fail(TURBO_E_INVALID_ARGUMENT, std::string("rocm: '") + name + "' names no GEMM block shape");
        return TURBO_OK;
    });
}

int32_t turbo_rocm_session_packing(void *session, int32_t *start, int32_t *len, int32_t *at, uint32_t *tokens,
                                   turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        std::lock_guard<std::recursive_mutex> g(s->ctx->lock);
        OnDevice on(s->ctx->ordinal);
        int32_t t = 0;
        check(hipMemcpy(&t, s->pk.tokens, 4, hipMemcpyDeviceToHost), "packing");
        check(hipMemcpy(start, s->pk.start, (size_t)s->batch * 4, hipMemcpyDeviceToHost), "packing");
        check(hipMemcpy(len, s->pk.len, (size_t)s->batch * 4, hipMemcpyDeviceToHost), "packing");
        check(hipMemcpy(at, s->pk.at, (size_t)t * 4, hipMemcpyDeviceToHost), "packing");
        *tokens = (uint32_t)t;
        return TURBO_OK;
    });
}

int32_t turbo_rocm_session_hidden(void *session, float *out, uint64_t floats, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        const uint64_t n = (uint64_t)s->tokens * s->model->hidden;
        if (floats < n) fail(TURBO_E_INVALID_ARGUMENT, "rocm: the hidden states need " + std::to_string(n) + " floats");
        std::lock_guard<std::recursive_mutex> g(s->ctx->lock);
        OnDevice on(s->ctx->ordinal);
        check(hipMemcpy(out, s->x, n * 4, hipMemcpyDeviceToHost), "hidden states");
        return TURBO_OK;
    });
}

int32_t turbo_rocm_session_timing(void *session, uint32_t on_, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        OnDevice on(s->ctx->ordinal);
        if (on_ && s->ev.empty()) {
            s->ev.resize(2 * (16 + 16 * s->model->layers * Session::MAX_PARTS));
            for (auto &e : s->ev) check(hipEventCreate(&e), "hipEventCreate");
            s->ev_name.assign(s->ev.size() / 2, nullptr);
            check(hipEventCreate(&s->ev0), "hipEventCreate");
        }
        s->timing = on_ != 0;
        return TURBO_OK;
    });
}

int32_t turbo_rocm_session_times(void *session, char *out, uint32_t len, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        // The last timed run's events (it has synchronized), summed by
        // kernel name in first-launch order.
        std::vector<std::string> order;
        std::map<std::string, std::pair<double, uint32_t>> by;
        OnDevice on(s->ctx->ordinal);
        for (size_t i = 0; s->timing && i + 1 < s->ev_used; i += 2) {
            float ms = 0;
            (void)hipEventElapsedTime(&ms, s->ev[i], s->ev[i + 1]);
            const std::string n = s->ev_name[i / 2];
            if (!by.count(n)) order.push_back(n);
            by[n].first += ms;
            by[n].second += 1;
        }
        std::string t;
        for (auto &n : order) {
            char line[128];
            std::snprintf(line, sizeof line, "%s %.6f %u\n", n.c_str(), by[n].first, by[n].second);
            t += line;
        }
        if (len) std::snprintf(out, len, "%s", t.c_str());
        return TURBO_OK;
    });
}

int32_t turbo_rocm_session_intervals(void *session, char *out, uint32_t len, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        // The last timed run's launches in the order they were made: name,
        // then start and end in ms from the run's start.
        std::string t;
        OnDevice on(s->ctx->ordinal);
        for (size_t i = 0; s->timing && s->ev0 && i + 1 < s->ev_used; i += 2) {
            float a = 0, b = 0;
            check(hipEventElapsedTime(&a, s->ev0, s->ev[i]), "the run's events");
            check(hipEventElapsedTime(&b, s->ev0, s->ev[i + 1]), "the run's events");
            char line[128];
            std::snprintf(line, sizeof line, "%s %.6f %.6f\n", s->ev_name[i / 2], a, b);
            t += line;
        }
        if (len) std::snprintf(out, len, "%s", t.c_str());
        return TURBO_OK;
    });
}

int32_t turbo_rocm_session_replay(void *session, uint32_t runs, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        if (s->tokens == 0) fail(TURBO_E_INVALID_STATE, "rocm: the session has no rows written");
        std::lock_guard<std::recursive_mutex> g(s->ctx->lock);
        OnDevice on(s->ctx->ordinal);
        for (uint32_t i = 0; i < runs; ++i) launch_run(*s);
        check(hipStreamSynchronize(s->ctx->stream), "replay");
        return TURBO_OK;
    });
}

int32_t turbo_rocm_session_graphs(void *session, uint64_t *captured, uint64_t *launched, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        *captured = s->captures;
        *launched = s->graph_launches;
        return TURBO_OK;
    });
}

int32_t turbo_rocm_session_choices(void *session, char *out, uint32_t len, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = static_cast<Session *>(session);
        if (len) std::snprintf(out, len, "%s", s->choices.c_str());
        return TURBO_OK;
    });
}

// The hooks' dtype: TURBO_DTYPE_F16, BF16, I8 or F32.
static Dt hook_dt(uint32_t dtype) {
    switch (dtype) {
    case TURBO_DTYPE_F16: return Dt::F16;
    case TURBO_DTYPE_BF16: return Dt::BF16;
    case TURBO_DTYPE_I8: return Dt::I8;
    case TURBO_DTYPE_F32: return Dt::F32;
    default: fail(TURBO_E_INVALID_ENUM, "rocm: dtype " + std::to_string(dtype));
    }
}

// F32 operands on the device in the GEMM's operand type: narrowed copies,
// or int8 rows with their scales (into e).
struct Operands {
    DevPtr a, w, scales;
    const void *pa = nullptr, *pw = nullptr;
    Operands(Dt dt, const float *a32, const float *w32, size_t M, size_t N, size_t K, EpiArgs &e) {
        const size_t na = M * K, nw = N * K;
        pa = a32;
        pw = w32;
        if (dt == Dt::F32) return;
        a.reset(dev_alloc(na * 2, "gemm operands"));
        w.reset(dev_alloc(nw * 2, "gemm operands"));
        if (dt == Dt::I8) {
            scales.reset(dev_alloc((M + N) * 4, "gemm operands"));
            float *sa = static_cast<float *>(scales.get()), *sw = sa + M;
            check(quantize_rows(nullptr, a32, Dt::F32, (int)M, (int)K, (int)K, (int8_t *)a.get(), sa), "gemm operands");
            check(quantize_rows(nullptr, w32, Dt::F32, (int)N, (int)K, (int)K, (int8_t *)w.get(), sw), "gemm operands");
            e.a_scale = sa;
            e.w_scale = sw;
        } else {
            check(narrow(nullptr, a32, a.get(), na, dt, nullptr), "gemm operands");
            check(narrow(nullptr, w32, w.get(), nw, dt, nullptr), "gemm operands");
        }
        pa = a.get();
        pw = w.get();
    }
};

int32_t turbo_rocm_gemm_check(uint32_t ordinal, uint32_t dtype, uint32_t M, uint32_t N, uint32_t K, const float *A,
                              const float *W, const float *bias, float *out, uint32_t tile, turbo_error *err) {
    return guarded(err, [&] {
        if (ordinal >= devices().size()) fail(TURBO_E_DEVICE_NOT_FOUND, "rocm: no device");
        const Dt dt = hook_dt(dtype);
        OnDevice on(devices()[ordinal]);
        const size_t na = (size_t)M * K, nw = (size_t)N * K;
        DevPtr a32(dev_alloc(na * 4, "gemm check")), w32(dev_alloc(nw * 4, "gemm check"));
        DevPtr b(dev_alloc((size_t)N * 4, "gemm check")), o(dev_alloc((size_t)M * N * 4, "gemm check"));
        check(hipMemcpy(a32.get(), A, na * 4, hipMemcpyHostToDevice), "gemm check");
        check(hipMemcpy(w32.get(), W, nw * 4, hipMemcpyHostToDevice), "gemm check");
        if (bias) check(hipMemcpy(b.get(), bias, (size_t)N * 4, hipMemcpyHostToDevice), "gemm check");
        EpiArgs e;
        e.kind = Epi::Plain;
        e.bias = bias ? (const float *)b.get() : nullptr;
        e.out = o.get();
        e.ldo = (int)N;
        Operands ops(dt, (const float *)a32.get(), (const float *)w32.get(), M, N, K, e);
        check(gemm(nullptr, dt, (int)M, (int)N, (int)K, ops.pa, (int)K, ops.pw, e, (int)tile), "gemm check");
        check(hipDeviceSynchronize(), "gemm check");
        check(hipMemcpy(out, o.get(), (size_t)M * N * 4, hipMemcpyDeviceToHost), "gemm check");
        return TURBO_OK;
    });
}

int32_t turbo_rocm_gemm_time(uint32_t ordinal, uint32_t dtype, uint32_t M, uint32_t N, uint32_t K, uint32_t tile,
                             uint32_t iters, float *ms, turbo_error *err) {
    return guarded(err, [&] {
        if (ordinal >= devices().size()) fail(TURBO_E_DEVICE_NOT_FOUND, "rocm: no device");
        if (iters == 0) fail(TURBO_E_INVALID_ARGUMENT, "rocm: iters");
        const Dt dt = hook_dt(dtype);
        OnDevice on(devices()[ordinal]);
        DevPtr a32(dev_alloc((size_t)M * K * 4, "gemm time")), w32(dev_alloc((size_t)N * K * 4, "gemm time"));
        DevPtr x(dev_alloc((size_t)M * N * 4, "gemm time")), b(dev_alloc((size_t)N * 4, "gemm time"));
        // Uniform operands in [-1, 1) and [-1/16, 1/16): the multipliers
        // toggle as they do on real activations and weights (a constant
        // pattern draws less power and runs faster).
        check(fill_uniform(nullptr, (float *)a32.get(), (size_t)M * K, 1.0f, 1), "gemm time");
        check(fill_uniform(nullptr, (float *)w32.get(), (size_t)N * K, 0.0625f, 2), "gemm time");
        check(hipMemset(x.get(), 0, (size_t)M * N * 4), "gemm time");
        check(hipMemset(b.get(), 0, (size_t)N * 4), "gemm time");
        EpiArgs e;
        e.kind = Epi::Residual;
        e.bias = (const float *)b.get();
        e.x = (float *)x.get();
        e.ldo = (int)N;
        Operands ops(dt, (const float *)a32.get(), (const float *)w32.get(), M, N, K, e);
        hipEvent_t e0, e1;
        check(hipEventCreate(&e0), "gemm time");
        check(hipEventCreate(&e1), "gemm time");
        for (int i = 0; i < 3; ++i)
            check(gemm(nullptr, dt, (int)M, (int)N, (int)K, ops.pa, (int)K, ops.pw, e, (int)tile), "gemm time");
        check(hipEventRecord(e0, nullptr), "gemm time");
        for (uint32_t i = 0; i < iters; ++i)
            check(gemm(nullptr, dt, (int)M, (int)N, (int)K, ops.pa, (int)K, ops.pw, e, (int)tile), "gemm time");
        check(hipEventRecord(e1, nullptr), "gemm time");
        check(hipEventSynchronize(e1), "gemm time");
        float t = 0;
        check(hipEventElapsedTime(&t, e0, e1), "gemm time");
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        *ms = t / iters;
        return TURBO_OK;
    });
}

int32_t turbo_rocm_copy_probe(uint32_t ordinal, uint64_t bytes, uint32_t iters, float *ms, turbo_error *err) {
    return guarded(err, [&] {
        if (ordinal >= devices().size()) fail(TURBO_E_DEVICE_NOT_FOUND, "rocm: no device");
        if (iters == 0 || bytes == 0 || bytes % 16 != 0) fail(TURBO_E_INVALID_ARGUMENT, "rocm: bytes and iters");
        OnDevice on(devices()[ordinal]);
        DevPtr src(dev_alloc(bytes, "copy probe")), dst(dev_alloc(bytes, "copy probe"));
        check(hipMemset(src.get(), 1, bytes), "copy probe");
        hipEvent_t e0, e1;
        check(hipEventCreate(&e0), "copy probe");
        check(hipEventCreate(&e1), "copy probe");
        check(copy_bytes(nullptr, src.get(), dst.get(), bytes), "copy probe");
        check(hipEventRecord(e0, nullptr), "copy probe");
        for (uint32_t i = 0; i < iters; ++i) check(copy_bytes(nullptr, src.get(), dst.get(), bytes), "copy probe");
        check(hipEventRecord(e1, nullptr), "copy probe");
        check(hipEventSynchronize(e1), "copy probe");
        float t = 0;
        check(hipEventElapsedTime(&t, e0, e1), "copy probe");
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        *ms = t / iters;
        return TURBO_OK;
    });
}

int32_t turbo_rocm_mfma_probe(uint32_t ordinal, uint32_t random, uint32_t iters, float *tflops, float *mhz,
                              turbo_error *err) {
    return guarded(err, [&] {
        if (ordinal >= devices().size()) fail(TURBO_E_DEVICE_NOT_FOUND, "rocm: no device");
        if (iters == 0 || !tflops || !mhz) fail(TURBO_E_INVALID_ARGUMENT, "rocm: iters, tflops and mhz");
        OnDevice on(devices()[ordinal]);
        int cus = 0;
        check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, devices()[ordinal]), "mfma probe");
        DevPtr out(dev_alloc(256 * 4, "mfma probe")), clk(dev_alloc(16, "mfma probe"));
        float *o = static_cast<float *>(out.get());
        unsigned long long *c = static_cast<unsigned long long *>(clk.get());
        hipEvent_t e0, e1;
        check(hipEventCreate(&e0), "mfma probe");
        check(hipEventCreate(&e1), "mfma probe");
        check(mfma_probe(nullptr, cus, 100, (int)random, o, c), "mfma probe");
        check(hipEventRecord(e0, nullptr), "mfma probe");
        check(mfma_probe(nullptr, cus, (int)iters, (int)random, o, c), "mfma probe");
        check(hipEventRecord(e1, nullptr), "mfma probe");
        check(hipEventSynchronize(e1), "mfma probe");
        float ms = 0;
        check(hipEventElapsedTime(&ms, e0, e1), "mfma probe");
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        unsigned long long counts[2] = {0, 0};
        check(hipMemcpy(counts, c, 16, hipMemcpyDeviceToHost), "mfma probe");
        // 4 waves a workgroup, 8 products a round, 2 * 32 * 32 * 16 flops a product.
        *tflops = (float)((double)cus * 4 * iters * 8 * 32768.0 / (ms * 1e-3) / 1e12);
        *mhz = counts[1] ? (float)(100.0 * (double)counts[0] / (double)counts[1]) : 0.0f;
        return TURBO_OK;
    });
}

}  // extern "C"
