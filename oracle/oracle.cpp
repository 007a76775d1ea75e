// The oracle: TurboEmbed's CPU encoder restated in C++ for checking the rocm
// backend, and for the CPU baseline the benchmark reports. Test
// infrastructure only; see oracle.h.
//
// It follows the reference's CPU path (core/src/cpu/) operation for
// operation, so that its results are the ones that path gives up to the
// order-preserving changes noted at each function:
//   - packing             core/src/cpu/encoder/mod.rs:379-424
//   - lookup + LayerNorm  core/src/cpu/encoder/job.rs:113-129, kernels/rowwise.rs:9-29
//   - linear layers       core/src/cpu/kernels/gemm.rs:66-142 (one FMA chain over
//                         k = 0..K-1 per output, then the bias; kernels/mod.rs:5-19)
//   - attention           core/src/cpu/kernels/attend.rs:84-322
//   - GELU, exp, SiLU     core/src/cpu/kernels/rowwise.rs:31-113
//   - RoPE, gated MLP     core/src/cpu/kernels/pairs.rs:40-216
//   - rotary layer loop   core/src/cpu/encoder/rotary/mod.rs:88-175
//   - pooling, L2         core/src/cpu/encoder/mod.rs:426-482, job.rs:169-191
// Built with -ffp-contract=off: every multiply-add the reference does not
// fuse is rounded twice here too, and every one it fuses is an explicit fmaf.
#include <immintrin.h>
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <stdexcept>
#include <string>
#include <thread>

#include <pthread.h>
#include <sched.h>
#include <vector>

namespace {

constexpr uint32_t kLanes = 16;        // attention's vector lanes (attend.rs:23)
// A limit on the gated product act(gate) * up (0: none). The CPU path holds
// it in F32; a device tier that stores it in F16 saturates it at 65504 (the
// reference's CUDA backend, core/cuda/rotary.cuh:31-45), and the tests check
// that tier against this oracle with the same limit set.
std::atomic<float> gated_limit{0.0f};
constexpr float kNegInf = -std::numeric_limits<float>::infinity();

struct Failure : std::runtime_error {
    int32_t code;
    Failure(int32_t c, const std::string &m) : std::runtime_error(m), code(c) {}
};

// ---- Scalar functions (rowwise.rs) ----------------------------------------

inline float bits_to_float(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
inline uint32_t float_to_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

// Cephes expf as rowwise.rs:31-53 writes it: 0 under -80, clamped at 88.
float cephes_exp(float x) {
    const float lo = -80.0f;
    float c = std::min(std::max(x, lo), 88.0f);
    if (std::isnan(x)) c = x;
    const float n = std::floor(c * 1.44269504088896340736f + 0.5f);
    float r = c - n * 0.693359375f;
    r = r - n * -2.12194440e-4f;
    const float r2 = r * r;
    float p = 1.9875691e-4f * r + 1.3982e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    const float e = p * r2 + r + 1.0f;
    const uint32_t n_int = float_to_bits(n + 12582912.0f) - 0x4b400000u;
    const float scale = bits_to_float((n_int + 127u) << 23);
    return x < lo ? 0.0f : e * scale;
}

// Dekker's product with Veltkamp's split and Knuth's sum (rowwise.rs:94-113).
inline void two_product(float a, float b, float &p, float &e) {
    auto split = [](float v, float &hi, float &lo) {
        const float c = 4097.0f * v;
        hi = c - (c - v);
        lo = v - hi;
    };
    p = a * b;
    float ah, al, bh, bl;
    split(a, ah, al);
    split(b, bh, bl);
    e = ((ah * bh - p) + ah * bl + al * bh) + al * bl;
}
inline void two_sum(float a, float b, float &s, float &e) {
    s = a + b;
    const float bb = s - a;
    e = (a - (s - bb)) + (b - bb);
}

// GELU by erf through Numerical Recipes' erfcc fit, the exponent's -x^2/2
// carried exactly (rowwise.rs:55-83).
float gelu_erf(float x) {
    const float xc = std::min(std::max(x, -16.0f), 16.0f);
    const float z = std::fabs(xc) * 0.70710678118654752440f;
    const float t = 1.0f / (1.0f + 0.5f * z);
    const float p =
        -1.26551223f +
        t * (1.00002368f +
             t * (0.37409196f +
                  t * (0.09678418f +
                       t * (-0.18628806f +
                            t * (0.27886807f +
                                 t * (-1.13520398f + t * (1.48851587f + t * (-0.8221522f + t * 0.17087277f))))))));
    float sq, sq_lo;
    two_product(xc, xc, sq, sq_lo);
    const float hi = -0.5f * sq, lo = -0.5f * sq_lo;
    float a, e;
    two_sum(hi, p, a, e);
    const float r = t * (cephes_exp(a) * (1.0f + (e + lo)));
    return 0.5f * x * (x >= 0.0f ? 2.0f - r : r);
}

float silu(float x) { return x / (1.0f + cephes_exp(-x)); }

// LayerNorm with the mean and biased variance summed in F64 over eight lanes
// (rowwise.rs:3-29). b NULL is a zero bias, added as the reference adds its
// zero vector.
void layer_norm(float *y, const float *w, const float *b, uint32_t n, float eps) {
    auto lanes8 = [](const double *s) { return ((s[0] + s[4]) + (s[1] + s[5])) + ((s[2] + s[6]) + (s[3] + s[7])); };
    double s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t i = 0; i < n; ++i) s[i % 8] += (double)y[i];
    const double mean = lanes8(s) / (double)n;
    double v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t i = 0; i < n; ++i) {
        const double c = (double)y[i] - mean;
        v[i % 8] += c * c;
    }
    const double var = lanes8(v) / (double)n;
    const double inv = 1.0 / std::sqrt(var + (double)eps);
    for (uint32_t i = 0; i < n; ++i) y[i] = (float)(((double)y[i] - mean) * inv) * w[i] + (b ? b[i] : 0.0f);
}

// DeBERTa's LayerNorm (core/src/deberta/math.rs:9-27): the mean and the
// biased variance summed in F64 in order, the scale 1 / sqrt(var + eps) in
// F64, y = (x - mean) * scale * w + b in F64, rounded once. eps is the
// architecture's (F64).
void deberta_norm(float *y, const float *w, const float *b, uint32_t n, double eps) {
    double sum = 0.0;
    for (uint32_t i = 0; i < n; ++i) sum += (double)y[i];
    const double mean = sum / (double)n;
    double var = 0.0;
    for (uint32_t i = 0; i < n; ++i) var += ((double)y[i] - mean) * ((double)y[i] - mean);
    var /= (double)n;
    const double scale = 1.0 / std::sqrt(var + eps);
    for (uint32_t i = 0; i < n; ++i) y[i] = (float)(((double)y[i] - mean) * scale * (double)w[i] + (double)b[i]);
}

// The relative row of a signed distance (core/src/deberta/math.rs:30-40,
// transformers' make_log_bucket_position): distances within half the
// buckets are their own row; beyond, ceil(ln(|d| / mid) / ln((max - 1) / mid)
// * (mid - 1)) + mid with F32 logarithms, signed, offset by the buckets and
// clamped to the table.
uint32_t deberta_bucket(int64_t distance, uint32_t buckets, uint32_t maximum) {
    const int64_t mid = buckets / 2;
    const int64_t mag0 = distance < 0 ? -distance : distance;
    int64_t mag = mag0;
    if (mag0 > mid) {
        const float a = std::log((float)mag0 / (float)mid), c = std::log((float)(maximum - 1) / (float)mid);
        mag = (int64_t)std::ceil(a / c * (float)(mid - 1)) + mid;
    }
    const int64_t signed_mag = distance < 0 ? -mag : mag;
    return (uint32_t)std::min<int64_t>(std::max<int64_t>(signed_mag + buckets, 0), 2 * (int64_t)buckets - 1);
}

// ---- Threads ----------------------------------------------------------------

// Whether worker threads pin themselves, thread i to the i-th CPU this
// process may run on (a timing baseline's threads then do not migrate).
std::atomic<int> pin_threads{0};

void pin_to(uint32_t i) {
    cpu_set_t allowed;
    if (sched_getaffinity(0, sizeof allowed, &allowed) != 0) return;
    const int n = CPU_COUNT(&allowed);
    if (n <= 0) return;
    int want = (int)(i % (uint32_t)n);
    for (int c = 0; c < CPU_SETSIZE; ++c)
        if (CPU_ISSET(c, &allowed) && want-- == 0) {
            cpu_set_t one;
            CPU_ZERO(&one);
            CPU_SET(c, &one);
            (void)pthread_setaffinity_np(pthread_self(), sizeof one, &one);
            return;
        }
}

// Runs fn(task) for task in [0, tasks) on `threads` threads. A task computes
// each of its outputs whole, so the bits never depend on the thread count.
void parallel(uint32_t threads, size_t tasks, const std::function<void(size_t)> &fn) {
    if (tasks == 0) return;
    const uint32_t n = (uint32_t)std::min<size_t>(threads, tasks);
    if (n <= 1) {
        for (size_t t = 0; t < tasks; ++t) fn(t);
        return;
    }
    std::atomic<size_t> next{0};
    std::vector<std::thread> pool;
    pool.reserve(n);
    const bool pin = pin_threads.load() != 0;
    for (uint32_t i = 0; i < n; ++i)
        pool.emplace_back([&, i] {
            if (pin) pin_to(i);
            for (size_t t; (t = next.fetch_add(1)) < tasks;) fn(t);
        });
    for (auto &th : pool) th.join();
}

// ---- Weights ----------------------------------------------------------------

float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else {  // subnormal: exact as a float
            float f = std::ldexp((float)m, -24);
            u = float_to_bits(f) | s;
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e - 15 + 127) << 23) | (m << 13);
    }
    return bits_to_float(u);
}

// A linear layer's weight W [n, k] laid out k-major, wt[k][n], so that a
// step of the reduction reads the row of n outputs at once.
struct Linear {
    uint32_t n = 0, k = 0;
    std::vector<float> wt;   // [k][n]
    std::vector<float> bias; // [n], zeros where the model has none
    // The same weights as panels of 16 outputs, [n / 16][k][16] (whole
    // panels only): a panel's reduction reads consecutive memory.
    std::vector<float> panels;
};

// The rows of W's parts one after another (each [n_i, k] row-major), in the
// order `rows` lists them, as a k-major Linear.
Linear pack_rows(const std::vector<const float *> &rows, uint32_t k) {
    Linear l;
    l.n = (uint32_t)rows.size();
    l.k = k;
    l.wt.assign((size_t)l.n * k, 0.0f);
    for (uint32_t o = 0; o < l.n; ++o)
        for (uint32_t kk = 0; kk < k; ++kk) l.wt[(size_t)kk * l.n + o] = rows[o][kk];
    l.panels.assign((size_t)(l.n / 16) * 16 * k, 0.0f);
    for (uint32_t o = 0; o < l.n / 16 * 16; ++o)
        for (uint32_t kk = 0; kk < k; ++kk) l.panels[((size_t)(o / 16) * k + kk) * 16 + o % 16] = rows[o][kk];
    l.bias.assign(l.n, 0.0f);
    return l;
}

struct Layer {
    Linear qkv, out, ffn_in, ffn_out;
    const float *attn_ln_w = nullptr, *attn_ln_b = nullptr;
    const float *ffn_ln_w = nullptr, *ffn_ln_b = nullptr;
};

struct Model {
    uint32_t family, layers, hidden, heads, d, inter, vocab, positions, types, position_offset;
    // DeBERTa-v2: the relative table's half rows and the distance the log
    // buckets reach; the normalized relative rows [2 buckets, H], and each
    // layer's shared-key projections of them, query then key [2 buckets][2 H].
    bool deberta = false;
    uint32_t buckets = 0, max_rel = 0;
    double eps64 = 0.0;
    std::vector<float> reln;
    std::vector<std::vector<float>> pos_qk;
    float eps;
    uint32_t ahead;       // keys past a query it reads; UINT32_MAX for the whole row
    bool rotary = false, modern = false, silu_act = false;
    uint32_t window = UINT32_MAX, global_every = 0, pairs = 0;
    const float *rope = nullptr;
    std::vector<std::vector<float>> widened;   // F16/BF16 tensors in F32
    std::vector<const float *> t;               // every tensor in F32
    std::vector<Layer> ls;
    const float *word = nullptr, *pos = nullptr, *type = nullptr, *emb_w = nullptr, *emb_b = nullptr,
                *final_w = nullptr;
};

const float *tensor_f32(Model &m, const turbo_backend_tensor &t, uint32_t dtype) {
    if (!t.data) return nullptr;
    if (dtype == TURBO_DTYPE_F32) return static_cast<const float *>(t.data);
    const size_t n = t.bytes / 2;
    std::vector<float> w(n);
    const uint16_t *src = static_cast<const uint16_t *>(t.data);
    for (size_t i = 0; i < n; ++i)
        w[i] = dtype == TURBO_DTYPE_F16 ? half_to_float(src[i]) : bits_to_float((uint32_t)src[i] << 16);
    m.widened.push_back(std::move(w));
    return m.widened.back().data();
}

void load(Model &m, const turbo_backend_model *d) {
    m.family = d->family;
    if (d->family != TURBO_FAMILY_BERT && d->family != TURBO_FAMILY_ROBERTA && d->family != TURBO_FAMILY_MODERNBERT &&
        d->family != TURBO_FAMILY_NOMIC_BERT && d->family != TURBO_FAMILY_DEBERTA_V2)
        throw Failure(TURBO_E_UNSUPPORTED, "family " + std::to_string(d->family) + " is not an encoder the oracle runs");
    if (d->dtype != TURBO_DTYPE_F32 && d->dtype != TURBO_DTYPE_F16 && d->dtype != TURBO_DTYPE_BF16)
        throw Failure(TURBO_E_UNSUPPORTED, "dtype " + std::to_string(d->dtype));
    m.layers = d->layers;
    m.hidden = d->hidden;
    m.heads = d->heads;
    m.d = d->hidden / d->heads;
    m.inter = d->intermediate;
    m.vocab = d->vocab_size;
    m.positions = d->max_positions;
    m.types = d->token_types;
    m.position_offset = d->position_offset;
    m.eps = (float)d->layer_norm_eps;
    m.ahead = d->lookahead == 0 ? UINT32_MAX : d->lookahead;
    m.rotary = d->family == TURBO_FAMILY_MODERNBERT || d->family == TURBO_FAMILY_NOMIC_BERT;
    m.modern = d->family == TURBO_FAMILY_MODERNBERT;
    const uint32_t H = m.hidden, I = m.inter;
    m.t.resize(d->tensor_count);
    for (uint32_t i = 0; i < d->tensor_count; ++i) m.t[i] = tensor_f32(m, d->tensors[i], d->dtype);
    m.deberta = d->family == TURBO_FAMILY_DEBERTA_V2;
    if (!m.rotary) {
        const uint32_t emb = m.deberta ? TURBO_DEBERTA_EMBEDDING_TENSORS : TURBO_BERT_EMBEDDING_TENSORS;
        const uint32_t need = emb + m.layers * TURBO_BERT_LAYER_TENSORS;
        if (d->tensor_count != need) throw Failure(TURBO_E_INVALID_ARGUMENT, "tensor_count");
        if (m.deberta) {
            if (d->struct_size < offsetof(turbo_backend_model, max_relative_positions) + 4 || d->position_buckets < 2 ||
                d->max_relative_positions < 2)
                throw Failure(TURBO_E_INVALID_ARGUMENT, "a DeBERTa-v2 model needs position_buckets and max_relative_positions");
            m.buckets = d->position_buckets;
            m.max_rel = d->max_relative_positions;
            m.eps64 = d->layer_norm_eps;
            m.word = m.t[TURBO_DEBERTA_WORD_EMBEDDINGS];
            m.emb_w = m.t[TURBO_DEBERTA_EMBEDDINGS_LN_WEIGHT];
            m.emb_b = m.t[TURBO_DEBERTA_EMBEDDINGS_LN_BIAS];
            // The relative rows through their own LayerNorm (core/src/deberta/weights.rs:91-92).
            const float *rel = m.t[TURBO_DEBERTA_RELATIVE_EMBEDDINGS];
            m.reln.assign(rel, rel + (size_t)2 * m.buckets * H);
            for (uint32_t r = 0; r < 2 * m.buckets; ++r)
                deberta_norm(&m.reln[(size_t)r * H], m.t[TURBO_DEBERTA_RELATIVE_LN_WEIGHT],
                             m.t[TURBO_DEBERTA_RELATIVE_LN_BIAS], H, d->layer_norm_eps);
        } else {
            m.word = m.t[TURBO_BERT_WORD_EMBEDDINGS];
            m.pos = m.t[TURBO_BERT_POSITION_EMBEDDINGS];
            m.type = m.t[TURBO_BERT_TOKEN_TYPE_EMBEDDINGS];
            m.emb_w = m.t[TURBO_BERT_EMBEDDINGS_LN_WEIGHT];
            m.emb_b = m.t[TURBO_BERT_EMBEDDINGS_LN_BIAS];
        }
        for (uint32_t l = 0; l < m.layers; ++l) {
            auto w = [&](uint32_t r) { return m.t[emb + l * TURBO_BERT_LAYER_TENSORS + r]; };
            Layer L;
            std::vector<const float *> rows;
            for (uint32_t part : {TURBO_BERT_Q_WEIGHT, TURBO_BERT_K_WEIGHT, TURBO_BERT_V_WEIGHT})
                for (uint32_t o = 0; o < H; ++o) rows.push_back(w(part) + (size_t)o * H);
            L.qkv = pack_rows(rows, H);
            for (uint32_t o = 0; o < H; ++o) {
                L.qkv.bias[o] = w(TURBO_BERT_Q_BIAS)[o];
                L.qkv.bias[H + o] = w(TURBO_BERT_K_BIAS)[o];
                L.qkv.bias[2 * H + o] = w(TURBO_BERT_V_BIAS)[o];
            }
            auto plain = [&](uint32_t wi, uint32_t bi, uint32_t n, uint32_t k) {
                std::vector<const float *> r;
                for (uint32_t o = 0; o < n; ++o) r.push_back(w(wi) + (size_t)o * k);
                Linear lin = pack_rows(r, k);
                std::copy(w(bi), w(bi) + n, lin.bias.begin());
                return lin;
            };
            L.out = plain(TURBO_BERT_ATTN_OUT_WEIGHT, TURBO_BERT_ATTN_OUT_BIAS, H, H);
            L.ffn_in = plain(TURBO_BERT_FFN_IN_WEIGHT, TURBO_BERT_FFN_IN_BIAS, I, H);
            L.ffn_out = plain(TURBO_BERT_FFN_OUT_WEIGHT, TURBO_BERT_FFN_OUT_BIAS, H, I);
            L.attn_ln_w = w(TURBO_BERT_ATTN_LN_WEIGHT);
            L.attn_ln_b = w(TURBO_BERT_ATTN_LN_BIAS);
            L.ffn_ln_w = w(TURBO_BERT_FFN_LN_WEIGHT);
            L.ffn_ln_b = w(TURBO_BERT_FFN_LN_BIAS);
            if (m.deberta) {
                // Shared keys: the layer's query and key projections of every
                // normalized relative row, an in-order FMA chain then the bias
                // (core/src/deberta/weights.rs:98-106).
                std::vector<float> pq((size_t)2 * m.buckets * 2 * H);
                for (uint32_t r = 0; r < 2 * m.buckets; ++r)
                    for (uint32_t o = 0; o < 2 * H; ++o) {
                        float acc = 0.0f;
                        for (uint32_t k = 0; k < H; ++k)
                            acc = __builtin_fmaf(m.reln[(size_t)r * H + k], L.qkv.wt[(size_t)k * L.qkv.n + o], acc);
                        pq[(size_t)r * 2 * H + o] = acc + L.qkv.bias[o];
                    }
                m.pos_qk.push_back(std::move(pq));
            }
            m.ls.push_back(std::move(L));
        }
        return;
    }
    // The rotary families (core/src/cpu/rotary.rs:18-66 checks; pairs.rs packs).
    if (d->struct_size < offsetof(turbo_backend_model, global_every) + 4)
        throw Failure(TURBO_E_INVALID_STRUCT_SIZE, "a rotary model needs the rotary fields");
    if (m.d % 2 || d->rope_pairs * 2 != m.d || !d->rope_table)
        throw Failure(TURBO_E_INVALID_ARGUMENT, "a rotary head is an even width, twice rope_pairs, with a table");
    m.pairs = d->rope_pairs;
    m.rope = d->rope_table;
    m.window = d->attention_window == 0 ? UINT32_MAX : d->attention_window / 2;
    m.global_every = d->global_every;
    m.silu_act = d->activation == TURBO_ACTIVATION_SILU;
    const uint32_t emb = m.modern ? TURBO_MODERNBERT_EMBEDDING_TENSORS : TURBO_NOMIC_EMBEDDING_TENSORS;
    const uint32_t per = m.modern ? TURBO_MODERNBERT_LAYER_TENSORS : TURBO_NOMIC_LAYER_TENSORS;
    if (d->tensor_count != emb + m.layers * per) throw Failure(TURBO_E_INVALID_ARGUMENT, "tensor_count");
    if (m.modern) {
        m.word = m.t[TURBO_MODERNBERT_WORD_EMBEDDINGS];
        m.emb_w = m.t[TURBO_MODERNBERT_EMBEDDINGS_LN_WEIGHT];
        m.final_w = m.t[TURBO_MODERNBERT_FINAL_NORM_WEIGHT];
    } else {
        m.word = m.t[TURBO_NOMIC_WORD_EMBEDDINGS];
        m.type = m.t[TURBO_NOMIC_TOKEN_TYPE_EMBEDDINGS];
        m.emb_w = m.t[TURBO_NOMIC_EMBEDDINGS_LN_WEIGHT];
        m.emb_b = m.t[TURBO_NOMIC_EMBEDDINGS_LN_BIAS];
    }
    for (uint32_t l = 0; l < m.layers; ++l) {
        auto w = [&](uint32_t r) { return m.t[emb + l * per + r]; };
        Layer L;
        // Q and K rows pair-adjacent per head, (c, c + d/2); V as stored
        // (pairs.rs:146-161).
        const float *qkv = w(m.modern ? TURBO_MODERNBERT_QKV_WEIGHT : TURBO_NOMIC_QKV_WEIGHT);
        std::vector<const float *> rows;
        for (uint32_t third = 0; third < 2; ++third)
            for (uint32_t head = 0; head < H; head += m.d)
                for (uint32_t c = 0; c < m.d / 2; ++c) {
                    rows.push_back(qkv + (size_t)(third * H + head + c) * H);
                    rows.push_back(qkv + (size_t)(third * H + head + c + m.d / 2) * H);
                }
        for (uint32_t o = 2 * H; o < 3 * H; ++o) rows.push_back(qkv + (size_t)o * H);
        L.qkv = pack_rows(rows, H);
        std::vector<const float *> r;
        const float *ow = w(m.modern ? TURBO_MODERNBERT_ATTN_OUT_WEIGHT : TURBO_NOMIC_ATTN_OUT_WEIGHT);
        for (uint32_t o = 0; o < H; ++o) r.push_back(ow + (size_t)o * H);
        L.out = pack_rows(r, H);
        // Gate row j then up row j (pairs.rs:163-166).
        const float *gate, *up;
        if (m.modern) {
            gate = w(TURBO_MODERNBERT_FFN_IN_WEIGHT);
            up = gate + (size_t)I * H;
        } else {
            gate = w(TURBO_NOMIC_FFN_GATE_WEIGHT);
            up = w(TURBO_NOMIC_FFN_UP_WEIGHT);
        }
        r.clear();
        for (uint32_t j = 0; j < I; ++j) {
            r.push_back(gate + (size_t)j * H);
            r.push_back(up + (size_t)j * H);
        }
        L.ffn_in = pack_rows(r, H);
        r.clear();
        const float *fo = w(m.modern ? TURBO_MODERNBERT_FFN_OUT_WEIGHT : TURBO_NOMIC_FFN_OUT_WEIGHT);
        for (uint32_t o = 0; o < H; ++o) r.push_back(fo + (size_t)o * I);
        L.ffn_out = pack_rows(r, I);
        if (m.modern) {
            L.attn_ln_w = w(TURBO_MODERNBERT_ATTN_LN_WEIGHT);  // NULL on layer 0
            L.ffn_ln_w = w(TURBO_MODERNBERT_FFN_LN_WEIGHT);
        } else {
            L.attn_ln_w = w(TURBO_NOMIC_ATTN_LN_WEIGHT);
            L.attn_ln_b = w(TURBO_NOMIC_ATTN_LN_BIAS);
            L.ffn_ln_w = w(TURBO_NOMIC_FFN_LN_WEIGHT);
            L.ffn_ln_b = w(TURBO_NOMIC_FFN_LN_BIAS);
        }
        m.ls.push_back(std::move(L));
    }
}

// ---- Packing (encoder/mod.rs:379-424) ----------------------------------------

struct Packing {
    std::vector<uint32_t> start, len, at;
    uint32_t tokens = 0;
};

Packing pack(const int32_t *mask, uint32_t batch, uint32_t seq, uint32_t stride, const turbo_token_range *ranges,
             uint32_t count) {
    Packing p;
    p.start.assign(batch, 0);
    p.len.assign(batch, 0);
    std::vector<uint32_t> reach(batch, 0);
    for (uint32_t i = 0; i < count; ++i) reach[ranges[i].row] = std::max(reach[ranges[i].row], ranges[i].end);
    uint32_t t = 0;
    for (uint32_t r = 0; r < batch; ++r) {
        uint32_t live = 0;
        for (uint32_t q = seq; q > 0; --q)
            if (mask[(size_t)r * stride + q - 1] != 0) {
                live = q;
                break;
            }
        const uint32_t len = count ? std::max(live, reach[r]) : live;
        p.start[r] = t;
        p.len[r] = len;
        for (uint32_t q = 0; q < len; ++q) p.at.push_back(r * seq + q);
        t += len;
    }
    p.tokens = t;
    return p;
}

// ---- One run ------------------------------------------------------------------

struct Run {
    const Model &m;
    uint32_t threads;
    uint32_t batch, seq;
    std::vector<uint32_t> ids, types;
    std::vector<uint8_t> mask;
    Packing pk;
    std::vector<float> x, xn, qkv, ctx, ffn;
    Run(const Model &mm, uint32_t th) : m(mm), threads(th) {}

    uint32_t T() const { return pk.tokens; }

    // y[t][o] = epi(chain_k x[t][k] * w[o][k], o) for every packed token t: each
    // output one chain of fused multiply-adds over k in order (gemm.rs:66-142).
    // (Blocks of 6 rows x 16 columns: the 96 chains stay in 12 AVX2 registers
    // over the whole k loop; the order of each chain is unchanged.)
    template <class Epi>
    void linear(const float *xin, uint32_t ldx, const Linear &w, Epi epi) {
        // A task: one 16-column panel of the weights (it stays in the core's
        // cache) over RG blocks of rows.
        constexpr uint32_t RB = 6, CB = 16, RG = 8;
        const size_t rblocks = (T() + RB - 1) / RB, cblocks = (w.n + CB - 1) / CB, rgroups = (rblocks + RG - 1) / RG;
        parallel(threads, rgroups * cblocks, [&](size_t task) {
          const size_t cb = task % cblocks, rg = task / cblocks;
          for (size_t rb = rg * RG; rb < std::min(rblocks, rg * RG + RG); ++rb) {
            const uint32_t r0 = (uint32_t)rb * RB, c0 = (uint32_t)cb * CB;
            const uint32_t rows = std::min(RB, T() - r0), cols = std::min(CB, w.n - c0);
            alignas(64) float acc[RB][CB];
            for (uint32_t i = 0; i < RB; ++i)
                for (uint32_t j = 0; j < CB; ++j) acc[i][j] = 0.0f;
            if (cols == CB && rows == RB) {
                // _mm256_fmadd_ps: eight fmaf, each rounded once.
                const float *xr[RB];
                for (uint32_t i = 0; i < RB; ++i) xr[i] = xin + (size_t)(r0 + i) * ldx;
                __m256 c[RB][2];
#pragma GCC unroll 6
                for (uint32_t i = 0; i < RB; ++i) c[i][0] = c[i][1] = _mm256_setzero_ps();
                const float *panel = &w.panels[(size_t)cb * w.k * CB];
                for (uint32_t k = 0; k < w.k; ++k) {
                    const float *wr = panel + (size_t)k * CB;
                    const __m256 w0 = _mm256_loadu_ps(wr), w1 = _mm256_loadu_ps(wr + 8);
#pragma GCC unroll 6
                    for (uint32_t i = 0; i < RB; ++i) {
                        const __m256 a = _mm256_broadcast_ss(xr[i] + k);
                        c[i][0] = _mm256_fmadd_ps(a, w0, c[i][0]);
                        c[i][1] = _mm256_fmadd_ps(a, w1, c[i][1]);
                    }
                }
#pragma GCC unroll 6
                for (uint32_t i = 0; i < RB; ++i) {
                    _mm256_store_ps(acc[i], c[i][0]);
                    _mm256_store_ps(acc[i] + 8, c[i][1]);
                }
            } else if (cols == CB) {
                for (uint32_t k = 0; k < w.k; ++k) {
                    const float *wr = &w.wt[(size_t)k * w.n + c0];
                    for (uint32_t i = 0; i < rows; ++i) {
                        const float a = xin[(size_t)(r0 + i) * ldx + k];
                        for (uint32_t j = 0; j < CB; ++j) acc[i][j] = __builtin_fmaf(a, wr[j], acc[i][j]);
                    }
                }
            } else {
                for (uint32_t k = 0; k < w.k; ++k) {
                    const float *wr = &w.wt[(size_t)k * w.n + c0];
                    for (uint32_t i = 0; i < rows; ++i) {
                        const float a = xin[(size_t)(r0 + i) * ldx + k];
                        for (uint32_t j = 0; j < cols; ++j) acc[i][j] = __builtin_fmaf(a, wr[j], acc[i][j]);
                    }
                }
            }
            for (uint32_t i = 0; i < rows; ++i) epi(r0 + i, c0, cols, acc[i]);
          }
        });
    }

    // Position of packed token t: its column in its row.
    uint32_t column(uint32_t t) const { return pk.at[t] % seq; }

    void lookup() {
        const uint32_t H = m.hidden;
        parallel(threads, (T() + 15) / 16, [&](size_t c) {
            for (uint32_t t = (uint32_t)c * 16; t < std::min<uint32_t>(T(), (uint32_t)c * 16 + 16); ++t) {
                const uint32_t at = pk.at[t];
                float *dst = &x[(size_t)t * H];
                const float *w = m.word + (size_t)ids[at] * H;
                if (m.deberta) {
                    // A masked position is zero after the embedding; a live one
                    // its row through the embedding norm (core/src/deberta/mod.rs:245-252).
                    if (!mask[at]) {
                        std::fill(dst, dst + H, 0.0f);
                    } else {
                        std::copy(w, w + H, dst);
                        deberta_norm(dst, m.emb_w, m.emb_b, H, m.eps64);
                    }
                    continue;
                }
                if (!m.rotary) {
                    const float *ps = m.pos + (size_t)(at % seq + m.position_offset) * H;
                    const float *tt = m.type + (size_t)types[at] * H;
                    for (uint32_t i = 0; i < H; ++i) dst[i] = w[i] + ps[i] + tt[i];
                } else {
                    std::copy(w, w + H, dst);
                    if (m.type) {
                        const float *tt = m.type + (size_t)types[at] * H;
                        for (uint32_t i = 0; i < H; ++i) dst[i] += tt[i];
                    }
                }
                layer_norm(dst, m.emb_w, m.emb_b, H, m.eps);
            }
        });
    }

    void norm(float *buf, const float *w, const float *b) {
        const uint32_t H = m.hidden;
        parallel(threads, (T() + 15) / 16, [&](size_t c) {
            for (uint32_t t = (uint32_t)c * 16; t < std::min<uint32_t>(T(), (uint32_t)c * 16 + 16); ++t) {
                if (m.deberta) deberta_norm(&buf[(size_t)t * H], w, b, H, m.eps64);
                else layer_norm(&buf[(size_t)t * H], w, b, H, m.eps);
            }
        });
    }

    // DeBERTa's disentangled attention of layer l (core/src/deberta/attention.rs:207-315):
    // for each live query i and live key j, the score
    // (q_i . k_j + q_i . pos_k[b] + k_j . pos_q[b]) / sqrt(3 d), b the bucket of
    // the columns' distance, each dot an in-order FMA chain; the row's
    // softmax over the live keys, and the context as an in-order FMA chain
    // over them. A masked position attends uniformly to every position
    // through the row's last live one: the mean of their values in F64.
    void attention_deberta(uint32_t l) {
        const uint32_t H = m.hidden, d = m.d, ld = 3 * H;
        const float inv = (float)(1.0 / std::sqrt(3.0 * (double)d));
        const float *pq = m.pos_qk[l].data();
        parallel(threads, (size_t)batch * m.heads, [&](size_t task) {
            const uint32_t r = (uint32_t)(task / m.heads), head = (uint32_t)(task % m.heads);
            const uint32_t start = pk.start[r], len = pk.len[r];
            if (len == 0) return;
            const uint8_t *mk = &mask[(size_t)r * seq];
            std::vector<uint32_t> live;
            for (uint32_t p = 0; p < len; ++p)
                if (mk[p]) live.push_back(p);
            const uint32_t nv = (uint32_t)live.size();
            const float *qv = &qkv[(size_t)start * ld];
            auto dot = [&](const float *a, const float *b) {
                float acc = 0.0f;
                for (uint32_t c = 0; c < d; ++c) acc = __builtin_fmaf(a[c], b[c], acc);
                return acc;
            };
            std::vector<float> sc(nv);
            for (uint32_t ii = 0; ii < nv; ++ii) {
                const uint32_t pi = live[ii];
                const float *q = qv + (size_t)pi * ld + head * d;
                for (uint32_t jj = 0; jj < nv; ++jj) {
                    const uint32_t pj = live[jj];
                    const float *k = qv + (size_t)pj * ld + H + head * d;
                    const uint32_t bk = deberta_bucket((int64_t)pi - (int64_t)pj, m.buckets, m.max_rel);
                    const float *row = pq + (size_t)bk * 2 * H;
                    sc[jj] = (dot(q, k) + dot(q, row + H + head * d) + dot(k, row + head * d)) * inv;
                }
                float mx = kNegInf;
                for (uint32_t jj = 0; jj < nv; ++jj)
                    if (sc[jj] > mx) mx = sc[jj];
                float lanes[kLanes];
                for (uint32_t w = 0; w < kLanes; ++w) lanes[w] = 0.0f;
                for (uint32_t jj = 0; jj < nv; ++jj) {
                    sc[jj] = cephes_exp(sc[jj] - mx);
                    lanes[jj % kLanes] += sc[jj];
                }
                for (uint32_t w = kLanes / 2; w > 0; w /= 2)
                    for (uint32_t x = 0; x < w; ++x) lanes[x] += lanes[x + w];
                const float rinv = 1.0f / lanes[0];
                for (uint32_t jj = 0; jj < nv; ++jj) sc[jj] *= rinv;
                float *out = &ctx[(size_t)(start + pi) * H + head * d];
                for (uint32_t c = 0; c < d; ++c) {
                    float acc = 0.0f;
                    for (uint32_t jj = 0; jj < nv; ++jj)
                        acc = __builtin_fmaf(sc[jj], qv[(size_t)live[jj] * ld + 2 * H + head * d + c], acc);
                    out[c] = acc;
                }
            }
            for (uint32_t p = 0; p < len; ++p) {
                if (mk[p]) continue;
                float *out = &ctx[(size_t)(start + p) * H + head * d];
                for (uint32_t c = 0; c < d; ++c) {
                    double sum = 0.0;
                    for (uint32_t j = 0; j < len; ++j) sum += (double)qv[(size_t)j * ld + 2 * H + head * d + c];
                    out[c] = (float)(sum / (double)len);
                }
            }
        });
    }

    void norm_into(const float *w, const float *b) {
        const uint32_t H = m.hidden;
        parallel(threads, (T() + 15) / 16, [&](size_t c) {
            for (uint32_t t = (uint32_t)c * 16; t < std::min<uint32_t>(T(), (uint32_t)c * 16 + 16); ++t) {
                std::copy(&x[(size_t)t * H], &x[(size_t)t * H] + H, &xn[(size_t)t * H]);
                layer_norm(&xn[(size_t)t * H], w, b, H, m.eps);
            }
        });
    }

    // Softmax attention of one row and head (attend.rs:84-322). Queries are
    // handled one at a time here; the reference's groups of queries share loads
    // only, and each query's sums keep their order whatever its group. A key
    // outside a query's window or band scores -inf over the whole row instead
    // of over the group's span: the extra keys add exact zeros to the lanes'
    // sums and fmaf(0, v, acc) leaves the context's chains unchanged.
    void attention(uint32_t window) {
        const uint32_t H = m.hidden, d = m.d, ld = 3 * H;
        const float scale = 1.0f / std::sqrt((float)d);
        parallel(threads, (size_t)batch * m.heads, [&](size_t task) {
            const uint32_t r = (uint32_t)(task / m.heads), head = (uint32_t)(task % m.heads);
            const uint32_t start = pk.start[r], len = pk.len[r];
            if (len == 0) return;
            const uint32_t lp = (len + kLanes - 1) / kLanes * kLanes;
            const uint8_t *mk = &mask[(size_t)r * seq];
            std::vector<float> masked(lp), sc(lp);
            for (uint32_t j = 0; j < lp; ++j) masked[j] = (j < len && mk[j]) ? 0.0f : kNegInf;
            const float *qv = &qkv[(size_t)start * ld];
            // (With d a multiple of 8, eight keys' chains, or eight context
            // columns' chains, run side by side in AVX2 registers, each in
            // the order below: the same bits.)
            const bool vec = d % 8 == 0;
            std::vector<float> kt;
            if (vec) {
                // K^T of the head: d rows of lp keys, zeros past len.
                kt.assign((size_t)d * lp, 0.0f);
                for (uint32_t j = 0; j < len; ++j)
                    for (uint32_t c = 0; c < d; ++c) kt[(size_t)c * lp + j] = qv[(size_t)j * ld + H + head * d + c];
            }
            for (uint32_t i = 0; i < len; ++i) {
                const float *q = qv + (size_t)i * ld + head * d;
                if (vec) {
                    // 32 keys (four chains of eight) at a time, then 16.
                    uint32_t j0 = 0;
                    for (; j0 + 32 <= lp; j0 += 32) {
                        __m256 a[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
                        for (uint32_t c = 0; c < d; ++c) {
                            const __m256 qc = _mm256_broadcast_ss(q + c);
                            const float *kr = &kt[(size_t)c * lp + j0];
                            for (int g = 0; g < 4; ++g) a[g] = _mm256_fmadd_ps(qc, _mm256_loadu_ps(kr + 8 * g), a[g]);
                        }
                        alignas(32) float acc[32];
                        for (int g = 0; g < 4; ++g) _mm256_store_ps(acc + 8 * g, a[g]);
                        for (uint32_t jj = 0; jj < 32; ++jj) sc[j0 + jj] = acc[jj] * scale + masked[j0 + jj];
                    }
                    for (; j0 < lp; j0 += 16) {
                        __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
                        for (uint32_t c = 0; c < d; ++c) {
                            const __m256 qc = _mm256_broadcast_ss(q + c);
                            a0 = _mm256_fmadd_ps(qc, _mm256_loadu_ps(&kt[(size_t)c * lp + j0]), a0);
                            a1 = _mm256_fmadd_ps(qc, _mm256_loadu_ps(&kt[(size_t)c * lp + j0 + 8]), a1);
                        }
                        alignas(32) float acc[16];
                        _mm256_store_ps(acc, a0);
                        _mm256_store_ps(acc + 8, a1);
                        for (uint32_t jj = 0; jj < 16; ++jj) sc[j0 + jj] = acc[jj] * scale + masked[j0 + jj];
                    }
                } else {
                    for (uint32_t j = 0; j < lp; ++j) {
                        float acc = 0.0f;
                        if (j < len) {
                            const float *k = qv + (size_t)j * ld + H + head * d;
                            for (uint32_t c = 0; c < d; ++c) acc = __builtin_fmaf(q[c], k[c], acc);
                        }
                        // The slots past len hold zeros in the reference's kt.
                        const float s = acc * scale;
                        sc[j] = s + masked[j];
                    }
                }
                if (m.ahead < len)
                    for (uint32_t j = std::min<uint64_t>((uint64_t)i + m.ahead + 1, len); j < len; ++j) sc[j] = kNegInf;
                if (window < len)
                    for (uint32_t j = 0; j < len; ++j)
                        if ((j + window < i) || (j > i + window)) sc[j] = kNegInf;
                float mx = kNegInf;
                for (uint32_t j = 0; j < lp; ++j)
                    if (sc[j] > mx) mx = sc[j];
                float *out = &ctx[(size_t)(start + i) * H + head * d];
                if (mx == kNegInf) {
                    for (uint32_t c = 0; c < d; ++c) out[c] = 0.0f;
                    continue;
                }
                for (uint32_t j = 0; j < lp; ++j) sc[j] = cephes_exp(sc[j] - mx);
                float lanes[kLanes];
                for (uint32_t l = 0; l < kLanes; ++l) lanes[l] = 0.0f;
                for (uint32_t j = 0; j < lp; ++j) lanes[j % kLanes] += sc[j];
                for (uint32_t w = kLanes / 2; w > 0; w /= 2)
                    for (uint32_t l = 0; l < w; ++l) lanes[l] += lanes[l + w];
                const float inv = 1.0f / lanes[0];
                for (uint32_t j = 0; j < lp; ++j) sc[j] = sc[j] * inv;
                if (vec) {
                    // Up to eight groups of eight columns side by side.
                    for (uint32_t c0 = 0; c0 < d; c0 += 64) {
                        const uint32_t ng = std::min<uint32_t>(8, (d - c0) / 8);
                        __m256 acc[8];
                        for (uint32_t g = 0; g < 8; ++g) acc[g] = _mm256_setzero_ps();
                        for (uint32_t j = 0; j < len; ++j) {
                            const __m256 p = _mm256_broadcast_ss(&sc[j]);
                            const float *vr = qv + (size_t)j * ld + 2 * H + head * d + c0;
                            for (uint32_t g = 0; g < ng; ++g) acc[g] = _mm256_fmadd_ps(p, _mm256_loadu_ps(vr + 8 * g), acc[g]);
                        }
                        for (uint32_t g = 0; g < ng; ++g) _mm256_storeu_ps(out + c0 + 8 * g, acc[g]);
                    }
                } else {
                    for (uint32_t c = 0; c < d; ++c) {
                        float acc = 0.0f;
                        for (uint32_t j = 0; j < len; ++j)
                            acc = __builtin_fmaf(sc[j], qv[(size_t)j * ld + 2 * H + head * d + c], acc);
                        out[c] = acc;
                    }
                }
            }
        });
    }

    // The mean of row r's live tokens among columns [c0, c1) (or of every
    // column there when none is live) from states `src`, output_dim values,
    // summed in F32 in column order, times one over the count (mod.rs:443-468).
    void mean(const float *src, uint32_t r, uint32_t c0, uint32_t c1, float *dst, uint32_t od) const {
        const uint32_t H = m.hidden;
        for (uint32_t i = 0; i < od; ++i) dst[i] = 0.0f;
        const uint8_t *mk = &mask[(size_t)r * seq];
        bool live_only = false;
        for (uint32_t p = c0; p < c1; ++p) live_only |= mk[p] != 0;
        uint32_t n = 0;
        for (uint32_t p = c0; p < c1; ++p) {
            if (live_only && !mk[p]) continue;
            const float *row = src + (size_t)(pk.start[r] + p) * H;
            for (uint32_t i = 0; i < od; ++i) dst[i] += row[i];
            ++n;
        }
        const float inv = 1.0f / (float)n;
        for (uint32_t i = 0; i < od; ++i) dst[i] *= inv;
    }

    // L2 with the norm summed in F64, floored at 1e-12 (mod.rs:470-482).
    static void finish(float *dst, uint32_t od, uint32_t normalize) {
        if (normalize != TURBO_NORMALIZE_L2) return;
        double s = 0.0;
        for (uint32_t i = 0; i < od; ++i) s += (double)dst[i] * (double)dst[i];
        const double norm = std::max(std::sqrt(s), 1e-12);
        const float inv = (float)(1.0 / norm);
        for (uint32_t i = 0; i < od; ++i) dst[i] *= inv;
    }
};

void encode(const Model &m, const turbo_backend_embed_rows *rows, const turbo_token_range *ranges, uint32_t count,
            uint32_t threads, float *out, float *hidden) {
    if (rows->head) throw Failure(TURBO_E_UNSUPPORTED, "encode pools vectors; the head is applied after it");
    // Layer reads (core/src/cpu/encoder/mod.rs:292-303): the last `taps`
    // layers' states pooled per range, or with tap_alone the model cut after
    // the first of them, read plainly.
    const uint32_t taps = rows->taps > 1 ? rows->taps : 1;
    if (taps > 1 && (count == 0 || taps > m.layers))
        throw Failure(TURBO_E_INVALID_ARGUMENT, "oracle: layer reads need ranges and at most the model's layers");
    if (rows->tap_alone && taps == 1) throw Failure(TURBO_E_INVALID_ARGUMENT, "oracle: tap_alone with one layer read");
    const uint32_t nl = rows->tap_alone ? m.layers + 1 - taps : m.layers;
    const uint32_t reads = rows->tap_alone ? 1 : taps;
    Run run(m, threads);
    const uint32_t B = rows->batch, S = rows->seq, stride = rows->row_stride ? rows->row_stride : rows->seq;
    run.batch = B;
    run.seq = S;
    run.ids.resize((size_t)B * S);
    run.types.resize((size_t)B * S);
    run.mask.resize((size_t)B * S);
    for (uint32_t r = 0; r < B; ++r)
        for (uint32_t p = 0; p < S; ++p) {
            const size_t src = (size_t)r * stride + p, dst = (size_t)r * S + p;
            run.ids[dst] = (uint32_t)rows->ids[src];
            run.mask[dst] = (uint8_t)rows->mask[src];
            run.types[dst] = rows->types ? (uint32_t)rows->types[src] : 0;
        }
    run.pk = pack(rows->mask, B, S, stride, ranges, count);
    const uint32_t T = run.T(), H = m.hidden, I = m.inter;
    run.x.assign((size_t)T * H, 0.0f);
    run.qkv.assign((size_t)T * 3 * H, 0.0f);
    run.ctx.assign((size_t)T * H, 0.0f);
    run.ffn.assign((size_t)T * I, 0.0f);
    if (m.modern) run.xn.assign((size_t)T * H, 0.0f);
    run.lookup();
    float *x = run.x.data();
    auto residual = [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc, const Linear &w) {
        float *y = x + (size_t)t * H + c0;
        for (uint32_t j = 0; j < cols; ++j) y[j] += acc[j] + w.bias[c0 + j];
    };
    const uint32_t od = rows->output_dim;
    // Each range pooled from src into block k of out (mod.rs:336-345).
    auto pool_ranges = [&](const float *src, uint32_t k) {
        for (uint32_t i = 0; i < count; ++i) {
            const turbo_token_range g = ranges[i];
            float *dst = out + ((size_t)k * count + i) * od;
            run.mean(src, g.row, g.start, std::min(g.end, run.pk.len[g.row]), dst, od);
            Run::finish(dst, od, rows->normalize);
        }
    };
    // After layer l: a read before the last layer run goes into its block; a
    // ModernBERT read is final_norm(x) (rotary/mod.rs:161-168).
    std::vector<float> normed;
    auto tapped = [&](uint32_t l) {
        if (reads == 1 || l + 1 >= nl || l + reads < nl) return;
        const float *src = x;
        if (m.modern) {
            normed.assign(run.x.begin(), run.x.end());
            run.norm(normed.data(), m.final_w, nullptr);
            src = normed.data();
        }
        pool_ranges(src, l + reads - nl);
    };
    for (uint32_t l = 0; l < nl; ++l) {
        const Layer &L = m.ls[l];
        if (!m.rotary) {
            run.linear(x, H, L.qkv, [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc) {
                float *y = &run.qkv[(size_t)t * 3 * H + c0];
                for (uint32_t j = 0; j < cols; ++j) y[j] = acc[j] + L.qkv.bias[c0 + j];
            });
            if (m.deberta) run.attention_deberta(l);
            else run.attention(UINT32_MAX);
            run.linear(run.ctx.data(), H, L.out,
                       [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc) { residual(t, c0, cols, acc, L.out); });
            run.norm(x, L.attn_ln_w, L.attn_ln_b);
            run.linear(x, H, L.ffn_in, [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc) {
                float *y = &run.ffn[(size_t)t * I + c0];
                for (uint32_t j = 0; j < cols; ++j) y[j] = gelu_erf(acc[j] + L.ffn_in.bias[c0 + j]);
            });
            run.linear(run.ffn.data(), I, L.ffn_out, [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc) {
                residual(t, c0, cols, acc, L.ffn_out);
            });
            run.norm(x, L.ffn_ln_w, L.ffn_ln_b);
            tapped(l);
            continue;
        }
        // Rotary layer (rotary/mod.rs:119-160).
        const bool global = m.global_every == 0 || l % m.global_every == 0;
        const size_t half = (size_t)m.positions * m.pairs;
        const float *cosb = m.rope + (global ? 0 : 2 * half), *sinb = cosb + half;
        const float *src = x;
        if (m.modern && l > 0) {
            run.norm_into(L.attn_ln_w, nullptr);
            src = run.xn.data();
        }
        // RoPE epilogue over pair-adjacent Q and K columns (pairs.rs:66-108).
        run.linear(src, H, L.qkv, [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc) {
            float *y = &run.qkv[(size_t)t * 3 * H];
            const uint32_t p = run.column(t);
            for (uint32_t j = 0; j < cols; j += 2) {
                const uint32_t c = c0 + j;
                const float x1 = acc[j] + L.qkv.bias[c], x2 = acc[j + 1] + L.qkv.bias[c + 1];
                if (c >= 2 * H) {
                    y[c] = x1;
                    y[c + 1] = x2;
                    continue;
                }
                const uint32_t pr = (c % m.d) / 2;
                const float cs = cosb[(size_t)p * m.pairs + pr], sn = sinb[(size_t)p * m.pairs + pr];
                const float a1 = x1 * cs, b1 = x2 * sn, a2 = x2 * cs, b2 = x1 * sn;
                y[c] = a1 - b1;
                y[c + 1] = a2 + b2;
            }
        });
        run.attention(global ? UINT32_MAX : m.window);
        run.linear(run.ctx.data(), H, L.out,
                   [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc) { residual(t, c0, cols, acc, L.out); });
        if (!m.modern) run.norm(x, L.attn_ln_w, L.attn_ln_b);
        else run.norm_into(L.ffn_ln_w, nullptr);
        // Gated epilogue: y[t, c/2] = act(gate) * up (pairs.rs:111-144).
        run.linear(m.modern ? run.xn.data() : x, H, L.ffn_in, [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc) {
            float *y = &run.ffn[(size_t)t * I + c0 / 2];
            for (uint32_t j = 0; j < cols / 2; ++j) {
                const float g = acc[2 * j] + L.ffn_in.bias[c0 + 2 * j];
                const float u = acc[2 * j + 1] + L.ffn_in.bias[c0 + 2 * j + 1];
                const float v = (m.silu_act ? silu(g) : gelu_erf(g)) * u, lim = gated_limit.load();
                y[j] = lim > 0.0f ? (v > lim ? lim : v < -lim ? -lim : v) : v;
            }
        });
        run.linear(run.ffn.data(), I, L.ffn_out,
                   [&](uint32_t t, uint32_t c0, uint32_t cols, const float *acc) { residual(t, c0, cols, acc, L.ffn_out); });
        if (!m.modern) run.norm(x, L.ffn_ln_w, L.ffn_ln_b);
        tapped(l);
    }
    if (m.modern) run.norm(x, m.final_w, nullptr);
    if (hidden) std::copy(run.x.begin(), run.x.end(), hidden);
    if (count == 0) {
        for (uint32_t r = 0; r < B; ++r) {
            float *dst = out + (size_t)r * od;
            const uint32_t start = run.pk.start[r], len = run.pk.len[r];
            if (rows->pooling == TURBO_POOLING_CLS) std::copy(x + (size_t)start * H, x + (size_t)start * H + od, dst);
            else if (rows->pooling == TURBO_POOLING_LAST)
                std::copy(x + (size_t)(start + len - 1) * H, x + (size_t)(start + len - 1) * H + od, dst);
            else run.mean(x, r, 0, len, dst, od);
            Run::finish(dst, od, rows->normalize);
        }
        return;
    }
    pool_ranges(x, reads - 1);
}

void say(char *why, uint32_t len, const char *msg) {
    if (why && len) {
        std::snprintf(why, len, "%s", msg);
    }
}

}  // namespace

// Seconds the last oracle_encode spent encoding (its rows' pass alone, not
// the weights' layout before it): the benchmark's CPU figure.
std::atomic<double> last_encode_s{0.0};

extern "C" {

int32_t oracle_encode(const turbo_backend_model *d, const turbo_backend_embed_rows *rows,
                      const turbo_token_range *ranges, uint32_t count, uint32_t threads, float *out, float *hidden,
                      char *why, uint32_t why_len) {
    try {
        if (threads == 0) threads = std::max(1u, std::thread::hardware_concurrency());
        Model m;
        load(m, d);
        if (!rows->head) {
            const auto t0 = std::chrono::steady_clock::now();
            encode(m, rows, ranges, count, threads, out, hidden);
            last_encode_s.store(std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
            say(why, why_len, "");
            return TURBO_OK;
        }
        // A range write through the span head (turbo_backend.h:418-422):
        // each range's mean over all hidden values, not normalized, then
        // the head's rows summed in F64 from the bias and rounded to F32
        // once (core/src/qa/session.rs:268-276).
        if (!d->head || d->head_out == 0 || count == 0)
            throw Failure(TURBO_E_INVALID_ARGUMENT, "oracle: a head write needs ranges and a model with a head");
        const uint32_t H = d->hidden, O = d->head_out;
        const turbo_backend_tensor &hw = d->head[0], &hb = d->head[1];
        if (hw.bytes != (uint64_t)O * H * 4 || hb.bytes != (uint64_t)O * 4)
            throw Failure(TURBO_E_INVALID_ARGUMENT, "oracle: the head is [head_out, hidden] and [head_out] F32");
        turbo_backend_embed_rows plain = *rows;
        plain.head = 0;
        plain.output_dim = H;
        plain.normalize = TURBO_NORMALIZE_NONE;
        std::vector<float> v((size_t)count * H);
        encode(m, &plain, ranges, count, threads, v.data(), hidden);
        const float *w = static_cast<const float *>(hw.data), *b = static_cast<const float *>(hb.data);
        for (uint32_t i = 0; i < count; ++i)
            for (uint32_t o = 0; o < O; ++o) {
                double acc = (double)b[o];
                for (uint32_t c = 0; c < H; ++c) acc += (double)w[(size_t)o * H + c] * (double)v[(size_t)i * H + c];
                out[(size_t)i * O + o] = (float)acc;
            }
        say(why, why_len, "");
        return TURBO_OK;
    } catch (const Failure &f) {
        say(why, why_len, f.what());
        return f.code;
    } catch (const std::exception &e) {
        say(why, why_len, e.what());
        return TURBO_E_INTERNAL;
    }
}

uint32_t oracle_pack(const int32_t *mask, uint32_t batch, uint32_t seq, uint32_t row_stride,
                     const turbo_token_range *ranges, uint32_t count, uint32_t *start, uint32_t *len, uint32_t *at) {
    const Packing p = pack(mask, batch, seq, row_stride ? row_stride : seq, ranges, count);
    std::copy(p.start.begin(), p.start.end(), start);
    std::copy(p.len.begin(), p.len.end(), len);
    std::copy(p.at.begin(), p.at.end(), at);
    return p.tokens;
}

float oracle_exp(float x) { return cephes_exp(x); }

double oracle_last_encode_seconds() { return last_encode_s.load(); }
void oracle_set_gated_limit(float limit) { gated_limit.store(limit); }
void oracle_set_pinning(int32_t on) { pin_threads.store(on ? 1 : 0); }
uint32_t oracle_deberta_bucket(int64_t distance, uint32_t buckets, uint32_t maximum) {
    return deberta_bucket(distance, buckets, maximum);
}
float oracle_gelu(float x) { return gelu_erf(x); }
float oracle_silu(float x) { return silu(x); }
void oracle_layer_norm(float *y, const float *w, const float *b, uint32_t n, float eps) { layer_norm(y, w, b, n, eps); }

// int8: step = (max - min) / 255 in F32, 1 where that is 0; the code is
// clamp(floor((x - min) / step), 0, 255) - 128, a NaN in the bottom bucket
// (core/src/quantize.rs:60-70). ubinary: bit x > 0, eight to a byte, the first
// value in the top bit, a last byte padded with 0 bits (:72-83).
void oracle_quantize(const float *x, uint32_t rows, uint32_t dim, uint32_t mode, const float *ranges, uint8_t *out) {
    if (mode == 2) {
        for (uint32_t r = 0; r < rows; ++r)
            for (uint32_t d = 0; d < dim; ++d) {
                const float lo = ranges[d], hi = ranges[dim + d];
                float step = (hi - lo) / 255.0f;
                if (step == 0.0f) step = 1.0f;
                float q = std::floor((x[(size_t)r * dim + d] - lo) / step);
                q = q != q ? 0.0f : q < 0.0f ? 0.0f : q > 255.0f ? 255.0f : q;
                out[(size_t)r * dim + d] = (uint8_t)(int8_t)((int)q - 128);
            }
    } else {
        const uint32_t per = (dim + 7) / 8;
        for (uint32_t r = 0; r < rows; ++r)
            for (uint32_t b = 0; b < per; ++b) {
                uint32_t byte = 0;
                for (uint32_t k = 0; k < 8 && 8 * b + k < dim; ++k)
                    if (x[(size_t)r * dim + 8 * b + k] > 0.0f) byte |= 0x80u >> k;
                out[(size_t)r * per + b] = (uint8_t)byte;
            }
    }
}

}  // extern "C"
