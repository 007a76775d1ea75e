// A session's kernel choices: the GEMM block shape each of a layer's four
// products takes and the attention path, per bin of packed tokens. They come
// from the backend's rule, a cached choices string, the tuner's timings, or
// TURBO_ROCM_CHOICES, which forces them in every mode.
//
// The bins are the reference's (core/cuda/autotune.h:46-51; the core keys
// its cache by them, core/src/tuning.rs:119-126): bin i holds runs of more
// than BIN_EDGE[i - 1] and at most BIN_EDGE[i] packed tokens; a session has
// the bins its max_batch x max_seq reaches.
//
// A choices string, as format_choices writes it and parse_choices reads it:
//   <bin>:qkv=<tile>,out=<tile>,ffn1=<tile>,ffn2=<tile>,attn=<mfma|mfma128|simple>;...;forced=<knob>,...
// with a tile as the GEMM launcher names it ("auto" is its rule on the
// run's own shape). "all:" names every bin; the older single items
// "gemm=<tile>" and "attention=<path>" mean every product and every bin.
#pragma once

#include <stdint.h>

#include <climits>
#include <string>

namespace rocm {

constexpr int BINS = 5;
constexpr int BIN_EDGE[BINS] = {256, 1024, 4096, 16384, INT32_MAX};
constexpr const char *BIN_NAME[BINS] = {"le256", "le1k", "le4k", "le16k", "gt16k"};

// The bins a session of tcap packed tokens at most has: one at least.
inline int bins_for(uint64_t tcap) {
    int n = 1;
    while (n < BINS && (uint64_t)BIN_EDGE[n - 1] < tcap) ++n;
    return n;
}

// The bin of a run of `tokens` packed tokens, of `bins` bins.
inline int bin_of(uint32_t tokens, int bins) {
    int b = 0;
    while (b + 1 < bins && tokens > (uint32_t)BIN_EDGE[b]) ++b;
    return b;
}

// The token count the tuner times a bin at: its upper edge, or the
// session's capacity for the last bin it has.
inline uint32_t bin_tokens(int b, uint64_t tcap) {
    const uint64_t edge = (uint64_t)BIN_EDGE[b];
    return (uint32_t)(edge < tcap ? edge : tcap);
}

enum GemmSlot : int { G_QKV = 0, G_OUT = 1, G_FFN1 = 2, G_FFN2 = 3, G_COUNT = 4 };
constexpr const char *GEMM_NAME[G_COUNT] = {"qkv", "out", "ffn1", "ffn2"};

// What a choice was fixed by rather than left to the rule or the tuner.
enum Knob : uint32_t { KNOB_TILE = 1, KNOB_ATTN = 2 };

// The attention paths: the matrix-core kernel on 256-query workgroups of 8
// waves, or on 128-query workgroups of 4 (twice the workgroups, each
// streaming its keys for half the queries), and the scalar kernel.
enum AttnPath : int { ATTN_MFMA = 0, ATTN_SIMPLE = 1, ATTN_MFMA128 = 2, ATTN_PATHS = 3 };
constexpr const char *ATTN_NAME[ATTN_PATHS] = {"mfma", "simple", "mfma128"};

struct BinChoice {
    int tile[G_COUNT] = {0, 0, 0, 0};   // 0: the launcher's rule on the run's shape
    int attn = ATTN_MFMA;
    uint32_t tile_forced[G_COUNT] = {0, 0, 0, 0};
    uint32_t attn_forced = 0;
};

struct Choices {
    int bins = 1;
    BinChoice bin[BINS];
};

// The knobs forced anywhere in c (KNOB_* bits).
uint32_t forced_knobs(const Choices &c);
// Whether every GEMM's tile and every attention path was forced.
bool all_forced(const Choices &c);

std::string format_choices(const Choices &c);

// Sets what s names, marking it forced when `force`; bins the session does
// not have are left alone. False with why filled for an unknown item or
// value (nothing is changed then).
bool parse_choices(const char *s, Choices *c, bool force, std::string *why);

}  // namespace rocm
