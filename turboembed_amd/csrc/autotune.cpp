// Choices strings: format and parse (the format is described in autotune.h).
#include "autotune.h"

#include <cstring>
#include <vector>

#include "kernels.h"

namespace rocm {

uint32_t forced_knobs(const Choices &c) {
    uint32_t k = 0;
    for (int b = 0; b < c.bins; ++b) {
        k |= c.bin[b].attn_forced;
        for (int g = 0; g < G_COUNT; ++g) k |= c.bin[b].tile_forced[g];
    }
    return k;
}

bool all_forced(const Choices &c) {
    for (int b = 0; b < c.bins; ++b) {
        if (!c.bin[b].attn_forced) return false;
        for (int g = 0; g < G_COUNT; ++g)
            if (!c.bin[b].tile_forced[g]) return false;
    }
    return true;
}

std::string format_choices(const Choices &c) {
    std::string s;
    for (int b = 0; b < c.bins; ++b) {
        const BinChoice &x = c.bin[b];
        s += BIN_NAME[b];
        s += ':';
        for (int g = 0; g < G_COUNT; ++g) {
            s += GEMM_NAME[g];
            s += '=';
            s += gemm_tile_name(x.tile[g]);
            s += ',';
        }
        s += "attn=";
        s += ATTN_NAME[x.attn >= 0 && x.attn < ATTN_PATHS ? x.attn : ATTN_MFMA];
        s += ';';
    }
    const uint32_t k = forced_knobs(c);
    s += "forced=";
    if (!k) s += "none";
    if (k & KNOB_TILE) s += "tile";
    if ((k & KNOB_TILE) && (k & KNOB_ATTN)) s += ',';
    if (k & KNOB_ATTN) s += "attn";
    return s;
}

namespace {

struct Item {
    int bin;   // -1: every bin
    std::string key, value;
};

bool split_items(const char *s, std::vector<Item> *out, std::string *why) {
    const std::string all(s);
    size_t i = 0;
    while (i < all.size()) {
        size_t semi = all.find(';', i);
        if (semi == std::string::npos) semi = all.size();
        std::string part = all.substr(i, semi - i);
        i = semi + 1;
        while (!part.empty() && part.front() == ' ') part.erase(part.begin());
        while (!part.empty() && part.back() == ' ') part.pop_back();
        if (part.empty()) continue;
        int bin = -1;
        const size_t colon = part.find(':');
        std::string body = part;
        if (colon != std::string::npos) {
            const std::string name = part.substr(0, colon);
            body = part.substr(colon + 1);
            if (name != "all") {
                bin = -2;
                for (int b = 0; b < BINS; ++b)
                    if (name == BIN_NAME[b]) bin = b;
                if (bin == -2) {
                    *why = "unknown bin '" + name + "'";
                    return false;
                }
            }
        }
        size_t j = 0;
        while (j <= body.size()) {
            size_t comma = body.find(',', j);
            if (comma == std::string::npos) comma = body.size();
            const std::string kv = body.substr(j, comma - j);
            j = comma + 1;
            if (kv.empty()) continue;
            const size_t eq = kv.find('=');
            if (eq == std::string::npos) {
                *why = "item '" + kv + "' has no '='";
                return false;
            }
            out->push_back({bin, kv.substr(0, eq), kv.substr(eq + 1)});
        }
    }
    return true;
}

}  // namespace

bool parse_choices(const char *s, Choices *c, bool force, std::string *why) {
    if (!s) return true;
    std::vector<Item> items;
    if (!split_items(s, &items, why)) return false;
    Choices next = *c;
    for (const Item &it : items) {
        if (it.key == "forced") continue;
        const int b0 = it.bin < 0 ? 0 : it.bin, b1 = it.bin < 0 ? BINS : it.bin + 1;
        int slot = -1;
        for (int g = 0; g < G_COUNT; ++g)
            if (it.key == GEMM_NAME[g]) slot = g;
        if (slot >= 0 || it.key == "gemm") {
            const int tile = gemm_tile_by_name(it.value.data(), it.value.size());
            if (tile < 0) {
                *why = "unknown tile '" + it.value + "' for " + it.key;
                return false;
            }
            for (int b = b0; b < b1; ++b)
                for (int g = 0; g < G_COUNT; ++g) {
                    if (slot >= 0 && g != slot) continue;
                    next.bin[b].tile[g] = tile;
                    if (force) next.bin[b].tile_forced[g] = KNOB_TILE;
                }
        } else if (it.key == "attn" || it.key == "attention") {
            int path = -1;
            for (int a = 0; a < ATTN_PATHS; ++a)
                if (it.value == ATTN_NAME[a]) path = a;
            if (path < 0) {
                *why = "unknown attention path '" + it.value + "'";
                return false;
            }
            for (int b = b0; b < b1; ++b) {
                next.bin[b].attn = path;
                if (force) next.bin[b].attn_forced = KNOB_ATTN;
            }
        } else {
            *why = "unknown item '" + it.key + "'";
            return false;
        }
    }
    *c = next;
    return true;
}

}  // namespace rocm
