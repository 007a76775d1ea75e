// The checks TurboEmbed's core makes of a write before it calls a backend
// (reference core/src/session/tokens.rs:274-384), restated so that a caller
// without the Rust core, this project's Python host side, holds rows to the
// same rules and gets the same statuses. Host code only.
#include <cstdio>
#include <string>

#include "turbo/turbo_seam.h"
#include "turbo_rocm.h"

namespace {

int32_t refuse(turbo_error *err, int32_t code, const std::string &m) {
    if (err) {
        err->code = code;
        err->field = 0;
        std::snprintf(err->message, sizeof err->message, "%s", m.c_str());
    }
    return code;
}

int32_t ok(turbo_error *err) {
    if (err) {
        err->code = 0;
        err->field = 0;
        err->message[0] = 0;
    }
    return TURBO_OK;
}

}  // namespace

extern "C" {

int32_t turbo_rocm_check_tokens(uint32_t batch, uint32_t seq, uint32_t row_stride, const int32_t *ids,
                                const int32_t *mask, const int32_t *types, uint32_t max_batch, uint32_t max_seq,
                                uint32_t vocab, uint32_t token_types, uint32_t max_tokens, turbo_error *err) {
    if (batch == 0 || seq == 0)
        return refuse(err, TURBO_E_INVALID_SHAPE,
                      "batch " + std::to_string(batch) + " by seq " + std::to_string(seq) + ": neither may be 0");
    if (batch > max_batch)
        return refuse(err, TURBO_E_CAPACITY, "batch " + std::to_string(batch) + " is over the session's max_batch " +
                                                 std::to_string(max_batch));
    if (seq > max_seq)
        return refuse(err, TURBO_E_CAPACITY,
                      "seq " + std::to_string(seq) + " is over the session's max_seq " + std::to_string(max_seq));
    const uint32_t stride = row_stride == 0 ? seq : row_stride;
    if (stride < seq)
        return refuse(err, TURBO_E_INVALID_SHAPE,
                      "row_stride " + std::to_string(stride) + " is under seq " + std::to_string(seq));
    if (!ids || !mask) return refuse(err, TURBO_E_INVALID_ARGUMENT, "ids and mask may not be NULL");
    const uint32_t ntypes = token_types ? token_types : 1;
    for (uint32_t r = 0; r < batch; ++r) {
        const size_t at = (size_t)r * stride;
        uint32_t live = 0;
        for (uint32_t p = 0; p < seq; ++p) {
            const int32_t id = ids[at + p], m = mask[at + p];
            if (id < 0 || (uint32_t)id >= vocab)
                return refuse(err, TURBO_E_INVALID_ARGUMENT,
                              "ids[" + std::to_string(r) + "][" + std::to_string(p) + "] is " + std::to_string(id) +
                                  ", outside the model's vocabulary of " + std::to_string(vocab));
            if (m == 1) live = p + 1;
            else if (m != 0)
                return refuse(err, TURBO_E_INVALID_ARGUMENT, "mask[" + std::to_string(r) + "][" + std::to_string(p) +
                                                                 "] is " + std::to_string(m) + ", not 0 or 1");
            if (types && (types[at + p] < 0 || (uint32_t)types[at + p] >= ntypes))
                return refuse(err, TURBO_E_INVALID_ARGUMENT,
                              "types[" + std::to_string(r) + "][" + std::to_string(p) + "] is " +
                                  std::to_string(types[at + p]) + ", and the model has " + std::to_string(ntypes) +
                                  " token types");
        }
        if (live == 0)
            return refuse(err, TURBO_E_INVALID_ARGUMENT,
                          "mask row " + std::to_string(r) + " has no 1: a row needs a token");
        if (max_tokens != 0 && live > max_tokens)
            return refuse(err, TURBO_E_CAPACITY, "row " + std::to_string(r) + ": " + std::to_string(live) +
                                                     " tokens through its last live one is over max_tokens " +
                                                     std::to_string(max_tokens));
    }
    return ok(err);
}

int32_t turbo_rocm_check_ranges(uint32_t batch, uint32_t seq, uint32_t row_stride, const int32_t *mask,
                                const turbo_token_range *ranges, uint32_t count, uint32_t max_ranges,
                                turbo_error *err) {
    if (count == 0) return refuse(err, TURBO_E_INVALID_ARGUMENT, "count is 0: a run needs at least one range");
    if (!ranges) return refuse(err, TURBO_E_INVALID_ARGUMENT, "ranges is NULL and count is " + std::to_string(count));
    if (count > max_ranges)
        return refuse(err, TURBO_E_CAPACITY, std::to_string(count) + " ranges is over the session's max_ranges " +
                                                 std::to_string(max_ranges));
    const uint32_t stride = row_stride == 0 ? seq : row_stride;
    for (uint32_t i = 0; i < count; ++i) {
        const turbo_token_range g = ranges[i];
        const std::string at = "ranges[" + std::to_string(i) + "]: ";
        if (g.row >= batch)
            return refuse(err, TURBO_E_INVALID_ARGUMENT,
                          at + "row " + std::to_string(g.row) + " is not under batch " + std::to_string(batch));
        if (g.start >= g.end)
            return refuse(err, TURBO_E_INVALID_ARGUMENT,
                          at + "start " + std::to_string(g.start) + " is not under end " + std::to_string(g.end));
        if (g.end > seq)
            return refuse(err, TURBO_E_INVALID_ARGUMENT,
                          at + "end " + std::to_string(g.end) + " is over seq " + std::to_string(seq));
        bool live = false;
        for (uint32_t p = g.start; p < g.end && !live; ++p) live = mask[(size_t)g.row * stride + p] == 1;
        if (!live)
            return refuse(err, TURBO_E_UNSUPPORTED_OPTION,
                          at + "columns " + std::to_string(g.start) + " to " + std::to_string(g.end) + " of row " +
                              std::to_string(g.row) +
                              " hold no token whose mask is 1, and the rocm backend does not compute mask-0 columns");
    }
    return ok(err);
}

}  // extern "C"
