// The rocm backend's host side: the turbo_backend table TurboEmbed's core
// calls (reference include/turbo/turbo_backend.h:455-627), over HIP on
// MI355X (gfx950) devices.
//
// Ownership follows the seam: a context owns a HIP stream; a model owns its
// weights on the device (F32, plus the narrowed copies a session's precision
// needs, made on first need and shared); a session owns every byte a run
// touches, allocated at creation, so a run allocates nothing. A run is one
// pass of kernels on the context's stream, then one synchronization.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "turbo/turbo_seam.h"
#include "turbo_rocm.h"
#include "kernels.h"
#include "session.h"

using namespace rocm;

namespace rocm {

// ---- Errors ---------------------------------------------------------------------

[[noreturn]] void fail(int32_t code, const std::string &m, uint32_t field) { throw Failure{code, field, m}; }

void check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        fail(TURBO_E_RUNTIME, std::string("rocm: ") + what + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
    }
}

void fill(turbo_error *err, int32_t code, uint32_t field, const std::string &m) {
    if (!err) return;
    err->code = code;
    err->field = field;
    std::snprintf(err->message, sizeof err->message, "%s", m.c_str());
}

std::atomic<uint64_t> device_allocs{0};
static thread_local uint64_t device_allocs_here = 0;

void counted_device_alloc() {
    device_allocs.fetch_add(1, std::memory_order_relaxed);
    ++device_allocs_here;
}

uint64_t device_allocs_on_thread() { return device_allocs_here; }

void *dev_alloc(size_t bytes, const char *what) {
    void *p = nullptr;
    if (bytes == 0) bytes = 256;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
        (void)hipGetLastError();
        fail(TURBO_E_OUT_OF_MEMORY,
             std::string("rocm: ") + what + ": " + std::to_string(bytes) + " bytes of device memory");
    }
    check(e, what);
    counted_device_alloc();
    return p;
}

// Never throws: the release functions use it too. A device that cannot be
// made current fails the next HIP call instead.
OnDevice::OnDevice(int ordinal) {
    if (hipGetDevice(&prev) != hipSuccess) {
        (void)hipGetLastError();
        prev = -1;
    }
    if (prev != ordinal && hipSetDevice(ordinal) != hipSuccess) (void)hipGetLastError();
}
OnDevice::~OnDevice() {
    int now = -1;
    if (prev >= 0 && hipGetDevice(&now) == hipSuccess && now != prev) (void)hipSetDevice(prev);
}

// Only gfx950 devices are listed: the kernels are built for that alone.
const std::vector<int> &devices() {
    static std::vector<int> list;
    static std::once_flag once;
    std::call_once(once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();
            return;
        }
        for (int i = 0; i < n; ++i) {
            hipDeviceProp_t p;
            if (hipGetDeviceProperties(&p, i) != hipSuccess) {
                (void)hipGetLastError();
                continue;
            }
            if (std::strncmp(p.gcnArchName, "gfx950", 6) == 0) list.push_back(i);
        }
    });
    return list;
}

void Context::say(uint32_t level, const std::string &m) const {
    if (!log) return;
    turbo_text t{m.c_str(), m.size()};
    log(log_user_data, level, t);
}

}  // namespace rocm

namespace {

#define ROCM_STR2(x) #x
#define ROCM_STR(x) ROCM_STR2(x)
// The HIP runtime this build compiled against.
constexpr const char *RUNTIME_VERSION =
    "HIP " ROCM_STR(HIP_VERSION_MAJOR) "." ROCM_STR(HIP_VERSION_MINOR) "." ROCM_STR(HIP_VERSION_PATCH);
const char *runtime_version_string() { return RUNTIME_VERSION; }

// ---- Devices and capability ---------------------------------------------------------

int32_t device_count(uint32_t *out, turbo_error *err) {
    return guarded(err, [&] {
        *out = (uint32_t)devices().size();
        return TURBO_OK;
    });
}

int32_t device_info(uint32_t ordinal, turbo_device_info *out, turbo_error *err) {
    return guarded(err, [&] {
        if (ordinal >= devices().size()) fail(TURBO_E_DEVICE_NOT_FOUND, "rocm: no device " + std::to_string(ordinal));
        const int dev = devices()[ordinal];
        hipDeviceProp_t p;
        check(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
        OnDevice on(dev);
        size_t free_b = 0, total_b = 0;
        check(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
        int driver = 0;
        (void)hipDriverGetVersion(&driver);
        out->kind = TURBO_DEVICE_GPU;
        out->ordinal = ordinal;
        out->unified_memory = 0;
        out->memory_total = total_b;
        out->memory_free = free_b;
        std::snprintf(out->arch, sizeof out->arch, "%s", "mi355x");
        std::snprintf(out->name, sizeof out->name, "%s (%s)", p.name, p.gcnArchName);
        std::snprintf(out->vendor, sizeof out->vendor, "%s", "AMD");
        std::snprintf(out->runtime_version, sizeof out->runtime_version, "%s", runtime_version_string());
        std::snprintf(out->driver_version, sizeof out->driver_version, "%d", driver);
        return TURBO_OK;
    });
}

// Fields of turbo_embed_options a run honors: normalize (4), pooling (5)
// and output_dim (6), every value of each; layers (9) and layer_alone (10),
// read from the BERT, RoBERTa, ModernBERT and nomic-bert encoders. Field n
// is bit n - 1 (core/src/session/tokens.rs:157-162).
constexpr uint32_t EMBED_HONORED = (1u << 3) | (1u << 4) | (1u << 5) | (1u << 8) | (1u << 9);

// Every task the core maps onto the embedding encoder runs here: EMBED,
// RERANK (CLS rows for the core's host head) and EXTRACTIVE_QA (range writes
// through the span head, token_head = 1). The core asks with the model's own
// task before it opens the session with EMBED (reference
// core/src/session/create.rs:61-62, 93-111; the CUDA backend answers
// EXPERIMENTAL whatever the task, core/cuda/backend.cpp:411-434).
int32_t capability(uint32_t ordinal, uint32_t task, uint32_t precision, uint32_t *status, uint32_t *dtype,
                   uint32_t *options_honored, char *reason, uint32_t reason_len, turbo_error *err) {
    return guarded(err, [&] {
        if (ordinal >= devices().size()) fail(TURBO_E_DEVICE_NOT_FOUND, "rocm: no device " + std::to_string(ordinal));
        if (task != TURBO_TASK_EMBED && task != TURBO_TASK_RERANK && task != TURBO_TASK_EXTRACTIVE_QA) {
            *status = TURBO_CAP_UNSUPPORTED;
            *dtype = 0;
            *options_honored = 0;
            if (reason_len)
                std::snprintf(reason, reason_len, "task %u: the rocm backend runs the embed, rerank and extractive QA "
                              "encoders", task);
            return TURBO_OK;
        }
        *status = TURBO_CAP_EXPERIMENTAL;
        *dtype = precision == TURBO_PRECISION_FASTEST ? TURBO_DTYPE_F16 : TURBO_DTYPE_F32;
        *options_honored = EMBED_HONORED;
        if (reason_len) reason[0] = 0;
        return TURBO_OK;
    });
}

// ---- Contexts and buffers ---------------------------------------------------------------

int32_t context_create(uint32_t ordinal, turbo_log_fn log, void *ud, void **out, turbo_error *err) {
    return guarded(err, [&] {
        if (ordinal >= devices().size()) fail(TURBO_E_DEVICE_NOT_FOUND, "rocm: no device " + std::to_string(ordinal));
        auto c = std::make_unique<Context>();
        c->ordinal = devices()[ordinal];
        c->log = log;
        c->log_user_data = ud;
        OnDevice on(c->ordinal);
        // The device's fixed staging area (the no-allocation buffer_quantize):
        // its address on this device, looked up with the device current.
        check(static_scratch(c->ordinal, &c->scratch), "the device's staging area");
        if (hipHostMalloc(&c->read_stage, Context::READ_STAGE, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            c->read_stage = nullptr;
        }
        // Default priority on every stream: the one stream priority every run
        // uses. The side streams carry a split run's other parts of rows; the
        // events fork them from the first and join them back.
        check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        bool ok = hipEventCreateWithFlags(&c->fork, hipEventDisableTiming) == hipSuccess;
        for (int i = 0; i < Context::SIDES && ok; ++i)
            ok = hipStreamCreateWithFlags(&c->side[i], hipStreamNonBlocking) == hipSuccess &&
                 hipEventCreateWithFlags(&c->join[i], hipEventDisableTiming) == hipSuccess;
        if (!ok) {
            for (int i = 0; i < Context::SIDES; ++i) {
                if (c->join[i]) (void)hipEventDestroy(c->join[i]);
                if (c->side[i]) (void)hipStreamDestroy(c->side[i]);
            }
            if (c->fork) (void)hipEventDestroy(c->fork);
            (void)hipStreamDestroy(c->stream);
            if (c->read_stage) (void)hipHostFree(c->read_stage);
            fail(TURBO_E_RUNTIME, "rocm: the context's side streams and their events");
        }
        *out = c.release();
        return TURBO_OK;
    });
}

void context_release(void *ctx) {
    if (!ctx) return;
    Context *c = static_cast<Context *>(ctx);
    {
        OnDevice on(c->ordinal);
        (void)hipStreamSynchronize(c->stream);
        for (int i = 0; i < Context::SIDES; ++i) {
            (void)hipStreamSynchronize(c->side[i]);
            (void)hipEventDestroy(c->join[i]);
            (void)hipStreamDestroy(c->side[i]);
        }
        (void)hipEventDestroy(c->fork);
        (void)hipStreamDestroy(c->stream);
        if (c->read_stage) (void)hipHostFree(c->read_stage);
    }
    delete c;
}

uint64_t desc_bytes(const turbo_buffer_desc *d) {
    if (d->bytes) return d->bytes;
    uint64_t el = 0;
    switch (d->dtype) {
    case TURBO_DTYPE_I8:
    case TURBO_DTYPE_U8: el = 1; break;
    case TURBO_DTYPE_F16:
    case TURBO_DTYPE_BF16: el = 2; break;
    case TURBO_DTYPE_I32:
    case TURBO_DTYPE_F32: el = 4; break;
    default: el = 8;
    }
    uint64_t n = d->shape[0];
    if (d->ndim == 2) n *= d->shape[1];
    return n * el;
}

int32_t buffer_alloc(void *ctx, const turbo_buffer_desc *desc, void **out, void **host, turbo_error *err) {
    return guarded(err, [&] {
        Context *c = static_cast<Context *>(ctx);
        OnDevice on(c->ordinal);
        auto b = std::make_unique<Buffer>();
        b->ctx = c;
        b->placement = desc->placement;
        b->bytes = desc_bytes(desc);
        b->owned = true;
        switch (desc->placement) {
        case TURBO_PLACE_DEVICE: b->dev = dev_alloc(b->bytes, "buffer_alloc"); break;
        case TURBO_PLACE_PINNED:
            check(hipHostMalloc(&b->host, b->bytes, hipHostMallocDefault), "hipHostMalloc");
            counted_device_alloc();   // page-locked memory is the driver's
            b->dev = b->host;
            break;
        case TURBO_PLACE_SHARED:
            // One allocation both address: pinned, mapped host memory (the
            // device reads and writes it over the bus). Managed memory is
            // not host-addressable on a device without XNACK.
            check(hipHostMalloc(&b->host, b->bytes ? b->bytes : 1, hipHostMallocDefault), "hipHostMalloc");
            counted_device_alloc();   // page-locked memory is the driver's
            b->dev = b->host;
            break;
        case TURBO_PLACE_HOST:
            b->host = std::malloc(b->bytes ? b->bytes : 1);
            if (!b->host) fail(TURBO_E_OUT_OF_MEMORY, "rocm: host buffer");
            break;
        default: fail(TURBO_E_INVALID_ENUM, "rocm: placement " + std::to_string(desc->placement));
        }
        *host = b->placement == TURBO_PLACE_DEVICE ? nullptr : b->host;
        *out = b.release();
        return TURBO_OK;
    });
}

int32_t buffer_import(void *ctx, const turbo_buffer_desc *desc, const turbo_native_handle *handle, void **out,
                      void **host, turbo_error *err) {
    return guarded(err, [&] {
        Context *c = static_cast<Context *>(ctx);
        auto b = std::make_unique<Buffer>();
        b->ctx = c;
        b->placement = desc->placement;
        b->bytes = desc_bytes(desc);
        b->owned = false;
        char *p = reinterpret_cast<char *>(handle->handle) + handle->offset;
        if (handle->kind == TURBO_HANDLE_CUDA_PTR && desc->placement == TURBO_PLACE_DEVICE) {
            b->dev = p;
        } else if (handle->kind == TURBO_HANDLE_HOST_PTR && desc->placement != TURBO_PLACE_DEVICE) {
            b->host = p;
            b->dev = p;
        } else {
            fail(TURBO_E_UNSUPPORTED, "rocm: handle kind " + std::to_string(handle->kind) + " for placement " +
                                          std::to_string(desc->placement));
        }
        *host = desc->placement == TURBO_PLACE_DEVICE ? nullptr : b->host;
        *out = b.release();
        return TURBO_OK;
    });
}

void buffer_release(void *buf) {
    if (!buf) return;
    Buffer *b = static_cast<Buffer *>(buf);
    if (b->owned) {
        OnDevice on(b->ctx->ordinal);
        switch (b->placement) {
        case TURBO_PLACE_DEVICE: (void)hipFree(b->dev); break;
        case TURBO_PLACE_SHARED:
        case TURBO_PLACE_PINNED: (void)hipHostFree(b->host); break;
        case TURBO_PLACE_HOST: std::free(b->host); break;
        }
    }
    delete b;
}

int32_t buffer_export(void *buf, uint32_t kind, turbo_native_handle *out, turbo_error *err) {
    return guarded(err, [&] {
        Buffer *b = static_cast<Buffer *>(buf);
        if (kind == TURBO_HANDLE_CUDA_PTR && b->dev) {
            out->kind = kind;
            out->handle = reinterpret_cast<uint64_t>(b->dev);
            out->aux = (uint64_t)b->ctx->ordinal;
            out->offset = 0;
            return TURBO_OK;
        }
        if (kind == TURBO_HANDLE_HOST_PTR && b->host) {
            out->kind = kind;
            out->handle = reinterpret_cast<uint64_t>(b->host);
            out->aux = 0;
            out->offset = 0;
            return TURBO_OK;
        }
        fail(TURBO_E_UNSUPPORTED, "rocm: this buffer has no handle of kind " + std::to_string(kind));
    });
}

int32_t buffer_read(void *buf, void *dst, uint64_t bytes, turbo_error *err) {
    return guarded(err, [&] {
        Buffer *b = static_cast<Buffer *>(buf);
        if (bytes > b->bytes) fail(TURBO_E_INVALID_ARGUMENT, "rocm: read of " + std::to_string(bytes) +
                                                                 " bytes from a buffer of " + std::to_string(b->bytes));
        std::lock_guard<std::recursive_mutex> g(b->ctx->lock);
        OnDevice on(b->ctx->ordinal);
        // A device buffer's bytes go to the context's pinned stage on the
        // stream (a DMA that starts as soon as the run before it ends), then
        // to dst on the host: a copy straight into pageable memory first
        // waits for the stream and then stages through the runtime's buffers
        // (BERT-base 64 x 512 write + run + read: 7.77 -> 7.6 ms).
        if (b->placement == TURBO_PLACE_DEVICE && b->ctx->read_stage && bytes <= Context::READ_STAGE) {
            check(hipMemcpyAsync(b->ctx->read_stage, b->dev, bytes, hipMemcpyDeviceToHost, b->ctx->stream),
                  "buffer_read");
            check(hipStreamSynchronize(b->ctx->stream), "buffer_read");
            std::memcpy(dst, b->ctx->read_stage, bytes);
            return TURBO_OK;
        }
        check(hipMemcpyAsync(dst, b->dev ? b->dev : b->host, bytes, hipMemcpyDefault, b->ctx->stream), "buffer_read");
        check(hipStreamSynchronize(b->ctx->stream), "buffer_read");
        return TURBO_OK;
    });
}

// The checks buffer_quantize and its no-allocation variant share: the
// codes' mode, a device-addressable buffer holding rows x dim F32 values,
// finite int8 ranges with min <= max. Returns the codes' bytes (0: nothing
// to do).
uint64_t quantize_codes_bytes(const Buffer *b, uint32_t quantization, const float *int8_ranges, uint32_t rows,
                              uint32_t dim) {
    if (quantization != TURBO_QUANTIZE_INT8 && quantization != TURBO_QUANTIZE_UBINARY)
        fail(TURBO_E_INVALID_ARGUMENT, "rocm: quantization " + std::to_string(quantization) +
                                           " is not int8 or ubinary");
    if (!b->dev || (b->placement != TURBO_PLACE_DEVICE && b->placement != TURBO_PLACE_SHARED))
        fail(TURBO_E_INVALID_ARGUMENT, "rocm: buffer_quantize needs a device or shared buffer");
    const uint64_t floats = (uint64_t)rows * dim;
    if (floats * 4 > b->bytes)
        fail(TURBO_E_INVALID_ARGUMENT, "rocm: " + std::to_string(rows) + " by " + std::to_string(dim) +
                                           " values over the buffer's " + std::to_string(b->bytes) + " bytes");
    if (rows == 0 || dim == 0) return 0;
    if (rows > (uint32_t)INT32_MAX || dim > (uint32_t)INT32_MAX)
        fail(TURBO_E_INVALID_ARGUMENT, "rocm: rows and dim must fit in 31 bits");
    const bool i8 = quantization == TURBO_QUANTIZE_INT8;
    if (i8) {
        if (!int8_ranges) fail(TURBO_E_INVALID_ARGUMENT, "rocm: int8 codes need the [2, dim] ranges");
        for (uint32_t d = 0; d < dim; ++d)
            if (!std::isfinite(int8_ranges[d]) || !std::isfinite(int8_ranges[dim + d]) ||
                int8_ranges[d] > int8_ranges[dim + d])
                fail(TURBO_E_INVALID_ARGUMENT, "rocm: int8 ranges of dimension " + std::to_string(d));
    }
    return i8 ? floats : (uint64_t)rows * ((dim + 7) / 8);
}

// On-device vector codes (turbo_backend.h:610-626): the first rows x dim F32
// values of a device buffer as int8 or ubinary codes, written over the
// buffer's leading bytes. The codes go to a temporary device buffer first,
// so the write never races the read; the int8 ranges are sent to the device.
// Both allocations and the ranges' bytes are added to the run's counts.
int32_t buffer_quantize(void *buf, uint32_t quantization, const float *int8_ranges, uint32_t rows, uint32_t dim,
                        turbo_backend_run *run, turbo_error *err) {
    return guarded(err, [&] {
        Buffer *b = static_cast<Buffer *>(buf);
        const uint64_t code_bytes = quantize_codes_bytes(b, quantization, int8_ranges, rows, dim);
        if (code_bytes == 0) return TURBO_OK;
        const bool i8 = quantization == TURBO_QUANTIZE_INT8;
        std::lock_guard<std::recursive_mutex> g(b->ctx->lock);
        OnDevice on(b->ctx->ordinal);
        const uint64_t dev0 = device_allocs_on_thread();
        DevPtr codes(dev_alloc(code_bytes, "quantized codes"));
        DevPtr ranges;
        hipStream_t st = b->ctx->stream;
        if (i8) {
            ranges.reset(dev_alloc((size_t)2 * dim * 4, "int8 ranges"));
            check(hipMemcpyAsync(ranges.get(), int8_ranges, (size_t)2 * dim * 4, hipMemcpyHostToDevice, st),
                  "int8 ranges");
        }
        check(quantize_codes(st, static_cast<const float *>(b->dev), (int)rows, (int)dim, (int)quantization,
                             static_cast<const float *>(ranges.get()), static_cast<uint8_t *>(codes.get())),
              "buffer_quantize");
        check(hipMemcpyAsync(b->dev, codes.get(), code_bytes, hipMemcpyDeviceToDevice, st), "buffer_quantize");
        check(hipStreamSynchronize(st), "buffer_quantize");
        if (run) {
            run->device_allocs += device_allocs_on_thread() - dev0;
            if (i8) run->h2d_bytes += (uint64_t)2 * dim * 4;
        }
        return TURBO_OK;
    });
}

// ---- Models ------------------------------------------------------------------------

int32_t model_load_fn(void *ctx, const turbo_backend_model *desc, void **out, turbo_error *err) {
    return guarded(err, [&] {
        *out = model_load(static_cast<Context *>(ctx), desc);
        return TURBO_OK;
    });
}

void model_release_fn(void *model) { model_release(static_cast<Model *>(model)); }

// ---- Sessions ------------------------------------------------------------------------

int32_t session_open_fn(void *model, const turbo_backend_session_desc *desc, turbo_backend_tuning *tuning,
                        uint32_t *compute_dtype, void **out, turbo_error *err) {
    return guarded(err, [&] {
        Session *s = session_open(static_cast<Model *>(model), desc, tuning);
        *compute_dtype = s->compute_dtype;
        *out = s;
        return TURBO_OK;
    });
}

int32_t session_create_tuned_fn(void *model, uint32_t task, uint32_t max_batch, uint32_t max_seq, uint32_t precision,
                                 turbo_backend_tuning *tuning, uint32_t *compute_dtype, void **out, turbo_error *err) {
    turbo_backend_session_desc d{};
    d.struct_size = sizeof d;
    d.task = task;
    d.max_batch = max_batch;
    d.max_seq = max_seq;
    d.precision = precision;
    d.max_ranges = max_batch;
    return session_open_fn(model, &d, tuning, compute_dtype, out, err);
}

int32_t session_create_fn(void *model, uint32_t task, uint32_t max_batch, uint32_t max_seq, uint32_t precision,
                          uint32_t *compute_dtype, void **out, turbo_error *err) {
    return session_create_tuned_fn(model, task, max_batch, max_seq, precision, nullptr, compute_dtype, out, err);
}

void session_release_fn(void *session) { session_release(static_cast<Session *>(session)); }

int32_t embed_write_fn(void *session, const turbo_backend_embed_rows *rows, turbo_error *err) {
    return guarded(err, [&] {
        session_write(static_cast<Session *>(session), rows, nullptr, 0);
        return TURBO_OK;
    });
}

int32_t embed_write_ranges_fn(void *session, const turbo_backend_embed_rows *rows, const turbo_token_range *ranges,
                              uint32_t count, turbo_error *err) {
    return guarded(err, [&] {
        if (count == 0) fail(TURBO_E_INVALID_ARGUMENT, "rocm: a range write needs at least one range");
        session_write(static_cast<Session *>(session), rows, ranges, count);
        return TURBO_OK;
    });
}

int32_t session_run_fn(void *session, turbo_backend_run *out, turbo_error *err) {
    return guarded(err, [&] {
        session_run(static_cast<Session *>(session), out);
        return TURBO_OK;
    });
}

}  // namespace

extern "C" {

const turbo_backend turbo_rocm_backend = {
    sizeof(turbo_backend),
    0,
    "rocm",
    RUNTIME_VERSION,
    device_count,
    device_info,
    capability,
    context_create,
    context_release,
    buffer_alloc,
    buffer_import,
    buffer_release,
    buffer_export,
    model_load_fn,
    model_release_fn,
    session_create_fn,
    session_release_fn,
    embed_write_fn,
    session_run_fn,
    buffer_read,
    TURBO_FORMAT_BIT(TURBO_FORMAT_SAFETENSORS),
    0,
    session_create_tuned_fn,
    session_open_fn,
    embed_write_ranges_fn,
    1,   // token_head: model_load takes a QA model's span head; headed range writes apply it
    0,
    buffer_quantize,
};

// buffer_quantize without an allocation: the same codes, staged in the
// device's fixed staging area (STATIC_SCRATCH_BYTES: the codes, then the
// int8 ranges on a 256-byte boundary) instead of memory allocated per call.
// Calls whose codes and ranges exceed it are refused before any device work.
// Every call on one GPU shares the area, so calls that overlap on one GPU
// (through two contexts) race; calls through one context are serialized by
// its lock. Nothing in the area needs clearing: every code byte is written.
// One lock per device for its fixed staging area: every context on a GPU
// shares the area, so a call holds its device's lock from the ranges' copy
// in to the codes' copy out (the seam's threading rule: a backend takes its
// own locks, reference include/turbo/turbo_backend.h:19-20).
static std::mutex scratch_locks[MAX_DEVICES];

int32_t turbo_rocm_buffer_quantize_static(void *buf, uint32_t quantization, const float *int8_ranges, uint32_t rows,
                                          uint32_t dim, turbo_backend_run *run, turbo_error *err) {
    return guarded(err, [&] {
        const uint64_t dev0 = device_allocs_on_thread();
        Buffer *b = static_cast<Buffer *>(buf);
        const uint64_t code_bytes = quantize_codes_bytes(b, quantization, int8_ranges, rows, dim);
        if (code_bytes == 0) return TURBO_OK;
        const bool i8 = quantization == TURBO_QUANTIZE_INT8;
        const uint64_t ranges_at = (code_bytes + 255) & ~(uint64_t)255;
        const uint64_t need = i8 ? ranges_at + (uint64_t)2 * dim * 4 : code_bytes;
        if (need > STATIC_SCRATCH_BYTES)
            fail(TURBO_E_INVALID_ARGUMENT, "rocm: buffer_quantize_static stages at most " +
                                               std::to_string(STATIC_SCRATCH_BYTES) + " bytes (the codes, then the "
                                               "int8 ranges); " + std::to_string(rows) + " by " + std::to_string(dim) +
                                               " values need " + std::to_string(need));
        std::lock_guard<std::recursive_mutex> g(b->ctx->lock);
        if (b->ctx->ordinal < 0 || b->ctx->ordinal >= MAX_DEVICES)
            fail(TURBO_E_RUNTIME, "rocm: device " + std::to_string(b->ctx->ordinal) + " has no staging area");
        std::lock_guard<std::mutex> area_lock(scratch_locks[b->ctx->ordinal]);
        OnDevice on(b->ctx->ordinal);
        void *area = b->ctx->scratch;
        if (!area) fail(TURBO_E_RUNTIME, "rocm: the device's staging area was not found at context creation");
        uint8_t *codes = static_cast<uint8_t *>(area);
        const float *ranges = i8 ? reinterpret_cast<const float *>(codes + ranges_at) : nullptr;
        hipStream_t st = b->ctx->stream;
        if (i8)
            check(hipMemcpyAsync(codes + ranges_at, int8_ranges, (size_t)2 * dim * 4, hipMemcpyHostToDevice, st),
                  "int8 ranges");
        check(quantize_codes(st, static_cast<const float *>(b->dev), (int)rows, (int)dim, (int)quantization, ranges,
                             codes),
              "buffer_quantize_static");
        check(hipMemcpyAsync(b->dev, codes, code_bytes, hipMemcpyDeviceToDevice, st), "buffer_quantize_static");
        check(hipStreamSynchronize(st), "buffer_quantize_static");
        if (run) {
            if (i8) run->h2d_bytes += (uint64_t)2 * dim * 4;
            run->device_allocs += device_allocs_on_thread() - dev0;
        }
        return TURBO_OK;
    });
}

}  // extern "C"
