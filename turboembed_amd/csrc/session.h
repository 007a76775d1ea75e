// The rocm backend's handles and their shared helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <array>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "turbo/turbo_seam.h"
#include "autotune.h"
#include "kernels.h"

namespace rocm {

// Log levels of turbo_log_fn (reference include/turbo/turbo.h:276).
constexpr uint32_t LOG_WARNING = 1, LOG_INFO = 2, LOG_DEBUG = 3;

struct Failure {
    int32_t code;
    uint32_t field;
    std::string message;
};

[[noreturn]] void fail(int32_t code, const std::string &m, uint32_t field = 0);
void check(hipError_t e, const char *what);
void fill(turbo_error *err, int32_t code, uint32_t field, const std::string &m);
void *dev_alloc(size_t bytes, const char *what);
const std::vector<int> &devices();

// Device allocations (device memory, and page-locked host memory, which is
// the driver's) made by the backend, in the process and on the calling
// thread: a call reports the change of the thread's count across it.
extern std::atomic<uint64_t> device_allocs;
void counted_device_alloc();
uint64_t device_allocs_on_thread();
// The backend's own heap allocations, every one its code makes (allocs.cpp:
// the library is linked with malloc and operator new wrapped), on every
// thread and on the calling thread: a run reports the change of the calling
// thread's count across it (reference core/cuda/backend.cpp:146-175).
extern std::atomic<uint64_t> host_allocs;
uint64_t host_allocs_on_thread();

// Every entry point: a status, the caller's turbo_error filled, nothing
// thrown across the boundary (reference include/turbo/turbo_backend.h:10-12).
template <class F> int32_t guarded(turbo_error *err, F &&f) {
    try {
        const int32_t rc = f();
        if (rc == TURBO_OK) fill(err, 0, 0, "");
        return rc;
    } catch (const Failure &e) {
        fill(err, e.code, e.field, e.message);
        return e.code;
    } catch (const std::bad_alloc &) {
        fill(err, TURBO_E_OUT_OF_MEMORY, 0, "rocm: host memory exhausted");
        return TURBO_E_OUT_OF_MEMORY;
    } catch (...) {
        fill(err, TURBO_E_INTERNAL, 0, "rocm: unexpected exception");
        return TURBO_E_INTERNAL;
    }
}

// Holds a device current for a scope, and gives the caller's back.
struct OnDevice {
    int prev = -1;
    explicit OnDevice(int ordinal);
    ~OnDevice();
};

struct DevFree {
    void operator()(void *p) const {
        if (p) (void)hipFree(p);
    }
};
using DevPtr = std::unique_ptr<void, DevFree>;

struct Context {
    int ordinal = 0;                 // the HIP device
    hipStream_t stream = nullptr;
    // A split run's streams after the first, and the events that fork them
    // from it and join them back.
    static constexpr int SIDES = 3;
    hipStream_t side[SIDES] = {};
    hipEvent_t fork = nullptr, join[SIDES] = {};
    turbo_log_fn log = nullptr;
    void *log_user_data = nullptr;
    // A launch through its sync, reads, and a session's open (whose tuner
    // writes and runs rows under it).
    std::recursive_mutex lock;
    void *scratch = nullptr;         // the device's fixed staging area (static_scratch)
    // Pinned host memory that buffer_read copies device buffers through (a
    // copy into pageable memory waits for the stream, then stages through the
    // runtime's own buffers): null if it could not be allocated.
    static constexpr size_t READ_STAGE = (size_t)4 << 20;
    void *read_stage = nullptr;
    void say(uint32_t level, const std::string &m) const;
};

struct Buffer {
    Context *ctx = nullptr;
    uint32_t placement = 0;
    void *dev = nullptr;    // device address (or the host one for host-visible memory)
    void *host = nullptr;
    uint64_t bytes = 0;
    bool owned = false;
};

// One layer's GEMM weights in one dtype: [n, k] row-major, as the kernels
// read them; int8 weights with a scale per output row.
struct LayerWeights {
    const void *qkv, *out, *ffn_in, *ffn_out;
    const float *s_qkv = nullptr, *s_out = nullptr, *s_ffn_in = nullptr, *s_ffn_out = nullptr;
};

struct Model {
    Context *ctx = nullptr;
    uint32_t family = 0, dtype = 0, layers = 0, hidden = 0, heads = 0, inter = 0, vocab = 0, positions = 0,
             types = 0, position_offset = 0;
    float eps = 0;
    bool rotary = false, modern = false, silu = false;
    bool int8 = false;   // the model asks for int8 GEMMs (compute_dtype I8) below EXACT
    uint32_t window = 0, global_every = 0, pairs = 0;   // window: keys each side, 0 for none
    DevPtr f32;                                         // every tensor in F32, one allocation
    // F32 device pointers (NULL where absent).
    const float *word = nullptr, *pos = nullptr, *type = nullptr, *emb_w = nullptr, *emb_b = nullptr,
                *final_w = nullptr, *rope = nullptr;
    // The span head, [head_out, hidden] and [head_out] F32 (head_out 0: none).
    const float *head_w = nullptr, *head_b = nullptr;
    uint32_t head_out = 0;
    struct Layer {
        const float *wqkv, *bqkv, *wo, *bo, *ln1_w, *ln1_b, *w1, *b1, *w2, *b2, *ln2_w, *ln2_b;
        size_t n_qkv, n_in;   // output rows of the QKV and FFN-in products
        const float *pos_qk;  // DeBERTa-v2: [2 buckets][2 H] query then key projections of the relative rows
    };
    // DeBERTa-v2: every layer's relative projections, and the relative row
    // of each distance d in [-(positions - 1), positions - 1] at d + positions - 1.
    bool deberta = false;
    DevPtr rel_pos, rel_table;
    // The relative row of consecutive distances grows by 0 or 1 (so 63 of
    // them span at most 64 rows: the matrix-core form's tiles hold that many).
    bool rel_tiles = false;
    size_t rel_rows = 0;   // 2 position_buckets
    DevPtr rel_narrowed[4];
    bool rel_overflow[4] = {};
    const void *rel_pos_in(Dt dt);
    std::vector<Layer> ls;
    // Narrowed GEMM weights, per dtype (index Dt), made on first need.
    std::mutex lock;
    DevPtr narrowed[4];
    std::vector<LayerWeights> gemm_w[4];
    bool f16_overflow = false;
    std::vector<LayerWeights> &weights_in(Dt dt);
};

struct Session {
    Model *model = nullptr;
    Context *ctx = nullptr;
    uint32_t task = 0, max_batch = 0, max_seq = 0, max_ranges = 0, precision = 0, compute_dtype = 0;
    Dt dt = Dt::F32;    // GEMM operands
    Dt act = Dt::F32;   // activations between the GEMMs: dt, or F16 for I8
    size_t tcap = 0;
    std::vector<DevPtr> owned;
    int32_t *ids = nullptr, *mask = nullptr, *types = nullptr;
    uint32_t *ranges = nullptr;
    Packing pk{};
    float *x = nullptr;      // [tcap, H] F32 residual stream
    void *xh = nullptr;      // [tcap, H] GEMM-operand copy (dt), or the pre-norm rows
    void *qkv = nullptr;     // [3][heads][tcap][d] (dt)
    void *ctxb = nullptr;    // [tcap, H] (dt)
    void *ffn = nullptr;     // [tcap, I] (dt)
    void *y = nullptr;       // [tcap, H] a residual product, in ydt, for the add + LayerNorm after it
    Dt ydt = Dt::F32;        // F16 for post-norm 16-bit sessions, else F32
    int8_t *aq = nullptr;    // I8: a GEMM's quantized operand [tcap, max(H, I)]
    float *ascale = nullptr; // I8: its per-token scales [tcap]
    float *out = nullptr;    // [max(max_batch, max_ranges), H] F32
    float *splitk_ws = nullptr;   // split K's F32 slices (not on the int8 tier)
    size_t splitk_floats = 0;
    PoolScratch pool_scratch;   // the means' chunk sums
    Buffer output;
    int32_t *staging = nullptr;   // pinned: ids, mask, types planes then ranges
    size_t staging_ints = 0;
    // The written run.
    bool written = false;
    uint32_t batch = 0, seq = 0, pooling = 0, normalize = 0, output_dim = 0, count = 0, tokens = 0, max_len = 0;
    bool has_types = false;
    bool head = false;   // ranges through the span head
    // Layer reads of a range write: the last `taps` layers' states, [taps,
    // count, output_dim]; with tap_alone, the first of them alone (the model
    // cut after layer L - taps + 1).
    uint32_t taps = 1;
    bool tap_alone = false;
    // A split run (parts > 1): the rows in `parts` parts of about equal
    // packed tokens, each part's layers on its own stream; part i is rows
    // [part_row[i], part_row[i + 1]), tokens [part_tok[i], part_tok[i + 1]),
    // its longest row part_len[i]. Two parts by default (measured on
    // BERT-base 64 x 512: 8.4 ms a batch against 9.0 with four and 9.2 with
    // one); TURBO_ROCM_SPLIT=n asks for n parts (0 or 1: none; at most 4).
    static constexpr int MAX_PARTS = rocm::MAX_PARTS;
    uint32_t split_parts = 2;
    uint32_t parts = 1, part_row[MAX_PARTS + 1] = {}, part_tok[MAX_PARTS + 1] = {}, part_len[MAX_PARTS] = {};
    uint64_t h2d = 0;
    // The run's dimensions: staged with the rows (pinned) and on the device,
    // where every kernel of a run reads them.
    RunDims *dims_host = nullptr, *dims_dev = nullptr;
    std::vector<uint32_t> row_lens;   // the write's row lengths (host, sized at open)
    std::vector<LayerWeights> *w = nullptr;
    // DeBERTa-v2: the model's relative projections in the operand type, or
    // null (the scalar attention on the F32 table).
    const void *rel_pos_t = nullptr;
    Choices kc;            // kernel choices per bin of packed tokens
    std::string choices;   // kc as a choices string
    // One graph per bin of packed tokens, captured at session_open with the
    // bin's kernel choices and grids sized for its largest run, and replayed
    // for every run of that bin whatever its rows (the kernels read the run's
    // extent from dims_dev). Runs that read layers before the last, and runs
    // timed launch by launch, launch their kernels directly. Off with
    // TURBO_ROCM_GRAPHS=0.
    bool graphs = true;
    uint32_t layers_limit = 0;   // the tuner's runs: the first layers alone (0: every layer)
    hipGraphExec_t graph[BINS] = {};
    uint32_t bin_parts[BINS] = {};   // parts a bin's graph runs (its runs use as many or fewer)
    uint64_t captures = 0, graph_launches = 0;   // counted for the graphs hook
    // Per-launch timing (a test and benchmark hook): events around each
    // kernel of a run on its own stream, by name, and the run's start.
    bool timing = false;
    hipEvent_t ev0 = nullptr;   // the timed run's start
    std::vector<hipEvent_t> ev;
    std::vector<const char *> ev_name;
    size_t ev_used = 0;
};

Model *model_load(Context *c, const turbo_backend_model *desc);
void model_release(Model *m);
Session *session_open(Model *m, const turbo_backend_session_desc *desc, turbo_backend_tuning *tuning);
void session_release(Session *s);
void session_write(Session *s, const turbo_backend_embed_rows *rows, const turbo_token_range *ranges, uint32_t count);
void session_run(Session *s, turbo_backend_run *out);
// Times the session's candidate kernels within budget_ms and keeps the
// fastest in s.kc; timing lines into *timings. Whether anything was timed.
bool tune(Session &s, uint32_t budget_ms, std::string *timings);
// One run's launches on the session's stream: its bin's graph, or the
// kernels launched directly.
void launch_run(Session &s);
// Captures each bin's graph (with TURBO_ROCM_GRAPHS not 0).
void capture_graphs(Session &s);

}  // namespace rocm
