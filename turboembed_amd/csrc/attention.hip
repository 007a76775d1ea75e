// Softmax attention within each packed row and head: ctx = softmax(Q K^T /
// sqrt(d) + mask) V over the row's live keys (reference
// core/src/cpu/kernels/attend.rs:84-322). Masked keys, and keys outside a
// sliding window, score minus infinity; a query whose keys are all masked
// gets a zero context (attend.rs:216-224).
//
// Q and K are head-major, [heads][tcap][d], so one head's keys of one row
// are contiguous rows of d values; V follows transposed, [heads][d][tcap], so
// one head's values of a run of keys are contiguous in each column.
#include "kernels.h"
#include "launch.h"
#include "devmath.h"

namespace rocm {

// The scalar path: one workgroup of SW waves per (64-query block, head, row),
// a lane per query; the keys are staged through LDS 64 at a time (32 at
// d = 128) and wave w takes keys w, w + SW, ... of each stage, with its own
// online softmax in F32 on Cephes' exp (a key's dot product in column order,
// one FMA chain). The waves' states then merge: each rescales its context and
// sum to the largest of their maxima, and wave 0 adds the contexts and sums in
// wave order. Every tier's reference path.
constexpr int SW = 4;
template <typename T, int D>
__global__ void __launch_bounds__(64 * SW) attention_simple_kernel(const T *__restrict__ qkv, int tcap, int heads,
                                                                   Packing p, const int32_t *__restrict__ mask,
                                                                   Span sp, int window, T *__restrict__ ctx) {
    const Live lv = live_of(sp);
    if ((int)blockIdx.z >= lv.rows) return;
    const int r = lv.row0 + blockIdx.z, head = blockIdx.y, q0 = blockIdx.x * 64, seq = lv.seq;
    const int len = p.len[r];
    if (q0 >= len) return;
    const int start = p.start[r];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, i = q0 + lane;
    const T *Q = qkv + ((size_t)head * tcap + start) * D;
    const T *K = qkv + ((size_t)(heads + head) * tcap + start) * D;
    const T *Vt = qkv + (size_t)2 * heads * tcap * D + (size_t)head * D * tcap + start;
    const int32_t *mk = mask + (size_t)r * seq;
    constexpr int KC = D <= 64 ? 64 : 32;   // keys staged a step
    constexpr int CH = D < 32 ? D : 32;     // context columns merged a round
    constexpr int KV = 2 * KC * (D + 1), RED = SW * 64 * CH;
    // K and V of the staged keys; after the loop, the merge's scratch.
    __shared__ float buf[KV > RED ? KV : RED];
    __shared__ float live[KC];
    __shared__ float mst[SW][64], lst[SW][64];
    float(*ks)[D + 1] = reinterpret_cast<float(*)[D + 1]>(buf);
    float(*vs)[D + 1] = reinterpret_cast<float(*)[D + 1]>(buf + KC * (D + 1));
    float q[D], acc[D];
    const float scale = 1.0f / sqrtf((float)D);
#pragma unroll
    for (int c = 0; c < D; ++c) {
        q[c] = i < len ? to_f32(Q[(size_t)i * D + c]) : 0.0f;
        acc[c] = 0.0f;
    }
    float mx = -INFINITY, l = 0.0f;
    for (int j0 = 0; j0 < len; j0 += KC) {
        __syncthreads();
        for (int x = threadIdx.x; x < KC * D; x += 64 * SW) {
            const int j = x / D, c = x % D;
            const bool in = j0 + j < len;
            ks[j][c] = in ? to_f32(K[(size_t)(j0 + j) * D + c]) : 0.0f;
            vs[j][c] = in ? to_f32(Vt[(size_t)c * tcap + j0 + j]) : 0.0f;
        }
        if (threadIdx.x < KC) live[threadIdx.x] = (j0 + (int)threadIdx.x < len && mk[j0 + threadIdx.x] != 0) ? 1.0f : 0.0f;
        __syncthreads();
        const int nj = min(KC, len - j0);
        for (int j = wave; j < nj; j += SW) {
            const int key = j0 + j;
            if (live[j] == 0.0f) continue;
            if (window < INT32_MAX && (key + window < i || key > i + window)) continue;
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < D; ++c) s = fmaf(q[c], ks[j][c], s);
            s *= scale;
            if (s > mx) {
                const float f = mx == -INFINITY ? 0.0f : dev_exp(mx - s);
                l *= f;
#pragma unroll
                for (int c = 0; c < D; ++c) acc[c] *= f;
                mx = s;
            }
            const float pj = dev_exp(s - mx);
            l += pj;
#pragma unroll
            for (int c = 0; c < D; ++c) acc[c] = fmaf(pj, vs[j][c], acc[c]);
        }
    }
    // Merge: every wave's state to the largest max (a wave that saw no key
    // weighs 0), then the contexts and sums in wave order.
    __syncthreads();
    mst[wave][lane] = mx;
    lst[wave][lane] = l;
    __syncthreads();
    float big = -INFINITY;
#pragma unroll
    for (int w = 0; w < SW; ++w) big = fmaxf(big, mst[w][lane]);
    const float f = mx == -INFINITY ? 0.0f : dev_exp(mx - big);
    float tot_l = 0.0f;
#pragma unroll
    for (int w = 0; w < SW; ++w) {
        const float mw = mst[w][lane];
        tot_l += (mw == -INFINITY ? 0.0f : dev_exp(mw - big)) * lst[w][lane];
    }
    const float inv = tot_l > 0.0f ? 1.0f / tot_l : 0.0f;
    T *out = ctx + (size_t)(start + i) * heads * D + head * D;
#pragma unroll
    for (int c0 = 0; c0 < D; c0 += CH) {
        __syncthreads();
#pragma unroll
        for (int c = 0; c < CH; ++c) buf[(wave * CH + c) * 64 + lane] = acc[c0 + c] * f;
        __syncthreads();
        if (wave == 0 && i < len) {
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                float t = 0.0f;
#pragma unroll
                for (int w = 0; w < SW; ++w) t += buf[(w * CH + c) * 64 + lane];
                out[c0 + c] = from_f32<T>(t * inv);
            }
        }
    }
}

template <typename T>
static hipError_t attention_t(hipStream_t s, const void *qkv, int tcap, int heads, int d, const Packing &p,
                              const int32_t *mask, const Span &sp, int max_rows, int max_len, int window, void *ctx) {
    const dim3 grid((max_len + 63) / 64, heads, max_rows);
#define ATT_CASE(D)                                                                                             \
    case D:                                                                                                     \
        enqueue((attention_simple_kernel<T, D>), grid, dim3(64 * SW), 0, s, (const T *)qkv, tcap,     \
                heads, p, mask, sp, window, (T *)ctx);                                               \
        break;
    switch (d) {
        ATT_CASE(8)
        ATT_CASE(16)
        ATT_CASE(32)
        ATT_CASE(64)
        ATT_CASE(128)
    default: return hipErrorInvalidValue;
    }
#undef ATT_CASE
    return hipGetLastError();
}


// ---- The matrix-core path (F16 and BF16 operands, F32 softmax and sums) ----------
//
// One workgroup of 4 waves per (256-query block, head, row); each wave owns
// 64 queries as two tiles of 32. Keys go 64 at a time through LDS: K as
// stored, and V already transposed by the QKV epilogue, both loaded as
// 16-byte vectors; each fragment a wave reads from LDS feeds both of its
// query tiles, so the LDS reads per product are half a 32-query wave's.
//
// Scores are computed transposed, S^T = K Q^T on v_mfma_f32_32x32x16, so that
// each lane holds one query of a tile (its column, lane % 32) and 16 of the
// 32 keys of a sub-block, the other 16 in the lane 32 away. The online
// softmax runs per 32-key sub-block and needs one cross-lane step there (the
// max with lane ^ 32); each query's running max is a lane's own scalar. The
// context is also computed transposed, O^T += V^T P^T: P^T is the B operand
// straight from the score registers (converted to the operand type), and O^T
// keeps a query per lane, so rescaling is a per-lane multiply.
//
// Key order inside a 32-key sub-block: MFMA row m of the scores reads key
// swap23(m) (bits 2 and 3 of m exchanged). Score register r of a lane in
// half h then holds key 16 (r / 8) + 8 h + r % 8, so registers 0..7 and
// 8..15 are each 8 consecutive keys: exactly the 8 k-slots the lane feeds
// the P^T V^T product per 16-key step, matching 16-byte reads of V^T rows.
// Softmax runs in base 2 on v_exp_f32 with the max already subtracted by
// the matrix cores: Q enters pre-scaled by log2(e)/sqrt(d), and each
// sub-block's score product starts with an all-ones tile times a tile
// holding -m/16 for each query (m its running max, kept at a value that tile
// represents exactly), so a score register holds s - m in log2 units and
// the softmax takes exp2 of it as it is. The row sums accumulate on the
// vector unit as v_dot2 of the 16-bit p values with 1s (F32): the sums of
// the very p values the context used. The context is rescaled only when a
// sub-block raises some query's max by more than 2^8. A query with no live
// key in reach gets a zero context.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));

template <typename T> struct AttnMma;
typedef _Float16 half2x_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2x_t __attribute__((ext_vector_type(2)));
template <> struct AttnMma<_Float16> {
    typedef half8_t frag;
    static __device__ __forceinline__ floatx16_t run(frag a, frag b, floatx16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    // c + the sum of the frag's 8 values (F32 accumulation, v_dot2 with 1s).
    static __device__ __forceinline__ float sum8(frag a, float c) {
#pragma unroll
        for (int e = 0; e < 8; e += 2)
            c = __builtin_amdgcn_fdot2(half2x_t{a[e], a[e + 1]}, half2x_t{(_Float16)1.0f, (_Float16)1.0f}, c, false);
        return c;
    }
};
template <> struct AttnMma<__bf16> {
    typedef bf16x8_t frag;
    static __device__ __forceinline__ floatx16_t run(frag a, frag b, floatx16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ float sum8(frag a, float c) {
#pragma unroll
        for (int e = 0; e < 8; e += 2)
            c = __builtin_amdgcn_fdot2_f32_bf16(bf16x2x_t{a[e], a[e + 1]}, bf16x2x_t{(__bf16)1.0f, (__bf16)1.0f}, c,
                                                false);
        return c;
    }
};

// The max of a lane's value and the value of the lane 32 away, in every
// lane: v_permlane32_swap exchanges the upper half of one copy with the lower
// half of the other, so the two copies hold each lane pair's two values (a
// vector op; a cross-lane shuffle would go through LDS).
__device__ __forceinline__ float max_across_halves(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ int swap23(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

// LDS rows of 128 bytes (64 keys of V^T, or one key's 64 columns of K) keep
// 16-byte chunk c at slot c ^ swz(row), as the GEMM's tiles do, so the
// fragment reads of 16 consecutive rows fall in distinct banks.
__device__ __forceinline__ int att_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <int N> __device__ __forceinline__ void att_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Keys stream through a STAGES-deep LDS ring filled by buffer loads straight
// into LDS (lane l of a load instruction writes 16 bytes at its base + 16 l;
// the MUBUF form counts on vmcnt alone, so the fragment reads' waits stay
// partial): each 64-key block is K (64 rows of d) and V^T (d rows of 64
// keys), 8 rows per instruction. Loads never leave the buffer: a key past the
// row's end reads a clamped address, and its score is -inf, so it weighs
// exactly 0 (the session zeroes Q, K and V once, so every value read is
// finite). Each block's live keys are a 64-bit mask, the same for the whole
// workgroup.
// WIN: a sliding window (window < INT32_MAX). Without one, every sub-block
// of a live wave has work, and the score products run unconditionally (a
// wave past its row's end computes scores it never uses): with no path that
// skips them, their registers need no zeroing for one.
template <typename T, int D, int QT, bool WIN, int QB, int STAGES, int BPB>
__global__ void __launch_bounds__(64 * (QB / (32 * QT))) attention_mfma_kernel(const T *__restrict__ qkv, int tcap,
                                                                               int heads, Span sp, int nqb, Packing p,
                                                                               const int32_t *__restrict__ mask,
                                                                               int window, T *__restrict__ ctx) {
    // QT query tiles of 32 a wave, WAVES waves over a block of QB queries.
    constexpr int WQ = 32 * QT, WAVES = QB / WQ, KB = 64;
    // Each block's K and V^T take 8 load instructions each (8 rows of 128
    // bytes an instruction), shared among the waves.
    constexpr int LPW = 8 / WAVES;
    static_assert(LPW * WAVES == 8, "the waves share a block's loads evenly");
    constexpr int KBYTES = KB * D * 2, VBYTES = D * KB * 2, SBYTES = KBYTES + VBYTES;
    constexpr int KROW = D * 2;   // bytes of one K row
    typedef typename AttnMma<T>::frag frag;
    typedef uint32_t vec4 __attribute__((ext_vector_type(4)));
    static_assert(D == 64, "the ring kernel is written for 64-wide heads");
    // The ring is dynamic LDS (STAGES * SBYTES bytes), then one live-key mask
    // per 64-key block of the longest row (the launch sizes both): memory the
    // compiler sees written only through the loads.
    extern __shared__ __attribute__((aligned(1024))) char ring[];
    uint64_t *live_bits = reinterpret_cast<uint64_t *>(ring + STAGES * SBYTES);

    // XCD-aware numbering of a 1-D grid: the hardware hands block L to XCD
    // L % 8, so the query blocks of one (row, head) pair take numbers 8 apart
    // (same XCD, dispatched together) and share its K and V through that
    // XCD's L2. Pairs go 8 to a group of 8 nqb blocks.
    const int L = blockIdx.x;
    const int pair = (L / (8 * nqb)) * 8 + L % 8, qb = (L / 8) % nqb;
    const Live lv = live_of(sp);
    // (The packing's pointers are tested too, never null, so their argument
    // words are read beside the run's dimensions, not after them.)
    if (pair >= heads * lv.rows || p.len == nullptr || p.start == nullptr) return;
    const int r = lv.row0 + pair / heads, head = pair % heads, q0 = qb * QB, seq = lv.seq;
    // Both reads go out together: the test takes the start too (never
    // negative), so the compiler cannot sink its read past the exit and
    // wait for the two one after the other.
    const int len = p.len[r], start = p.start[r];
    if (q0 >= len || start < 0) return;
    // The wave's number as a scalar (readfirstlane): everything derived from
    // it (its queries, its window tests, its branches) stays uniform.
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, ql = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qw = q0 + wave * WQ;   // this wave's first query
    const T *Q = qkv + ((size_t)head * tcap + start) * D;
    const T *K = qkv + ((size_t)(heads + head) * tcap + start) * D;
    const T *Vt = qkv + (size_t)2 * heads * tcap * D + (size_t)head * D * tcap;
    const int32_t *mk = mask + (size_t)r * seq;
    const bool wave_live = qw < len;   // a wave past the row's end loads and syncs but computes nothing

    // o[qt]: the context of tile qt, transposed; lsum[qt]: its softmax sums
    // over this lane's 16 keys of each sub-block.
    constexpr int NO = D / 32;
    floatx16_t o[QT][NO];
    float lsum[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        lsum[qt] = 0.0f;
#pragma unroll
        for (int t = 0; t < NO; ++t) o[qt][t] = floatx16_t{};
    }
    frag ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (T)1.0f;
    // The running max of each tile's query, in scaled (log2) units (0 before
    // its first live key). It moves only when a sub-block's max passes it by
    // more than RESCALE (p <= 2^RESCALE stays exact enough in the operand
    // type and finite in F32), so a wave rescales its context rarely; every p
    // and the sums share the max in use, so the quotient is the softmax
    // whatever that max is. mb holds it as the bias tile (every element
    // -m/16, so |m| reaches 16 times the operand type's largest value: far
    // past any score); thr is the growth a sub-block's max must pass to move
    // it (-inf until the first live key, whose sub-block's max it then
    // takes).
    constexpr float RESCALE = 8.0f;
    float m_run[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) m_run[qt] = 0.0f;
    frag mb[QT];
    float thr[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        thr[qt] = -INFINITY;
#pragma unroll
        for (int e = 0; e < 8; ++e) mb[qt][e] = (T)0.0f;
    }

    int k_lo = 0, k_hi = len;
    if (window < INT32_MAX) {
        k_lo = max(0, q0 - window) / KB * KB;
        k_hi = min(len, q0 + QB + window);
    }
    const int nb = (k_hi - k_lo + KB - 1) / KB;
    // Buffer resources over this head's K rows and V^T columns of the run.
#if defined(__HIP_DEVICE_COMPILE__)
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void *)K, (short)0, len * KROW, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void *)Vt, (short)0, (int)min((size_t)D * tcap * 2 + 256, (size_t)0x7fffffff), 0x00020000);
#endif
    // This lane's K row and V^T row within each of its load instructions.
    const int lrow = lane >> 3, lchunk = lane & 7;
    auto issue = [&](int stage, int kb) {
        char *base = ring + stage * SBYTES;
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int row = (wave * LPW + i) * 8 + lrow;             // key within the block
            const int key = min(kb + row, len - 1);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rk, (__attribute__((address_space(3))) void *)(base + (wave * LPW + i) * 8 * KROW), 16,
                key * KROW + 16 * (lchunk ^ att_swz(row)), 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int c = (wave * LPW + i) * 8 + lrow;               // column of d
            // Keys kb + 8 slot .. + 7 of column c; a chunk wholly past the
            // row reads the row's last chunk instead (it weighs 0).
            const int slot = lchunk ^ att_swz(c);
            int k0 = kb + 8 * slot;
            if (k0 >= len) k0 = max(0, (len - 1) & ~7);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rv, (__attribute__((address_space(3))) void *)(base + KBYTES + (wave * LPW + i) * 8 * 128), 16,
                (c * tcap + start + k0) * 2, 0, 0, 0);
        }
#else
        (void)base;
        (void)kb;
#endif
    };
    // The workgroup syncs once every BPB blocks; at each sync the loads of
    // the next BPB blocks AHEAD blocks on go out, into the slots of the BPB
    // blocks every wave has just finished.
    constexpr int AHEAD = STAGES - BPB;
    static_assert(AHEAD >= BPB, "a sync's blocks were issued at an earlier sync");
#pragma unroll
    for (int st = 0; st < AHEAD; ++st)
        if (st < nb) issue(st, k_lo + st * KB);
    // Q goes out after the first blocks' loads, and the masks' reads after
    // both, so one memory latency covers the three.
    frag qf[QT][D / 16];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const T *qrow = Q + (size_t)min(qw + 32 * qt + ql, len - 1) * D + h * 8;
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
            const vec4 v = *(const vec4 *)(qrow + s * 16);
            qf[qt][s] = *(const frag *)&v;
        }
    }
    // Every block's live keys, once, before the loop (a mask read inside it
    // would make its wave wait on the prefetch loads too): block b's 64 keys
    // as one 64-bit word, by wave b % WAVES, eight blocks' reads in flight at
    // once on long rows.
    for (int b0 = wave; b0 < nb; b0 += 8 * WAVES) {
        // Every lane reads, from a clamped block and key, and the empty asm
        // takes all eight values: the reads cannot sink into the branches
        // that use them, so they go out together and are waited for once.
        int32_t mv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) mv[u] = mk[min(k_lo + min(b0 + u * WAVES, nb - 1) * KB + lane, len - 1)];
        asm volatile("" ::"v"(mv[0]), "v"(mv[1]), "v"(mv[2]), "v"(mv[3]), "v"(mv[4]), "v"(mv[5]), "v"(mv[6]), "v"(mv[7]));
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int b = b0 + u * WAVES, key = k_lo + b * KB + lane;
            const uint64_t bits = __ballot(b < nb && key < len && mv[u] != 0);
            if (lane == 0 && b < nb) live_bits[b] = bits;
        }
    }
    // Q times log2(e)/sqrt(d), rounded to the operand type.
    const float scale = 1.4426950408889634f / sqrtf((float)D);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int s = 0; s < D / 16; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[qt][s][e] = (T)((float)qf[qt][s][e] * scale);

    for (int bi = 0; bi < nb; ++bi) {
        const int kb = k_lo + bi * KB;
        if (bi % BPB == 0) {
            // Blocks bi .. bi + BPB - 1 must have landed; blocks issued after
            // them may still be in flight.
            constexpr int LATER = AHEAD - BPB;
            if (LATER > 0 && min(LATER, nb - bi - BPB) >= LATER) att_wait_vmcnt<2 * LPW * LATER>();
            else att_wait_vmcnt<0>();
            __syncthreads();
#pragma unroll
            for (int j = 0; j < BPB; ++j)
                if (bi + AHEAD + j < nb) issue((bi + AHEAD + j) % STAGES, kb + (AHEAD + j) * KB);
        }
        const int stage = bi % STAGES;
        const char *kbase = ring + stage * SBYTES;
        const char *vbase = kbase + KBYTES;
        const uint64_t bits = live_bits[bi];

        // Both sub-blocks' scores first: the second's products are still in
        // the matrix cores while the first's softmax runs, and the first's
        // context products while the second's softmax runs. A wave computes
        // nothing past the row's end or outside its queries' windows
        // (wave-uniform).
        bool work[2];
        floatx16_t scs[2][QT];
        // The max both sub-blocks' scores were taken against (the first one's
        // softmax may move it before the second's runs).
        float m_used[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) m_used[qt] = m_run[qt];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const int ks = kb + sub * 32;
            work[sub] = wave_live && !(window < INT32_MAX && (ks + 31 < qw - window || ks > qw + WQ - 1 + window));
            floatx16_t a[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) a[qt] = floatx16_t{};
            if (!WIN || work[sub]) {
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) a[qt] = AttnMma<T>::run(ones, mb[qt], a[qt]);
                const int row = sub * 32 + swap23(ql);
#pragma unroll
                for (int s = 0; s < D / 16; ++s) {
                    const int c = 2 * s + h;
                    const frag kf = *(const frag *)(kbase + row * KROW + 16 * (c ^ att_swz(row)));
#pragma unroll
                    for (int qt = 0; qt < QT; ++qt) a[qt] = AttnMma<T>::run(kf, qf[qt][s], a[qt]);
                }
            }
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) scs[sub][qt] = a[qt];
        }
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const int ks = kb + sub * 32;   // the sub-block's first key
            if (!work[sub]) continue;
            floatx16_t (&sc)[QT] = scs[sub];
            if (sub == 1) {
                bool lagging = false;
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) lagging = lagging || m_run[qt] != m_used[qt];
                if (__ballot(lagging) != 0) {
#pragma unroll
                    for (int qt = 0; qt < QT; ++qt) {
                        const float lag = m_run[qt] - m_used[qt];
#pragma unroll
                        for (int rr = 0; rr < 16; ++rr) sc[qt][rr] -= lag;
                    }
                }
            }
            // Mask (a sub-block wholly live and in every query's window skips
            // the per-key tests) and take each tile's max of the raw scores
            // for this lane's query (the scale is positive, so it keeps their
            // order).
            const uint32_t sbits = (uint32_t)(bits >> (32 * sub));
            const bool all_live = sbits == ~0u && (window == INT32_MAX || (ks >= qw + WQ - 1 - window && ks + 31 <= qw + window));
            float mx[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                if (!all_live) {
                    // This lane's live keys in reach as a mask over the
                    // sub-block; register rr holds key 8 h + j, j = 16 (rr / 8) + rr % 8.
                    uint32_t okm = sbits;
                    if (window < INT32_MAX) {
                        const int query = qw + 32 * qt + ql;
                        const int lo = query - window - ks, hi = query + window - ks;   // keys lo .. hi of the sub-block
                        if (hi < 0 || lo > 31) {
                            okm = 0;
                        } else {
                            const uint32_t upto = hi >= 31 ? ~0u : (2u << hi) - 1;
                            const uint32_t from = lo <= 0 ? ~0u : ~((1u << lo) - 1);
                            okm &= upto & from;
                        }
                    }
                    const uint32_t word = okm >> (8 * h);
#pragma unroll
                    for (int rr = 0; rr < 16; ++rr) {
                        const int j = 16 * (rr >> 3) + (rr & 7);
                        sc[qt][rr] = (word >> j) & 1u ? sc[qt][rr] : -INFINITY;
                    }
                }
                // A chain of three-input maxima (v_max3_f32: 8 for 16 scores).
                float m = fmaxf(fmaxf(sc[qt][0], sc[qt][1]), sc[qt][2]);
#pragma unroll
                for (int rr = 3; rr < 16; rr += 2) m = fmaxf(fmaxf(m, sc[qt][rr]), rr + 1 < 16 ? sc[qt][rr + 1] : m);
                mx[qt] = max_across_halves(m);
            }
            // Every lane runs the same instructions below (the matrix cores
            // take the whole wave): a query with nothing live in reach yet adds
            // zeros and keeps its state (-inf > thr is false).
            bool grow[QT], any = false;
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                grow[qt] = mx[qt] > thr[qt];
                any = any || grow[qt];
            }
            if (__ballot(any) != 0) {
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    // The new max as the bias tile holds it, and the shift it
                    // makes: this sub-block's scores move down by it, the
                    // context so far by 2^-shift (nothing to scale before the
                    // first live key).
                    const T x = (T)((m_run[qt] + mx[qt]) * -0.0625f);
                    const float m_new = (float)x * -16.0f, shift = grow[qt] ? m_new - m_run[qt] : 0.0f;
                    const float f = grow[qt] && thr[qt] != -INFINITY ? __builtin_amdgcn_exp2f(-shift) : 1.0f;
#pragma unroll
                    for (int t = 0; t < NO; ++t) o[qt][t] *= f;
                    lsum[qt] *= f;
#pragma unroll
                    for (int rr = 0; rr < 16; ++rr) sc[qt][rr] -= shift;
                    if (grow[qt]) {
                        m_run[qt] = m_new;
                        thr[qt] = RESCALE;
#pragma unroll
                        for (int e = 0; e < 8; ++e) mb[qt][e] = x;
                    }
                }
            }
            frag pf[QT][2];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
                for (int step = 0; step < 2; ++step) {
                    T pv[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) pv[e] = from_f32<T>(__builtin_amdgcn_exp2f(sc[qt][step * 8 + e]));
                    pf[qt][step] = *(const frag *)pv;
                    lsum[qt] = AttnMma<T>::sum8(pf[qt][step], lsum[qt]);
                }
            }
#pragma unroll
            for (int step = 0; step < 2; ++step) {
#pragma unroll
                for (int t = 0; t < D / 32; ++t) {
                    const int row = 32 * t + ql;
                    const int c = sub * 4 + step * 2 + h;
                    const frag vf = *(const frag *)(vbase + row * 128 + 16 * (c ^ att_swz(row)));
#pragma unroll
                    for (int qt = 0; qt < QT; ++qt) o[qt][t] = AttnMma<T>::run(vf, pf[qt][step], o[qt][t]);
                }
            }
        }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        // A lane's sums cover its half's 16 keys of each sub-block (taken
        // with every lane of the wave active).
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum[qt]), __float_as_uint(lsum[qt]), false, false);
        const float l_tot = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        const int query = qw + 32 * qt + ql;
        if (query >= len) continue;
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        T *out = ctx + (size_t)(start + query) * heads * D + head * D;
#pragma unroll
        for (int t = 0; t < D / 32; ++t)
#pragma unroll
            for (int rr = 0; rr < 16; rr += 4) {
                const int c = 32 * t + 8 * (rr >> 2) + 4 * h;
                T v4[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) v4[q] = from_f32<T>(o[qt][t][rr + q] * inv);
                *(uint2 *)(out + c) = *(const uint2 *)v4;
            }
    }
}

// Query tiles of 32 a wave (1: 32 queries a wave, the registers for four
// waves a SIMD; 2: 64, each K and V fragment read from LDS feeding two
// tiles, 16% slower at 64 x 512 with two waves a SIMD); queries a workgroup
// (ATT_QB: 256, eight waves, or 128, four); LDS ring slots of 64 keys.
#ifndef ATT_QT
#define ATT_QT 1
#endif
#ifndef ATT_QB
#define ATT_QB 256
#endif
#ifndef ATT_STAGES
#define ATT_STAGES 4
#endif
// 64-key blocks a workgroup sync covers (2: one sync per 128 keys, the
// loads of the next two blocks issued at it, 64 KB of ring for two
// workgroups a CU).
#ifndef ATT_BPB
#define ATT_BPB 2
#endif

template <typename T, int QB>
static hipError_t attention_mfma_t(hipStream_t s, const void *qkv, int tcap, int heads, int d, const Packing &p,
                                   const int32_t *mask, const Span &sp, int max_rows, int max_len, int window,
                                   void *ctx) {
    constexpr int STAGES = ATT_STAGES, THREADS = 64 * (QB / (32 * ATT_QT));
    // A 1-D grid of groups of 8 (row, head) pairs times nqb query blocks.
    const int nqb = (max_len + QB - 1) / QB, pairs = heads * max_rows;
    const int blocks = ((pairs + 7) / 8) * 8 * nqb;
    if (d != 64) return hipErrorInvalidValue;
    // STAGES stages of K (64 x 64) and V^T (64 x 64) blocks, then a live mask
    // per 64-key block a workgroup can reach (its keys start on a multiple of
    // 64 at most 63 before the row's, so ceil(max_len / 64) + 1 blocks).
    const int bytes = STAGES * 2 * 64 * 64 * 2 + ((max_len + 127) / 64) * 8;
    if (bytes > 160 * 1024) return hipErrorInvalidValue;
    if (window < INT32_MAX)
        enqueue((attention_mfma_kernel<T, 64, ATT_QT, true, QB, STAGES, ATT_BPB>), dim3(blocks), dim3(THREADS), bytes,
                s, (const T *)qkv, tcap, heads, sp, nqb, p, mask, window, (T *)ctx);
    else
        enqueue((attention_mfma_kernel<T, 64, ATT_QT, false, QB, STAGES, ATT_BPB>), dim3(blocks), dim3(THREADS), bytes,
                s, (const T *)qkv, tcap, heads, sp, nqb, p, mask, window, (T *)ctx);
    return hipGetLastError();
}

template <typename T>
static hipError_t attention_mfma_path(hipStream_t s, const void *qkv, int tcap, int heads, int d, const Packing &p,
                                      const int32_t *mask, const Span &sp, int max_rows, int max_len, int window,
                                      void *ctx, int path) {
    if (path == 2)
        return attention_mfma_t<T, 128>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, window, ctx);
    return attention_mfma_t<T, ATT_QB>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, window, ctx);
}

hipError_t attention(hipStream_t s, Dt dt, const void *qkv, int tcap, int heads, int d, const Packing &p,
                     const int32_t *mask, const Span &sp, int max_rows, int max_len, int window, void *ctx,
                     int path) {
    if (max_len <= 0 || max_rows <= 0) return hipSuccess;
    if (path < 0 || path > 2) return hipErrorInvalidValue;
    const bool mfma = d == 64 && path != 1;
    switch (dt) {
    case Dt::F16:
        return mfma ? attention_mfma_path<_Float16>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, window, ctx,
                                                    path)
                    : attention_t<_Float16>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, window, ctx);
    case Dt::BF16:
        return mfma ? attention_mfma_path<__bf16>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, window, ctx,
                                                  path)
                    : attention_t<__bf16>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, window, ctx);
    default: return attention_t<float>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, window, ctx);
    }
}

// ---- DeBERTa-v2 ---------------------------------------------------------------------
//
// Disentangled attention (reference core/src/deberta/attention.rs:207-315):
// one workgroup per (row, head), wave w taking the row's queries w, w + 4,
// ... A live query's score against each live key is
// (q . k + q . pos_k[b] + k . pos_q[b]) / sqrt(3 d), three in-order F32 FMA
// chains over the head's d columns, b the relative row of the columns'
// distance (buckets[i - j + positions - 1]); the scores of the row's keys
// sit in the wave's LDS (4 x max_len floats), then the max, e^(s - max)
// and their sum by wave reductions, and the context as an F32 FMA chain
// over the keys, times one over the sum. A masked query attends uniformly to
// every position through the row's last live one: the mean of their values.
template <typename T>
__global__ void __launch_bounds__(256) deberta_attention_kernel(const T *__restrict__ qkv, int tcap, int heads, int d,
                                                                Packing p, const int32_t *__restrict__ mask, Span sp,
                                                                const float *__restrict__ pos,
                                                                const int32_t *__restrict__ buckets, int positions,
                                                                T *__restrict__ ctx, int lds_len) {
    extern __shared__ float scores[];
    const Live lv = live_of(sp);
    const int head = blockIdx.x % heads, seq = lv.seq;
    if ((int)blockIdx.x / heads >= lv.rows) return;
    const int r = lv.row0 + (int)blockIdx.x / heads;
    const int len = p.len[r], start = p.start[r];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float *sc = scores + wave * lds_len;
    const int H = heads * d;
    const T *Q = qkv + ((size_t)head * tcap + start) * d;
    const T *K = qkv + ((size_t)(heads + head) * tcap + start) * d;
    const T *Vt = qkv + (size_t)2 * heads * tcap * d + (size_t)head * d * tcap + start;
    const int32_t *mk = mask + (size_t)r * seq;
    const float inv = (float)(1.0 / sqrt(3.0 * (double)d));
    for (int i = wave; i < len; i += 4) {
        T *out = ctx + (size_t)(start + i) * H + head * d;
        if (mk[i] == 0) {
            for (int c = lane; c < d; c += 64) {
                float s = 0.0f;
                for (int j = 0; j < len; ++j) s += to_f32(Vt[(size_t)c * tcap + j]);
                out[c] = from_f32<T>(s / (float)len);
            }
            continue;
        }
        const T *q = Q + (size_t)i * d;
        float mx = -INFINITY;
        for (int j = lane; j < len; j += 64) {
            float s = -INFINITY;
            if (mk[j] != 0) {
                const T *k = K + (size_t)j * d;
                const float *row = pos + (size_t)buckets[i - j + positions - 1] * 2 * H;
                const float *pq = row + head * d, *pk = row + H + head * d;
                float a = 0.0f, b = 0.0f, e = 0.0f;
                for (int c = 0; c < d; ++c) {
                    const float qc = to_f32(q[c]), kc = to_f32(k[c]);
                    a = fmaf(qc, kc, a);
                    b = fmaf(qc, pk[c], b);
                    e = fmaf(kc, pq[c], e);
                }
                s = (a + b + e) * inv;
            }
            sc[j] = s;
            mx = fmaxf(mx, s);
        }
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        float sum = 0.0f;
        for (int j = lane; j < len; j += 64) {
            const float e = sc[j] == -INFINITY ? 0.0f : __expf(sc[j] - mx);
            sc[j] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        // Every lane reads every key's weight: this wave's LDS writes first.
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        const float rs = 1.0f / sum;
        for (int c = lane; c < d; c += 64) {
            float acc = 0.0f;
            for (int j = 0; j < len; ++j) acc = fmaf(sc[j], to_f32(Vt[(size_t)c * tcap + j]), acc);
            out[c] = from_f32<T>(acc * rs);
        }
        // The next query's scores overwrite these only after every lane read them.
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
    }
}

// The matrix-core form (F16 and BF16, 64-wide heads): one workgroup of 4
// waves per (128-query block, head, row), each wave 32 queries and its own
// pass over the row's keys, 32 at a time, with no workgroup sync. Scores are
// transposed as in attention_mfma_kernel (S^T = K Q^T, a query per lane,
// register r of half h holding key 16 (r / 8) + 8 h + r % 8), in log2 units:
// Q enters times log2(e)/sqrt(3 d) and so do the query projections of the
// relative rows. For a 32 x 32 tile the distances i - j take 63 values, so
// their relative rows are a run of at most 64 (the bucket of a distance
// never grows by more than one a step: the host checks its table). Two more
// products over those rows give every score's relative terms at once:
// C = PK Q^T (each query against each row's key projection) and
// P = K PQ^T (each key against each row's query projection), both put in the
// wave's LDS, from which each lane picks C[b(i - j)][i] and P[j][b(i - j)].
// The relative rows come narrowed to the operand type (the query half
// unscaled: P takes the scale as it leaves the accumulators). A tile whose
// 63 distances all fall in the buckets' linear half takes each score's row
// by arithmetic instead of the table.
// Then the online softmax per tile in F32 (exp2 of the score less the
// running max) and the context transposed, O^T += V^T P^T, with P^T taken
// from the score registers. A masked query (before the row's last live
// token) scores 0 against every position of the row: the mean of their
// values.
template <typename T>
__global__ void __launch_bounds__(256) deberta_attention_mfma_kernel(const T *__restrict__ qkv, int tcap, int heads, Span sp,
                                                           int nqb, Packing p, const int32_t *__restrict__ mask,
                                                           const T *__restrict__ pos,
                                                           const int32_t *__restrict__ buckets, int positions,
                                                           T *__restrict__ ctx) {
    constexpr int D = 64, QB = 128;
    typedef typename AttnMma<T>::frag frag;
    typedef uint32_t vec4 __attribute__((ext_vector_type(4)));
    // Per wave: C as [64 rows][32 queries], P as [32 keys][64 rows].
    __shared__ float cbuf[4][64 * 32], pbuf[4][32 * 64];
    const Live lv = live_of(sp);
    // The query blocks of a (row, head) pair take numbers 8 apart: one XCD,
    // whose L2 then holds the pair's keys, values and relative rows once.
    const int L = blockIdx.x;
    const int pair = (L / (8 * nqb)) * 8 + L % 8, qb = (L / 8) % nqb;
    if (pair >= heads * lv.rows) return;
    const int r = lv.row0 + pair / heads, head = pair % heads, seq = lv.seq;
    const int len = p.len[r], start = p.start[r];
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, ql = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qw = qb * QB + wave * 32;
    if (qw >= len) return;
    const int H = heads * D;
    const T *Q = qkv + ((size_t)head * tcap + start) * D;
    const T *K = qkv + ((size_t)(heads + head) * tcap + start) * D;
    const T *Vt = qkv + (size_t)2 * heads * tcap * D + (size_t)head * D * tcap;
    const int32_t *mk = mask + (size_t)r * seq;
    float *cw = cbuf[wave], *pw = pbuf[wave];
    const float scale = 1.4426950408889634f / sqrtf(3.0f * D);

    const int qi = min(qw + ql, len - 1);          // this lane's query (clamped past the row's end)
    const bool q_masked = mk[qi] == 0;
    frag qf[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
        const vec4 v = *(const vec4 *)(Q + (size_t)qi * D + s * 16 + h * 8);
        qf[s] = *(const frag *)&v;
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[s][e] = (T)((float)qf[s][e] * scale);
    }
#if defined(__HIP_DEVICE_COMPILE__)
    // V^T columns of this run start anywhere: 16-byte buffer loads at byte
    // offsets, bounded by the head's V^T block.
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void *)Vt, (short)0, (int)min((size_t)D * tcap * 2, (size_t)0x7fffffff), 0x00020000);
#endif
    floatx16_t o[2] = {floatx16_t{}, floatx16_t{}};
    float m_run = -INFINITY, lsum = 0.0f;
    const int qlast = min(qw + 31, len - 1);
    for (int ks = 0; ks < len; ks += 32) {
        const int klast = min(ks + 31, len - 1);
        // The tile's relative rows: b_lo .. b_hi, at most 64.
        const int b_lo = buckets[qw - klast + positions - 1], b_hi = buckets[qlast - ks + positions - 1];
        const bool linear = b_hi - b_lo == (qlast - ks) - (qw - klast);
        // Otherwise lane l holds the row of distance qw - klast + l (to the
        // tile's largest), and each score takes its row from that lane.
        int brow = 0;
        if (!linear) brow = buckets[min(qw - klast + lane, qlast - ks) + positions - 1];
        // Keys as the score product's rows: row m reads key swap23(m).
        frag kf[D / 16];
        {
            const int key = min(ks + swap23(ql), len - 1);
#pragma unroll
            for (int s = 0; s < D / 16; ++s) {
                const vec4 v = *(const vec4 *)(K + (size_t)key * D + s * 16 + h * 8);
                kf[s] = *(const frag *)&v;
            }
        }
        // C = PK Q^T, rows b_lo + 32 tb + m; then P = K PQ^T, columns b_lo + 32 tb + n.
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const T *row = pos + (size_t)min(b_lo + 32 * tb + ql, b_hi) * 2 * H + head * D + h * 8;
            floatx16_t c = floatx16_t{}, pp = floatx16_t{};
#pragma unroll
            for (int s = 0; s < D / 16; ++s) {
                const vec4 k4 = *(const vec4 *)(row + H + s * 16), q4 = *(const vec4 *)(row + s * 16);
                c = AttnMma<T>::run(*(const frag *)&k4, qf[s], c);
                pp = AttnMma<T>::run(kf[s], *(const frag *)&q4, pp);
            }
            // Output register rr of half h: row 8 (rr / 4) + 4 h + rr % 4, column ql.
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const int m = 8 * (rr >> 2) + 4 * h + (rr & 3);
                cw[(32 * tb + m) * 32 + ql] = c[rr];
                pw[swap23(m) * 64 + 32 * tb + ql] = pp[rr] * scale;
            }
        }
        floatx16_t sc = floatx16_t{};
#pragma unroll
        for (int s = 0; s < D / 16; ++s) sc = AttnMma<T>::run(kf[s], qf[s], sc);
        const uint64_t live = __ballot(ks + ql <= klast && mk[ks + ql] != 0);
        // This wave's LDS writes land before its lanes read each other's.
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        float mx = -INFINITY;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            const int jl = 16 * (rr >> 3) + 8 * h + (rr & 7), key = ks + jl;
            const int dist = qi - min(key, len - 1);
            const int t = linear ? dist - (qw - klast) : min(max(__shfl(brow, dist - (qw - klast), 64) - b_lo, 0), 63);
            const float v = sc[rr] + cw[t * 32 + ql] + pw[jl * 64 + t];
            const bool in_row = key < len;
            sc[rr] = q_masked ? (in_row ? 0.0f : -INFINITY) : ((live >> jl) & 1u ? v : -INFINITY);
            mx = fmaxf(mx, sc[rr]);
        }
        // Every lane has read C and P before the next tile writes them.
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        mx = max_across_halves(mx);
        const float m_new = fmaxf(m_run, mx);
        // Nothing live yet for this query: no weights, no rescale.
        const float f = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        o[0] *= f;
        o[1] *= f;
        lsum *= f;
        m_run = m_new;
        frag pf[2];
#pragma unroll
        for (int step = 0; step < 2; ++step) {
            T pv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                pv[e] = from_f32<T>(m_new == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[step * 8 + e] - m_new));
            pf[step] = *(const frag *)pv;
            lsum = AttnMma<T>::sum8(pf[step], lsum);
        }
#pragma unroll
        for (int step = 0; step < 2; ++step) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                frag vf;
#if defined(__HIP_DEVICE_COMPILE__)
                // Keys ks + 16 step + 8 h .. + 7 of column 32 t + ql; those past
                // the row's end weigh 0, whatever they read
                // (the next column's first values, or zeros past the block).
                const int c = 32 * t + ql, k0 = ks + 16 * step + 8 * h;
                const vec4 v = __builtin_bit_cast(vec4, __builtin_amdgcn_raw_buffer_load_b128(
                                                            rv, (c * tcap + start + k0) * 2, 0, 0));
                vf = *(const frag *)&v;
#else
                vf = frag{};
#endif
                o[t] = AttnMma<T>::run(vf, pf[step], o[t]);
            }
        }
    }
    const auto rs = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum), __float_as_uint(lsum), false, false);
    const float l_tot = __uint_as_float(rs[0]) + __uint_as_float(rs[1]);
    const int query = qw + ql;
    if (query >= len) return;
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    T *out = ctx + (size_t)(start + query) * H + head * D;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int rr = 0; rr < 16; rr += 4) {
            const int c = 32 * t + 8 * (rr >> 2) + 4 * h;
            T v4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v4[q] = from_f32<T>(o[t][rr + q] * inv);
            *(uint2 *)(out + c) = *(const uint2 *)v4;
        }
}

template <typename T>
static hipError_t deberta_t(hipStream_t s, const void *qkv, int tcap, int heads, int d, const Packing &p,
                            const int32_t *mask, const Span &sp, int max_rows, int max_len, const float *pos,
                            const int32_t *buckets, int positions, const void *pos_t, void *ctx) {
    if (max_len > positions) return hipErrorInvalidValue;
    if constexpr (sizeof(T) == 2) {
        if (pos_t && d == 64) {
            // A 1-D grid of groups of 8 (row, head) pairs times nqb query blocks.
            const int nqb = (max_len + 127) / 128, blocks = ((max_rows * heads + 7) / 8) * 8 * nqb;
            enqueue((deberta_attention_mfma_kernel<T>), dim3(blocks), dim3(256), 0, s, (const T *)qkv, tcap, heads,
                    sp, nqb, p, mask, (const T *)pos_t, buckets, positions, (T *)ctx);
            return hipGetLastError();
        }
    }
    const size_t lds = (size_t)4 * max_len * sizeof(float);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    enqueue((deberta_attention_kernel<T>), dim3(max_rows * heads), dim3(256), lds, s, (const T *)qkv, tcap,
            heads, d, p, mask, sp, pos, buckets, positions, (T *)ctx, max_len);
    return hipGetLastError();
}

hipError_t deberta_attention(hipStream_t s, Dt dt, const void *qkv, int tcap, int heads, int d, const Packing &p,
                             const int32_t *mask, const Span &sp, int max_rows, int max_len, const float *pos,
                             const int32_t *buckets, int positions, const void *pos_t, void *ctx) {
    if (max_len <= 0 || max_rows <= 0) return hipSuccess;
    switch (dt) {
    case Dt::F16:
        return deberta_t<_Float16>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, pos, buckets, positions,
                                   pos_t, ctx);
    case Dt::BF16:
        return deberta_t<__bf16>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, pos, buckets, positions,
                                 pos_t, ctx);
    default:
        return deberta_t<float>(s, qkv, tcap, heads, d, p, mask, sp, max_rows, max_len, pos, buckets, positions,
                                nullptr, ctx);
    }
}

}  // namespace rocm
