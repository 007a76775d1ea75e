// The encoder's linear layers on CDNA4 matrix cores: C = A W^T with both
// operands K-contiguous (A [M, K] activations, W [N, K] weights as the model
// stores them), F32 accumulation, and the epilogue fused into the store.
//
// Block: 256 threads = 4 waves in 2 x 2, each wave (BM/2) x (BN/2) of the
// output as 32 x 32 MFMA tiles (v_mfma_f32_32x32x16_{f16,bf16}, or
// v_mfma_f32_32x32x2f32 for the F32 tier). K advances BK at a time through
// two LDS buffers: the next tile's global loads are in flight in registers
// while the current one is multiplied, and one barrier a step separates the
// two. Rows of the LDS tiles are padded by 16 bytes so that the 16-byte
// fragment reads of 32 consecutive rows spread over the banks.
//
// Fragments: lane l feeds row (l % 32) of its A and B tiles, and the
// contiguous half (l / 32) of the BK columns, BK/2 elements read as 16-byte
// vectors. The matrix core sums over its k slots without regard to which
// memory column fed each slot, so A and B fed with the same column map give
// the product over all of K.
//
// Block numbering is XCD-aware: the hardware hands block b to XCD b % 8, so
// blocks are renumbered so that each XCD takes a contiguous run of output
// tiles, along N first: the run shares its A rows, which then stay in that
// XCD's L2.
#include <atomic>
#include <mutex>
#include <cstring>
#include <type_traits>

#include "kernels.h"
#include "launch.h"
#include "devmath.h"
#include "rowmath.h"

namespace rocm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mma;

typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef int int32x16 __attribute__((ext_vector_type(16)));

template <> struct Mma<_Float16> {
    static constexpr int EPM = 8;   // elements a lane feeds one MFMA
    typedef half8 frag;
    typedef floatx16 acc;
    static __device__ __forceinline__ floatx16 run(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <> struct Mma<__bf16> {
    static constexpr int EPM = 8;
    typedef bf16x8 frag;
    typedef floatx16 acc;
    static __device__ __forceinline__ floatx16 run(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

template <> struct Mma<int8_t> {
    static constexpr int EPM = 16;
    typedef int32x4 frag;
    typedef int32x16 acc;
    static __device__ __forceinline__ int32x16 run(frag a, frag b, int32x16 c) {
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
    }
};

template <> struct Mma<float> {
    static constexpr int EPM = 1;
    typedef float frag;
    typedef floatx16 acc;
    static __device__ __forceinline__ floatx16 run(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

// A gated unit's product act(gate) * up as stored: at an F16 output it
// saturates at F16's largest finite magnitude instead of rounding to
// infinity (a NaN stays NaN), as the reference's CUDA backend stores it
// (core/cuda/rotary.cuh:31-45); BF16 and F32 outputs hold it as it is.
template <typename T> __device__ __forceinline__ float gated_product(float g, float up) {
    const float v = __fmul_rn(g, up);
    if constexpr (std::is_same<T, _Float16>::value) return v > 65504.0f ? 65504.0f : v < -65504.0f ? -65504.0f : v;
    return v;
}

// The rows a GEMM launch multiplies: its span, and how far apart A's token
// rows are for the span's first token (the run's operand rows may be wider
// than the product's K).
struct GemmRows {
    Span sp;
    int a_tok;
};

// The span's first token moves the epilogue's row-major output (and the int8
// activation scales) down to it; the Q, K and V scatter (and the rotary
// epilogue's positions) take it as the token of row 0.
template <Epi KIND, typename OT>
__device__ __forceinline__ void place_epilogue(EpiArgs &e, const Live &lv) {
    e.tok0 = lv.tok0;
    if (e.a_scale) e.a_scale += lv.tok0;
    const size_t rows = (size_t)lv.tok0 * e.ldo;
    if constexpr (KIND == Epi::Plain) e.out = (float *)e.out + rows;
    else if constexpr (KIND == Epi::Bias) e.out = e.out_f32 ? (void *)((float *)e.out + rows) : (void *)((OT *)e.out + rows);
    else if constexpr (KIND == Epi::Gelu || KIND == Epi::Gated) e.out = (OT *)e.out + rows;
    else if constexpr (KIND == Epi::Residual) e.x += rows;
}

// The epilogue of one 32 x 32 MFMA tile, for this lane's column n and its 16
// rows m0 + 8 (r / 4) + 4 (lane / 32) + r % 4, v = acc + bias. The kind is a
// template argument, so each kernel carries one small epilogue, and what
// depends on the column alone is worked out once per tile.
template <typename T, Epi KIND>
__device__ __forceinline__ void epilogue_tile(const EpiArgs &e, int M, int N, int mt, int n, const floatx16 &acc) {
    const int lane = threadIdx.x & 63;
    const int mb = mt + (lane >> 5) * 4;   // row of register r: mb + 8 (r / 4) + r % 4
    const bool col_ok = n < N;
    const float bias = (e.bias && col_ok) ? e.bias[n] : 0.0f;
    if constexpr (KIND == Epi::Plain || KIND == Epi::Gelu || KIND == Epi::Residual || KIND == Epi::Bias) {
        if (!col_ok) return;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mb + (r >> 2) * 8 + (r & 3);
            if (m >= M) continue;
            const float v = acc[r] + bias;
            const size_t at = (size_t)m * e.ldo + n;
            if constexpr (KIND == Epi::Plain) ((float *)e.out)[at] = v;
            else if constexpr (KIND == Epi::Bias) {
                if (e.out_f32) ((float *)e.out)[at] = v;
                else if (sizeof(T) == 2 && e.out_bf16) ((__bf16 *)e.out)[at] = from_f32<__bf16>(v);
                else ((T *)e.out)[at] = from_f32<T>(v);
            }
            else if constexpr (KIND == Epi::Gelu)
                ((T *)e.out)[at] = from_f32<T>(sizeof(T) == 2 ? dev_gelu_fast(v) : dev_gelu(v));
            else e.x[at] = e.x[at] + v;
        }
    } else if constexpr (KIND == Epi::Qkv || KIND == Epi::QkvRope) {
        const int which = n / e.hidden, rem = n - which * e.hidden;
        const int head = rem / e.d, c = rem - head * e.d;
        T *out = (T *)e.out + (size_t)which * e.heads * e.tcap * e.d;
        const int half = e.d >> 1, pr = c >> 1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mb + (r >> 2) * 8 + (r & 3);
            float v = acc[r] + bias;
            if constexpr (KIND == Epi::QkvRope) {
                // Columns come pair-adjacent: the partner of n is n ^ 1, in
                // the neighbouring lane (column n sits in lane n % 32).
                const float w = __shfl_xor(v, 1, 64);
                if (which < 2 && col_ok && m < M) {
                    // Rounded products, then their sum or difference, in
                    // every instantiation (no fused multiply-add).
#pragma clang fp contract(off)
                    const int pos = e.pos[e.tok0 + m];
                    const float cs = e.cos[(size_t)pos * half + pr], sn = e.sin[(size_t)pos * half + pr];
                    // (x1, x2) -> (x1 cos - x2 sin, x2 cos + x1 sin)
                    v = (c & 1) ? v * cs + w * sn : v * cs - w * sn;
                }
            }
            if (!col_ok || m >= M) continue;
            // Q and K token-major per head; V transposed per head.
            const size_t t = (size_t)e.tok0 + m;
            const size_t at = which < 2 ? ((size_t)head * e.tcap + t) * e.d + c : ((size_t)head * e.d + c) * e.tcap + t;
            out[at] = from_f32<T>(v);
        }
    } else {   // Gated: out[m, n / 2] = act(gate) * up, gate and up in neighbouring columns
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mb + (r >> 2) * 8 + (r & 3);
            const float v = acc[r] + bias;
            const float up = __shfl_xor(v, 1, 64);
            if (!col_ok || m >= M || (n & 1)) continue;
            const float g = e.silu ? dev_silu(v) : sizeof(T) == 2 ? dev_gelu_fast(v) : dev_gelu(v);
            ((T *)e.out)[(size_t)m * e.ldo + (n >> 1)] = from_f32<T>(gated_product<T>(g, up));
        }
    }
}

// ks > 0: split K, the grid's y-th slice of ks columns of k (W's rows stay
// K long), its F32 sums (Plain epilogue, no bias) into slice y of the
// output, split_stride floats apart; splitk_reduce adds the slices.
template <typename T, int BM, int BN, int BK, Epi KIND>
__global__ void __launch_bounds__(256) gemm_kernel(Span sp, int a_tok, int N, int K, const T *__restrict__ A, int lda,
                                                   const T *__restrict__ W, EpiArgs e, int grid_n, int ks = 0,
                                                   size_t split_stride = 0) {
    constexpr int VEC = 16 / sizeof(T);          // elements in 16 bytes
    constexpr int STRIDE = BK + VEC;             // LDS row, padded by 16 bytes
    constexpr int TM = BM / 64, TN = BN / 64;    // MFMA tiles per wave (2 x 2 waves)
    constexpr int HALF = BK / 2;                 // the columns one lane reads
    constexpr int VROW = BK / VEC;               // 16-byte vectors in a tile row
    constexpr int LA = BM * VROW / 256, LB = BN * VROW / 256;
    static_assert(LA * 256 == BM * VROW && LB * 256 == BN * VROW, "tile loads split evenly over 256 threads");
    typedef typename Mma<T>::frag frag;
    constexpr int EPM = Mma<T>::EPM;
    typedef uint32_t vec4 __attribute__((ext_vector_type(4)));

    __shared__ __attribute__((aligned(16))) T lds[2][(BM + BN) * STRIDE];

    const Live lv = live_of(sp);
    const int M = lv.tokens;
    // XCD-aware renumbering of the block over the span's own tiles (the grid
    // may be sized for more rows: the blocks past them leave).
    const int live = (M + BM - 1) / BM * grid_n;
    if ((int)blockIdx.x >= live) return;
    A += (size_t)lv.tok0 * a_tok;
    // (A span whose rows pass a slice's would write into the next: such a
    // launch leaves, and the session never makes one.)
    if (ks && (size_t)(lv.tok0 + M) * N > split_stride) return;
    if (ks) e.out = (float *)e.out + blockIdx.y * split_stride;
    place_epilogue<KIND, T>(e, lv);
    const int per = live / 8;
    int b = blockIdx.x;
    if (b < per * 8) b = (b % 8) * per + b / 8;
    const int tile_n = b % grid_n, tile_m = b / grid_n;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    // This block's columns of k: all of them, or its split's.
    const int kb = ks ? (int)blockIdx.y * ks : 0, ke = ks ? min(K, kb + ks) : K;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    vec4 ra[LA], rb[LB];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int v = tid + 256 * i, r = v / VROW, c = (v % VROW) * VEC;
            const int gm = min(m0 + r, M - 1), gk = k0 + c;
            ra[i] = gk + VEC <= ke ? *(const vec4 *)(A + (size_t)gm * lda + gk) : vec4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int v = tid + 256 * i, r = v / VROW, c = (v % VROW) * VEC;
            const int gn = min(n0 + r, N - 1), gk = k0 + c;
            rb[i] = gk + VEC <= ke ? *(const vec4 *)(W + (size_t)gn * K + gk) : vec4{0, 0, 0, 0};
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int v = tid + 256 * i, r = v / VROW, c = (v % VROW) * VEC;
            *(vec4 *)&lds[buf][r * STRIDE + c] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int v = tid + 256 * i, r = v / VROW, c = (v % VROW) * VEC;
            *(vec4 *)&lds[buf][(BM + r) * STRIDE + c] = rb[i];
        }
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx16{};

    const int nk = (ke - kb + BK - 1) / BK;
    load(kb);
    store(0);
    __syncthreads();
    const int row_a = wm * (BM / 2) + (lane & 31), row_b = BM + wn * (BN / 2) + (lane & 31);
    const int col = (lane >> 5) * HALF;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load(kb + (kt + 1) * BK);
        const T *base = lds[buf];
#pragma unroll
        for (int s = 0; s < HALF / EPM; ++s) {
            frag fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) fa[i] = *(const frag *)&base[(row_a + i * 32) * STRIDE + col + s * EPM];
#pragma unroll
            for (int j = 0; j < TN; ++j) fb[j] = *(const frag *)&base[(row_b + j * 32) * STRIDE + col + s * EPM];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = Mma<T>::run(fa[i], fb[j], acc[i][j]);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }

    // Output element r of tile (i, j): column lane % 32, row 8 (r / 4) + 4 (lane / 32) + r % 4.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
            epilogue_tile<T, KIND>(e, M, N, m0 + wm * (BM / 2) + i * 32, n0 + wn * (BN / 2) + j * 32 + (lane & 31),
                                   acc[i][j]);
}

template <typename T, int BM, int BN, int BK, Epi KIND>
static hipError_t launch_k(hipStream_t s, const GemmRows &gr, int M, int N, int K, const void *A, int lda,
                           const void *W, const EpiArgs &e) {
    const int gn = (N + BN - 1) / BN, gm = (M + BM - 1) / BM;
    enqueue((gemm_kernel<T, BM, BN, BK, KIND>), dim3(gn * gm), dim3(256), 0, s, gr.sp, gr.a_tok, N, K,
            (const T *)A, lda, (const T *)W, e, gn, 0, (size_t)0);
    return hipGetLastError();
}

template <typename T, int BM, int BN, int BK>
static hipError_t launch(hipStream_t s, const GemmRows &gr, int M, int N, int K, const void *A, int lda, const void *W,
                         const EpiArgs &e) {
    switch (e.kind) {
    case Epi::Plain: return launch_k<T, BM, BN, BK, Epi::Plain>(s, gr, M, N, K, A, lda, W, e);
    case Epi::Qkv: return launch_k<T, BM, BN, BK, Epi::Qkv>(s, gr, M, N, K, A, lda, W, e);
    case Epi::Gelu: return launch_k<T, BM, BN, BK, Epi::Gelu>(s, gr, M, N, K, A, lda, W, e);
    case Epi::Residual: return launch_k<T, BM, BN, BK, Epi::Residual>(s, gr, M, N, K, A, lda, W, e);
    case Epi::QkvRope: return launch_k<T, BM, BN, BK, Epi::QkvRope>(s, gr, M, N, K, A, lda, W, e);
    case Epi::Gated: return launch_k<T, BM, BN, BK, Epi::Gated>(s, gr, M, N, K, A, lda, W, e);
    case Epi::Bias: return launch_k<T, BM, BN, BK, Epi::Bias>(s, gr, M, N, K, A, lda, W, e);
    }
    return hipErrorInvalidValue;
}


// ---- Split K for products too small to fill the chip --------------------------------
//
// A Bias product (out or FFN-out: N the hidden size) of few row tiles runs
// its K in `splits` slices, each slice's tiles a block of the grid's y-th
// row, their F32 sums into a workspace slice; then one pass adds the slices
// in slice order (no float atomics: the same bits every run), adds the bias
// and stores the product as the Bias epilogue does (F32, the operand type,
// or BF16). The reference's tuner offers split-K as its SkMode knob
// (core/cuda/kernels.h:166-175, core/cuda/kernels.cu:4449-4469).
template <typename T>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(Span sp, const float *__restrict__ ws, int splits,
                                                            size_t stride, int N, EpiArgs e) {
    const Live lv = live_of(sp);
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;   // 4 consecutive outputs a thread
    const int n = (int)(i * 4 % N), m = (int)(i * 4 / N);
    if (m >= lv.tokens || (size_t)(lv.tok0 + lv.tokens) * N > stride) return;
    const size_t at = (size_t)(lv.tok0 + m) * N + n;
    typedef float float4_v __attribute__((ext_vector_type(4)));
    float4_v v = *(const float4_v *)(ws + at);
    for (int s = 1; s < splits; ++s) v += *(const float4_v *)(ws + s * stride + at);
    float o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = v[q] + (e.bias ? e.bias[n + q] : 0.0f);
    const size_t out = (size_t)(lv.tok0 + m) * e.ldo + n;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (e.out_f32) ((float *)e.out)[out + q] = o[q];
        else if (sizeof(T) == 2 && e.out_bf16) ((__bf16 *)e.out)[out + q] = from_f32<__bf16>(o[q]);
        else ((T *)e.out)[out + q] = from_f32<T>(o[q]);
    }
}

template <typename T, int BM, int BN, int BK>
static hipError_t launch_split(hipStream_t s, const GemmRows &gr, int M, int N, int K, const void *A, int lda,
                               const void *W, const EpiArgs &e, int splits) {
    // Slices of whole BK steps; the workspace holds every slice's rows.
    const int ks = ((K + splits - 1) / splits + BK - 1) / BK * BK;
    splits = (K + ks - 1) / ks;
    const size_t stride = (size_t)M * N;
    if (e.kind != Epi::Bias || !e.ws || N % 4 != 0 || (size_t)splits * stride > e.ws_floats || e.ldo < N)
        return hipErrorInvalidValue;
    EpiArgs p;
    p.kind = Epi::Plain;
    p.out = e.ws;
    p.ldo = N;
    const int gn = (N + BN - 1) / BN, gm = (M + BM - 1) / BM;
    enqueue((gemm_kernel<T, BM, BN, BK, Epi::Plain>), dim3(gn * gm, splits), dim3(256), 0, s, gr.sp,
            gr.a_tok, N, K, (const T *)A, lda, (const T *)W, p, gn, ks, stride);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const size_t quads = stride / 4;
    enqueue((splitk_reduce_kernel<T>), dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, s, gr.sp, e.ws,
            splits, stride, N, e);
    return hipGetLastError();
}

// ---- The pipelined kernel (16-bit operands, K a multiple of 64) -------------------
//
// The same 2 x 2 waves of 32 x 32 MFMA tiles, fed by a STAGES-deep ring of
// LDS tiles that the hardware fills directly from global memory
// (global_load_lds_dwordx4: lane l of a wave writes its 16 bytes at the
// instruction's LDS base + 16 l), so no registers stage the operands and
// STAGES - 1 tiles are in flight while one is multiplied. A tile row is 64
// elements, 128 bytes, as 8 chunks of 16 bytes; chunk c of row r is kept at
// slot c ^ f(r), f(r) = (r & 7) ^ ((r >> 3) & 1), so the 16-byte fragment
// reads of 16 consecutive rows at one chunk fall in distinct banks whether
// the LDS serves 8 or 16 lanes of a 16-byte read per clock. A lane of a
// load instruction fills slot (lane & 7) of row (lane >> 3) of its 8-row
// group, so it fetches global chunk (lane & 7) ^ f(row).
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
// Rows of 64 bytes (BK 32) hold 4 chunks: chunk c of row r at slot
// c ^ (((r >> 1) & 3) ^ ((r >> 3) & 1)), distinct over 8 and over 16 rows alike.
__device__ __forceinline__ int swz4(int row) { return ((row >> 1) & 3) ^ ((row >> 3) & 1); }
template <int ROWB> __device__ __forceinline__ int swz_of(int row) { return ROWB == 128 ? swz(row) : swz4(row); }

// s_waitcnt vmcnt(N) with the other counters left free (gfx9 encoding).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The pipelined kernel's epilogue: each wave stages 32 rows of its tile at a
// time through its own LDS scratch (F32, rows padded by 4 floats), then reads
// them back along rows (or, for V^T, down columns), so every global access is
// a 16-byte vector of 8 consecutive outputs: coalesced stores of the outputs,
// and coalesced reads and writes of x for the residual. The values are the
// accumulators exactly; only the order of the stores changes.
constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }

// Stores through a buffer resource: a lane whose row lies past the output
// gets an offset past the resource's end and the hardware drops its store, so
// the store loop has no per-lane branches and the compiler can overlap each
// store's LDS reads with the previous store.
constexpr int OOB = 0x7fffffff;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// An int8 product's output: the int32 sum times both scales, plus the bias,
// each step rounded on its own, so every store path and block shape of the
// epilogue gives the same bits. (The contraction pragma, with plain
// operators: __fmul_rn and __fadd_rn still let the compiler fuse a product
// into the add after inlining.)
__device__ __forceinline__ float dequant(float acc, float as, float ws, float bias) {
#pragma clang fp contract(off)
    return acc * as * ws + bias;
}

template <typename T>
__device__ __forceinline__ u32x4_t pack8(const float (&v)[8]) {
    T tmp[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) tmp[q] = from_f32<T>(v[q]);
    return __builtin_bit_cast(u32x4_t, tmp);
}

template <typename T>
__device__ __forceinline__ u32x2_t pack4(const float (&v)[4]) {
    T tmp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) tmp[q] = from_f32<T>(v[q]);
    return __builtin_bit_cast(u32x2_t, tmp);
}

// The per-column constants a lane's epilogue uses (the int8 weight scales
// and biases; a 16-bit product's bias is in its accumulators from the
// start), read after the main loop and before the first store. A global load
// issued among the stores would make the wait for its value wait for every
// store before it too (the vector memory counter retires in order), so the
// epilogue reads nothing from global memory once its first store is out.
// int8 operands, whose bias follows the scales: the wave's COLS scales, then
// its COLS biases, NV values a lane, go to the wave's LDS (stage_cols) once
// the stages are free, and each store reads its columns' from there
// (registers for them all would spill the wide block shapes' accumulators).
template <int TN, int PASS, bool SCALED>
struct EpiCols {
    static constexpr int COLS = TN * 32, CH = COLS / 8, PH = CH / gcd_c(64, CH);
    static constexpr int NV = SCALED ? (2 * COLS + 63) / 64 : 1;
    float v[NV];
    const float *lds = nullptr;
};

template <Epi KIND, int TN, int PASS, bool SCALED>
__device__ __forceinline__ void load_cols(EpiCols<TN, PASS, SCALED> &c, const EpiArgs &e, int N, int nw) {
    using C = EpiCols<TN, PASS, SCALED>;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < C::NV; ++k) c.v[k] = 0.0f;
#if defined(__HIP_DEVICE_COMPILE__)
    // Buffer reads: columns at or past N read as 0 (their outputs are never stored).
    auto rsrc = [&](const float *p) {
        return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, N * 4, 0x00020000);
    };
    auto at = [&](const __amdgpu_buffer_rsrc_t &r, int n) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, n * 4, 0, 0));
    };
    if constexpr (SCALED) {
        // Value i of the wave: scale i (i < COLS), bias i - COLS (0 with no bias).
        const __amdgpu_buffer_rsrc_t rw = rsrc(e.w_scale);
        const __amdgpu_buffer_rsrc_t rb = rsrc(e.bias);
#pragma unroll
        for (int k = 0; k < C::NV; ++k) {
            const int i = lane + 64 * k;
            if (i < C::COLS) c.v[k] = at(rw, nw + i);
            else if (i < 2 * C::COLS && e.bias) c.v[k] = at(rb, nw + i - C::COLS);
        }
    }
#else
    (void)e;
    (void)N;
    (void)nw;
    (void)lane;
#endif
}

// The int8 epilogue's constants into the wave's LDS (2 COLS floats, 16-byte
// aligned), once the stages are free; the caller waits for the writes.
template <int TN, int PASS, bool SCALED>
__device__ __forceinline__ void stage_cols(EpiCols<TN, PASS, SCALED> &c, float *ccol) {
    using C = EpiCols<TN, PASS, SCALED>;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < C::NV; ++k)
        if (lane + 64 * k < 2 * C::COLS) ccol[lane + 64 * k] = c.v[k];
    c.lds = ccol;
}

// The scales and biases of the 8 columns from cc, from the staged constants.
template <int COLS>
__device__ __forceinline__ void chunk_cols(const float *ccol, int cc, float (&wsc)[8], float (&bias)[8]) {
    typedef float f4_t __attribute__((ext_vector_type(4)));
    const f4_t w0 = *(const f4_t *)(ccol + cc), w1 = *(const f4_t *)(ccol + cc + 4);
    const f4_t b0 = *(const f4_t *)(ccol + COLS + cc), b1 = *(const f4_t *)(ccol + COLS + cc + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) wsc[q] = w0[q], wsc[4 + q] = w1[q], bias[q] = b0[q], bias[4 + q] = b1[q];
}

// Head and column within the head of column `rem` of Q, K or V. (A lane's
// columns repeat from pass to pass, so the compiler computes these once.)
__device__ __forceinline__ void head_col(int rem, int d, int &head, int &c) {
    head = rem / d;
    c = rem - head * d;
}

// `ascale` (int8 operands): the activation scales of this wave's rows,
// staged in LDS before the first store.
// ROPE_AHEAD: a rotary pass too wide to defer its stores reads all its
// chunks' angles before its first store (the block shapes whose registers
// allow it).
template <typename T, Epi KIND, int TM, int TN, int PASS, bool SCALED, bool ROPE_AHEAD, typename ACC>
__device__ __forceinline__ void epilogue_lds(const EpiArgs &e, int M, int N, int mw, int nw, float *scratch,
                                             const float *ascale, const EpiCols<TN, PASS, SCALED> &cols,
                                             const ACC (&acc)[TM][TN]) {
    typedef float float4_t __attribute__((ext_vector_type(4)));
    constexpr int COLS = TN * 32, SROW = COLS + 4, CH = COLS / 8;   // 8-column chunks per row
    static_assert(PASS == 32 || PASS == 16, "32 or 16 rows a pass");
    const int lane = threadIdx.x & 63, h = lane >> 5, ql = lane & 31;
    constexpr bool QKV = KIND == Epi::Qkv || KIND == Epi::QkvRope;
    // The branch-free path: whole 8-column chunks, and an output region the
    // 32-bit buffer offsets reach (row-major from this wave's first row, or
    // one of the Q, K and V blocks).
    const int64_t region = QKV ? (int64_t)e.heads * e.tcap * e.d * (int64_t)sizeof(T)
                               : (int64_t)(M - mw) * e.ldo * (int64_t)((KIND == Epi::Plain || e.out_f32) ? 4 : sizeof(T));
    // (Marked likely where they branch, so the fast path's blocks are laid
    // out together: 1% off the headline step.)
    const bool fast = KIND != Epi::Residual && (N & 7) == 0 && region < OOB && (!QKV || (e.d & 7) == 0);
    const bool fast_v = fast && ((e.tcap | e.tok0) & 7) == 0;   // V^T: 8 tokens in 16 aligned bytes
    // Q, K and V: a wave's columns lie in one of them (every block shape
    // whose waves' width does not divide the hidden size is refused for
    // these products), so the block, and its first column, are the wave's.
    const int qkv_which = QKV ? uniform(nw / e.hidden) : 0, qkv_base = qkv_which * e.hidden;
#if defined(__HIP_DEVICE_COMPILE__)
    __amdgpu_buffer_rsrc_t rs;
    if constexpr (QKV) {
        const int which = qkv_which;
        rs = __builtin_amdgcn_make_buffer_rsrc((T *)e.out + (size_t)which * e.heads * e.tcap * e.d, (short)0,
                                               (int)region, 0x00020000);
    } else if constexpr (KIND != Epi::Residual) {
        void *base = (KIND == Epi::Plain || e.out_f32) ? (void *)((float *)e.out + (size_t)mw * e.ldo)
                                                       : (void *)((T *)e.out + (size_t)mw * e.ldo);
        rs = __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)(region > 0 && region < OOB ? region : 0), 0x00020000);
    }
#endif
#pragma unroll
    for (int pi = 0; pi < TM * (32 / PASS); ++pi) {
        const int i = pi / (32 / PASS), half = pi % (32 / PASS);
        // Registers to LDS: row 8 (r / 4) + 4 h + r % 4 of the 32, column
        // 32 j + ql; a 16-row pass takes registers r < 8 (rows 0-15), then the rest.
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if (PASS == 16 && (r >> 3) != half) continue;
                const int row = (r >> 2) * 8 + h * 4 + (r & 3) - (PASS == 16 ? half * 16 : 0);
                // (16-bit operands: the bias is in the accumulators.)
                scratch[row * SROW + j * 32 + ql] = (float)acc[i][j][r];
            }
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        const int mt = mw + i * 32 + half * PASS;
        if constexpr (KIND == Epi::Qkv || KIND == Epi::QkvRope) {
            if (qkv_which == 2) {
                // V^T: 8 consecutive tokens of a column (of V^T's row vr =
                // head * d + c) a lane.
                auto put_vt = [&](int vr, int m, const float (&v)[8]) {
                    T *out = (T *)e.out + (size_t)2 * e.heads * e.tcap * e.d + (size_t)vr * e.tcap + e.tok0;
#if defined(__HIP_DEVICE_COMPILE__)
                    if (__builtin_expect(fast_v, 1)) {
                        // From the V block: rows past M, and a tail of fewer than 8, are dropped.
                        const int off = m + 8 <= M ? (int)((((size_t)vr) * e.tcap + e.tok0 + m) * sizeof(T)) : OOB;
                        __builtin_amdgcn_raw_buffer_store_b128(pack8<T>(v), rs, off, 0, 0);
                        if (__builtin_expect(m + 8 > M && m < M, 0)) {
#pragma unroll
                            for (int q = 0; q < 8; ++q)
                                if (m + q < M) out[m + q] = from_f32<T>(v[q]);
                        }
                        return;
                    }
#endif
                    if (m + 8 <= M && ((e.tcap | e.tok0) & 7) == 0) {
                        store8<T>(out + m, v);
                    } else {
#pragma unroll
                        for (int q = 0; q < 8; ++q)
                            if (m + q < M) out[m + q] = from_f32<T>(v[q]);
                    }
                };
                if constexpr (KIND == Epi::Qkv && !SCALED && ((COLS / 2) * (PASS / 8)) % 64 == 0) {
                    // Two adjacent columns a lane (8-byte reads of the staged
                    // rows: half the LDS reads of one column a lane; the bias
                    // is in the staged values). A column pair lies in one
                    // head (d is even). (Not on the rotary shape: its
                    // read-ahead angles leave no registers for it.)
#pragma unroll
                    for (int k = 0; k < (COLS / 2) * (PASS / 8) / 64; ++k) {
                        const int u = lane + 64 * k, col = 2 * (u / (PASS / 8)), g = (u % (PASS / 8)) * 8;
                        const int n = nw + col;
                        if (n >= N) continue;
                        int head, c;
                        head_col(n - qkv_base, e.d, head, c);
                        float v0[8], v1[8];
#pragma unroll
                        for (int q = 0; q < 8; ++q) {
                            const float2 p2 = *(const float2 *)&scratch[(g + q) * SROW + col];
                            v0[q] = p2.x;
                            v1[q] = p2.y;
                        }
                        const int m = mt + g, vr = head * e.d + c;
                        put_vt(vr, m, v0);
                        put_vt(vr + 1, m, v1);
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < COLS * (PASS / 8) / 64; ++k) {
                        const int u = lane + 64 * k, col = u / (PASS / 8), g = (u % (PASS / 8)) * 8;
                        const int n = nw + col;
                        if (n >= N) continue;
                        int head, c;
                        head_col(n - qkv_base, e.d, head, c);
                        float v[8];
                        const int m = mt + g;
                        if constexpr (SCALED) {
                            const float ws = cols.lds[col], bias = cols.lds[COLS + col];
#pragma unroll
                            for (int q = 0; q < 8; ++q) v[q] = dequant(scratch[(g + q) * SROW + col], ascale[m + q - mw], ws, bias);
                        } else {
#pragma unroll
                            for (int q = 0; q < 8; ++q) v[q] = scratch[(g + q) * SROW + col];
                        }
                        T *out = (T *)e.out + (size_t)2 * e.heads * e.tcap * e.d + ((size_t)head * e.d + c) * e.tcap + e.tok0;
#if defined(__HIP_DEVICE_COMPILE__)
                        if (__builtin_expect(fast_v, 1)) {
                            // From the V block: rows past M, and a tail of fewer than 8, are dropped.
                            const int off = m + 8 <= M ? (int)((((size_t)head * e.d + c) * e.tcap + e.tok0 + m) * sizeof(T)) : OOB;
                            __builtin_amdgcn_raw_buffer_store_b128(pack8<T>(v), rs, off, 0, 0);
                            if (__builtin_expect(m + 8 > M && m < M, 0)) {
#pragma unroll
                                for (int q = 0; q < 8; ++q)
                                    if (m + q < M) out[m + q] = from_f32<T>(v[q]);
                            }
                        } else
#endif
                        if (m + 8 <= M && ((e.tcap | e.tok0) & 7) == 0) {
                            store8<T>(out + m, v);
                        } else {
#pragma unroll
                            for (int q = 0; q < 8; ++q)
                                if (m + q < M) out[m + q] = from_f32<T>(v[q]);
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
                continue;
            }
        }
        // Row-wise: 8 consecutive columns of one row a lane, item u = lane +
        // 64 k taking chunk u % CH of row u / CH. A lane's chunk repeats every
        // PH items (64 PH is a multiple of CH).
        constexpr int PH = EpiCols<TN, PASS, SCALED>::PH;
        static_assert((PASS * CH) % 64 == 0 && ((PASS * CH) / 64) % PH == 0, "whole items per lane");
#if defined(__HIP_DEVICE_COMPILE__)
        if constexpr (KIND != Epi::Residual) {
            if (__builtin_expect(fast, 1)) {
                const bool f32 = KIND == Epi::Plain || e.out_f32;
                // The rotary scatter stores its pass's chunks after the last
                // one is made: each chunk reads its token's position and
                // angles, and a load issued after a store waits for that
                // store too (the vector memory counter retires in order).
                // (Where the accumulators leave room: 128 registers a lane.)
                constexpr bool DEFER = KIND == Epi::QkvRope && TM * TN * 16 <= 128;
                constexpr int NK = PASS * CH / 64, NR = DEFER ? NK : 1;
                u32x4_t rope_out[NR];
                int rope_off[NR];
                // Elsewhere, where ROPE_AHEAD allows, every chunk's angles are
                // read before the pass's first store, so the pass waits on
                // earlier stores once (chunk by chunk it waits once a chunk:
                // ModernBERT's step 1.3-1.6% slower).
                constexpr int RG = KIND == Epi::QkvRope && !DEFER && !SCALED && ROPE_AHEAD ? NK : 1;
                if constexpr (RG > 1) {
#pragma unroll
                    for (int k0 = 0; k0 < NK; k0 += RG) {
                        float4_t gcs[RG], gsn[RG];
#pragma unroll
                        for (int g = 0; g < RG; ++g) {
                            const int k = k0 + g;
                            const int cc = ((lane + 64 * (k % PH)) % CH) * 8, n = nw + cc;
                            const int m = mt + (lane + 64 * k) / CH;
                            int head, c;
                            head_col(n - qkv_base, e.d, head, c);
                            const int pos = e.pos[e.tok0 + min(m, M - 1)], hd = e.d >> 1;
                            const size_t at = (size_t)pos * hd + (c >> 1);
                            gcs[g] = *(const float4_t *)(e.cos + at);
                            gsn[g] = *(const float4_t *)(e.sin + at);
                        }
#pragma unroll
                        for (int g = 0; g < RG; ++g) {
                            const int k = k0 + g;
                            const int cc = ((lane + 64 * (k % PH)) % CH) * 8, n = nw + cc;
                            const int row = (lane + 64 * k) / CH, m = mt + row;
                            const bool ok = m < M && n < N;
                            const float4_t lo = *(const float4_t *)&scratch[row * SROW + cc];
                            const float4_t hi = *(const float4_t *)&scratch[row * SROW + cc + 4];
                            float v[8];
#pragma unroll
                            for (int q = 0; q < 4; ++q) v[q] = lo[q], v[4 + q] = hi[q];
                            int head, c;
                            head_col(n - qkv_base, e.d, head, c);
#pragma unroll
                            for (int p = 0; p < 4; ++p) {
#pragma clang fp contract(off)
                                const float cs = gcs[g][p], sn = gsn[g][p];
                                const float x1 = v[2 * p], x2 = v[2 * p + 1];
                                v[2 * p] = x1 * cs - x2 * sn;
                                v[2 * p + 1] = x2 * cs + x1 * sn;
                            }
                            const int off = ok ? (int)((((size_t)head * e.tcap + e.tok0 + m) * e.d + c) * sizeof(T)) : OOB;
                            __builtin_amdgcn_raw_buffer_store_b128(pack8<T>(v), rs, off, 0, 0);
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                    continue;
                }
#pragma unroll
                for (int k = 0; k < NK; ++k) {
                    const int cc = ((lane + 64 * (k % PH)) % CH) * 8, n = nw + cc;
                    float bias[8], wsc[8];
                    if constexpr (SCALED) chunk_cols<COLS>(cols.lds, cc, wsc, bias);
                    const int row = (lane + 64 * k) / CH, m = mt + row;
                    const bool ok = m < M && n < N;
                    const float4_t lo = *(const float4_t *)&scratch[row * SROW + cc];
                    const float4_t hi = *(const float4_t *)&scratch[row * SROW + cc + 4];
                    const float as = SCALED ? ascale[m - mw] : 1.0f;
                    float v[8];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if constexpr (SCALED) {
                            v[q] = dequant(lo[q], as, wsc[q], bias[q]);
                            v[4 + q] = dequant(hi[q], as, wsc[4 + q], bias[4 + q]);
                        } else {
                            v[q] = lo[q];
                            v[4 + q] = hi[q];
                        }
                    }
                    const int rm = m - mw;   // row within the wave's region
                    if constexpr (KIND == Epi::Plain || KIND == Epi::Bias) {
                        if (f32) {
                            const int off = ok ? (rm * e.ldo + n) * 4 : OOB;
                            __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                                                          __float_as_uint(v[2]), __float_as_uint(v[3])},
                                                                  rs, off, 0, 0);
                            __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{__float_as_uint(v[4]), __float_as_uint(v[5]),
                                                                          __float_as_uint(v[6]), __float_as_uint(v[7])},
                                                                  rs, ok ? off + 16 : OOB, 0, 0);
                        } else {
                            // (out_bf16 is the launch's: a uniform branch.)
                            const int off = ok ? (rm * e.ldo + n) * (int)sizeof(T) : OOB;
                            if (sizeof(T) == 2 && e.out_bf16)
                                __builtin_amdgcn_raw_buffer_store_b128(pack8<__bf16>(v), rs, off, 0, 0);
                            else
                                __builtin_amdgcn_raw_buffer_store_b128(pack8<T>(v), rs, off, 0, 0);
                        }
                    } else if constexpr (KIND == Epi::Gelu) {
#pragma unroll
                        for (int q = 0; q < 8; ++q) v[q] = sizeof(T) == 2 ? dev_gelu_fast(v[q]) : dev_gelu(v[q]);
                        __builtin_amdgcn_raw_buffer_store_b128(pack8<T>(v), rs,
                                                              ok ? (rm * e.ldo + n) * (int)sizeof(T) : OOB, 0, 0);
                    } else if constexpr (KIND == Epi::Gated) {
                        // Columns (2p, 2p + 1) are gate and up of output column n / 2 + p.
                        float g4[4];
#pragma unroll
                        for (int p = 0; p < 4; ++p) {
                            const float g = e.silu ? dev_silu(v[2 * p])
                                                   : sizeof(T) == 2 ? dev_gelu_fast(v[2 * p]) : dev_gelu(v[2 * p]);
                            g4[p] = gated_product<T>(g, v[2 * p + 1]);
                        }
                        __builtin_amdgcn_raw_buffer_store_b64(pack4<T>(g4), rs,
                                                             ok ? (rm * e.ldo + (n >> 1)) * (int)sizeof(T) : OOB, 0, 0);
                    } else {   // Qkv, QkvRope: Q or K, token-major per head
                        int head, c;
                        head_col(n - qkv_base, e.d, head, c);
                        if constexpr (KIND == Epi::QkvRope) {
                            const int pos = e.pos[e.tok0 + min(m, M - 1)], hd = e.d >> 1;
                            // The chunk's 4 pairs' angles: 16 aligned bytes of
                            // each table (c is a multiple of 8, the tables' rows
                            // of d / 2 floats start on 16 bytes).
                            const size_t at = (size_t)pos * hd + (c >> 1);
                            const float4_t cs4 = *(const float4_t *)(e.cos + at), sn4 = *(const float4_t *)(e.sin + at);
#pragma unroll
                            for (int p = 0; p < 4; ++p) {
                                // Rounded products, then their difference or
                                // sum, in every instantiation (no fused
                                // multiply-add: split and unsplit runs launch
                                // different block shapes).
#pragma clang fp contract(off)
                                const float cs = cs4[p], sn = sn4[p];
                                const float x1 = v[2 * p], x2 = v[2 * p + 1];
                                v[2 * p] = x1 * cs - x2 * sn;
                                v[2 * p + 1] = x2 * cs + x1 * sn;
                            }
                        }
                        const int off = ok ? (int)((((size_t)head * e.tcap + e.tok0 + m) * e.d + c) * sizeof(T)) : OOB;
                        if constexpr (DEFER) {
                            rope_out[k] = pack8<T>(v);
                            rope_off[k] = off;
                        } else {
                            __builtin_amdgcn_raw_buffer_store_b128(pack8<T>(v), rs, off, 0, 0);
                        }
                    }
                }
                if constexpr (DEFER)
#pragma unroll
                    for (int k = 0; k < NK; ++k) __builtin_amdgcn_raw_buffer_store_b128(rope_out[k], rs, rope_off[k], 0, 0);
                __builtin_amdgcn_wave_barrier();
                continue;
            }
        }
#endif
#pragma unroll
        for (int k = 0; k < PASS * CH / 64; ++k) {
            const int cc = ((lane + 64 * (k % PH)) % CH) * 8, n = nw + cc;
            float bias[8], wsc[8];
            if constexpr (SCALED) chunk_cols<COLS>(cols.lds, cc, wsc, bias);
            const int row = (lane + 64 * k) / CH;
            const int m = mt + row;
            if (m >= M || n >= N) continue;
            const bool full = n + 8 <= N;
            float v[8];
            const float4_t lo = *(const float4_t *)&scratch[row * SROW + cc];
            const float4_t hi = *(const float4_t *)&scratch[row * SROW + cc + 4];
            const float as = SCALED ? ascale[m - mw] : 1.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if constexpr (SCALED) {
                    v[q] = dequant(lo[q], as, wsc[q], bias[q]);
                    v[4 + q] = dequant(hi[q], as, wsc[4 + q], bias[4 + q]);
                } else {
                    v[q] = lo[q];
                    v[4 + q] = hi[q];
                }
            }
            if constexpr (KIND == Epi::Plain || KIND == Epi::Bias) {
                if (KIND == Epi::Plain || e.out_f32) {
                    float *o = (float *)e.out + (size_t)m * e.ldo + n;
                    if (full) {
                        *(float4_t *)o = float4_t{v[0], v[1], v[2], v[3]};
                        *(float4_t *)(o + 4) = float4_t{v[4], v[5], v[6], v[7]};
                    } else {
                        for (int q = 0; n + q < N; ++q) o[q] = v[q];
                    }
                } else if (sizeof(T) == 2 && e.out_bf16) {
                    __bf16 *o = (__bf16 *)e.out + (size_t)m * e.ldo + n;
                    if (full) store8<__bf16>(o, v);
                    else for (int q = 0; n + q < N; ++q) o[q] = from_f32<__bf16>(v[q]);
                } else {
                    T *o = (T *)e.out + (size_t)m * e.ldo + n;
                    if (full) store8<T>(o, v);
                    else for (int q = 0; n + q < N; ++q) o[q] = from_f32<T>(v[q]);
                }
            } else if constexpr (KIND == Epi::Residual) {
                float *o = e.x + (size_t)m * e.ldo + n;
                if (full) {
                    const float4_t a = *(const float4_t *)o, b = *(const float4_t *)(o + 4);
                    *(float4_t *)o = float4_t{a[0] + v[0], a[1] + v[1], a[2] + v[2], a[3] + v[3]};
                    *(float4_t *)(o + 4) = float4_t{b[0] + v[4], b[1] + v[5], b[2] + v[6], b[3] + v[7]};
                } else {
                    for (int q = 0; n + q < N; ++q) o[q] = o[q] + v[q];
                }
            } else if constexpr (KIND == Epi::Gelu) {
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] = sizeof(T) == 2 ? dev_gelu_fast(v[q]) : dev_gelu(v[q]);
                T *o = (T *)e.out + (size_t)m * e.ldo + n;
                if (full) store8<T>(o, v);
                else for (int q = 0; n + q < N; ++q) o[q] = from_f32<T>(v[q]);
            } else if constexpr (KIND == Epi::Gated) {
                // Columns (2p, 2p + 1) are gate and up of output column n / 2 + p.
                T *o = (T *)e.out + (size_t)m * e.ldo + (n >> 1);
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    if (n + 2 * p + 1 >= N) break;
                    const float g = e.silu ? dev_silu(v[2 * p]) : sizeof(T) == 2 ? dev_gelu_fast(v[2 * p]) : dev_gelu(v[2 * p]);
                    o[p] = from_f32<T>(gated_product<T>(g, v[2 * p + 1]));
                }
            } else {   // Qkv, QkvRope: Q or K, token-major per head
                const int which = n / e.hidden, rem = n - which * e.hidden;
                const int head = rem / e.d, c = rem - head * e.d;
                if constexpr (KIND == Epi::QkvRope) {
                    const int pos = e.pos[e.tok0 + m], half = e.d >> 1;
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        // (Rounded products, as above.)
#pragma clang fp contract(off)
                        const int pr = (c >> 1) + p;
                        const float cs = e.cos[(size_t)pos * half + pr], sn = e.sin[(size_t)pos * half + pr];
                        const float x1 = v[2 * p], x2 = v[2 * p + 1];
                        v[2 * p] = x1 * cs - x2 * sn;
                        v[2 * p + 1] = x2 * cs + x1 * sn;
                    }
                }
                const size_t t = (size_t)e.tok0 + m;
                T *o = (T *)e.out + (size_t)which * e.heads * e.tcap * e.d + ((size_t)head * e.tcap + t) * e.d + c;
                if (full && (e.d & 7) == 0) store8<T>(o, v);
                else for (int q = 0; q < 8 && n + q < N; ++q) {
                    const int nq = n + q, wq = nq / e.hidden, rq = nq - wq * e.hidden, hq = rq / e.d, cq = rq - hq * e.d;
                    ((T *)e.out)[(size_t)wq * e.heads * e.tcap * e.d + ((size_t)hq * e.tcap + t) * e.d + cq] =
                        from_f32<T>(v[q]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// The pipelined kernel's shape: a BM x BN output tile, WM x WN waves, a
// STAGES-deep ring of BK-column stages.
template <typename T, int BM, int BN, int WM, int WN, int STAGES, int BK>
struct LdsTile {
    static constexpr int WAVES = WM * WN;
    static constexpr int EPC = 16 / (int)sizeof(T);                 // elements in a 16-byte chunk
    static constexpr int ROWB = BK * (int)sizeof(T), CHUNKS = ROWB / 16;   // bytes and chunks of a tile row
    static constexpr int RPI = 64 / CHUNKS;                         // rows one load instruction fills
    static constexpr int TILE = (BM + BN) * ROWB;                   // bytes of one stage
    static constexpr int TM = BM / WM / 32, TN = BN / WN / 32;      // MFMA tiles per wave
    static constexpr int LA = BM / RPI / WAVES, LB = BN / RPI / WAVES;   // load instructions per wave per stage
    static constexpr int L = LA + LB;
    static_assert(ROWB == 128 || ROWB == 64, "tile rows of 64 or 128 bytes");
    static_assert(LA * RPI * WAVES == BM && LB * RPI * WAVES == BN, "whole row groups per wave");
    static_assert(STAGES >= 2 && STAGES * TILE <= 160 * 1024, "LDS");
    static_assert((STAGES - 2) * L < 64, "vmcnt");
};

// The pipelined main loop: acc[i][j] (this wave's MFMA tiles, zeroed by the
// caller) takes the sums over all of K of the BM x BN tile whose first row
// and column are m0 and n0 (rows of A past M and of W past N read as the
// last ones). With `bias` (16-bit operands), every accumulator starts from
// its column's bias instead of 0 (columns past N from 0), so the epilogue
// has no bias to add: y = b + sum, one F32 rounding per product as before.
// Leaves every wave's last fragment reads done but the stages still in use:
// the caller syncs before it reuses the LDS.
template <typename T, int BM, int BN, int WM, int WN, int STAGES, int BK>
__device__ __forceinline__ void lds_mainloop(char *smem, const T *__restrict__ A, int lda, const T *__restrict__ W,
                                             int M, int N, int K, int m0, int n0, int wave, int lane,
                                             typename Mma<T>::acc (&acc)[BM / WM / 32][BN / WN / 32],
                                             const float *__restrict__ bias = nullptr) {
    using P = LdsTile<T, BM, BN, WM, WN, STAGES, BK>;
    constexpr int EPC = P::EPC, ROWB = P::ROWB, CHUNKS = P::CHUNKS, RPI = P::RPI, TILE = P::TILE;
    constexpr int TM = P::TM, TN = P::TN, LA = P::LA, LB = P::LB, L = P::L;
    typedef typename Mma<T>::frag frag;
    const int wm = wave / WN, wn = wave % WN;

    // The operands are read through buffer resources based at the tile's
    // first row (buffer_load_dwordx4 ... lds: the MUBUF form of the direct
    // load counts on vmcnt alone, so the compiler keeps the fragment reads'
    // lgkmcnt waits partial and the LDS reads stay pipelined). Each lane's
    // byte offset in each of its load instructions, rows past the operand's
    // last clamped to it.
    int src_a[LA], src_b[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int row = (wave * LA + i) * RPI + lane / CHUNKS;
        src_a[i] = (min(row, M - 1 - m0) * lda + EPC * ((lane % CHUNKS) ^ swz_of<ROWB>(row))) * (int)sizeof(T);
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
        const int row = (wave * LB + i) * RPI + lane / CHUNKS;
        src_b[i] = (min(row, N - 1 - n0) * K + EPC * ((lane % CHUNKS) ^ swz_of<ROWB>(row))) * (int)sizeof(T);
    }
    // (The host pass of the compiler sees no LDS address space or buffer
    // resources: the loads are device code alone.)
#if defined(__HIP_DEVICE_COMPILE__)
    const uint64_t bytes_a = ((uint64_t)(M - 1 - m0) * lda + K) * sizeof(T);
    const uint64_t bytes_b = (uint64_t)(N - n0) * K * sizeof(T);
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A + (size_t)m0 * lda), (short)0, (int)min(bytes_a, (uint64_t)0xffffffffu), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(W + (size_t)n0 * K), (short)0, (int)min(bytes_b, (uint64_t)0xffffffffu), 0x00020000);
#endif
    auto issue = [&](int stage, int k0) {
#if defined(__HIP_DEVICE_COMPILE__)
        char *base = smem + stage * TILE;
        const int kb = k0 * (int)sizeof(T);
#pragma unroll
        for (int i = 0; i < LA; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsa, (__attribute__((address_space(3))) void *)(base + (wave * LA + i) * RPI * ROWB), 16, src_a[i] + kb, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < LB; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsb, (__attribute__((address_space(3))) void *)(base + BM * ROWB + (wave * LB + i) * RPI * ROWB), 16,
                src_b[i] + kb, 0, 0, 0);
#else
        (void)stage;
        (void)k0;
#endif
    };

    const int nk = K / BK;
    // The bias of this lane's columns n0 + wn (BN / WN) + 32 j + (lane & 31),
    // read before the stages' loads so its wait leaves them in flight.
    float binit[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) binit[j] = 0.0f;
#if defined(__HIP_DEVICE_COMPILE__)
    if constexpr (sizeof(T) == 2) {
        if (bias) {
            const __amdgpu_buffer_rsrc_t rbias = __builtin_amdgcn_make_buffer_rsrc((void *)bias, (short)0, N * 4, 0x00020000);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                binit[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                         rbias, (n0 + wn * (BN / WN) + 32 * j + (lane & 31)) * 4, 0, 0));
        }
    }
#endif
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st)
        if (st < nk) issue(st, st * BK);
    if constexpr (sizeof(T) == 2) {
        if (bias) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = binit[j];
        }
    }
    const int ra = wm * (BM / WM) + (lane & 31), rb = wn * (BN / WN) + (lane & 31);
    const int h = lane >> 5;
    // Each lane's fragment addresses within a stage, for chunk pair (h, s).
    int off_a[TM], off_b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) off_a[i] = (ra + i * 32) * ROWB;
#pragma unroll
    for (int j = 0; j < TN; ++j) off_b[j] = BM * ROWB + (rb + j * 32) * ROWB;
    const int sw_a = swz_of<ROWB>(ra), sw_b = swz_of<ROWB>(rb);   // rows 32 apart share the swizzle
    // The fragments: both operands double-buffered (the next k-step's read
    // while this one's products run), or, when the accumulators leave too few
    // registers for that, A's held once and each of its rows read again for
    // the next k-step as soon as this step's products of that row are out.
    constexpr bool SINGLE_A = TM * TN * 16 + 2 * (TM + TN) * 4 > 216;
    frag fa[SINGLE_A ? 1 : 2][TM], fb[2][TN];
    auto fetch_a = [&](const char *base, int s, int set, int i) {
        fa[set][i] = *(const frag *)(base + off_a[i] + 16 * ((2 * s + h) ^ sw_a));
    };
    // (In the order the first products use them: A's first row tile, then
    // B's, then A's other row tiles.)
    auto fetch = [&](const char *base, int s, int set) {
        const int c = 2 * s + h;
        if (!SINGLE_A || set == 0) fetch_a(base, s, SINGLE_A ? 0 : set, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[set][j] = *(const frag *)(base + off_b[j] + 16 * (c ^ sw_b));
#pragma unroll
        for (int i = 1; i < TM; ++i)
            if (!SINGLE_A || set == 0) fetch_a(base, s, SINGLE_A ? 0 : set, i);
    };
    for (int kt = 0; kt < nk; ++kt) {
        // This wave's loads of stage kt have landed once at most the later
        // stages' are outstanding; then the barrier makes every wave's visible.
        const int later = min(STAGES - 2, nk - 1 - kt);
        if (later >= STAGES - 2) wait_vmcnt<(STAGES - 2) * L>();
        else if (STAGES > 3 && later == 1) wait_vmcnt<L>();
        else wait_vmcnt<0>();
        __syncthreads();
        // The stage's first fragment reads go out before its successor's
        // loads are issued, so the products restart as soon as they can
        // after the barrier (FFN-out, K 3072: -2.5%).
        const char *base = smem + (kt % STAGES) * TILE;
        fetch(base, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + STAGES - 1 < nk) issue((kt + STAGES - 1) % STAGES, (kt + STAGES - 1) * BK);
        // The next k-step's fragments are read while this one's products run.
        // (sched_barrier keeps the compiler from sinking those reads back
        // under the products that do not need them.)
#pragma unroll
        for (int s = 0; s < ROWB / 32; ++s) {
            if constexpr (SINGLE_A) {
                if (s + 1 < ROWB / 32) {
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        fb[(s + 1) & 1][j] = *(const frag *)(base + off_b[j] + 16 * ((2 * (s + 1) + h) ^ sw_b));
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < TM; ++i) {
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = Mma<T>::run(fa[0][i], fb[s & 1][j], acc[i][j]);
                    if (s + 1 < ROWB / 32) fetch_a(base, s + 1, 0, i);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                if (s + 1 < ROWB / 32) fetch(base, s + 1, (s + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = Mma<T>::run(fa[s & 1][i], fb[s & 1][j], acc[i][j]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

}

template <typename T, typename OT, int BM, int BN, int WM, int WN, int STAGES, int BK, int OCC, Epi KIND>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(OCC, OCC)))
gemm_lds_kernel(Span sp, int a_tok, int N, int K, const T *__restrict__ A, int lda, const T *__restrict__ W, EpiArgs e,
                int grid_n) {
    using P = LdsTile<T, BM, BN, WM, WN, STAGES, BK>;
    constexpr int WAVES = P::WAVES, TILE = P::TILE, TM = P::TM, TN = P::TN;
    typedef typename Mma<T>::acc acc_t;
    extern __shared__ __attribute__((aligned(1024))) char smem[];

    const Live lv = live_of(sp);
    const int M = lv.tokens;
    // XCD-aware renumbering over the span's own tiles; blocks past them leave.
    const int live = (M + BM - 1) / BM * grid_n;
    if ((int)blockIdx.x >= live) return;
    A += (size_t)lv.tok0 * a_tok;
    place_epilogue<KIND, OT>(e, lv);
    const int per = live / 8;
    int b = blockIdx.x;
    if (b < per * 8) b = (b % 8) * per + b / 8;
    const int tile_n = b % grid_n, tile_m = b / grid_n;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    // The wave index is uniform: kept in scalar registers, the LDS bases of
    // the direct loads (M0) need no per-load readfirstlane.
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    // 16 rows a pass (half the staging LDS of 32, and the same row-wise
    // stores); 32 for the QKV scatter when they fit, so each V^T column
    // gets 64 contiguous bytes a store instead of 32.
    constexpr bool QKV_KIND = KIND == Epi::Qkv || KIND == Epi::QkvRope;
    // (int8 operands: each wave's rows' activation scales, and its columns'
    // weight scales and biases, beside the staging rows.)
    constexpr int I8_LDS = sizeof(T) == 1 ? WAVES * (BM / WM + 2 * TN * 32) * 4 : 0;
    constexpr int PASS = QKV_KIND && WAVES * 32 * (TN * 32 + 4) * 4 + I8_LDS <= STAGES * TILE ? 32 : 16;
    static_assert(WAVES * PASS * (TN * 32 + 4) * 4 + I8_LDS <= STAGES * TILE, "epilogue staging fits the stages");
    const int mw = m0 + wm * (BM / WM), nw = n0 + wn * (BN / WN);


    acc_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};
    lds_mainloop<T, BM, BN, WM, WN, STAGES, BK>(smem, A, lda, W, M, N, K, m0, n0, wave, lane, acc,
                                                sizeof(T) == 2 ? e.bias : nullptr);

    // The epilogue's per-column constants, read now (not held through the
    // main loop) and before the first store, so no store waits behind them.
    EpiCols<TN, PASS, sizeof(T) == 1> cols;
    load_cols<KIND>(cols, e, N, nw);
    // Every wave is done with the stages: their LDS becomes each wave's
    // staging area for the stores (and, for int8 operands, for its rows'
    // activation scales, read before the first store).
    __syncthreads();
    float *ascale = reinterpret_cast<float *>(smem + STAGES * TILE) - (WAVES - wave) * (BM / WM);
    if constexpr (sizeof(T) == 1) {
#pragma unroll
        for (int r = lane; r < BM / WM; r += 64) ascale[r] = mw + r < M ? e.a_scale[mw + r] : 0.0f;
        stage_cols(cols, reinterpret_cast<float *>(smem + STAGES * TILE) - WAVES * (BM / WM) -
                             (WAVES - wave) * 2 * TN * 32);
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's scales are in LDS
        __builtin_amdgcn_wave_barrier();
    }
    // (With BK 32 and four stages the rotary 256 x 384 shape spills if its
    // angles are read ahead.)
    epilogue_lds<OT, KIND, TM, TN, PASS, sizeof(T) == 1, BK == 64>(e, M, N, mw, nw,
                                                         reinterpret_cast<float *>(smem) + wave * PASS * (TN * 32 + 4),
                                                         ascale, cols, acc);
}

template <typename T, int BM, int BN, int WM, int WN, int STAGES, int BK, int OCC, Epi KIND>
static hipError_t launch_lds_k(hipStream_t s, const GemmRows &gr, int M, int N, int K, const void *A, int lda,
                               const void *W, const EpiArgs &e) {
    // int8 operands write F16 activations.
    typedef typename std::conditional<sizeof(T) == 1, _Float16, T>::type OT;
    constexpr int bytes = STAGES * (BM + BN) * BK * (int)sizeof(T);
    // Dynamic LDS up to the device's 160 KB per workgroup needs no attribute on gfx950.
    const int gn = (N + BN - 1) / BN, gm = (M + BM - 1) / BM;
    enqueue((gemm_lds_kernel<T, OT, BM, BN, WM, WN, STAGES, BK, OCC, KIND>), dim3(gn * gm),
            dim3(64 * WM * WN), bytes, s, gr.sp, gr.a_tok, N, K, (const T *)A, lda, (const T *)W, e, gn);
    return hipGetLastError();
}

template <typename T, int BM, int BN, int WM, int WN, int STAGES, int BK = 64, int OCC = 1>
static hipError_t launch_lds(hipStream_t s, const GemmRows &gr, int M, int N, int K, const void *A, int lda,
                             const void *W, const EpiArgs &e) {
#define LDS_CASE(E) \
    case Epi::E: return launch_lds_k<T, BM, BN, WM, WN, STAGES, BK, OCC, Epi::E>(s, gr, M, N, K, A, lda, W, e);
    switch (e.kind) {
        LDS_CASE(Plain)
        LDS_CASE(Qkv)
        LDS_CASE(Gelu)
        LDS_CASE(Residual)
        LDS_CASE(QkvRope)
        LDS_CASE(Gated)
        LDS_CASE(Bias)
    }
#undef LDS_CASE
    return hipErrorInvalidValue;
}

// ---- Whole-row tiles: the residual add and the LayerNorm in the epilogue ------------
//
// A product whose N is the hidden size (attention-out, FFN-out) on BM x N
// tiles, so each workgroup holds whole rows: y = A W^T + b, the residual add
// and the row's LayerNorm happen in its epilogue, and y never goes to HBM
// (the reference's LN-fused tile: core/cuda/autotune.h:40-41,
// core/cuda/kernels.cu:2954-2955, chosen at core/cuda/backend.cpp:1807-1849).
// The epilogue takes the tile's rows 32 WM at a time (one 32-row MFMA band
// of every wave row): each wave stages its columns of them through LDS, y
// rounded to the operand type as the separate product stores it; then each
// 32-lane half norms whole rows with the row kernels' arithmetic
// (rowmath.h: the same lane map, sums and rounding), so every row gets the
// bits the product followed by add_layer_norm gives it. Post-norm rows
// whose residual is carried in the 16-bit operand rows (out_h): read and
// written there, and in F32 too with keep_f32.
template <typename T, int BM, int BN, int WM, int WN, int STAGES, int BK>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_ln_kernel(Span sp, int a_tok, int K, const T *__restrict__ A, int lda, const T *__restrict__ W, LnArgs e) {
    constexpr int WAVES = WM * WN, TM = BM / WM / 32, TN = BN / WN / 32, G = BN / 256;
    constexpr int STAGE_BYTES = (BM + BN) * BK * (int)sizeof(T);
    constexpr int PR = 32 * WM;         // rows a pass
    constexpr int YS = BN + 8;          // staged row stride: 16 bytes of padding
    constexpr int RH = PR / WAVES / 2;  // rows a half-wave norms a pass
    static_assert(BN % 256 == 0 && RH >= 1 && RH * 2 * WAVES == PR, "whole rows a half-wave");
    static_assert(PR * YS * (int)sizeof(T) + 2 * BN * 4 <= STAGES * STAGE_BYTES, "staging fits the stages");
    typedef typename Mma<T>::acc acc_t;
    extern __shared__ __attribute__((aligned(1024))) char smem[];

    const Live lv = live_of(sp);
    const int M = lv.tokens;
    // XCD-aware renumbering over the span's row tiles; blocks past them leave.
    const int live = (M + BM - 1) / BM;
    if ((int)blockIdx.x >= live) return;
    A += (size_t)lv.tok0 * a_tok;
    const int per = live / 8;
    int b = blockIdx.x;
    if (b < per * 8) b = (b % 8) * per + b / 8;
    const int m0 = b * BM;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    acc_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};
    // (The accumulators start from the bias, as the separate product's do.)
    lds_mainloop<T, BM, BN, WM, WN, STAGES, BK>(smem, A, lda, W, M, BN, K, m0, 0, wave, lane, acc, e.bias);

    const int h = lane >> 5, ql = lane & 31;
    __syncthreads();   // every wave is done with the stages
    T *ys = reinterpret_cast<T *>(smem);
    float *lw = reinterpret_cast<float *>(smem + PR * YS * (int)sizeof(T));   // the norm's weight, then its bias
    for (int c = tid; c < BN; c += 64 * WAVES) {
        lw[c] = e.ln_w[c];
        lw[BN + c] = e.ln_b ? e.ln_b[c] : 0.0f;
    }
    T *xh = reinterpret_cast<T *>(e.out_h) + (size_t)lv.tok0 * BN;
    float *xf = e.x + (size_t)lv.tok0 * BN;
    // The residual rows a half normalizes in pass i, 16 raw bytes of each
    // group: read a pass ahead, so their latency hides behind the pass
    // before (rows past M read row M - 1, and are not stored).
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    auto row_of = [&](int i, int q) {
        const int pr = (wave * 2 + h) * RH + q;
        return m0 + (pr / 32) * (BM / WM) + 32 * i + (pr % 32);
    };
    auto load_res = [&](int i, u32x4 (&r)[RH][G]) {
#pragma unroll
        for (int q = 0; q < RH; ++q) {
            const int m = min(row_of(i, q), M - 1);
#pragma unroll
            for (int g = 0; g < G; ++g) r[q][g] = *(const u32x4 *)(xh + (size_t)m * BN + 8 * (ql + 32 * g));
        }
    };
    u32x4 res[2][RH][G];
    load_res(0, res[0]);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        // Band i of this wave's rows is pass rows wm * 32 ..; register r of
        // MFMA tile (i, j) is row 8 (r / 4) + 4 h + r % 4, column 32 j + ql.
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = wm * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
                ys[row * YS + wn * (BN / WN) + 32 * j + ql] = from_f32<T>(acc[i][j][r]);
            }
        __syncthreads();
        if (i + 1 < TM) load_res(i + 1, res[(i + 1) & 1]);
#pragma unroll
        for (int q = 0; q < RH; ++q) {
            const int pr = (wave * 2 + h) * RH + q;   // the half's row of the pass
            const int m = row_of(i, q);
            if (m >= M) continue;   // (the same for the whole half)
            float v[G][8];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const int c = 8 * (ql + 32 * g);
                float a[8];
                load8(reinterpret_cast<const T *>(&res[i & 1][q][g]), v[g]);
                load8(ys + pr * YS + c, a);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[g][k] = v[g][k] + a[k];
            }
            float mean, inv;
            ln_pair_stats<G>(v, BN, ql, e.eps, mean, inv);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const int c = 8 * (ql + 32 * g);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[g][k] = ln_out(v[g][k], mean, inv, lw[c + k], lw[BN + c + k]);
                if (e.keep_f32) store8(xf + (size_t)m * BN + c, v[g]);
                store8(xh + (size_t)m * BN + c, v[g]);
            }
        }
        __syncthreads();   // the pass's rows are read before the next pass stages
    }
}

// The whole-row block shape: 128 x 768, 8 waves as 1 x 8 (each 128 x 96),
// 32 columns of k a stage in two stages (114 KB). (As 2 x 4 waves of 64 x
// 192, both fragment sets double-buffered, it needs more than 256
// registers; 16 columns of k in five stages, loads four steps ahead, made
// the FFN-out product slower: 278 against 207 us at 32768 rows.)
template <typename T, int WM, int WN, int STAGES, int BK>
static hipError_t launch_ln(hipStream_t s, const GemmRows &gr, int M, int K, const void *A, int lda, const void *W,
                            const LnArgs &e) {
    constexpr int BM = 128, BN = 768;
    constexpr int bytes = (BM + BN) * BK * (int)sizeof(T) * STAGES;
    enqueue((gemm_ln_kernel<T, BM, BN, WM, WN, STAGES, BK>), dim3((M + BM - 1) / BM), dim3(64 * WM * WN),
            bytes, s, gr.sp, gr.a_tok, K, (const T *)A, lda, (const T *)W, e);
    return hipGetLastError();
}

bool gemm_ln_takes(Dt dt, int hidden, int K, int lda, bool res_h) {
    return dt == Dt::F16 && hidden == 768 && res_h && K % 32 == 0 && lda % 8 == 0;
}

bool gemm_ln_tile(int tile) { return tile == LN_TILE; }

bool gemm_splitk_tile(int tile) { return tile == SPLITK_TILE_4 || tile == SPLITK_TILE_2; }

hipError_t gemm_ln(hipStream_t s, Dt dt, const Span &sp, int max_m, int hidden, int K, const void *A, int lda,
                   int a_tok, const void *W, const LnArgs &e, int tile) {
    if (max_m <= 0) return hipSuccess;
    if (!gemm_ln_takes(dt, hidden, K, lda, e.res_h != 0) || !e.out_h || !e.ln_w || (e.keep_f32 && !e.x))
        return hipErrorInvalidValue;
    if (tile == 0) tile = LN_TILE;
    if (!gemm_ln_tile(tile)) return hipErrorInvalidValue;
    if (gemm_made_to_fail(tile)) return hipErrorInvalidDeviceFunction;
    const GemmRows gr{sp, a_tok ? a_tok : lda};
    return launch_ln<_Float16, 1, 8, 2, 32>(s, gr, max_m, K, A, lda, W, e);
}

// The highest block-shape number.
constexpr int TILES = 19;

int gemm_tiles() { return TILES; }

// The block shape made to fail to launch, as on a device that cannot take
// it (a test hook; -1 for none): an explicit launch of it fails, the rule
// picks another, the tuner skips it and a session forcing it is refused.
static std::mutex fail_lock;
static int fail_tile = -1;

bool gemm_fail_variant(const char *name) {
    const int t = name && *name ? gemm_tile_by_name(name, std::strlen(name)) : -1;
    if (name && *name && t <= 0) return false;
    std::lock_guard<std::mutex> g(fail_lock);
    fail_tile = t;
    return true;
}

bool gemm_made_to_fail(int tile) {
    std::lock_guard<std::mutex> g(fail_lock);
    return tile > 0 && tile == fail_tile;
}

// Names of the block shapes, as a choices string spells them: output tile,
// then what sets it apart (r: operands staged through registers; k32: 32
// columns of k a stage; s<n>: n stages).
static const char *const TILE_NAME[TILES + 1] = {
    "auto",      "r128x128",   "r256x128",     "r64x128",    "256x128", "128x128", "128x256",
    "256x256",   "128x128s2",  "256x128k32",   "128x256k32", "256x128k32s3", "256x256k32", "256x192",
    "r64x64",    "256x384",    "256x384k32s4", "128x768ln", "r128x128sk4", "r64x64sk2"};

const char *gemm_tile_name(int tile) { return tile >= 0 && tile <= TILES ? TILE_NAME[tile] : "?"; }

int gemm_tile_by_name(const char *s, size_t n) {
    for (int t = 0; t <= TILES; ++t)
        if (std::strlen(TILE_NAME[t]) == n && std::strncmp(TILE_NAME[t], s, n) == 0) return t;
    // A bare number names a tile too.
    int v = 0;
    if (n == 0 || n > 2) return -1;
    for (size_t i = 0; i < n; ++i) {
        if (s[i] < '0' || s[i] > '9') return -1;
        v = v * 10 + (s[i] - '0');
    }
    return v <= TILES ? v : -1;
}

// Columns of one wave's output tile, per block shape (the staged shapes,
// 1-3 and 14, store column by column and take any).
static int wave_cols(int tile) {
    switch (tile) {
    case 6:
    case 10: return 128;
    case 13:
    case 15:
    case 16: return 96;
    case 4: case 5: case 7: case 8: case 9: case 11: case 12: return 64;
    default: return 1;
    }
}

// The tiles worth timing for a product of this type and shape: every
// pipelined shape when the operands take it, else the staged ones.
int gemm_candidates(Dt dt, int K, int lda, const EpiArgs &e, int *out, int cap) {
    int n = 0;
    auto add = [&](int t) {
        if (n < cap) out[n++] = t;
    };
    const bool qkv = e.kind == Epi::Qkv || e.kind == Epi::QkvRope;
    // Q, K and V must each start on a wave's column boundary.
    auto fits = [&](int t) { return !qkv || e.hidden % wave_cols(t) == 0; };
    if (dt == Dt::I8) {
        if (K % 128 == 0) add(7);
        // (Not with the rotary epilogue, whose angles spill this shape's registers.)
        if (K % 128 == 0 && fits(15) && e.kind != Epi::QkvRope) add(15);
        add(9);
        return n;
    }
    if (dt == Dt::F32 || K % 64 != 0 || lda % 8 != 0) {
        add(1);
        add(2);
        add(3);
        add(14);
        return n;
    }
    for (int t : {7, 13, 15, 16, 4, 6, 5, 9, 10})
        if (fits(t)) add(t);
    return n;
}

// The device's compute units, for the launch-shape choice.
// (Read once per device: an attribute query on every launch costs host time
// the device then spends idle between eagerly launched products.)
static int cu_count() {
    static std::atomic<int> cached[64];
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (dev >= 0 && dev < 64 && (n = cached[dev].load(std::memory_order_relaxed)) > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
    if (dev >= 0 && dev < 64) cached[dev].store(n, std::memory_order_relaxed);
    return n;
}

// The pipelined block shape for a large product: 256 x 256 output tiles,
// or 256 x 192 on a long inner dimension when they leave the compute units
// less idle over the launch's rounds of tiles (time ~ rounds x tile area).
// Measured on MI355X at 32768 tokens: 256 x 192 is faster at N = 768,
// K = 3072 (whole rounds against one and a half), slower at K = 768, where
// its 96-column waves' operand reads and epilogue cost more than the rounds
// save. Q, K and V must each start on a wave's column boundary (64 or 96).
static int wide_tile(int M, int N, int K, const EpiArgs &e) {
    const bool qkv = e.kind == Epi::Qkv || e.kind == Epi::QkvRope;
    const long cus = cu_count();
    auto cost = [&](int bm, int bn) {
        const long tiles = (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        return (double)((tiles + cus - 1) / cus) * bm * bn;
    };
    const bool can192 = (!qkv || e.hidden % 96 == 0) && K >= 2048;
    if (can192 && cost(256, 192) * 1.03 < cost(256, 256)) return 13;
    return 7;
}

// Block shapes by number: 1-3 and 14 stage operands through registers (any K
// a multiple of 8, and the F32 tier); 4-13, 15 and 16 are the pipelined
// kernel, for 16-bit operands with K a multiple of 64 (every encoder shape
// here).
template <typename T, int BK>
static hipError_t gemm_t(hipStream_t s, const GemmRows &gr, int M, int N, int K, const void *A, int lda, const void *W,
                         const EpiArgs &e,
                         int tile) {
    const bool pipelined = sizeof(T) == 2 && K % 64 == 0 && lda % 8 == 0;
    if (tile == 0) {
        tile = pipelined ? (M >= 2048 ? wide_tile(M, N, K, e) : 5) : 1;
        // The rule's next choices when its own cannot launch here.
        static const int PIPELINED[] = {7, 4, 5, 6, 8}, STAGED[] = {1, 2, 3, 14, 0};
        const int *next = pipelined ? PIPELINED : STAGED;
        for (int i = 0; gemm_made_to_fail(tile) && i < 5 && next[i]; ++i) tile = next[i];
    }
    if (gemm_made_to_fail(tile)) return hipErrorInvalidDeviceFunction;
    // A pipelined shape asked of an operand it cannot take runs the staged kernel.
    if (((tile >= 4 && tile <= 13) || tile == 15 || tile == 16) && !pipelined) tile = (N % 128 == 0 && M >= 8192) ? 2 : 1;
    // Q, K and V must each start on a wave's column boundary: a shape whose
    // waves are wider than 64 columns runs 64-column waves (K = hidden is a
    // multiple of 64 on the pipelined kernel) when they do not.
    if ((e.kind == Epi::Qkv || e.kind == Epi::QkvRope) && e.hidden % wave_cols(tile) != 0) tile = 7;
    switch (tile) {
    // Split K: the staged kernel's tiles over K in 4 (128 x 128) or 2 (64 x 64) slices.
    case SPLITK_TILE_4: return launch_split<T, 128, 128, BK>(s, gr, M, N, K, A, lda, W, e, 4);
    case SPLITK_TILE_2: return launch_split<T, 64, 64, BK>(s, gr, M, N, K, A, lda, W, e, 2);
    case 1: return launch<T, 128, 128, BK>(s, gr, M, N, K, A, lda, W, e);
    case 2: return launch<T, 256, 128, BK>(s, gr, M, N, K, A, lda, W, e);
    case 3: return launch<T, 64, 128, BK>(s, gr, M, N, K, A, lda, W, e);
    // 64 x 64: four times the workgroups of 128 x 128, for products too small to fill the chip.
    case 14: return launch<T, 64, 64, BK>(s, gr, M, N, K, A, lda, W, e);
    }
    if constexpr (sizeof(T) == 2) {
        switch (tile) {
        case 4: return launch_lds<T, 256, 128, 2, 2, 3>(s, gr, M, N, K, A, lda, W, e);
        case 5: return launch_lds<T, 128, 128, 2, 2, 4>(s, gr, M, N, K, A, lda, W, e);
        case 6: return launch_lds<T, 128, 256, 2, 2, 3>(s, gr, M, N, K, A, lda, W, e);
        case 7: return launch_lds<T, 256, 256, 2, 4, 2>(s, gr, M, N, K, A, lda, W, e);
        case 8: return launch_lds<T, 128, 128, 2, 2, 2>(s, gr, M, N, K, A, lda, W, e);
        // BK 32 with two workgroups a CU, so one's epilogue overlaps the other's products.
        case 9: return launch_lds<T, 256, 128, 2, 2, 2, 32, 2>(s, gr, M, N, K, A, lda, W, e);
        case 10: return launch_lds<T, 128, 256, 2, 2, 2, 32, 2>(s, gr, M, N, K, A, lda, W, e);
        case 11: return launch_lds<T, 256, 128, 2, 2, 3, 32, 2>(s, gr, M, N, K, A, lda, W, e);
        case 12: return launch_lds<T, 256, 256, 2, 4, 3, 32, 1>(s, gr, M, N, K, A, lda, W, e);
        // 8 waves as 4 x 2 of 64 x 96: N = 768, 2304 and 3072 in whole rounds of tiles.
        case 13: return launch_lds<T, 256, 192, 4, 2, 2>(s, gr, M, N, K, A, lda, W, e);
        // 8 waves as 2 x 4 of 128 x 96: a third less LDS reading per product than
        // 128 x 64 waves, and N = 768, 2304 and 3072 in whole rounds at 32768 rows.
        case 15: return launch_lds<T, 256, 384, 2, 4, 2>(s, gr, M, N, K, A, lda, W, e);
        // The same waves on 32 columns of k a stage, four stages (all 160 KB
        // of LDS): loads issued three steps ahead instead of one.
        case 16: return launch_lds<T, 256, 384, 2, 4, 4, 32, 1>(s, gr, M, N, K, A, lda, W, e);
        }
    }
    return hipErrorInvalidValue;
}

// The int8 tier: the pipelined kernel alone, on 128-byte rows (K a multiple
// of 128: 256 x 256 or 256 x 384 tiles) or 64-byte rows (K a multiple of 64).
static hipError_t gemm_i8(hipStream_t s, const GemmRows &gr, int M, int N, int K, const void *A, int lda, const void *W,
                          const EpiArgs &e,
                          int tile) {
    if (K % 64 != 0 || lda % 16 != 0 || !e.a_scale || !e.w_scale) return hipErrorInvalidValue;
    if (tile == 0) {
        tile = K % 128 == 0 ? 7 : 9;
        if (gemm_made_to_fail(tile)) tile = tile == 7 ? 9 : 7;
    }
    if ((tile == 7 || tile == 15) && K % 128 != 0) tile = 9;
    if (gemm_made_to_fail(tile)) return hipErrorInvalidDeviceFunction;
    switch (tile) {
    case 7: return launch_lds<int8_t, 256, 256, 2, 4, 2, 128, 1>(s, gr, M, N, K, A, lda, W, e);
    case 15: return launch_lds<int8_t, 256, 384, 2, 4, 2, 128, 1>(s, gr, M, N, K, A, lda, W, e);
    default: return launch_lds<int8_t, 256, 128, 2, 2, 2, 64, 2>(s, gr, M, N, K, A, lda, W, e);
    }
}

hipError_t gemm(hipStream_t s, Dt dt, const Span &sp, int M, int N, int K, const void *A, int lda, int a_tok,
                const void *W, const EpiArgs &e, int tile) {
    if (M <= 0) return hipSuccess;
    // The whole-row shapes take a LayerNorm with them: gemm_ln. Split K is
    // for Bias products with a workspace, off the int8 tier.
    if (gemm_ln_tile(tile)) return hipErrorInvalidValue;
    if (gemm_splitk_tile(tile) && (e.kind != Epi::Bias || !e.ws || dt == Dt::I8)) return hipErrorInvalidValue;
    const GemmRows gr{sp, a_tok ? a_tok : lda};
    if (dt == Dt::I8) return gemm_i8(s, gr, M, N, K, A, lda, W, e, tile);
    if (K % (16 / (int)dt_bytes(dt)) != 0 || lda % (16 / (int)dt_bytes(dt)) != 0) return hipErrorInvalidValue;
    if ((e.kind == Epi::QkvRope || e.kind == Epi::Gated) && N % 2 != 0) return hipErrorInvalidValue;
    switch (dt) {
    case Dt::F16: return gemm_t<_Float16, 32>(s, gr, M, N, K, A, lda, W, e, tile);
    case Dt::BF16: return gemm_t<__bf16, 32>(s, gr, M, N, K, A, lda, W, e, tile);
    default: return gemm_t<float, 16>(s, gr, M, N, K, A, lda, W, e, tile);
    }
}

// ---- MFMA rate probe ----------------------------------------------------------
//
// Every wave issues 8 independent v_mfma_f32_32x32x16_f16 chains for `iters`
// rounds: with fixed operands (the same in every round), or with random ones,
// four sets of fragments taken in turn, as a GEMM's change every k-step. The
// chip's clock under the load is the shader clock count over the 100 MHz
// real-time count of block 0's first wave.
__global__ void __launch_bounds__(256) mfma_probe_kernel(float *out, unsigned long long *clk, int iters, int random) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    typedef float f16x __attribute__((ext_vector_type(16)));
    f16x acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f16x{};
    h8 a[4], b[4];
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t h = (threadIdx.x * 8 + i + 2048 * v) * 0x9e3779b9u;
            h ^= h >> 16;
            h *= 0x7feb352du;
            h ^= h >> 15;
            a[v][i] = random ? (_Float16)((float)(h & 0xffff) / 32768.0f - 1.0f) : (_Float16)(0.5f + i);
            b[v][i] = random ? (_Float16)((float)(h >> 16) / 32768.0f - 1.0f) : (_Float16)0.25f;
        }
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[2 * v + j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[v], b[(v + j) & 3], acc[2 * v + j], 0, 0, 0);
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[j][r];
    if (s == 1234.5f) out[threadIdx.x] = s;   // keeps the products
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        clk[0] = t1 - t0;
        clk[1] = r1 - r0;
    }
}

hipError_t mfma_probe(hipStream_t s, int blocks, int iters, int random, float *out, unsigned long long *clk) {
    enqueue(mfma_probe_kernel, dim3(blocks), dim3(256), 0, s, out, clk, iters, random);
    return hipGetLastError();
}

}  // namespace rocm
