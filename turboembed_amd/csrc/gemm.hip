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
#include "kernels.h"
#include "devmath.h"

namespace rocm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mma;

template <> struct Mma<_Float16> {
    static constexpr int EPM = 8;   // elements a lane feeds one MFMA
    typedef half8 frag;
    static __device__ __forceinline__ floatx16 run(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <> struct Mma<__bf16> {
    static constexpr int EPM = 8;
    typedef bf16x8 frag;
    static __device__ __forceinline__ floatx16 run(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

template <> struct Mma<float> {
    static constexpr int EPM = 1;
    typedef float frag;
    static __device__ __forceinline__ floatx16 run(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

// The epilogue of one output element pair-aware: v is acc + bias at (m, n).
template <typename T>
__device__ __forceinline__ void epilogue_store(const EpiArgs &e, int M, int N, int m, int n, float acc) {
    const float v = acc + (e.bias ? e.bias[n] : 0.0f);
    switch (e.kind) {
    case Epi::Plain:
        if (m < M && n < N) ((float *)e.out)[(size_t)m * e.ldo + n] = v;
        break;
    case Epi::Gelu:
        if (m < M && n < N) ((T *)e.out)[(size_t)m * e.ldo + n] = from_f32<T>(dev_gelu(v));
        break;
    case Epi::Residual:
        if (m < M && n < N) {
            float *x = e.x + (size_t)m * e.ldo + n;
            *x = *x + v;
        }
        break;
    case Epi::Qkv: {
        if (m < M && n < N) {
            const int which = n / e.hidden, rem = n - which * e.hidden;
            const int head = rem / e.d, c = rem - head * e.d;
            ((T *)e.out)[(((size_t)which * e.heads + head) * e.tcap + m) * e.d + c] = from_f32<T>(v);
        }
        break;
    }
    case Epi::QkvRope: {
        // Columns come pair-adjacent: the partner of n is n ^ 1, in the
        // neighbouring lane (the MFMA layout puts column n in lane n % 32).
        const float w = __shfl_xor(v, 1, 64);
        if (m < M && n < N) {
            const int which = n / e.hidden, rem = n - which * e.hidden;
            const int head = rem / e.d, c = rem - head * e.d;
            float y = v;
            if (which < 2) {
                const int pos = e.at[m] % e.seq, pr = c >> 1;
                const float cs = e.cos[(size_t)pos * (e.d >> 1) + pr], sn = e.sin[(size_t)pos * (e.d >> 1) + pr];
                // (x1, x2) -> (x1 cos - x2 sin, x2 cos + x1 sin)
                y = (c & 1) ? __fadd_rn(__fmul_rn(v, cs), __fmul_rn(w, sn)) : __fsub_rn(__fmul_rn(v, cs), __fmul_rn(w, sn));
            }
            ((T *)e.out)[(((size_t)which * e.heads + head) * e.tcap + m) * e.d + c] = from_f32<T>(y);
        }
        break;
    }
    case Epi::Gated: {
        const float up = __shfl_xor(v, 1, 64);
        if (m < M && n < N && (n & 1) == 0) {
            const float g = e.silu ? dev_silu(v) : dev_gelu(v);
            ((T *)e.out)[(size_t)m * e.ldo + (n >> 1)] = from_f32<T>(__fmul_rn(g, up));
        }
        break;
    }
    }
}

template <typename T, int BM, int BN, int BK>
__global__ void __launch_bounds__(256) gemm_kernel(int M, int N, int K, const T *__restrict__ A, int lda,
                                                   const T *__restrict__ W, EpiArgs e, int grid_n) {
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

    // XCD-aware renumbering of the block.
    const int nb = gridDim.x, per = nb / 8;
    int b = blockIdx.x;
    if (b < per * 8) b = (b % 8) * per + b / 8;
    const int tile_n = b % grid_n, tile_m = b / grid_n;
    const int m0 = tile_m * BM, n0 = tile_n * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    vec4 ra[LA], rb[LB];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            const int v = tid + 256 * i, r = v / VROW, c = (v % VROW) * VEC;
            const int gm = min(m0 + r, M - 1), gk = k0 + c;
            ra[i] = gk + VEC <= K ? *(const vec4 *)(A + (size_t)gm * lda + gk) : vec4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            const int v = tid + 256 * i, r = v / VROW, c = (v % VROW) * VEC;
            const int gn = min(n0 + r, N - 1), gk = k0 + c;
            rb[i] = gk + VEC <= K ? *(const vec4 *)(W + (size_t)gn * K + gk) : vec4{0, 0, 0, 0};
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

    const int nk = (K + BK - 1) / BK;
    load(0);
    store(0);
    __syncthreads();
    const int row_a = wm * (BM / 2) + (lane & 31), row_b = BM + wn * (BN / 2) + (lane & 31);
    const int col = (lane >> 5) * HALF;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load((kt + 1) * BK);
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
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                epilogue_store<T>(e, M, N, m, n, acc[i][j][r]);
            }
        }
}

template <typename T, int BM, int BN, int BK>
static hipError_t launch(hipStream_t s, int M, int N, int K, const void *A, int lda, const void *W, const EpiArgs &e) {
    const int gn = (N + BN - 1) / BN, gm = (M + BM - 1) / BM;
    hipLaunchKernelGGL((gemm_kernel<T, BM, BN, BK>), dim3(gn * gm), dim3(256), 0, s, M, N, K, (const T *)A, lda,
                       (const T *)W, e, gn);
    return hipGetLastError();
}

int gemm_tiles() { return 3; }

template <typename T, int BK>
static hipError_t gemm_t(hipStream_t s, int M, int N, int K, const void *A, int lda, const void *W, const EpiArgs &e,
                         int tile) {
    if (tile == 0) tile = (N % 128 == 0 && M >= 8192) ? 2 : 1;
    switch (tile) {
    case 1: return launch<T, 128, 128, BK>(s, M, N, K, A, lda, W, e);
    case 2: return launch<T, 256, 128, BK>(s, M, N, K, A, lda, W, e);
    case 3: return launch<T, 64, 128, BK>(s, M, N, K, A, lda, W, e);
    default: return hipErrorInvalidValue;
    }
}

hipError_t gemm(hipStream_t s, Dt dt, int M, int N, int K, const void *A, int lda, const void *W, const EpiArgs &e,
                int tile) {
    if (M <= 0) return hipSuccess;
    if (K % (16 / (int)dt_bytes(dt)) != 0 || lda % (16 / (int)dt_bytes(dt)) != 0) return hipErrorInvalidValue;
    if ((e.kind == Epi::QkvRope || e.kind == Epi::Gated) && N % 2 != 0) return hipErrorInvalidValue;
    switch (dt) {
    case Dt::F16: return gemm_t<_Float16, 32>(s, M, N, K, A, lda, W, e, tile);
    case Dt::BF16: return gemm_t<__bf16, 32>(s, M, N, K, A, lda, W, e, tile);
    default: return gemm_t<float, 16>(s, M, N, K, A, lda, W, e, tile);
    }
}

}  // namespace rocm
