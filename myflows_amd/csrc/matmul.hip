// The teaching matmul family behind native.matmul: C(M,N) = A(M,K) B(K,N), all row-major, with
// three summation modes. These kernels are the accuracy references of the API; the fast path is the
// MFMA engine in gemm.hip.
//
// Summation modes (per output element, terms taken in increasing k):
//   SEQUENTIAL   one FMA chain over all K terms.
//   GROUPED      an FMA chain inside each group of G consecutive terms; each group's chain is folded
//                into a compensated pair (sum, err) with Knuth's TwoSum, so the error no longer
//                grows with K.
//   DOT2         Ogita, Rump and Oishi, "Accurate sum and dot product", SIAM J. Sci. Comput. 26(6),
//                2005, Algorithm Dot2: every product is split exactly (TwoProduct via FMA) and added
//                with TwoSum, as if accumulated in twice the working precision and rounded once.
// The error-free transformations are compiled with contraction off; the FMA in TwoProduct is
// explicit. Group sizes: 32 for the one-thread-per-output and register-blocked kernels, TILE for
// the tiled and LDS kernels, so the register-blocked kernel repeats the exact operation sequence of
// the one-thread-per-output kernel and the two agree bit for bit.
#include "common.h"

namespace mfh {
namespace {

enum SumMode { SEQUENTIAL = 0, GROUPED = 1, DOT2 = 2 };

// Knuth's TwoSum: hi + lo == a + b exactly, hi = fl(a + b).
__device__ __forceinline__ void knuth_two_sum(float a, float b, float& hi, float& lo) {
#pragma clang fp contract(off)
    hi = a + b;
    const float b_virtual = hi - a;
    const float a_virtual = hi - b_virtual;
    lo = (a - a_virtual) + (b - b_virtual);
}

// Running state of one output element.
template <int MODE>
struct DotState {
    float chain = 0.f;  // SEQUENTIAL, GROUPED: the current FMA chain
    float sum = 0.f;    // GROUPED, DOT2: compensated pair
    float err = 0.f;

    __device__ __forceinline__ void term(float a, float b) {
#pragma clang fp contract(off)
        if constexpr (MODE == DOT2) {
            const float product = a * b;
            const float product_err = __builtin_fmaf(a, b, -product);
            float hi, lo;
            knuth_two_sum(sum, product, hi, lo);
            err = err + (lo + product_err);
            sum = hi;
        } else {
            chain = __builtin_fmaf(a, b, chain);
        }
    }

    __device__ __forceinline__ void close_group() {
#pragma clang fp contract(off)
        if constexpr (MODE == GROUPED) {
            float hi, lo;
            knuth_two_sum(sum, chain, hi, lo);
            err = err + lo;
            sum = hi;
            chain = 0.f;
        }
    }

    __device__ __forceinline__ float value() {
#pragma clang fp contract(off)
        if constexpr (MODE == SEQUENTIAL) return chain;
        close_group();
        return sum + err;
    }
};

// Row `a` (stride 1) times column `b` (stride ldb) from global memory, groups of G terms.
template <int G, int MODE>
__device__ __forceinline__ float global_dot(const float* a, const float* b, int ldb, int K) {
    DotState<MODE> st;
    for (int k0 = 0; k0 < K; k0 += G) {
        const int k1 = min(k0 + G, K);
        for (int k = k0; k < k1; ++k) st.term(a[k], b[static_cast<long long>(k) * ldb]);
        st.close_group();
    }
    return st.value();
}

// One thread per output element on a 1-D grid of 256-thread workgroups.
template <int MODE>
__global__ __launch_bounds__(256) void matmul_per_output(const float* A, const float* B, float* C, int M, int N,
                                                         int K) {
    const long long e = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (e >= static_cast<long long>(M) * N) return;
    const int i = static_cast<int>(e / N), j = static_cast<int>(e % N);
    C[e] = global_dot<32, MODE>(A + static_cast<long long>(i) * K, B + j, N, K);
}

// TILE x TILE workgroups, one per output tile, operands straight from global memory.
template <int TILE, int MODE>
__global__ __launch_bounds__(TILE* TILE) void matmul_tiled(const float* A, const float* B, float* C, int M, int N,
                                                           int K) {
    const int i = blockIdx.y * TILE + threadIdx.y, j = blockIdx.x * TILE + threadIdx.x;
    if (i < M && j < N) C[static_cast<long long>(i) * N + j] = global_dot<TILE, MODE>(A + static_cast<long long>(i) * K, B + j, N, K);
}

// TILE x TILE tiles of A and B staged in LDS; each staged element is used TILE times.
template <int TILE, int MODE>
__global__ __launch_bounds__(TILE* TILE) void matmul_lds(const float* A, const float* B, float* C, int M, int N,
                                                         int K) {
    __shared__ float a_tile[TILE][TILE + 1];
    __shared__ float b_tile[TILE][TILE + 1];
    const int c = threadIdx.x, r = threadIdx.y;
    const int i = blockIdx.y * TILE + r, j = blockIdx.x * TILE + c;
    DotState<MODE> st;
    for (int k0 = 0; k0 < K; k0 += TILE) {
        a_tile[r][c] = (i < M && k0 + c < K) ? A[static_cast<long long>(i) * K + k0 + c] : 0.f;
        b_tile[r][c] = (k0 + r < K && j < N) ? B[static_cast<long long>(k0 + r) * N + j] : 0.f;
        __syncthreads();
        const int depth = min(TILE, K - k0);
        for (int k = 0; k < depth; ++k) st.term(a_tile[r][k], b_tile[k][c]);
        st.close_group();
        __syncthreads();
    }
    if (i < M && j < N) C[static_cast<long long>(i) * N + j] = st.value();
}

// Register-blocked: 64 x 64 workgroup tiles, 256 threads with 4 x 4 outputs each (rows ry + 16 u,
// columns rx + 16 v), 32-deep LDS stages. Each stage is one group of 32 terms, in increasing k.
template <int MODE>
__global__ __launch_bounds__(256) void matmul_register(const float* A, const float* B, float* C, int M, int N,
                                                       int K) {
    constexpr int T = 64, D = 32;
    __shared__ float a_stage[D][T + 1];
    __shared__ float b_stage[D][T + 1];
    const int tid = threadIdx.x, rx = tid % 16, ry = tid / 16;
    const int i0 = blockIdx.y * T, j0 = blockIdx.x * T;
    DotState<MODE> st[4][4];
    for (int k0 = 0; k0 < K; k0 += D) {
        for (int f = tid; f < T * D; f += 256) {
            const int ar = f / D, ak = f % D;  // A: 64 rows x 32 k, read along k
            a_stage[ak][ar] = (i0 + ar < M && k0 + ak < K) ? A[static_cast<long long>(i0 + ar) * K + k0 + ak] : 0.f;
            const int bk = f / T, bc = f % T;  // B: 32 k x 64 columns, read along columns
            b_stage[bk][bc] = (k0 + bk < K && j0 + bc < N) ? B[static_cast<long long>(k0 + bk) * N + j0 + bc] : 0.f;
        }
        __syncthreads();
        const int depth = min(D, K - k0);
        for (int k = 0; k < depth; ++k) {
            float av[4], bv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) av[u] = a_stage[k][ry + 16 * u];
#pragma unroll
            for (int v = 0; v < 4; ++v) bv[v] = b_stage[k][rx + 16 * v];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) st[u][v].term(av[u], bv[v]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) st[u][v].close_group();
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int i = i0 + ry + 16 * u, j = j0 + rx + 16 * v;
            if (i < M && j < N) C[static_cast<long long>(i) * N + j] = st[u][v].value();
        }
}

template <int MODE>
int launch_mode(int variant, int tile, const float* a, const float* b, float* c, int M, int N, int K,
                hipStream_t stream) {
    if (variant == 0) {
        launch(matmul_per_output<MODE>, blocks_for(static_cast<std::int64_t>(M) * N, 256), 256, 0, stream, a, b, c, M, N,
                                                                                                       K);
        return MFH_CHECK_LAUNCH("matmul_per_output", stream);
    }
    if (variant == 4) {
        if (blocks_for(M, 64) > GRID_YZ_LIMIT) return MFH_FAIL(ERR_ARG, "matmul rows exceed the grid limit");
        launch(matmul_register<MODE>, dim3(blocks_for(N, 64), blocks_for(M, 64)), 256, 0, stream, a, b, c, M, N, K);
        return MFH_CHECK_LAUNCH("matmul_register", stream);
    }
    if (blocks_for(M, tile) > GRID_YZ_LIMIT) return MFH_FAIL(ERR_ARG, "matmul rows exceed the grid limit");
    const dim3 grid(blocks_for(N, tile), blocks_for(M, tile)), block(tile, tile);
    if (variant == 1) {
        if (tile == 16) launch(matmul_tiled<16, MODE>, grid, block, 0, stream, a, b, c, M, N, K);
        else launch(matmul_tiled<32, MODE>, grid, block, 0, stream, a, b, c, M, N, K);
        return MFH_CHECK_LAUNCH("matmul_tiled", stream);
    }
    if (tile == 16) launch(matmul_lds<16, MODE>, grid, block, 0, stream, a, b, c, M, N, K);
    else launch(matmul_lds<32, MODE>, grid, block, 0, stream, a, b, c, M, N, K);
    return MFH_CHECK_LAUNCH("matmul_lds", stream);
}

}  // namespace

int launch_matmul(int variant, int tile, int accumulate, const float* a, const float* b, float* c, int M, int N,
                  int K, hipStream_t stream) {
    switch (accumulate) {
        case SEQUENTIAL: return launch_mode<SEQUENTIAL>(variant, tile, a, b, c, M, N, K, stream);
        case GROUPED: return launch_mode<GROUPED>(variant, tile, a, b, c, M, N, K, stream);
        default: return launch_mode<DOT2>(variant, tile, a, b, c, M, N, K, stream);
    }
}

}  // namespace mfh
