// The lecture matmul family behind native.matmul: C(M,N) = A(M,K) B(K,N), all row-major, with
// three summation modes. These kernels are the correctness and accuracy references of the API;
// the fast path is the MFMA engine in gemm.hip.
//   accumulate 0: sequential FMA.
//   accumulate 1: FMA inside groups of G consecutive terms; groups are combined with TwoSum and the
//                 rounding errors are carried in a separate compensation term (Kahan-style).
//   accumulate 2: Dot2 of Ogita, Rump and Oishi (SIAM J. Sci. Comput. 26(6), 2005): TwoProduct and
//                 TwoSum on every term, i.e. the dot product as if accumulated in twice the working
//                 precision and rounded once.
// Error-free transformations must not be contracted into FMAs, so they are compiled with
// contraction off; the FMA in TwoProduct is explicit.
#include "common.h"

namespace mfh {
namespace {

__device__ __forceinline__ void two_sum(float a, float b, float& s, float& e) {
#pragma clang fp contract(off)
    s = a + b;
    const float z = s - a;
    e = (a - (s - z)) + (b - z);
}

template <int ACC>
struct Accum;

template <>
struct Accum<0> {
    float s = 0.f;
    __device__ __forceinline__ void add(float a, float b) { s = __builtin_fmaf(a, b, s); }
    __device__ __forceinline__ void group_end() {}
    __device__ __forceinline__ float result() { return s; }
};

template <>
struct Accum<1> {
    float s = 0.f, c = 0.f, part = 0.f;
    __device__ __forceinline__ void add(float a, float b) { part = __builtin_fmaf(a, b, part); }
    __device__ __forceinline__ void group_end() {
#pragma clang fp contract(off)
        float t, e;
        two_sum(s, part, t, e);
        c = c + e;
        s = t;
        part = 0.f;
    }
    __device__ __forceinline__ float result() {
#pragma clang fp contract(off)
        group_end();
        return s + c;
    }
};

template <>
struct Accum<2> {
    float s = 0.f, c = 0.f;
    __device__ __forceinline__ void add(float a, float b) {
#pragma clang fp contract(off)
        const float p = a * b;
        const float pe = __builtin_fmaf(a, b, -p);
        float t, se;
        two_sum(s, p, t, se);
        c = c + (se + pe);
        s = t;
    }
    __device__ __forceinline__ void group_end() {}
    __device__ __forceinline__ float result() {
#pragma clang fp contract(off)
        return s + c;
    }
};

// Row of A (stride 1) times column of B (stride N) from global memory, in groups of G terms.
template <int G, int ACC>
__device__ __forceinline__ float dot_global(const float* a, const float* b, int N, int K) {
    Accum<ACC> acc;
    for (int k0 = 0; k0 < K; k0 += G) {
        const int k1 = min(k0 + G, K);
        for (int k = k0; k < k1; ++k) acc.add(a[k], b[static_cast<long long>(k) * N]);
        acc.group_end();
    }
    return acc.result();
}

// basic: one thread per output element on a 1-D grid.
template <int ACC>
__global__ __launch_bounds__(256) void matmul_basic(const float* A, const float* B, float* C, int M, int N, int K) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * N) return;
    const int row = idx / N, col = idx % N;
    C[idx] = dot_global<32, ACC>(A + static_cast<long long>(row) * K, B + col, N, K);
}

// tiled: TILE x TILE thread blocks, one per output tile, operands straight from global memory.
template <int TILE, int ACC>
__global__ __launch_bounds__(TILE* TILE) void matmul_tiled(const float* A, const float* B, float* C, int M, int N,
                                                           int K) {
    const int row = blockIdx.y * TILE + threadIdx.y, col = blockIdx.x * TILE + threadIdx.x;
    if (row >= M || col >= N) return;
    C[static_cast<long long>(row) * N + col] = dot_global<TILE, ACC>(A + static_cast<long long>(row) * K, B + col, N, K);
}

// shared: TILE x TILE tiles of A and B staged in LDS, each element reused TILE times.
template <int TILE, int ACC>
__global__ __launch_bounds__(TILE* TILE) void matmul_shared(const float* A, const float* B, float* C, int M, int N,
                                                            int K) {
    __shared__ float As[TILE][TILE + 1];
    __shared__ float Bs[TILE][TILE + 1];
    const int tx = threadIdx.x, ty = threadIdx.y;
    const int row = blockIdx.y * TILE + ty, col = blockIdx.x * TILE + tx;
    Accum<ACC> acc;
    for (int k0 = 0; k0 < K; k0 += TILE) {
        As[ty][tx] = (row < M && k0 + tx < K) ? A[static_cast<long long>(row) * K + k0 + tx] : 0.f;
        Bs[ty][tx] = (k0 + ty < K && col < N) ? B[static_cast<long long>(k0 + ty) * N + col] : 0.f;
        __syncthreads();
        const int kn = min(TILE, K - k0);
        for (int k = 0; k < kn; ++k) acc.add(As[ty][k], Bs[k][tx]);
        acc.group_end();
        __syncthreads();
    }
    if (row < M && col < N) C[static_cast<long long>(row) * N + col] = acc.result();
}

// register: 64 x 64 block tiles, 256 threads with 4 x 4 outputs each (rows ty + 16 i, columns
// tx + 16 j), BK = 32 deep LDS stages. Every output sums k = 0 .. K-1 in order with a group end
// after each 32 terms, exactly the operation sequence of matmul_basic, so the two agree bit for bit.
template <int ACC>
__global__ __launch_bounds__(256) void matmul_register(const float* A, const float* B, float* C, int M, int N, int K) {
    constexpr int BT = 64, BK = 32;
    __shared__ float As[BK][BT + 1];
    __shared__ float Bs[BK][BT + 1];
    const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    const int m0 = blockIdx.y * BT, n0 = blockIdx.x * BT;
    Accum<ACC> acc[4][4];
    for (int k0 = 0; k0 < K; k0 += BK) {
        for (int f = tid; f < BT * BK; f += 256) {
            const int r = f / BK, k = f % BK;  // A: 64 rows x 32 k, read along k
            const int row = m0 + r;
            As[k][r] = (row < M && k0 + k < K) ? A[static_cast<long long>(row) * K + k0 + k] : 0.f;
            const int kb = f / BT, c = f % BT;  // B: 32 k x 64 columns, read along columns
            const int col = n0 + c;
            Bs[kb][c] = (k0 + kb < K && col < N) ? B[static_cast<long long>(k0 + kb) * N + col] : 0.f;
        }
        __syncthreads();
        const int kn = min(BK, K - k0);
        for (int k = 0; k < kn; ++k) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[k][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[k][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j].add(a[i], b[j]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j].group_end();
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = m0 + ty + 16 * i, col = n0 + tx + 16 * j;
            if (row < M && col < N) C[static_cast<long long>(row) * N + col] = acc[i][j].result();
        }
}

template <int ACC>
int launch_acc(int variant, int tile, const float* a, const float* b, float* c, int M, int N, int K,
               hipStream_t stream) {
    if (variant == 0) {
        matmul_basic<ACC><<<blocks_for(static_cast<std::int64_t>(M) * N, 256), 256, 0, stream>>>(a, b, c, M, N, K);
        return MFH_CHECK_LAUNCH("matmul_basic", stream);
    }
    if (variant == 4) {
        if (blocks_for(M, 64) > GRID_YZ_LIMIT) return MFH_FAIL(ERR_ARG, "matmul rows exceed the grid limit");
        matmul_register<ACC><<<dim3(blocks_for(N, 64), blocks_for(M, 64)), 256, 0, stream>>>(a, b, c, M, N, K);
        return MFH_CHECK_LAUNCH("matmul_register", stream);
    }
    if (blocks_for(M, tile) > GRID_YZ_LIMIT) return MFH_FAIL(ERR_ARG, "matmul rows exceed the grid limit");
    const dim3 grid(blocks_for(N, tile), blocks_for(M, tile)), block(tile, tile);
    if (variant == 1) {
        if (tile == 16) matmul_tiled<16, ACC><<<grid, block, 0, stream>>>(a, b, c, M, N, K);
        else matmul_tiled<32, ACC><<<grid, block, 0, stream>>>(a, b, c, M, N, K);
        return MFH_CHECK_LAUNCH("matmul_tiled", stream);
    }
    if (tile == 16) matmul_shared<16, ACC><<<grid, block, 0, stream>>>(a, b, c, M, N, K);
    else matmul_shared<32, ACC><<<grid, block, 0, stream>>>(a, b, c, M, N, K);
    return MFH_CHECK_LAUNCH("matmul_shared", stream);
}

}  // namespace

int launch_matmul(int variant, int tile, int accumulate, const float* a, const float* b, float* c, int M, int N,
                  int K, hipStream_t stream) {
    switch (accumulate) {
        case 0: return launch_acc<0>(variant, tile, a, b, c, M, N, K, stream);
        case 1: return launch_acc<1>(variant, tile, a, b, c, M, N, K, stream);
        default: return launch_acc<2>(variant, tile, a, b, c, M, N, K, stream);
    }
}

}  // namespace mfh
