// The network head and loss around the last convolution: the global average pool (forward and
// backward), the mean squared error (loss and gradient) and FP64 column sums (a Linear layer's
// bias gradient). Each repeats the float32 rounding steps of the operator it replaces, with the
// sums formed in FP64 in a fixed order, so every result is reproducible bit for bit:
//   * plane means y[p] = float(FP64 sum of x[p, 0..hw) / hw)              (mean in FP64, rounded once)
//   * their gradient dx[p, i] (+)= dy[p] / float(hw)                     (one float32 division)
//   * loss = float(FP64 sum of float32 (d * d) / count), d = pred - target (float32 difference and
//     square, as the operator's diff * diff)
//   * its gradient g[i] (+)= seed * ((2 * d) / float(count))             (float32, in that order)
//   * column sums out[j] = float(FP64 sum over rows of src[r, j]), rows in order.
#include <cstdint>

#include "common.h"

namespace mfh {
namespace {

constexpr int HEAD_THREADS = 256;
constexpr int LOSS_THREADS = 1024;  // one workgroup forms the loss

__global__ __launch_bounds__(HEAD_THREADS) void plane_mean_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                  long long planes, int hw) {
    const long long p = static_cast<long long>(blockIdx.x) * HEAD_THREADS + threadIdx.x;
    if (p >= planes) return;
    const float* __restrict__ src = x + p * hw;
    double s = 0.0;
    for (int i = 0; i < hw; ++i) s += static_cast<double>(src[i]);
    y[p] = static_cast<float>(s / static_cast<double>(hw));
}

__global__ __launch_bounds__(HEAD_THREADS) void plane_mean_backward_kernel(const float* __restrict__ dy, float* dx,
                                                                           long long count, int hw, int add) {
#pragma clang fp contract(off)
    const long long i = static_cast<long long>(blockIdx.x) * HEAD_THREADS + threadIdx.x;
    if (i >= count) return;
    const float v = dy[i / hw] / static_cast<float>(hw);
    dx[i] = add ? dx[i] + v : v;
}

// One workgroup: thread t adds the squares of elements t, t + LOSS_THREADS, ... in FP64; the
// thread sums are then combined by a fixed tree in LDS.
__global__ __launch_bounds__(LOSS_THREADS) void mse_loss_kernel(const float* __restrict__ pred,
                                                                const float* __restrict__ target,
                                                                float* __restrict__ loss, long long count) {
#pragma clang fp contract(off)
    __shared__ double partial[LOSS_THREADS];
    double s = 0.0;
    for (long long i = threadIdx.x; i < count; i += LOSS_THREADS) {
        const float d = pred[i] - target[i];
        const float square = d * d;
        s += static_cast<double>(square);
    }
    partial[threadIdx.x] = s;
    __syncthreads();
    for (int half = LOSS_THREADS / 2; half > 0; half >>= 1) {
        if (static_cast<int>(threadIdx.x) < half) partial[threadIdx.x] += partial[threadIdx.x + half];
        __syncthreads();
    }
    // The mean of no elements is NaN, as the operator's FP64 mean of an empty array.
    if (threadIdx.x == 0)
        loss[0] = count > 0 ? static_cast<float>(partial[0] / static_cast<double>(count)) : __builtin_nanf("");
}

__global__ __launch_bounds__(HEAD_THREADS) void mse_grad_kernel(const float* __restrict__ pred,
                                                                const float* __restrict__ target,
                                                                const float* __restrict__ seed, float* grad,
                                                                long long count, float divisor, int add) {
#pragma clang fp contract(off)
    const long long i = static_cast<long long>(blockIdx.x) * HEAD_THREADS + threadIdx.x;
    if (i >= count) return;
    const float d = pred[i] - target[i];
    const float v = seed[0] * ((2.0f * d) / divisor);
    grad[i] = add ? grad[i] + v : v;
}

__global__ __launch_bounds__(HEAD_THREADS) void column_sums_kernel(const float* __restrict__ src,
                                                                   float* __restrict__ out, long long rows,
                                                                   long long cols) {
    const long long j = static_cast<long long>(blockIdx.x) * HEAD_THREADS + threadIdx.x;
    if (j >= cols) return;
    double s = 0.0;
    long long r = 0;
    for (; r + 8 <= rows; r += 8) {  // eight loads in flight, added in row order
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = src[(r + u) * cols + j];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += static_cast<double>(v[u]);
    }
    for (; r < rows; ++r) s += static_cast<double>(src[r * cols + j]);
    out[j] = static_cast<float>(s);
}

}  // namespace

int launch_plane_mean(const float* x, float* y, std::int64_t planes, int hw, hipStream_t stream) {
    if (planes == 0) return OK;
    launch(plane_mean_kernel, blocks_for(planes, HEAD_THREADS), HEAD_THREADS, 0, stream, x, y, planes, hw);
    return MFH_CHECK_LAUNCH("plane_mean", stream);
}

int launch_plane_mean_backward(const float* dy, float* dx, std::int64_t planes, int hw, bool add, hipStream_t stream) {
    const std::int64_t count = planes * hw;
    if (count == 0) return OK;
    launch(plane_mean_backward_kernel, blocks_for(count, HEAD_THREADS), HEAD_THREADS, 0, stream, dy, dx, count, hw,
                                                                                           add ? 1 : 0);
    return MFH_CHECK_LAUNCH("plane_mean_backward", stream);
}

int launch_mse_loss(const float* pred, const float* target, float* loss, std::int64_t count, hipStream_t stream) {
    launch(mse_loss_kernel, 1, LOSS_THREADS, 0, stream, pred, target, loss, count);
    return MFH_CHECK_LAUNCH("mse_loss", stream);
}

int launch_mse_grad(const float* pred, const float* target, const float* seed, float* grad, std::int64_t count,
                    bool add, hipStream_t stream) {
    if (count == 0) return OK;
    const float divisor = static_cast<float>(count > 0 ? count : 1);
    launch(mse_grad_kernel, blocks_for(count, HEAD_THREADS), HEAD_THREADS, 0, stream, pred, target, seed, grad, count,
                                                                                divisor, add ? 1 : 0);
    return MFH_CHECK_LAUNCH("mse_grad", stream);
}

int launch_column_sums(const float* src, float* out, std::int64_t rows, std::int64_t cols, hipStream_t stream) {
    if (cols == 0) return OK;
    launch(column_sums_kernel, blocks_for(cols, HEAD_THREADS), HEAD_THREADS, 0, stream, src, out, rows, cols);
    return MFH_CHECK_LAUNCH("column_sums", stream);
}

}  // namespace mfh
