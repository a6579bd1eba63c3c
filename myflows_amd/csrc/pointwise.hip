// Elementwise kernels around the convolution path: ReLU forward/backward and a multi-tensor Adam
// step.
//
// Adam applies, per element and with every operation rounded to float32 in this order (no
// contraction, IEEE division and square root):
//   gs = decay != 0 ? g * scale + decay * p : (scale == 1 ? g : g * scale)
//   m  = b1 * m + (1 - b1) * gs
//   v  = b2 * v + (1 - b2) * (gs * gs)
//   p  = p - (lr * (m / bc1)) / (sqrt(v / bc2) + eps)
// One launch covers up to ADAM_GROUP tensors whose descriptors travel in the kernel arguments, so
// the step needs no device-side table and no host-to-device copy; workgroup w finds its tensor
// from the running workgroup offsets.
#include "common.h"

namespace mfh {
namespace {

constexpr int EW_THREADS = 256;
constexpr int ADAM_GROUP = 16;

__global__ __launch_bounds__(EW_THREADS) void relu_forward_kernel(const float* __restrict__ x,
                                                                  float* __restrict__ y, long long count) {
    const long long i = static_cast<long long>(blockIdx.x) * EW_THREADS + threadIdx.x;
    if (i >= count) return;
    const float v = x[i];
    y[i] = v < 0.0f ? 0.0f : v;  // NaN stays NaN
}

template <bool LEAKY>
__global__ __launch_bounds__(EW_THREADS) void relu_backward_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ g, float* out,
                                                                   long long count, float alpha, int add) {
#pragma clang fp contract(off)
    const long long i = static_cast<long long>(blockIdx.x) * EW_THREADS + threadIdx.x;
    if (i >= count) return;
    const float grad = g[i];
    const float v = x[i] > 0.0f ? grad : (LEAKY ? alpha * grad : 0.0f);
    out[i] = add ? out[i] + v : v;
}

struct AdamGroup {
    AdamTensor t[ADAM_GROUP];
    unsigned first_block[ADAM_GROUP + 1];  // workgroups [first_block[i], first_block[i + 1]) update t[i]
    int count;
};

__global__ __launch_bounds__(EW_THREADS) void adam_kernel(AdamGroup group, AdamScalars s) {
#pragma clang fp contract(off)
    int k = 0;
    while (k + 1 < group.count && blockIdx.x >= group.first_block[k + 1]) ++k;
    const AdamTensor& t = group.t[k];
    const long long i = static_cast<long long>(blockIdx.x - group.first_block[k]) * EW_THREADS + threadIdx.x;
    if (i >= t.size) return;
    float m = t.m[i], v = t.v[i], p = t.param[i];
    const float g = t.grad[i];
    float gs;
    if (t.decay != 0.0f) gs = g * s.grad_scale + t.decay * p;  // decoupled into the gradient, scale applied
    else gs = s.grad_scale == 1.0f ? g : g * s.grad_scale;
    m = s.b1 * m + s.omb1 * gs;
    v = s.b2 * v + s.omb2 * (gs * gs);
    const float denom = sqrtf(v / t.bc2) + s.eps;
    p = p - (t.lr * (m / t.bc1)) / denom;
    t.m[i] = m;
    t.v[i] = v;
    t.param[i] = p;
}

}  // namespace

int launch_relu_forward(const float* x, float* y, std::int64_t count, hipStream_t stream) {
    if (count == 0) return OK;
    relu_forward_kernel<<<blocks_for(count, EW_THREADS), EW_THREADS, 0, stream>>>(x, y, count);
    return MFH_CHECK_LAUNCH("relu_forward", stream);
}

int launch_relu_backward(const float* x, const float* g, float* out, std::int64_t count, float alpha, bool add,
                         hipStream_t stream) {
    if (count == 0) return OK;
    const unsigned blocks = blocks_for(count, EW_THREADS);
    if (alpha != 0.0f) relu_backward_kernel<true><<<blocks, EW_THREADS, 0, stream>>>(x, g, out, count, alpha, add);
    else relu_backward_kernel<false><<<blocks, EW_THREADS, 0, stream>>>(x, g, out, count, alpha, add);
    return MFH_CHECK_LAUNCH("relu_backward", stream);
}

int launch_adam(const AdamTensor* tensors, int count, const AdamScalars& s, hipStream_t stream) {
    for (int base = 0; base < count; base += ADAM_GROUP) {
        AdamGroup group{};
        unsigned blocks = 0;
        for (int k = 0; k < ADAM_GROUP && base + k < count; ++k) {
            group.t[group.count] = tensors[base + k];
            group.first_block[group.count] = blocks;
            blocks += blocks_for(tensors[base + k].size, EW_THREADS);
            ++group.count;
        }
        group.first_block[group.count] = blocks;
        if (blocks == 0) continue;
        adam_kernel<<<blocks, EW_THREADS, 0, stream>>>(group, s);
        MFH_TRY(MFH_CHECK_LAUNCH("adam", stream));
    }
    return OK;
}

}  // namespace mfh
