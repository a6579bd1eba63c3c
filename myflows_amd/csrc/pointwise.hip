// Elementwise kernels around the convolution path: ReLU forward/backward, a zero fill and a
// multi-tensor Adam step.
//
// Adam applies, per element and with every operation rounded to float32 in this order (no
// contraction, IEEE division and square root):
//   gs = decay != 0 ? g * scale + decay * p : (scale == 1 ? g : g * scale)
//   m  = b1 * m + (1 - b1) * gs
//   v  = b2 * v + (1 - b2) * (gs * gs)
//   p  = p - (lr * (m / bc1)) / (sqrt(v / bc2) + eps)
// One launch covers up to ADAM_GROUP tensors whose descriptors travel in the kernel arguments, so
// the step needs no device-side table and no host-to-device copy; workgroup w finds its tensor
// from the running workgroup offsets. A tensor whose size is a multiple of 4 with 16-byte aligned
// arrays takes four elements per thread (16-byte loads and stores), others one.
#include <cstdint>

#include "common.h"

namespace mfh {
namespace {

constexpr int EW_THREADS = 256;
constexpr int ADAM_GROUP = 48;

__global__ __launch_bounds__(EW_THREADS) void relu_forward_kernel(const float* __restrict__ x,
                                                                  float* __restrict__ y, long long count) {
    const long long i = static_cast<long long>(blockIdx.x) * EW_THREADS + threadIdx.x;
    if (i >= count) return;
    const float v = x[i];
    y[i] = v < 0.0f ? 0.0f : v;  // NaN stays NaN
}

__global__ __launch_bounds__(EW_THREADS) void fill_kernel(float* __restrict__ p, long long count, float value) {
    const long long i = static_cast<long long>(blockIdx.x) * EW_THREADS + threadIdx.x;
    if (i < count) p[i] = value;
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
    unsigned char vec[ADAM_GROUP];         // 1: four elements per thread
    int count;
};

static_assert(sizeof(AdamGroup) + sizeof(AdamScalars) <= 4096, "Adam descriptors must fit the kernel arguments");

__device__ __forceinline__ void adam_update(float& p, float& m, float& v, float g, const AdamTensor& t,
                                            const AdamScalars& s) {
#pragma clang fp contract(off)
    float gs;
    if (t.decay != 0.0f) gs = g * s.grad_scale + t.decay * p;  // decoupled into the gradient, scale applied
    else gs = s.grad_scale == 1.0f ? g : g * s.grad_scale;
    m = s.b1 * m + s.omb1 * gs;
    v = s.b2 * v + s.omb2 * (gs * gs);
    const float denom = sqrtf(v / t.bc2) + s.eps;
    p = p - (t.lr * (m / t.bc1)) / denom;
}

__global__ __launch_bounds__(EW_THREADS) void adam_kernel(AdamGroup group, AdamScalars s) {
    int k = 0;
    while (k + 1 < group.count && blockIdx.x >= group.first_block[k + 1]) ++k;
    const AdamTensor& t = group.t[k];
    const long long local = blockIdx.x - group.first_block[k];
    if (group.vec[k]) {
        const long long i = (local * EW_THREADS + threadIdx.x) * 4;
        if (i >= t.size) return;
        float4 m = *reinterpret_cast<const float4*>(t.m + i), v = *reinterpret_cast<const float4*>(t.v + i);
        float4 p = *reinterpret_cast<const float4*>(t.param + i);
        const float4 g = *reinterpret_cast<const float4*>(t.grad + i);
        adam_update(p.x, m.x, v.x, g.x, t, s);
        adam_update(p.y, m.y, v.y, g.y, t, s);
        adam_update(p.z, m.z, v.z, g.z, t, s);
        adam_update(p.w, m.w, v.w, g.w, t, s);
        *reinterpret_cast<float4*>(t.m + i) = m;
        *reinterpret_cast<float4*>(t.v + i) = v;
        *reinterpret_cast<float4*>(t.param + i) = p;
        return;
    }
    const long long i = local * EW_THREADS + threadIdx.x;
    if (i >= t.size) return;
    float m = t.m[i], v = t.v[i], p = t.param[i];
    adam_update(p, m, v, t.grad[i], t, s);
    t.m[i] = m;
    t.v[i] = v;
    t.param[i] = p;
}

bool aligned16(const void* q) { return (reinterpret_cast<std::uintptr_t>(q) & 15) == 0; }

}  // namespace

int launch_relu_forward(const float* x, float* y, std::int64_t count, hipStream_t stream) {
    if (count == 0) return OK;
    launch(relu_forward_kernel, blocks_for(count, EW_THREADS), EW_THREADS, 0, stream, x, y, count);
    return MFH_CHECK_LAUNCH("relu_forward", stream);
}

int launch_fill(float* p, std::int64_t count, float value, hipStream_t stream) {
    if (count == 0) return OK;
    launch(fill_kernel, blocks_for(count, EW_THREADS), EW_THREADS, 0, stream, p, count, value);
    return MFH_CHECK_LAUNCH("fill", stream);
}

int launch_fill_zero(float* p, std::int64_t count, hipStream_t stream) { return launch_fill(p, count, 0.0f, stream); }

int launch_relu_backward(const float* x, const float* g, float* out, std::int64_t count, float alpha, bool add,
                         hipStream_t stream) {
    if (count == 0) return OK;
    const unsigned blocks = blocks_for(count, EW_THREADS);
    if (alpha != 0.0f) launch(relu_backward_kernel<true>, blocks, EW_THREADS, 0, stream, x, g, out, count, alpha, add);
    else launch(relu_backward_kernel<false>, blocks, EW_THREADS, 0, stream, x, g, out, count, alpha, add);
    return MFH_CHECK_LAUNCH("relu_backward", stream);
}

int launch_adam(const AdamTensor* tensors, int count, const AdamScalars& s, hipStream_t stream) {
    for (int base = 0; base < count; base += ADAM_GROUP) {
        AdamGroup group{};
        unsigned blocks = 0;
        for (int k = 0; k < ADAM_GROUP && base + k < count; ++k) {
            const AdamTensor& t = tensors[base + k];
            const bool vec = t.size % 4 == 0 && aligned16(t.param) && aligned16(t.grad) && aligned16(t.m) &&
                             aligned16(t.v);
            group.t[group.count] = t;
            group.vec[group.count] = vec ? 1 : 0;
            group.first_block[group.count] = blocks;
            blocks += blocks_for(vec ? t.size / 4 : t.size, EW_THREADS);
            ++group.count;
        }
        group.first_block[group.count] = blocks;
        if (blocks == 0) continue;
        launch(adam_kernel, blocks, EW_THREADS, 0, stream, group, s);
        MFH_TRY(MFH_CHECK_LAUNCH("adam", stream));
    }
    return OK;
}

}  // namespace mfh
