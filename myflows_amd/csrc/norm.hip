// Batch normalisation of an NCHW tensor over the N*H*W positions of each channel, forward and
// backward, with an optional residual add and ReLU fused into the same passes.
//
// Forward (training): three launches.
//   1. norm_partials<STATS>: workgroup (s, c) sums d = x - x[n=0, c, 0] and d*d over slice s of
//      channel c in FP64 (the shift keeps the one-pass variance from cancelling);
//   2. norm_stats_finalize: per channel, adds the slices in slice order, forms the FP64 mean and
//      biased variance, stores the mean as the unevaluated float pair hi + lo (about 48 bits), the
//      inverse standard deviation rounded once, and updates the running statistics;
//   3. norm_apply: y = (((x - hi) - lo) * inv_std) * gamma + beta [+ residual] [ReLU], each
//      operation rounded to float32 in that order (no contraction), as the NumPy path computes it.
// Backward: norm_partials<GRADS> sums g and g * (x - mean) in FP64 (g = dy, or dy gated by the
// fused ReLU's output, also written to the residual gradient), norm_grad_finalize forms dgamma,
// dbeta and the coefficients of dx = a * ((g - k1) - ((x - hi) - lo) * k2), and norm_dx applies them.
// Every sum has a fixed order (lanes, then waves, then slices), so results are reproducible.
#include "common.h"
#include "fastdiv.h"

namespace mfh {
namespace {

constexpr int PT = 256;              // threads per partial-sum workgroup
constexpr int MIN_SLICE = 2048;      // fewest positions a slice covers
constexpr int APPLY_THREADS = 256;

enum PartialMode { STATS = 0, GRADS = 1 };

struct PartialArgs {
    const float* x;
    const float* dy;
    const float* gate;
    const float* mean;
    float* residual_grad;
    double* partial;
    int C, HW, total, chunk;
    FastDiv div_hw;
    int add_residual;
};

// Sum of (a, b) over the workgroup: a fixed xor-butterfly inside each wave64, then the wave sums in
// wave order. The result is valid in thread 0.
__device__ __forceinline__ void workgroup_sum(double& a, double& b) {
    __shared__ double wave_a[PT / 64], wave_b[PT / 64];
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        a += __shfl_xor(a, offset, 64);
        b += __shfl_xor(b, offset, 64);
    }
    const int wave = threadIdx.x / 64;
    if (threadIdx.x % 64 == 0) {
        wave_a[wave] = a;
        wave_b[wave] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        a = wave_a[0];
        b = wave_b[0];
#pragma unroll
        for (int w = 1; w < PT / 64; ++w) {
            a += wave_a[w];
            b += wave_b[w];
        }
    }
}

template <int MODE>
__global__ __launch_bounds__(PT) void norm_partials_kernel(PartialArgs p) {
    const int s = blockIdx.x, c = blockIdx.y, slices = gridDim.x;
    const int j0 = s * p.chunk, j1 = min(p.total, j0 + p.chunk);
    const int plane = p.C * p.HW;
    // STATS: shift by the channel's first element; GRADS: centre on the saved FP64 mean (hi + lo).
    const double centre = MODE == STATS ? static_cast<double>(p.x[c * p.HW])
                                        : static_cast<double>(p.mean[c]) + static_cast<double>(p.mean[p.C + c]);
    double a = 0.0, b = 0.0;
    for (int j = j0 + threadIdx.x; j < j1; j += PT) {
        int hw;
        const int n = p.div_hw.divmod(j, hw);
        const int at = n * plane + c * p.HW + hw;
        const double d = static_cast<double>(p.x[at]) - centre;
        if constexpr (MODE == STATS) {
            a += d;
            b = fma(d, d, b);
        } else {
            const float g = p.gate && !(p.gate[at] > 0.0f) ? 0.0f : p.dy[at];
            if (p.residual_grad) p.residual_grad[at] = p.add_residual ? p.residual_grad[at] + g : g;
            a += static_cast<double>(g);
            b = fma(static_cast<double>(g), d, b);
        }
    }
    workgroup_sum(a, b);
    if (threadIdx.x == 0) {
        p.partial[(static_cast<long long>(c) * slices + s) * 2] = a;
        p.partial[(static_cast<long long>(c) * slices + s) * 2 + 1] = b;
    }
}

__global__ __launch_bounds__(128) void norm_stats_finalize_kernel(const double* __restrict__ partial,
                                                                  const float* __restrict__ x, float* mean,
                                                                  float* inv_std, float* running_mean,
                                                                  float* running_var, int C, int HW, int slices,
                                                                  double count, double momentum, double eps,
                                                                  double var_scale, int training) {
    const int c = blockIdx.x * 128 + threadIdx.x;
    if (c >= C) return;
    double mu, var;
    if (training) {
        double sum = 0.0, sq = 0.0;
        for (int s = 0; s < slices; ++s) {
            sum += partial[(static_cast<long long>(c) * slices + s) * 2];
            sq += partial[(static_cast<long long>(c) * slices + s) * 2 + 1];
        }
        const double shifted = sum / count;
        var = fmax(sq / count - shifted * shifted, 0.0);
        mu = static_cast<double>(x[c * HW]) + shifted;
        running_mean[c] = static_cast<float>((1.0 - momentum) * static_cast<double>(running_mean[c]) + momentum * mu);
        running_var[c] =
            static_cast<float>((1.0 - momentum) * static_cast<double>(running_var[c]) + momentum * var * var_scale);
    } else {
        mu = static_cast<double>(running_mean[c]);
        var = static_cast<double>(running_var[c]);
    }
    const float hi = static_cast<float>(mu);
    mean[c] = hi;
    mean[C + c] = static_cast<float>(mu - static_cast<double>(hi));
    inv_std[c] = static_cast<float>(1.0 / sqrt(var + eps));
}

__global__ __launch_bounds__(128) void norm_grad_finalize_kernel(const double* __restrict__ partial,
                                                                 const float* __restrict__ gamma,
                                                                 const float* __restrict__ inv_std, float* gamma_grad,
                                                                 float* beta_grad, float* coef, int C, int slices,
                                                                 double count, int training, int add_gamma,
                                                                 int add_beta) {
    const int c = blockIdx.x * 128 + threadIdx.x;
    if (c >= C) return;
    double sdy = 0.0, sdyx = 0.0;
    for (int s = 0; s < slices; ++s) {
        sdy += partial[(static_cast<long long>(c) * slices + s) * 2];
        sdyx += partial[(static_cast<long long>(c) * slices + s) * 2 + 1];
    }
    const double istd = static_cast<double>(inv_std[c]);
    const double dgamma = istd * sdyx;
    if (gamma_grad) gamma_grad[c] = add_gamma ? gamma_grad[c] + static_cast<float>(dgamma) : static_cast<float>(dgamma);
    if (beta_grad) beta_grad[c] = add_beta ? beta_grad[c] + static_cast<float>(sdy) : static_cast<float>(sdy);
    coef[c] = static_cast<float>(static_cast<double>(gamma[c]) * istd);
    coef[C + c] = training ? static_cast<float>(sdy / count) : 0.0f;
    coef[2 * C + c] = training ? static_cast<float>(istd * dgamma / count) : 0.0f;
}

// Channel of flat NCHW element e: (e / HW) % C.
struct ChannelOf {
    FastDiv div_hw, div_c;
    __device__ __forceinline__ int operator()(int e) const {
        int c;
        div_c.divmod(div_hw.div(e), c);
        return c;
    }
};

__global__ __launch_bounds__(APPLY_THREADS) void norm_apply_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ mean,
                                                                   const float* __restrict__ inv_std,
                                                                   const float* __restrict__ gamma,
                                                                   const float* __restrict__ beta,
                                                                   const float* __restrict__ residual,
                                                                   float* __restrict__ y, int total, int C,
                                                                   ChannelOf channel_of, int relu) {
#pragma clang fp contract(off)
    const int e = blockIdx.x * APPLY_THREADS + threadIdx.x;
    if (e >= total) return;
    const int c = channel_of(e);
    float v = (((x[e] - mean[c]) - mean[C + c]) * inv_std[c]) * gamma[c] + beta[c];
    if (residual) v = v + residual[e];
    if (relu) v = v < 0.0f ? 0.0f : v;  // NaN stays NaN
    y[e] = v;
}

__global__ __launch_bounds__(APPLY_THREADS) void norm_dx_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ dy,
                                                                const float* __restrict__ gate,
                                                                const float* __restrict__ mean,
                                                                const float* __restrict__ coef, float* dx, int total,
                                                                int C, ChannelOf channel_of, int training, int add) {
#pragma clang fp contract(off)
    const int e = blockIdx.x * APPLY_THREADS + threadIdx.x;
    if (e >= total) return;
    const int c = channel_of(e);
    const float g = gate && !(gate[e] > 0.0f) ? 0.0f : dy[e];
    const float a = coef[c];
    float v;
    if (training) v = a * ((g - coef[C + c]) - ((x[e] - mean[c]) - mean[C + c]) * coef[2 * C + c]);
    else v = a * g;
    dx[e] = add ? dx[e] + v : v;
}

ChannelOf channel_of(const NormShape& s) { return ChannelOf{FastDiv(s.HW), FastDiv(s.C)}; }

int run_partials(int mode, const NormShape& s, const PartialArgs& args, hipStream_t stream) {
    const dim3 grid(norm_slices(s), s.C);
    if (mode == STATS) norm_partials_kernel<STATS><<<grid, PT, 0, stream>>>(args);
    else norm_partials_kernel<GRADS><<<grid, PT, 0, stream>>>(args);
    return MFH_CHECK_LAUNCH(mode == STATS ? "norm_partials<stats>" : "norm_partials<grads>", stream);
}

}  // namespace

int norm_slices(const NormShape& s) {
    const std::int64_t positions = static_cast<std::int64_t>(s.N) * s.HW;
    const std::int64_t wanted = (4LL * device_cu_count() + s.C - 1) / s.C;
    const std::int64_t most = std::max<std::int64_t>(1, positions / MIN_SLICE);
    return static_cast<int>(std::max<std::int64_t>(1, std::min(wanted, most)));
}

std::int64_t norm_workspace_doubles(const NormShape& s) {
    // FP64 (sum, second sum) per slice and channel, then 3 * C floats of dx coefficients.
    return 2LL * s.C * norm_slices(s) + (3LL * s.C + 1) / 2;
}

int norm_forward(const NormShape& s, const NormForward& f, hipStream_t stream) {
    const int total = s.N * s.C * s.HW;
    const int slices = norm_slices(s);
    if (f.training) {
        PartialArgs args{};
        args.x = f.x;
        args.partial = f.partial;
        args.C = s.C;
        args.HW = s.HW;
        args.total = s.N * s.HW;
        args.chunk = (args.total + slices - 1) / slices;
        args.div_hw = FastDiv(s.HW);
        MFH_TRY(run_partials(STATS, s, args, stream));
    }
    norm_stats_finalize_kernel<<<blocks_for(s.C, 128), 128, 0, stream>>>(
        f.partial, f.x, f.mean, f.inv_std, f.running_mean, f.running_var, s.C, s.HW, slices,
        static_cast<double>(s.N) * s.HW, f.momentum, f.eps, f.var_scale, f.training ? 1 : 0);
    MFH_TRY(MFH_CHECK_LAUNCH("norm_stats_finalize", stream));
    norm_apply_kernel<<<blocks_for(total, APPLY_THREADS), APPLY_THREADS, 0, stream>>>(
        f.x, f.mean, f.inv_std, f.gamma, f.beta, f.residual, f.y, total, s.C, channel_of(s), f.relu ? 1 : 0);
    return MFH_CHECK_LAUNCH("norm_apply", stream);
}

int norm_backward(const NormShape& s, const NormBackward& b, hipStream_t stream) {
    const int total = s.N * s.C * s.HW;
    const int slices = norm_slices(s);
    const bool sums = b.gamma_grad || b.beta_grad || (b.training && b.x_grad);
    if (sums || b.residual_grad) {
        PartialArgs args{};
        args.x = b.x;
        args.dy = b.dy;
        args.gate = b.gate;
        args.mean = b.mean;
        args.residual_grad = b.residual_grad;
        args.add_residual = b.add_residual ? 1 : 0;
        args.partial = b.partial;
        args.C = s.C;
        args.HW = s.HW;
        args.total = s.N * s.HW;
        args.chunk = (args.total + slices - 1) / slices;
        args.div_hw = FastDiv(s.HW);
        MFH_TRY(run_partials(GRADS, s, args, stream));
    }
    if (!b.x_grad && !sums) return OK;
    norm_grad_finalize_kernel<<<blocks_for(s.C, 128), 128, 0, stream>>>(
        b.partial, b.gamma, b.inv_std, b.gamma_grad, b.beta_grad, b.coef, s.C, sums ? slices : 0,
        static_cast<double>(s.N) * s.HW, b.training ? 1 : 0, b.add_gamma ? 1 : 0, b.add_beta ? 1 : 0);
    MFH_TRY(MFH_CHECK_LAUNCH("norm_grad_finalize", stream));
    if (!b.x_grad) return OK;
    norm_dx_kernel<<<blocks_for(total, APPLY_THREADS), APPLY_THREADS, 0, stream>>>(
        b.x, b.dy, b.gate, b.mean, b.coef, b.x_grad, total, s.C, channel_of(s), b.training ? 1 : 0,
        b.add_x ? 1 : 0);
    return MFH_CHECK_LAUNCH("norm_dx", stream);
}

}  // namespace mfh
