// Batch normalisation of an NCHW tensor over the N*H*W positions of each channel, forward and
// backward, with an optional residual add and ReLU fused into the same passes.
//
// Forward (training): two launches.
//   1. norm_partials<STATS>: workgroup (s, c) sums d = x - x[n=0, c, 0] and d*d over slice s of
//      channel c in FP64 (the shift keeps the one-pass variance from cancelling);
//   2. norm_apply: every workgroup first finalises the channels its elements belong to (adds the
//      slices in slice order, forms the FP64 mean and biased variance, the mean as the unevaluated
//      float pair hi + lo (about 48 bits) and the inverse standard deviation rounded once), then
//      y = (((x - hi) - lo) * inv_std) * gamma + beta [+ residual] [ReLU], each operation rounded to
//      float32 in that order (no contraction), as the NumPy path computes it. The workgroup that
//      holds the first element of image 0 of a channel also stores that channel's mean / inv_std
//      and updates its running statistics, so each is written exactly once.
// Backward: norm_partials<GRADS> sums g and g * (x - mean) in FP64 (g = dy, or dy gated by the
// fused ReLU's output, also written to the residual gradient); norm_dx finalises the channels it
// touches (dgamma, dbeta and the coefficients of dx = a * ((g - k1) - ((x - hi) - lo) * k2)) and
// applies them. Every sum has a fixed order (four interleaved chains per thread, then lanes, waves
// and slices), so results are reproducible; every workgroup finalises a channel with the same
// arithmetic, so they all agree.
// When a channel has at most CHANNEL_FUSED_MAX positions it is a single slice, and each pass is one
// launch of one workgroup per channel (norm_forward_channel / norm_backward_channel): the partial
// sums, the finalisation and the element pass in a row, with the arithmetic of the two-launch path.
#include <initializer_list>

#include "common.h"
#include "fastdiv.h"
#include "pool_rules.h"

namespace mfh {
namespace {

constexpr int PT = 256;           // threads per partial-sum workgroup (WIDE_PT for a one-slice channel of
                                  // at least WIDE_MIN positions, that one workgroup sums alone)
constexpr int WIDE_PT = 1024;
constexpr int WIDE_MIN = 4096;
constexpr int CHAINS = 4;         // independent load / add chains per thread in the partial sums
constexpr int MIN_SLICE = 2048;   // fewest positions a slice covers
constexpr int APPLY_THREADS = 256;
constexpr int APPLY_ELEMS = 16;   // elements per thread in norm_apply / norm_dx
constexpr int APPLY_SPAN = APPLY_THREADS * APPLY_ELEMS;
constexpr int MAX_PLANES = 128;   // (n, c) planes a workgroup finalises at once; more are taken in rounds
constexpr int CHANNEL_FUSED_MAX = 8192;  // positions per channel up to which a pass is one launch

enum PartialMode { STATS = 0, GRADS = 1 };

struct PartialArgs {
    const float* x;
    const float* dy;
    const float* gate;
    const float* mean;
    const float* inv_std;  // the forward's, for a gate recomputed from x (norm_partials_pool_kernel)
    float* residual_grad;
    double* partial;
    int C, HW, total, chunk;
    FastDiv div_hw;
    int add_residual;
    int vec;  // quads may be moved as float4s: every tensor of the pass is 16-byte aligned
};

// Four consecutive floats at v[at .. at + 3], as one 16-byte access when `vec`.
__device__ __forceinline__ void load_quad(const float* v, int at, int vec, float (&out)[4]) {
    if (vec) {
        const float4 t = *reinterpret_cast<const float4*>(v + at);
        out[0] = t.x; out[1] = t.y; out[2] = t.z; out[3] = t.w;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) out[u] = v[at + u];
    }
}
__device__ __forceinline__ void store_quad(float* v, int at, int vec, const float (&in)[4]) {
    if (vec) {
        *reinterpret_cast<float4*>(v + at) = make_float4(in[0], in[1], in[2], in[3]);
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) v[at + u] = in[u];
    }
}

// Sum of (a, b) over the workgroup: a fixed xor-butterfly inside each wave64, then the wave sums in
// wave order. The result is valid in thread 0.
template <int T>
__device__ __forceinline__ void workgroup_sum(double& a, double& b) {
    __shared__ double wave_a[T / 64], wave_b[T / 64];
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
        for (int w = 1; w < T / 64; ++w) {
            a += wave_a[w];
            b += wave_b[w];
        }
    }
}

// The gated gradient of four positions: dy, zero where the fused ReLU's output is not positive.
__device__ __forceinline__ void gated_quad(const PartialArgs& p, int at, float (&g)[4]) {
    load_quad(p.dy, at, p.vec, g);
    if (p.gate) {
        float t[4];
        load_quad(p.gate, at, p.vec, t);
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (!(t[u] > 0.0f)) g[u] = 0.0f;
    }
}

// Workgroup (s, c) of T threads sums slice s of channel c, in CHAINS = 4 chains per thread that are
// added in chain order at the end; the sums are valid in thread 0.
//   * QUAD (H*W a multiple of 4; the slice bounds are then multiples of 4 too): thread t takes the
//     quads of positions [j, j + 4) at j = j0 + 4 (t + i T), i = 0, 1, ..., chain u the u-th
//     position of each; a quad lies in one plane, so it is one 16-byte load per tensor.
//   * otherwise: positions j, j + T, j + 2 T, j + 3 T (chains 0-3), then the next 4 T.
template <int MODE, int T, bool QUAD>
__device__ __forceinline__ void channel_partial(const PartialArgs& p, int c, int s, double& sa, double& sb) {
    const int j0 = s * p.chunk, j1 = min(p.total, j0 + p.chunk);
    const int plane = p.C * p.HW;
    // STATS: shift by the channel's first element; GRADS: centre on the saved FP64 mean (hi + lo).
    const double centre = MODE == STATS ? static_cast<double>(p.x[c * p.HW])
                                        : static_cast<double>(p.mean[c]) + static_cast<double>(p.mean[p.C + c]);
    double a[CHAINS] = {}, b[CHAINS] = {};
    if constexpr (QUAD) {
        // Two quads per iteration, both loaded before either is summed.
        for (int base = j0 + 4 * threadIdx.x; base < j1; base += 8 * T) {
            float xv[2][4] = {}, gv[2][4] = {};
            int at[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int j = base + h * 4 * T;
                int hw;
                const int n = p.div_hw.divmod(j < j1 ? j : j0, hw);
                at[h] = n * plane + c * p.HW + hw;
                if (j < j1) {
                    load_quad(p.x, at[h], p.vec, xv[h]);
                    if constexpr (MODE == GRADS) gated_quad(p, at[h], gv[h]);
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (base + h * 4 * T >= j1) continue;
                if constexpr (MODE == GRADS) {
                    if (p.residual_grad) {
                        float r[4] = {};
                        if (p.add_residual) load_quad(p.residual_grad, at[h], p.vec, r);
#pragma unroll
                        for (int u = 0; u < 4; ++u) r[u] = p.add_residual ? r[u] + gv[h][u] : gv[h][u];
                        store_quad(p.residual_grad, at[h], p.vec, r);
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const double d = static_cast<double>(xv[h][u]) - centre;
                    if constexpr (MODE == STATS) {
                        a[u] += d;
                        b[u] = fma(d, d, b[u]);
                    } else {
                        a[u] += static_cast<double>(gv[h][u]);
                        b[u] = fma(static_cast<double>(gv[h][u]), d, b[u]);
                    }
                }
            }
        }
    }
    for (int base = j0 + threadIdx.x; !QUAD && base < j1; base += CHAINS * T) {
        float xv[CHAINS], gv[CHAINS];
        int at[CHAINS];
#pragma unroll
        for (int u = 0; u < CHAINS; ++u) {
            const int j = base + u * T;
            int hw;
            const int n = p.div_hw.divmod(j < j1 ? j : j0, hw);
            at[u] = n * plane + c * p.HW + hw;
            xv[u] = j < j1 ? p.x[at[u]] : 0.0f;
            if constexpr (MODE == GRADS) {
                float g = 0.0f;
                if (j < j1) g = p.gate && !(p.gate[at[u]] > 0.0f) ? 0.0f : p.dy[at[u]];
                gv[u] = g;
            }
        }
#pragma unroll
        for (int u = 0; u < CHAINS; ++u) {
            if (base + u * T >= j1) continue;
            const double d = static_cast<double>(xv[u]) - centre;
            if constexpr (MODE == STATS) {
                a[u] += d;
                b[u] = fma(d, d, b[u]);
            } else {
                if (p.residual_grad)
                    p.residual_grad[at[u]] = p.add_residual ? p.residual_grad[at[u]] + gv[u] : gv[u];
                a[u] += static_cast<double>(gv[u]);
                b[u] = fma(static_cast<double>(gv[u]), d, b[u]);
            }
        }
    }
    sa = a[0];
    sb = b[0];
#pragma unroll
    for (int u = 1; u < CHAINS; ++u) {
        sa += a[u];
        sb += b[u];
    }
    workgroup_sum<T>(sa, sb);
}

template <int MODE, int T, bool QUAD>
__global__ __launch_bounds__(T) void norm_partials_kernel(PartialArgs p) {
    raise_wave_priority();
    const int s = blockIdx.x, c = blockIdx.y, slices = gridDim.x;
    double sa, sb;
    channel_partial<MODE, T, QUAD>(p, c, s, sa, sb);
    if (threadIdx.x == 0) {
        p.partial[(static_cast<long long>(c) * slices + s) * 2] = sa;
        p.partial[(static_cast<long long>(c) * slices + s) * 2 + 1] = sb;
    }
}

// Sum of channel c's slice partials in slice order. The loads of SLICES_AHEAD slices are issued
// before their additions, which still run one at a time in slice order.
constexpr int SLICES_AHEAD = 8;
__device__ __forceinline__ void slice_sums(const double* __restrict__ partial, int c, int slices, double& a,
                                           double& b) {
    a = 0.0;
    b = 0.0;
    const double* row = partial + static_cast<long long>(c) * slices * 2;
    int s = 0;
    for (; s + SLICES_AHEAD <= slices; s += SLICES_AHEAD) {
        double2 v[SLICES_AHEAD];
#pragma unroll
        for (int u = 0; u < SLICES_AHEAD; ++u) v[u] = *reinterpret_cast<const double2*>(row + 2 * (s + u));
#pragma unroll
        for (int u = 0; u < SLICES_AHEAD; ++u) {
            a += v[u].x;
            b += v[u].y;
        }
    }
    for (; s < slices; ++s) {
        a += row[2 * s];
        b += row[2 * s + 1];
    }
}

struct ApplyArgs {
    const float* x;
    const float* gamma;
    const float* beta;
    const float* residual;
    float* y;
    float* mean;     // 2 x C (hi, lo), written by the first-element workgroups
    float* inv_std;  // C
    float* running_mean;
    float* running_var;
    const double* partial;
    int total, C, HW, slices, training, relu;
    double count, momentum, eps, var_scale;
    FastDiv div_hw, div_c;
};

struct DxArgs {
    const float* x;
    const float* dy;
    const float* gate;
    const float* gamma;
    const float* mean;
    const float* inv_std;
    float* dx;
    float* gamma_grad;
    float* beta_grad;
    const double* partial;
    int total, C, HW, slices, training, add, add_gamma, add_beta, sums;
    double count;
    FastDiv div_hw, div_c;
};

// The planes [p0, p1] that elements [e0, e0 + APPLY_SPAN) of a workgroup touch; plane pl is
// (n, c) = (pl / C, pl % C). A plane's first element lies in exactly one workgroup.
__device__ __forceinline__ void planes_of(int e0, int total, const FastDiv& div_hw, int& p0, int& p1) {
    p0 = div_hw.div(e0);
    p1 = div_hw.div(min(total, e0 + APPLY_SPAN) - 1);
}

// A channel's forward coefficients from its FP64 (shifted sum, second sum) when training, else from
// the running statistics: the mean as the float pair hi + lo, inv_std rounded once.
struct ApplyCoef {
    double mu, var;
    float hi, lo, istd;
};
__device__ __forceinline__ ApplyCoef apply_coef(const ApplyArgs& p, int c, double sum, double sq) {
    ApplyCoef k;
    if (p.training) {
        const double shifted = sum / p.count;
        k.var = fmax(sq / p.count - shifted * shifted, 0.0);
        k.mu = static_cast<double>(p.x[c * p.HW]) + shifted;
    } else {
        k.mu = static_cast<double>(p.running_mean[c]);
        k.var = static_cast<double>(p.running_var[c]);
    }
    k.hi = static_cast<float>(k.mu);
    k.lo = static_cast<float>(k.mu - static_cast<double>(k.hi));
    k.istd = static_cast<float>(1.0 / sqrt(k.var + p.eps));
    return k;
}

// The saved mean / inv_std of channel c and, when training, its running statistics.
__device__ __forceinline__ void store_statistics(const ApplyArgs& p, int c, const ApplyCoef& k) {
    p.mean[c] = k.hi;
    p.mean[p.C + c] = k.lo;
    p.inv_std[c] = k.istd;
    if (p.training) {
        p.running_mean[c] =
            static_cast<float>((1.0 - p.momentum) * static_cast<double>(p.running_mean[c]) + p.momentum * k.mu);
        p.running_var[c] = static_cast<float>((1.0 - p.momentum) * static_cast<double>(p.running_var[c]) +
                                              p.momentum * k.var * p.var_scale);
    }
}

// (((x - hi) - lo) * inv_std) * gamma + beta, rounded per operation.
__device__ __forceinline__ float affine_value(float x, float m_hi, float m_lo, float istd, float g, float b) {
#pragma clang fp contract(off)
    return (((x - m_hi) - m_lo) * istd) * g + b;
}

__device__ __forceinline__ float relu_value(float v) { return v < 0.0f ? 0.0f : v; }  // NaN stays NaN

// y = (((x - hi) - lo) * inv_std) * gamma + beta [+ residual] [ReLU], rounded per operation.
__device__ __forceinline__ float apply_value(const ApplyArgs& p, float x, float r, float m_hi, float m_lo, float istd,
                                             float g, float b) {
#pragma clang fp contract(off)
    float v = affine_value(x, m_hi, m_lo, istd, g, b);
    if (p.residual) v = v + r;
    if (p.relu) v = relu_value(v);
    return v;
}

// norm_apply with the statistics finalised in the workgroup: coefficients (hi, lo, inv_std, gamma,
// beta) of the planes it touches go to LDS, then every element is normalised.
template <int VEC>
__global__ __launch_bounds__(APPLY_THREADS) void norm_apply_kernel(ApplyArgs p) {
#pragma clang fp contract(off)
    raise_wave_priority();
    __shared__ float coef[5][MAX_PLANES];
    const int e0 = blockIdx.x * APPLY_SPAN;
    int p0, p1;
    planes_of(e0, p.total, p.div_hw, p0, p1);
    for (int first = p0; first <= p1; first += MAX_PLANES) {
        const int last = min(p1, first + MAX_PLANES - 1);
        for (int i = threadIdx.x; i <= last - first; i += APPLY_THREADS) {
            const int pl = first + i;
            int c;
            p.div_c.divmod(pl, c);
            double sum = 0.0, sq = 0.0;
            if (p.training) slice_sums(p.partial, c, p.slices, sum, sq);
            const ApplyCoef k = apply_coef(p, c, sum, sq);
            coef[0][i] = k.hi;
            coef[1][i] = k.lo;
            coef[2][i] = k.istd;
            coef[3][i] = p.gamma[c];
            coef[4][i] = p.beta[c];
            if (pl < p.C && static_cast<long long>(pl) * p.HW >= e0)  // image 0's plane of channel c starts here
                store_statistics(p, c, k);
        }
        __syncthreads();
        const int lo_e = max(e0, first * p.HW), hi_e = min(min(p.total, e0 + APPLY_SPAN), (last + 1) * p.HW);
        // A thread's ITER groups of VEC elements, APPLY_THREADS * VEC apart: every load is issued
        // before the first store (the stores could alias the loads for the compiler).
        constexpr int ITER = APPLY_ELEMS / VEC;
        float xv[ITER][VEC], rv[ITER][VEC] = {};
#pragma unroll
        for (int b = 0; b < ITER; ++b) {
            const int e = lo_e + (b * APPLY_THREADS + threadIdx.x) * VEC;
            if (e >= hi_e) continue;
            if constexpr (VEC == 4) {
                const float4 x4 = *reinterpret_cast<const float4*>(p.x + e);
                xv[b][0] = x4.x; xv[b][1] = x4.y; xv[b][2] = x4.z; xv[b][3] = x4.w;
                if (p.residual) {
                    const float4 r4 = *reinterpret_cast<const float4*>(p.residual + e);
                    rv[b][0] = r4.x; rv[b][1] = r4.y; rv[b][2] = r4.z; rv[b][3] = r4.w;
                }
            } else {
                xv[b][0] = p.x[e];
                if (p.residual) rv[b][0] = p.residual[e];
            }
        }
#pragma unroll
        for (int b = 0; b < ITER; ++b) {
            const int e = lo_e + (b * APPLY_THREADS + threadIdx.x) * VEC;
            if (e >= hi_e) continue;
            // The VEC elements' planes: i, then i + 1 from the element at `next` on (when H*W is
            // not a multiple of VEC a float4 may cross into the next plane).
            const int i = p.div_hw.div(e) - first;
            const int next = (first + i + 1) * p.HW - e;
            float out[VEC];
#pragma unroll
            for (int u = 0; u < VEC; ++u) {
                const int j = u < next ? i : i + 1;
                out[u] = apply_value(p, xv[b][u], rv[b][u], coef[0][j], coef[1][j], coef[2][j], coef[3][j],
                                     coef[4][j]);
            }
            if constexpr (VEC == 4) *reinterpret_cast<float4*>(p.y + e) = make_float4(out[0], out[1], out[2], out[3]);
            else p.y[e] = out[0];
        }
        __syncthreads();
    }
}

// A channel's dx coefficients from its FP64 (sum g, sum g (x - mean)): dx = a ((g - k1) - x_hat k2)
// when training (a g otherwise), and dgamma.
struct DxCoef {
    double dgamma;
    float a, k1, k2;
};
__device__ __forceinline__ DxCoef dx_coef(const DxArgs& p, int c, double sdy, double sdyx) {
    DxCoef k;
    const double istd = static_cast<double>(p.inv_std[c]);
    k.dgamma = istd * sdyx;
    k.a = static_cast<float>(static_cast<double>(p.gamma[c]) * istd);
    k.k1 = p.training ? static_cast<float>(sdy / p.count) : 0.0f;
    k.k2 = p.training ? static_cast<float>(istd * k.dgamma / p.count) : 0.0f;
    return k;
}

__device__ __forceinline__ void store_param_grads(const DxArgs& p, int c, const DxCoef& k, double sdy) {
    if (p.gamma_grad)
        p.gamma_grad[c] = p.add_gamma ? p.gamma_grad[c] + static_cast<float>(k.dgamma) : static_cast<float>(k.dgamma);
    if (p.beta_grad) p.beta_grad[c] = p.add_beta ? p.beta_grad[c] + static_cast<float>(sdy) : static_cast<float>(sdy);
}

// dx of one element from its (already gated) output gradient g.
__device__ __forceinline__ float dx_of_gated(const DxArgs& p, float x, float g, float prev, float a, float k1, float k2,
                                             float m_hi, float m_lo) {
#pragma clang fp contract(off)
    const float v = p.training ? a * ((g - k1) - ((x - m_hi) - m_lo) * k2) : a * g;
    return p.add ? prev + v : v;
}

__device__ __forceinline__ float dx_value(const DxArgs& p, float x, float dy, float gate, float prev, float a, float k1,
                                          float k2, float m_hi, float m_lo) {
    const float g = p.gate && !(gate > 0.0f) ? 0.0f : dy;
    return dx_of_gated(p, x, g, prev, a, k1, k2, m_hi, m_lo);
}

// norm_dx with dgamma / dbeta and the dx coefficients finalised in the workgroup.
template <int VEC>
__global__ __launch_bounds__(APPLY_THREADS) void norm_dx_kernel(DxArgs p) {
#pragma clang fp contract(off)
    raise_wave_priority();
    __shared__ float coef[5][MAX_PLANES];
    const int e0 = blockIdx.x * APPLY_SPAN;
    int p0, p1;
    planes_of(e0, p.total, p.div_hw, p0, p1);
    for (int first = p0; first <= p1; first += MAX_PLANES) {
        const int last = min(p1, first + MAX_PLANES - 1);
        for (int i = threadIdx.x; i <= last - first; i += APPLY_THREADS) {
            const int pl = first + i;
            int c;
            p.div_c.divmod(pl, c);
            double sdy = 0.0, sdyx = 0.0;
            if (p.sums) slice_sums(p.partial, c, p.slices, sdy, sdyx);
            const DxCoef k = dx_coef(p, c, sdy, sdyx);
            coef[0][i] = k.a;
            coef[1][i] = k.k1;
            coef[2][i] = k.k2;
            coef[3][i] = p.mean[c];
            coef[4][i] = p.mean[p.C + c];
            if (pl < p.C && static_cast<long long>(pl) * p.HW >= e0) store_param_grads(p, c, k, sdy);
        }
        __syncthreads();
        if (p.dx) {
            const int lo_e = max(e0, first * p.HW), hi_e = min(min(p.total, e0 + APPLY_SPAN), (last + 1) * p.HW);
            constexpr int ITER = APPLY_ELEMS / VEC;  // loads first, as in norm_apply
            float xv[ITER][VEC], gv[ITER][VEC], tv[ITER][VEC] = {}, prev[ITER][VEC] = {};
#pragma unroll
            for (int b = 0; b < ITER; ++b) {
                const int e = lo_e + (b * APPLY_THREADS + threadIdx.x) * VEC;
                if (e >= hi_e) continue;
                if constexpr (VEC == 4) {
                    const float4 x4 = *reinterpret_cast<const float4*>(p.x + e);
                    const float4 d4 = *reinterpret_cast<const float4*>(p.dy + e);
                    xv[b][0] = x4.x; xv[b][1] = x4.y; xv[b][2] = x4.z; xv[b][3] = x4.w;
                    gv[b][0] = d4.x; gv[b][1] = d4.y; gv[b][2] = d4.z; gv[b][3] = d4.w;
                    if (p.gate) {
                        const float4 t4 = *reinterpret_cast<const float4*>(p.gate + e);
                        tv[b][0] = t4.x; tv[b][1] = t4.y; tv[b][2] = t4.z; tv[b][3] = t4.w;
                    }
                    if (p.add) {
                        const float4 o4 = *reinterpret_cast<const float4*>(p.dx + e);
                        prev[b][0] = o4.x; prev[b][1] = o4.y; prev[b][2] = o4.z; prev[b][3] = o4.w;
                    }
                } else {
                    xv[b][0] = p.x[e];
                    gv[b][0] = p.dy[e];
                    if (p.gate) tv[b][0] = p.gate[e];
                    if (p.add) prev[b][0] = p.dx[e];
                }
            }
#pragma unroll
            for (int b = 0; b < ITER; ++b) {
                const int e = lo_e + (b * APPLY_THREADS + threadIdx.x) * VEC;
                if (e >= hi_e) continue;
                const int i = p.div_hw.div(e) - first;  // planes i and i + 1, as in norm_apply
                const int next = (first + i + 1) * p.HW - e;
                float out[VEC];
#pragma unroll
                for (int u = 0; u < VEC; ++u) {
                    const int j = u < next ? i : i + 1;
                    out[u] = dx_value(p, xv[b][u], gv[b][u], tv[b][u], prev[b][u], coef[0][j], coef[1][j], coef[2][j],
                                      coef[3][j], coef[4][j]);
                }
                if constexpr (VEC == 4)
                    *reinterpret_cast<float4*>(p.dx + e) = make_float4(out[0], out[1], out[2], out[3]);
                else p.dx[e] = out[0];
            }
        }
        __syncthreads();
    }
}

// One workgroup per channel when a channel is a single slice (at most CHANNEL_FUSED_MAX positions):
// the partial-sum pass, the finalisation and the element pass of norm_apply (forward) or norm_dx
// (backward) in one launch. Thread t holds its positions of the channel in registers, loaded once,
// and adds them into the same four chains in the same order as channel_partial, so the results are
// the bits of the two-launch path: QUAD, the quads j = 4 (t + i T) + u (chain u); otherwise
// j = t + i T (chain i % 4). Position j is (n, hw) = (j / HW, j % HW).
template <int T, bool QUAD>
struct ChannelSlots {
    static constexpr int PER = CHANNEL_FUSED_MAX / T;  // positions per thread
    static constexpr int GROUPS = QUAD ? PER / 4 : PER;
    static constexpr int WIDTH = QUAD ? 4 : 1;
    // First position of group i of this thread.
    static __device__ __forceinline__ int first(int i) { return QUAD ? 4 * (threadIdx.x + i * T) : threadIdx.x + i * T; }
    // Chain of position u of group i.
    static __device__ __forceinline__ int chain(int i, int u) { return QUAD ? u : i % CHAINS; }
};

template <int W>
__device__ __forceinline__ void load_group(const float* v, int at, int vec, float (&out)[W]) {
    if constexpr (W == 4) load_quad(v, at, vec, out);
    else out[0] = v[at];
}
template <int W>
__device__ __forceinline__ void store_group(float* v, int at, int vec, const float (&in)[W]) {
    if constexpr (W == 4) store_quad(v, at, vec, in);
    else v[at] = in[0];
}

// A convolution output not yet formed: the FP32 split-K slices of its product, slice z holding
// channel c's position j (= n * HW + hw) at partial[z * slice_floats + c * (N * HW) + j]. A
// position's value is their FP64 sum in slice order, rounded once, plus the channel's bias in
// FP32: the product's own slice reduction (gemm.hip split_reduce_vec4_kernel, finish_output), so x
// gets the same bits.
struct SplitSource {
    const float* partial;
    long long slice_floats;
    int slices;
    const float* bias;  // per channel, optional
    float* x;           // where the formed convolution output is stored
};

template <int W>
__device__ __forceinline__ void split_group(const SplitSource& src, int c, long long at, int vec, float (&out)[W]) {
    double sum[W] = {};
    if (W == 4 && vec) {
        for (int z = 0; z < src.slices; ++z) {
            const float4 t = *reinterpret_cast<const float4*>(src.partial + z * src.slice_floats + at);
            const float v[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int u = 0; u < W; ++u) sum[u] += static_cast<double>(v[u]);
        }
    } else {
        for (int z = 0; z < src.slices; ++z)
#pragma unroll
            for (int u = 0; u < W; ++u) sum[u] += static_cast<double>(src.partial[z * src.slice_floats + at + u]);
    }
    const float b = src.bias ? src.bias[c] : 0.0f;
#pragma unroll
    for (int u = 0; u < W; ++u) {
        out[u] = static_cast<float>(sum[u]);
        if (src.bias) out[u] += b;
    }
}

// SPLIT: x is formed from src first (and stored), then normalised as below, in one launch.
template <int T, bool QUAD, bool SPLIT = false>
__global__ __launch_bounds__(T) void norm_forward_channel_kernel(PartialArgs pa, ApplyArgs p, SplitSource src) {
    raise_wave_priority();
    using S = ChannelSlots<T, QUAD>;
    constexpr int G = S::GROUPS, W = S::WIDTH;
    __shared__ float coef[3];
    const int c = blockIdx.x, total = pa.total, plane = p.C * p.HW;
    const long long channel = static_cast<long long>(c) * total;  // channel c's first position in a slice
    double centre;
    if constexpr (SPLIT) {
        float first[1];
        split_group<1>(src, c, channel, 0, first);
        centre = static_cast<double>(first[0]);
    } else {
        centre = static_cast<double>(p.x[c * p.HW]);
    }
    float xv[G][W] = {}, rv[G][W] = {};  // x and the residual, both loaded before the sums
    int at[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const int j = S::first(i);
        int hw;
        const int n = p.div_hw.divmod(j < total ? j : 0, hw);
        at[i] = n * plane + c * p.HW + hw;
        if (j < total) {
            if constexpr (SPLIT) split_group<W>(src, c, channel + j, pa.vec, xv[i]);
            else load_group<W>(p.x, at[i], pa.vec, xv[i]);
            if (p.residual) load_group<W>(p.residual, at[i], pa.vec, rv[i]);
        }
    }
    if constexpr (SPLIT) {
#pragma unroll
        for (int i = 0; i < G; ++i)
            if (S::first(i) < total) store_group<W>(src.x, at[i], pa.vec, xv[i]);
    }
    double a[CHAINS] = {}, b[CHAINS] = {};
#pragma unroll
    for (int i = 0; i < G; ++i) {
        if (S::first(i) >= total) continue;
#pragma unroll
        for (int u = 0; u < W; ++u) {
            const double d = static_cast<double>(xv[i][u]) - centre;
            a[S::chain(i, u)] += d;
            b[S::chain(i, u)] = fma(d, d, b[S::chain(i, u)]);
        }
    }
    double sa = a[0], sb = b[0];
#pragma unroll
    for (int u = 1; u < CHAINS; ++u) {
        sa += a[u];
        sb += b[u];
    }
    workgroup_sum<T>(sa, sb);
    if (threadIdx.x == 0) {
        double sum = 0.0, sq = 0.0;  // the one-slice slice_sums
        sum += sa;
        sq += sb;
        const ApplyCoef k = apply_coef(p, c, sum, sq);
        coef[0] = k.hi;
        coef[1] = k.lo;
        coef[2] = k.istd;
        store_statistics(p, c, k);
    }
    __syncthreads();
    const float m_hi = coef[0], m_lo = coef[1], istd = coef[2], g = p.gamma[c], bt = p.beta[c];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        if (S::first(i) >= total) continue;
        float out[W];
#pragma unroll
        for (int u = 0; u < W; ++u) out[u] = apply_value(p, xv[i][u], rv[i][u], m_hi, m_lo, istd, g, bt);
        store_group<W>(p.y, at[i], pa.vec, out);
    }
}

// SPLIT: dy is formed from src first (the split-K slices of the product whose output gradient it
// is) and stored, then used as below, in one launch.
template <int T, bool QUAD, bool SPLIT = false>
__global__ __launch_bounds__(T) void norm_backward_channel_kernel(PartialArgs pa, DxArgs p, SplitSource src) {
    raise_wave_priority();
    using S = ChannelSlots<T, QUAD>;
    constexpr int G = S::GROUPS, W = S::WIDTH;
    __shared__ float coef[3];
    const int c = blockIdx.x, total = pa.total, plane = p.C * p.HW;
    const double centre = static_cast<double>(p.mean[c]) + static_cast<double>(p.mean[p.C + c]);
    const long long channel = static_cast<long long>(c) * total;  // channel c's first position in a slice
    float xv[G][W] = {}, dv[G][W] = {}, tv[G][W] = {};
    int at[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const int j = S::first(i);
        int hw;
        const int n = p.div_hw.divmod(j < total ? j : 0, hw);
        at[i] = n * plane + c * p.HW + hw;
        if (j < total) {
            load_group<W>(p.x, at[i], pa.vec, xv[i]);
            if constexpr (SPLIT) split_group<W>(src, c, channel + j, pa.vec, dv[i]);
            else load_group<W>(p.dy, at[i], pa.vec, dv[i]);
            if (p.gate) load_group<W>(p.gate, at[i], pa.vec, tv[i]);
        }
    }
    if constexpr (SPLIT) {
#pragma unroll
        for (int i = 0; i < G; ++i)
            if (S::first(i) < total) store_group<W>(src.x, at[i], pa.vec, dv[i]);
    }
    double a[CHAINS] = {}, b[CHAINS] = {};
#pragma unroll
    for (int i = 0; i < G; ++i) {
        if (S::first(i) >= total) continue;
        float gv[W];
#pragma unroll
        for (int u = 0; u < W; ++u) gv[u] = p.gate && !(tv[i][u] > 0.0f) ? 0.0f : dv[i][u];
        if (pa.residual_grad) {
            float r[W] = {};
            if (pa.add_residual) load_group<W>(pa.residual_grad, at[i], pa.vec, r);
#pragma unroll
            for (int u = 0; u < W; ++u) r[u] = pa.add_residual ? r[u] + gv[u] : gv[u];
            store_group<W>(pa.residual_grad, at[i], pa.vec, r);
        }
#pragma unroll
        for (int u = 0; u < W; ++u) {
            const double d = static_cast<double>(xv[i][u]) - centre;
            a[S::chain(i, u)] += static_cast<double>(gv[u]);
            b[S::chain(i, u)] = fma(static_cast<double>(gv[u]), d, b[S::chain(i, u)]);
        }
    }
    double sa = a[0], sb = b[0];
#pragma unroll
    for (int u = 1; u < CHAINS; ++u) {
        sa += a[u];
        sb += b[u];
    }
    workgroup_sum<T>(sa, sb);
    if (threadIdx.x == 0) {
        double sdy = 0.0, sdyx = 0.0;  // the one-slice slice_sums
        sdy += sa;
        sdyx += sb;
        const DxCoef k = dx_coef(p, c, sdy, sdyx);
        coef[0] = k.a;
        coef[1] = k.k1;
        coef[2] = k.k2;
        store_param_grads(p, c, k, sdy);
    }
    __syncthreads();
    if (!p.dx) return;
    const float ka = coef[0], k1 = coef[1], k2 = coef[2], m_hi = p.mean[c], m_lo = p.mean[p.C + c];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        if (S::first(i) >= total) continue;
        float prev[W] = {}, out[W];
        if (p.add) load_group<W>(p.dx, at[i], pa.vec, prev);
#pragma unroll
        for (int u = 0; u < W; ++u) out[u] = dx_value(p, xv[i][u], dv[i][u], tv[i][u], prev[u], ka, k1, k2, m_hi, m_lo);
        store_group<W>(p.dx, at[i], pa.vec, out);
    }
}

// ---- Batch norm + ReLU + max-pool as one unit (a stem: conv -> BN -> ReLU -> max-pool) ----------
// The ReLU output y is never stored. Forward: after norm_partials<STATS>, one workgroup per (n, c)
// plane normalises the plane into LDS with norm_apply's arithmetic and pools it there with the
// pooling kernels' window rule (argmax = flat index into the N x C x H x W tensor y would be).
// Backward: the pooled gradient and argmax of the planes a workgroup covers are staged in LDS; each
// element's gradient is the pooling backward's sum (pool_pixel_grad), gated by ReLU(BN(x)) > 0
// recomputed from x with the forward's coefficients (the same float operations as the stored y).
// The partial sums run over the slices and chains of norm_partials<GRADS> and the dx pass uses
// norm_dx's arithmetic, so the unit gives the bits of the separate BN+ReLU and max-pool passes.
struct PoolShape {
    int H, W, OH, OW, KH, KW, SH, SW;
    FastDiv div_ow, div_w, div_sh, div_sw;
};

struct PoolGrad {
    const float* dy;    // (N, C, OH, OW) gradient of the pooled output
    const int* argmax;  // (N, C, OH, OW) flat indices into x's shape
    const float* gamma;
    const float* beta;
};

constexpr int POOL_STAGE_FLOATS = 16384;  // LDS floats a fused workgroup may stage (64 KB)

// Stages planes [n_lo, n_lo + count) of channel c: their pooled gradient, then their argmax.
__device__ __forceinline__ void stage_pool_grads(const PoolGrad& g, int C, int c, int ohw, int n_lo, int count,
                                                 float* grad, int* where) {
    const int total = count * ohw;
    for (int k = threadIdx.x; k < total; k += blockDim.x) {
        const int n = n_lo + k / ohw, o = k - (k / ohw) * ohw;
        const long long at = (static_cast<long long>(n) * C + c) * ohw + o;
        grad[k] = g.dy[at];
        where[k] = g.argmax[at];
    }
}

// Forward: one workgroup per plane pl = n * C + c; y of the plane in LDS, then the pooled plane.
__global__ __launch_bounds__(APPLY_THREADS) void norm_apply_pool_kernel(ApplyArgs p, PoolShape q, float* __restrict__ pooled,
                                                                      int* __restrict__ argmax, int vec) {
#pragma clang fp contract(off)
    raise_wave_priority();
    extern __shared__ float plane_y[];  // H * W floats
    __shared__ float coef[3];
    const int pl = blockIdx.x;
    int c;
    p.div_c.divmod(pl, c);
    if (threadIdx.x == 0) {
        double sum = 0.0, sq = 0.0;
        if (p.training) slice_sums(p.partial, c, p.slices, sum, sq);
        const ApplyCoef k = apply_coef(p, c, sum, sq);
        coef[0] = k.hi;
        coef[1] = k.lo;
        coef[2] = k.istd;
        if (pl < p.C) store_statistics(p, c, k);  // image 0's plane: once per channel
    }
    __syncthreads();
    const float m_hi = coef[0], m_lo = coef[1], istd = coef[2], g = p.gamma[c], b = p.beta[c];
    const long long base = static_cast<long long>(pl) * p.HW;
    if (vec) {  // H*W % 4 == 0 and x 16-byte aligned
        for (int e = 4 * threadIdx.x; e < p.HW; e += 4 * APPLY_THREADS) {
            const float4 x4 = *reinterpret_cast<const float4*>(p.x + base + e);
            plane_y[e] = relu_value(affine_value(x4.x, m_hi, m_lo, istd, g, b));
            plane_y[e + 1] = relu_value(affine_value(x4.y, m_hi, m_lo, istd, g, b));
            plane_y[e + 2] = relu_value(affine_value(x4.z, m_hi, m_lo, istd, g, b));
            plane_y[e + 3] = relu_value(affine_value(x4.w, m_hi, m_lo, istd, g, b));
        }
    } else {
        for (int e = threadIdx.x; e < p.HW; e += APPLY_THREADS)
            plane_y[e] = relu_value(affine_value(p.x[base + e], m_hi, m_lo, istd, g, b));
    }
    __syncthreads();
    const int ohw = q.OH * q.OW;
    for (int o = threadIdx.x; o < ohw; o += APPLY_THREADS) {
        int ow;
        const int oh = q.div_ow.divmod(o, ow);
        int best;
        const float v = window_max(plane_y, oh * q.SH * q.W + ow * q.SW, q.W, q.KH, q.KW, best);
        const long long out = static_cast<long long>(pl) * ohw + o;
        pooled[out] = v;
        argmax[out] = static_cast<int>(base + best);
    }
}

// The gated gradient of element (n, hw) of channel c, whose flat index is `at`: its pooling gradient
// from the staged planes (n relative to the first staged plane), zero where ReLU(BN(x)) <= 0.
__device__ __forceinline__ float pooled_grad(const float* grad, const int* where, int n_rel, int hw, int at, float x,
                                             const PoolShape& q, float m_hi, float m_lo, float istd, float gm,
                                             float bt) {
    int iw;
    const int ih = q.div_w.divmod(hw, iw);
    const float y = relu_value(affine_value(x, m_hi, m_lo, istd, gm, bt));
    if (!(y > 0.0f)) return 0.0f;
    return pool_pixel_grad(grad, where, n_rel, ih, iw, at, q.OH, q.OW, q.KH, q.KW, q.div_sh, q.div_sw);
}

// The gated gradients of the quad of positions hw .. hw + 3 (one plane row when `rows`, i.e. W a
// multiple of 4: the covering windows are then scanned once for the four) of staged plane n_rel,
// first flat index `at`.
__device__ __forceinline__ void pooled_quad(const float* grad, const int* where, int n_rel, int hw, int at,
                                            const float (&x)[4], const PoolShape& q, float m_hi, float m_lo,
                                            float istd, float gm, float bt, bool rows, float (&g)[4]) {
    if (rows) {
        int iw;
        const int ih = q.div_w.divmod(hw, iw);
        const float4 g4 = pool_quad_grad(grad, where, n_rel, ih, iw, at, q.OH, q.OW, q.KH, q.KW, q.div_sh, q.div_sw);
        g[0] = g4.x; g[1] = g4.y; g[2] = g4.z; g[3] = g4.w;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (!(relu_value(affine_value(x[u], m_hi, m_lo, istd, gm, bt)) > 0.0f)) g[u] = 0.0f;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            g[u] = pooled_grad(grad, where, n_rel, hw + u, at + u, x[u], q, m_hi, m_lo, istd, gm, bt);
    }
}

// Backward partial sums: workgroup (s, c) covers slice s of channel c, in the order of
// norm_partials<GRADS> (quads when QUAD).
template <int T, bool QUAD>
__global__ __launch_bounds__(T) void norm_partials_pool_kernel(PartialArgs p, PoolShape q, PoolGrad pg, int rows) {
    raise_wave_priority();
    extern __shared__ float staged[];
    const int s = blockIdx.x, c = blockIdx.y, slices = gridDim.x;
    const int j0 = s * p.chunk, j1 = min(p.total, j0 + p.chunk);
    const int ohw = q.OH * q.OW;
    const int n_lo = j0 < j1 ? p.div_hw.div(j0) : 0;
    const int count = j0 < j1 ? p.div_hw.div(j1 - 1) - n_lo + 1 : 0;
    float* grad = staged;
    int* where = reinterpret_cast<int*>(staged + count * ohw);
    stage_pool_grads(pg, p.C, c, ohw, n_lo, count, grad, where);
    __syncthreads();
    const int plane = p.C * p.HW;
    const float m_hi = p.mean[c], m_lo = p.mean[p.C + c], istd = p.inv_std[c], gm = pg.gamma[c], bt = pg.beta[c];
    const double centre = static_cast<double>(m_hi) + static_cast<double>(m_lo);
    double a[CHAINS] = {}, b[CHAINS] = {};
    if constexpr (QUAD) {
        for (int base = j0 + 4 * threadIdx.x; base < j1; base += 8 * T) {
            float xv[2][4] = {}, gv[2][4] = {};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int j = base + h * 4 * T;
                if (j >= j1) continue;
                int hw;
                const int n = p.div_hw.divmod(j, hw);
                const int at = n * plane + c * p.HW + hw;
                load_quad(p.x, at, p.vec, xv[h]);
                pooled_quad(grad, where, n - n_lo, hw, at, xv[h], q, m_hi, m_lo, istd, gm, bt, rows != 0, gv[h]);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (base + h * 4 * T >= j1) continue;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const double d = static_cast<double>(xv[h][u]) - centre;
                    a[u] += static_cast<double>(gv[h][u]);
                    b[u] = fma(static_cast<double>(gv[h][u]), d, b[u]);
                }
            }
        }
    }
    for (int base = j0 + threadIdx.x; !QUAD && base < j1; base += CHAINS * T) {
        float xv[CHAINS], gv[CHAINS];
#pragma unroll
        for (int u = 0; u < CHAINS; ++u) {
            const int j = base + u * T;
            int hw;
            const int n = p.div_hw.divmod(j < j1 ? j : j0, hw);
            const int at = n * plane + c * p.HW + hw;
            xv[u] = j < j1 ? p.x[at] : 0.0f;
            gv[u] = j < j1 ? pooled_grad(grad, where, n - n_lo, hw, at, xv[u], q, m_hi, m_lo, istd, gm, bt) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < CHAINS; ++u) {
            if (base + u * T >= j1) continue;
            const double d = static_cast<double>(xv[u]) - centre;
            a[u] += static_cast<double>(gv[u]);
            b[u] = fma(static_cast<double>(gv[u]), d, b[u]);
        }
    }
    double sa = a[0], sb = b[0];
#pragma unroll
    for (int u = 1; u < CHAINS; ++u) {
        sa += a[u];
        sb += b[u];
    }
    workgroup_sum<T>(sa, sb);
    if (threadIdx.x == 0) {
        p.partial[(static_cast<long long>(c) * slices + s) * 2] = sa;
        p.partial[(static_cast<long long>(c) * slices + s) * 2 + 1] = sb;
    }
}

// Backward dx: one workgroup per plane pl = n * C + c, as norm_dx with the pooled gradient staged.
__global__ __launch_bounds__(APPLY_THREADS) void norm_dx_pool_kernel(DxArgs p, PoolShape q, PoolGrad pg, int vec) {
#pragma clang fp contract(off)
    raise_wave_priority();
    extern __shared__ float staged[];
    __shared__ float coef[3];
    const int pl = blockIdx.x;
    int c;
    const int n = p.div_c.divmod(pl, c);
    const int ohw = q.OH * q.OW;
    float* grad = staged;
    int* where = reinterpret_cast<int*>(staged + ohw);
    stage_pool_grads(pg, p.C, c, ohw, n, 1, grad, where);
    if (threadIdx.x == 0) {
        double sdy = 0.0, sdyx = 0.0;
        if (p.sums) slice_sums(p.partial, c, p.slices, sdy, sdyx);
        const DxCoef k = dx_coef(p, c, sdy, sdyx);
        coef[0] = k.a;
        coef[1] = k.k1;
        coef[2] = k.k2;
        if (pl < p.C) store_param_grads(p, c, k, sdy);
    }
    __syncthreads();
    if (!p.dx) return;
    const float ka = coef[0], k1 = coef[1], k2 = coef[2], m_hi = p.mean[c], m_lo = p.mean[p.C + c];
    const float istd = p.inv_std[c], gm = pg.gamma[c], bt = pg.beta[c];
    const int base = pl * p.HW;
    if (vec) {  // W % 4 == 0, x and dx 16-byte aligned: four adjacent pixels of one row
        for (int e = 4 * threadIdx.x; e < p.HW; e += 4 * APPLY_THREADS) {
            const float4 x4 = *reinterpret_cast<const float4*>(p.x + base + e);
            const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
            float4 prev = make_float4(0.f, 0.f, 0.f, 0.f);
            if (p.add) prev = *reinterpret_cast<const float4*>(p.dx + base + e);
            const float ps[4] = {prev.x, prev.y, prev.z, prev.w};
            int iw;
            const int ih = q.div_w.divmod(e, iw);
            const float4 g4 = pool_quad_grad(grad, where, 0, ih, iw, base + e, q.OH, q.OW, q.KH, q.KW, q.div_sh, q.div_sw);
            const float gs[4] = {g4.x, g4.y, g4.z, g4.w};
            float out[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float y = relu_value(affine_value(xs[u], m_hi, m_lo, istd, gm, bt));
                out[u] = dx_of_gated(p, xs[u], y > 0.0f ? gs[u] : 0.0f, ps[u], ka, k1, k2, m_hi, m_lo);
            }
            *reinterpret_cast<float4*>(p.dx + base + e) = make_float4(out[0], out[1], out[2], out[3]);
        }
    } else {
        for (int e = threadIdx.x; e < p.HW; e += APPLY_THREADS) {
            const float x = p.x[base + e];
            const float gv = pooled_grad(grad, where, 0, e, base + e, x, q, m_hi, m_lo, istd, gm, bt);
            p.dx[base + e] = dx_of_gated(p, x, gv, p.add ? p.dx[base + e] : 0.0f, ka, k1, k2, m_hi, m_lo);
        }
    }
}

// Whether a pass sums each channel with WIDE_PT threads: a one-slice channel of at least WIDE_MIN
// positions (one workgroup per channel then has too few to keep 256 threads' loads in flight; on
// MI355X layer3's 5120 positions take 6 / 8 us per forward / backward pass at 1024 threads against
// 9 / 16.5 at 256). The partial-sum pass and the one-launch channel kernels decide alike, so they
// sum in the same order.
bool wide_sums(const NormShape& s) {
    return norm_slices(s) == 1 && static_cast<std::int64_t>(s.N) * s.HW >= WIDE_MIN;
}

bool aligned16(const void* q) { return (reinterpret_cast<std::uintptr_t>(q) & 15) == 0; }

// Whether a channel's positions are summed in quads (channel_partial): H*W a multiple of 4. It depends
// on the shape only, so every pass over a shape sums in the same order.
bool quad_order(const NormShape& s) { return s.HW % 4 == 0; }

// Positions per partial-sum slice: a multiple of 4 in quad order, so that a quad lies in one slice.
int slice_chunk(const NormShape& s, int slices) {
    const std::int64_t total = static_cast<std::int64_t>(s.N) * s.HW;
    std::int64_t chunk = (total + slices - 1) / slices;
    if (quad_order(s)) chunk = (chunk + 3) / 4 * 4;
    return static_cast<int>(chunk);
}

// The float4 flag of a pass: all of its tensors 16-byte aligned (quad order only).
int quad_vec(const NormShape& s, std::initializer_list<const void*> tensors) {
    if (!quad_order(s)) return 0;
    for (const void* t : tensors)
        if (t && !aligned16(t)) return 0;
    return 1;
}

template <int MODE, bool QUAD>
void launch_partials(const NormShape& s, const PartialArgs& args, hipStream_t stream) {
    const dim3 grid(norm_slices(s), s.C);
    if (wide_sums(s)) launch(norm_partials_kernel<MODE, WIDE_PT, QUAD>, grid, WIDE_PT, 0, stream, args);
    else launch(norm_partials_kernel<MODE, PT, QUAD>, grid, PT, 0, stream, args);
}

template <bool SPLIT>
void launch_forward_channel(const NormShape& s, const PartialArgs& args, const ApplyArgs& a, const SplitSource& src,
                            hipStream_t stream) {
    const bool wide = wide_sums(s);
    if (quad_order(s)) {
        if (wide) launch(norm_forward_channel_kernel<WIDE_PT, true, SPLIT>, s.C, WIDE_PT, 0, stream, args, a, src);
        else launch(norm_forward_channel_kernel<PT, true, SPLIT>, s.C, PT, 0, stream, args, a, src);
    } else {
        if (wide) launch(norm_forward_channel_kernel<WIDE_PT, false, SPLIT>, s.C, WIDE_PT, 0, stream, args, a, src);
        else launch(norm_forward_channel_kernel<PT, false, SPLIT>, s.C, PT, 0, stream, args, a, src);
    }
}

int run_partials(int mode, const NormShape& s, const PartialArgs& args, hipStream_t stream) {
    const bool quad = quad_order(s);
    if (mode == STATS) (quad ? launch_partials<STATS, true> : launch_partials<STATS, false>)(s, args, stream);
    else (quad ? launch_partials<GRADS, true> : launch_partials<GRADS, false>)(s, args, stream);
    return MFH_CHECK_LAUNCH(mode == STATS ? "norm_partials<stats>" : "norm_partials<grads>", stream);
}

// Whether the element passes can take float4s: every workgroup's span starts on a multiple of 4
// (APPLY_SPAN is one) and is one round of planes (so its first element is the span's), and the
// tensor's length is a multiple of 4. A float4 then lies in one plane or crosses into the next.
bool vec4_spans(const NormShape& s) {
    const std::int64_t total = static_cast<std::int64_t>(s.N) * s.C * s.HW;
    return total % 4 == 0 && (s.HW % 4 == 0 || APPLY_SPAN / s.HW + 2 <= MAX_PLANES);
}

}  // namespace

int norm_slices(const NormShape& s) {
    const std::int64_t positions = static_cast<std::int64_t>(s.N) * s.HW;
    if (positions <= CHANNEL_FUSED_MAX) return 1;  // one workgroup per channel, one launch per pass
    const std::int64_t wanted = (8LL * device_cu_count() + s.C - 1) / s.C;
    const std::int64_t most = std::max<std::int64_t>(1, positions / MIN_SLICE);
    // At least two slices: one slice means the one-launch channel kernels, which hold at most
    // CHANNEL_FUSED_MAX positions (a wide layer, C >= 8 * CUs, would otherwise get one).
    return static_cast<int>(std::max<std::int64_t>(2, std::min(wanted, most)));
}

std::int64_t norm_workspace_doubles(const NormShape& s) {
    // FP64 (sum, second sum) per slice and channel.
    return 2LL * s.C * norm_slices(s);
}

// The arguments of the forward kernels of one batch-norm pass.
static void forward_args(const NormShape& s, const NormForward& f, int slices, PartialArgs& args, ApplyArgs& a) {
    const int total = s.N * s.C * s.HW;
    args = PartialArgs{};
    args.x = f.x;
    args.partial = f.partial;
    args.C = s.C;
    args.HW = s.HW;
    args.total = s.N * s.HW;
    args.chunk = slice_chunk(s, slices);
    args.div_hw = FastDiv(s.HW);
    args.vec = quad_vec(s, {f.x, f.y, f.residual});
    a = ApplyArgs{};
    a.x = f.x;
    a.gamma = f.gamma;
    a.beta = f.beta;
    a.residual = f.residual;
    a.y = f.y;
    a.mean = f.mean;
    a.inv_std = f.inv_std;
    a.running_mean = f.running_mean;
    a.running_var = f.running_var;
    a.partial = f.partial;
    a.total = total;
    a.C = s.C;
    a.HW = s.HW;
    a.slices = slices;
    a.training = f.training ? 1 : 0;
    a.relu = f.relu ? 1 : 0;
    a.count = static_cast<double>(s.N) * s.HW;
    a.momentum = f.momentum;
    a.eps = f.eps;
    a.var_scale = f.var_scale;
    a.div_hw = FastDiv(s.HW);
    a.div_c = FastDiv(s.C);
}

int norm_forward(const NormShape& s, const NormForward& f, hipStream_t stream) {
    const int total = s.N * s.C * s.HW;
    const int slices = norm_slices(s);
    PartialArgs args;
    ApplyArgs a;
    forward_args(s, f, slices, args, a);
    const bool vec = vec4_spans(s) && aligned16(f.x) && aligned16(f.y) && (!f.residual || aligned16(f.residual));
    if (f.training && slices == 1) {
        launch_forward_channel<false>(s, args, a, SplitSource{}, stream);
        return MFH_CHECK_LAUNCH("norm_forward_channel", stream);
    }
    if (f.training) MFH_TRY(run_partials(STATS, s, args, stream));
    const unsigned blocks = blocks_for(total, APPLY_SPAN);
    if (vec) launch(norm_apply_kernel<4>, blocks, APPLY_THREADS, 0, stream, a);
    else launch(norm_apply_kernel<1>, blocks, APPLY_THREADS, 0, stream, a);
    return MFH_CHECK_LAUNCH("norm_apply", stream);
}

int norm_forward_split(const NormShape& s, const NormForward& f, const float* partial, int slices, const float* bias,
                       float* x, hipStream_t stream) {
    if (!f.training || norm_slices(s) != 1)
        return MFH_FAIL(ERR_ARG, "forming x inside batch norm needs a training pass of one launch per channel "
                                 "(N*H*W at most 8192); reduce the slices first (mfh_split_reduce)");
    PartialArgs args;
    ApplyArgs a;
    forward_args(s, f, 1, args, a);
    args.vec = quad_vec(s, {x, f.y, f.residual, partial});
    const SplitSource src{partial, static_cast<long long>(s.C) * s.N * s.HW, slices, bias, x};
    launch_forward_channel<true>(s, args, a, src, stream);
    return MFH_CHECK_LAUNCH("norm_forward_channel<split>", stream);
}

namespace {

PoolShape pool_shape_of(const PoolDims& d) {
    PoolShape q{};
    q.H = d.H;
    q.W = d.W;
    q.OH = d.OH;
    q.OW = d.OW;
    q.KH = d.KH;
    q.KW = d.KW;
    q.SH = d.SH;
    q.SW = d.SW;
    q.div_ow = FastDiv(d.OW);
    q.div_w = FastDiv(d.W);
    q.div_sh = FastDiv(d.SH);
    q.div_sw = FastDiv(d.SW);
    return q;
}

// Most planes that one partial-sum slice (of norm_partials' chunk of positions) overlaps.
int planes_per_slice(const NormShape& s) {
    const std::int64_t total = static_cast<std::int64_t>(s.N) * s.HW;
    const int slices = norm_slices(s);
    const std::int64_t chunk = slice_chunk(s, slices);
    std::int64_t most = 0;
    for (std::int64_t j0 = 0; j0 < total; j0 += chunk) {
        const std::int64_t j1 = std::min(total, j0 + chunk);
        most = std::max(most, (j1 - 1) / s.HW - j0 / s.HW + 1);
    }
    return static_cast<int>(most);
}

}  // namespace

bool norm_pool_supported(const NormShape& s, const PoolDims& d) {
    const std::int64_t ohw = static_cast<std::int64_t>(d.OH) * d.OW;
    return d.H * d.W == s.HW && s.HW <= POOL_STAGE_FLOATS && 2 * ohw <= POOL_STAGE_FLOATS &&
           2 * ohw * planes_per_slice(s) <= POOL_STAGE_FLOATS;
}

int norm_relu_pool_forward(const NormShape& s, const NormForward& f, const PoolDims& d, float* pooled, int* argmax,
                           hipStream_t stream) {
    if (!norm_pool_supported(s, d)) return MFH_FAIL(ERR_ARG, "batch-norm + max-pool planes exceed the fused kernels' LDS");
    const int slices = norm_slices(s);
    PartialArgs args{};
    args.x = f.x;
    args.partial = f.partial;
    args.C = s.C;
    args.HW = s.HW;
    args.total = s.N * s.HW;
    args.chunk = slice_chunk(s, slices);
    args.div_hw = FastDiv(s.HW);
    args.vec = quad_vec(s, {f.x});
    ApplyArgs a{};
    a.x = f.x;
    a.gamma = f.gamma;
    a.beta = f.beta;
    a.mean = f.mean;
    a.inv_std = f.inv_std;
    a.running_mean = f.running_mean;
    a.running_var = f.running_var;
    a.partial = f.partial;
    a.total = s.N * s.C * s.HW;
    a.C = s.C;
    a.HW = s.HW;
    a.slices = slices;
    a.training = f.training ? 1 : 0;
    a.relu = 1;
    a.count = static_cast<double>(s.N) * s.HW;
    a.momentum = f.momentum;
    a.eps = f.eps;
    a.var_scale = f.var_scale;
    a.div_hw = FastDiv(s.HW);
    a.div_c = FastDiv(s.C);
    if (f.training) MFH_TRY(run_partials(STATS, s, args, stream));
    const int vec = s.HW % 4 == 0 && aligned16(f.x) ? 1 : 0;
    launch(norm_apply_pool_kernel, static_cast<unsigned>(s.N * s.C), APPLY_THREADS, s.HW * sizeof(float), stream, a, pool_shape_of(d), pooled, argmax, vec);
    return MFH_CHECK_LAUNCH("norm_apply_pool", stream);
}

int norm_relu_pool_backward(const NormShape& s, const NormBackward& b, const PoolDims& d, const float* pooled_grad,
                            const int* argmax, const float* beta, hipStream_t stream) {
    if (!norm_pool_supported(s, d)) return MFH_FAIL(ERR_ARG, "batch-norm + max-pool planes exceed the fused kernels' LDS");
    const int slices = norm_slices(s);
    const bool sums = b.gamma_grad || b.beta_grad || (b.training && b.x_grad);
    const PoolShape q = pool_shape_of(d);
    const PoolGrad pg{pooled_grad, argmax, b.gamma, beta};
    const int ohw = d.OH * d.OW;
    if (sums) {
        PartialArgs args{};
        args.x = b.x;
        args.mean = b.mean;
        args.inv_std = b.inv_std;
        args.partial = b.partial;
        args.C = s.C;
        args.HW = s.HW;
        args.total = s.N * s.HW;
        args.chunk = slice_chunk(s, slices);
        args.div_hw = FastDiv(s.HW);
        const size_t lds = static_cast<size_t>(planes_per_slice(s)) * ohw * 2 * sizeof(float);
        args.vec = quad_vec(s, {b.x});
        const int rows = d.W % 4 == 0 ? 1 : 0;
        const bool wide = wide_sums(s);
        const dim3 grid(slices, s.C);
        if (quad_order(s)) {
            if (wide) launch(norm_partials_pool_kernel<WIDE_PT, true>, grid, WIDE_PT, lds, stream, args, q, pg, rows);
            else launch(norm_partials_pool_kernel<PT, true>, grid, PT, lds, stream, args, q, pg, rows);
        } else {
            if (wide) launch(norm_partials_pool_kernel<WIDE_PT, false>, grid, WIDE_PT, lds, stream, args, q, pg, rows);
            else launch(norm_partials_pool_kernel<PT, false>, grid, PT, lds, stream, args, q, pg, rows);
        }
        MFH_TRY(MFH_CHECK_LAUNCH("norm_partials_pool", stream));
    }
    if (!b.x_grad && !sums) return OK;
    DxArgs dx{};
    dx.x = b.x;
    dx.gamma = b.gamma;
    dx.mean = b.mean;
    dx.inv_std = b.inv_std;
    dx.dx = b.x_grad;
    dx.gamma_grad = b.gamma_grad;
    dx.beta_grad = b.beta_grad;
    dx.partial = b.partial;
    dx.total = s.N * s.C * s.HW;
    dx.C = s.C;
    dx.HW = s.HW;
    dx.slices = slices;
    dx.training = b.training ? 1 : 0;
    dx.add = b.add_x ? 1 : 0;
    dx.add_gamma = b.add_gamma ? 1 : 0;
    dx.add_beta = b.add_beta ? 1 : 0;
    dx.sums = sums ? 1 : 0;
    dx.count = static_cast<double>(s.N) * s.HW;
    dx.div_hw = FastDiv(s.HW);
    dx.div_c = FastDiv(s.C);
    const int vec = d.W % 4 == 0 && aligned16(b.x) && (!b.x_grad || aligned16(b.x_grad)) ? 1 : 0;
    launch(norm_dx_pool_kernel, static_cast<unsigned>(s.N * s.C), APPLY_THREADS, static_cast<size_t>(ohw) * 2 * sizeof(float),
                          stream, dx, q, pg, vec);
    return MFH_CHECK_LAUNCH("norm_dx_pool", stream);
}

namespace {

template <bool SPLIT>
void launch_backward_channel(const NormShape& s, const PartialArgs& args, const DxArgs& d, const SplitSource& src,
                             hipStream_t stream) {
    const bool wide = wide_sums(s);
    if (quad_order(s)) {
        if (wide) launch(norm_backward_channel_kernel<WIDE_PT, true, SPLIT>, s.C, WIDE_PT, 0, stream, args, d, src);
        else launch(norm_backward_channel_kernel<PT, true, SPLIT>, s.C, PT, 0, stream, args, d, src);
    } else {
        if (wide) launch(norm_backward_channel_kernel<WIDE_PT, false, SPLIT>, s.C, WIDE_PT, 0, stream, args, d, src);
        else launch(norm_backward_channel_kernel<PT, false, SPLIT>, s.C, PT, 0, stream, args, d, src);
    }
}

void backward_args(const NormShape& s, const NormBackward& b, int slices, bool sums, PartialArgs& args, DxArgs& d) {
    args = PartialArgs{};
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
    args.chunk = slice_chunk(s, slices);
    args.div_hw = FastDiv(s.HW);
    args.vec = quad_vec(s, {b.x, b.dy, b.gate, b.residual_grad, b.x_grad});
    d = DxArgs{};
    d.x = b.x;
    d.dy = b.dy;
    d.gate = b.gate;
    d.gamma = b.gamma;
    d.mean = b.mean;
    d.inv_std = b.inv_std;
    d.dx = b.x_grad;
    d.gamma_grad = b.gamma_grad;
    d.beta_grad = b.beta_grad;
    d.partial = b.partial;
    d.total = s.N * s.C * s.HW;
    d.C = s.C;
    d.HW = s.HW;
    d.slices = slices;
    d.training = b.training ? 1 : 0;
    d.add = b.add_x ? 1 : 0;
    d.add_gamma = b.add_gamma ? 1 : 0;
    d.add_beta = b.add_beta ? 1 : 0;
    d.sums = sums ? 1 : 0;
    d.count = static_cast<double>(s.N) * s.HW;
    d.div_hw = FastDiv(s.HW);
    d.div_c = FastDiv(s.C);
}

}  // namespace

int norm_backward(const NormShape& s, const NormBackward& b, hipStream_t stream) {
    const int total = s.N * s.C * s.HW;
    const int slices = norm_slices(s);
    const bool sums = b.gamma_grad || b.beta_grad || (b.training && b.x_grad);
    PartialArgs args;
    DxArgs d;
    backward_args(s, b, slices, sums, args, d);
    const bool fused = sums && slices == 1;
    if ((sums || b.residual_grad) && !fused) MFH_TRY(run_partials(GRADS, s, args, stream));
    if (!b.x_grad && !sums) return OK;
    const bool vec = vec4_spans(s) && aligned16(b.x) && aligned16(b.dy) && (!b.gate || aligned16(b.gate)) &&
                     (!b.x_grad || aligned16(b.x_grad));
    if (fused) {
        launch_backward_channel<false>(s, args, d, SplitSource{}, stream);
        return MFH_CHECK_LAUNCH("norm_backward_channel", stream);
    }
    const unsigned blocks = blocks_for(total, APPLY_SPAN);
    if (vec) launch(norm_dx_kernel<4>, blocks, APPLY_THREADS, 0, stream, d);
    else launch(norm_dx_kernel<1>, blocks, APPLY_THREADS, 0, stream, d);
    return MFH_CHECK_LAUNCH("norm_dx", stream);
}

int norm_backward_split(const NormShape& s, const NormBackward& b, const float* partial, int slices, float* dy,
                        hipStream_t stream) {
    const bool sums = b.gamma_grad || b.beta_grad || (b.training && b.x_grad);
    if (!sums || norm_slices(s) != 1)
        return MFH_FAIL(ERR_ARG, "forming dy inside the batch-norm backward needs a pass that sums over one launch "
                                 "per channel (N*H*W at most 8192, with a gradient of gamma, beta or, training, x); "
                                 "reduce the slices first (mfh_split_reduce)");
    if (b.dy != dy) return MFH_FAIL(ERR_ARG, "the formed dy must be the pass's dy");
    PartialArgs args;
    DxArgs d;
    backward_args(s, b, 1, sums, args, d);
    args.vec = quad_vec(s, {b.x, b.dy, b.gate, b.residual_grad, b.x_grad, partial});
    const SplitSource src{partial, static_cast<long long>(s.C) * s.N * s.HW, slices, nullptr, dy};
    launch_backward_channel<true>(s, args, d, src, stream);
    return MFH_CHECK_LAUNCH("norm_backward_channel<split>", stream);
}

}  // namespace mfh
