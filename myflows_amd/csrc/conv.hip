// Bandwidth-bound kernels of the convolution and pooling path: im2col, col2im (gather from the
// transposed column gradient), the NCHW epilogue (bias + activation), the transposed/gated dy with
// FP64 bias partials, the fixed-order FP64 partial reduction, the GEMM bias epilogue and max-pool
// forward/backward.
//
// Layouts (row-major, NCHW): cols[(n*OH + oh)*OW + ow][(ci*KH + kh)*KW + kw] is the im2col matrix
// (M = N*OH*OW rows, K = CI*KH*KW features); rows[(n*OHW + p)][co] is a GEMM output before the
// epilogue; gcT[n][(ci*KH + kh)*KW + kw][oh*OW + ow] is the per-image transposed column gradient.
// Every reduction sums in a fixed order, so each kernel is bitwise reproducible.
#include <algorithm>

#include "common.h"
#include "fastdiv.h"
#include "pool_rules.h"

namespace mfh {
namespace {

// One thread per cols element. The index decomposition uses FastDiv; the x reads of neighbouring
// threads (consecutive kw, then kh/ci) hit the same cache lines, the writes are fully coalesced.
__global__ __launch_bounds__(256) void im2col_kernel(const float* __restrict__ x, float* __restrict__ cols, int total,
                                                     FastDiv div_k, FastDiv div_kw, FastDiv div_kh, FastDiv div_ow,
                                                     FastDiv div_oh, int CI, int H, int W, int SH, int SW, int PH,
                                                     int PW) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    int feature, kw, kh, ow, oh;
    const int row = div_k.divmod(idx, feature);
    const int t = div_kw.divmod(feature, kw);
    const int ci = div_kh.divmod(t, kh);
    const int t2 = div_ow.divmod(row, ow);
    const int n = div_oh.divmod(t2, oh);
    const int ih = oh * SH - PH + kh;
    const int iw = ow * SW - PW + kw;
    float v = 0.0f;
    if (ih >= 0 && ih < H && iw >= 0 && iw < W) v = x[((n * CI + ci) * H + ih) * W + iw];
    cols[idx] = v;
}

// The same matrix four features at a time (K % 4 == 0): thread t writes cols elements 4t .. 4t+3 of
// one row with one 16-byte store, stepping (ci, kh, kw) forward from the first without divisions.
__global__ __launch_bounds__(256) void im2col_vec4_kernel(const float* __restrict__ x, float* __restrict__ cols,
                                                          int quads, FastDiv div_k, FastDiv div_kw, FastDiv div_kh,
                                                          FastDiv div_ow, FastDiv div_oh, int CI, int KH, int KW,
                                                          int H, int W, int SH, int SW, int PH, int PW) {
    const int q = blockIdx.x * 256 + threadIdx.x;
    if (q >= quads) return;
    const int first = q * 4;
    int feature, kw, kh, ow, oh;
    const int row = div_k.divmod(first, feature);
    const int t = div_kw.divmod(feature, kw);
    int ci = div_kh.divmod(t, kh);
    const int t2 = div_ow.divmod(row, ow);
    const int n = div_oh.divmod(t2, oh);
    const int ih0 = oh * SH - PH, iw0 = ow * SW - PW;
    const float* image = x + static_cast<long long>(n) * CI * H * W;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ih = ih0 + kh, iw = iw0 + kw;
        v[j] = (ih >= 0 && ih < H && iw >= 0 && iw < W) ? image[(ci * H + ih) * W + iw] : 0.0f;
        if (++kw == KW) {
            kw = 0;
            if (++kh == KH) {
                kh = 0;
                ++ci;
            }
        }
    }
    *reinterpret_cast<float4*>(cols + first) = make_float4(v[0], v[1], v[2], v[3]);
}

// dx[n, ci, ih, iw] = sum over every window position (oh, ow) that reads (ih, iw), visited in
// increasing (oh, ow) order, of the column gradient of feature f = (ci*KH + kh)*KW + kw at that
// position. The column gradient is feature-major, element (f, n, oh*OW + ow) at
// f * f_stride + n * n_stride + oh*OW + ow ([f][n*OH*OW + p] or [n][f][p]), so for a fixed (kh, kw)
// the threads of consecutive iw read consecutive ow: the gather is coalesced. No atomics, so the
// result is deterministic.
// FKH, FKW, FSH, FSW > 0: the kernel for that window and stride, with every tap's read issued
// before the sums (taps outside the image add nothing: the sum starts at +0 and never is -0, so
// skipping a term and adding +0 give the same bits); 0: any window, read window by window.
template <int FKH, int FKW, int FSH, int FSW>
__global__ __launch_bounds__(256) void col2im_t_kernel(const float* __restrict__ gcT, float* __restrict__ dx,
                                                       int total, FastDiv div_w, FastDiv div_h, FastDiv div_ci,
                                                       int CI, int KH, int KW, int OH, int OW, int SH, int SW,
                                                       FastDiv div_sh, FastDiv div_sw, int PH, int PW,
                                                       long long f_stride, long long n_stride, int accumulate) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    int iw, ih, ci;
    const int t = div_w.divmod(idx, iw);
    const int t2 = div_h.divmod(t, ih);
    const int n = div_ci.divmod(t2, ci);
    const int hp = ih + PH, wp = iw + PW;  // coordinates in the zero-padded input
    float sum = 0.0f;
    if constexpr (FKH > 0) {
        const float* image = gcT + n * n_stride + static_cast<long long>(ci) * FKH * FKW * f_stride;
        // Taps in the order of increasing (oh, ow): kh, then kw, descending.
        float v[FKH * FKW];
#pragma unroll
        for (int a = 0; a < FKH; ++a) {
            const int kh = FKH - 1 - a, oh_s = hp - kh;  // oh * FSH
            const int oh = oh_s / FSH;
            const bool row_ok = oh_s >= 0 && oh_s % FSH == 0 && oh < OH;
#pragma unroll
            for (int b = 0; b < FKW; ++b) {
                const int kw = FKW - 1 - b, ow_s = wp - kw;
                const int ow = ow_s / FSW;
                const bool ok = row_ok && ow_s >= 0 && ow_s % FSW == 0 && ow < OW;
                v[a * FKW + b] = ok ? image[(kh * FKW + kw) * f_stride + oh * OW + ow] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < FKH * FKW; ++u) sum += v[u];
    } else {
        // Windows oh with oh*SH <= hp <= oh*SH + KH - 1, likewise ow.
        const int oh_lo = hp >= KH ? div_sh.div(hp - KH) + 1 : 0;
        const int oh_hi = min(OH - 1, div_sh.div(hp));
        const int ow_lo = wp >= KW ? div_sw.div(wp - KW) + 1 : 0;
        const int ow_hi = min(OW - 1, div_sw.div(wp));
        const float* image = gcT + n * n_stride + static_cast<long long>(ci) * KH * KW * f_stride;
        for (int oh = oh_lo; oh <= oh_hi; ++oh) {
            const int kh = hp - oh * SH;
            const float* row = image + kh * KW * f_stride + oh * OW;
            for (int ow = ow_lo; ow <= ow_hi; ++ow) {
                const int kw = wp - ow * SW;
                sum += row[kw * f_stride + ow];
            }
        }
    }
    dx[idx] = accumulate ? dx[idx] + sum : sum;
}

constexpr int TILE = 64;   // pixels x channels per transpose tile (one wave64 per row of the tile)
constexpr int TROWS = 4;   // waves per block; each thread covers TILE / TROWS tile rows

// rows (N*OHW, CO) -> y (N, CO, OHW), y = act(rows + bias). The transpose goes through a padded
// LDS tile so that the read (along CO) and the write (along OHW) are both coalesced. LeakyReLU is
// only fused for alpha > 0, so y > 0 exactly when the pre-activation is > 0 (the backward gate).
__global__ __launch_bounds__(TILE* TROWS) void conv_epilogue_kernel(const float* __restrict__ rows,
                                                                    const float* __restrict__ bias,
                                                                    float* __restrict__ y, int OHW, int CO, int act,
                                                                    float alpha) {
    __shared__ float tile[TILE][TILE + 1];
    const int n = blockIdx.z, p0 = blockIdx.x * TILE, c0 = blockIdx.y * TILE;
    const int tx = threadIdx.x, ty = threadIdx.y;
    const float* src = rows + static_cast<long long>(n) * OHW * CO;
    float* dst = y + static_cast<long long>(n) * CO * OHW;
#pragma unroll
    for (int j = ty; j < TILE; j += TROWS) {
        const int p = p0 + j, c = c0 + tx;
        if (p < OHW && c < CO) tile[tx][j] = src[p * CO + c];
    }
    __syncthreads();
#pragma unroll
    for (int j = ty; j < TILE; j += TROWS) {
        const int c = c0 + j, p = p0 + tx;
        if (p < OHW && c < CO) {
            float v = tile[j][tx];
            if (bias) v += bias[c];
            if (act == ACT_RELU) v = v < 0.0f ? 0.0f : v;  // NaN stays NaN, like max(0, v) in NumPy
            else if (act == ACT_LEAKY_RELU) v = v > 0.0f ? v : alpha * v;
            dst[c * OHW + p] = v;
        }
    }
}

// dy (N, CO, OHW) -> dyT (N*OHW, CO), gated by the fused activation through the forward output y,
// plus per-channel FP64 sums of the gated dy. Block (bx, by, n) walks the pixel tiles bx,
// bx + gridDim.x, ... in order; each thread sums its tile rows in FP64 and the 64 lanes of a wave
// combine with a fixed butterfly, so partial[(n * gridDim.x + bx) * CO + c] is reproducible.
__global__ __launch_bounds__(TILE* TROWS) void conv_grad_rows_kernel(const float* __restrict__ dy,
                                                                     const float* __restrict__ gate_y,
                                                                     float* __restrict__ dyT,
                                                                     double* __restrict__ partial, int OHW, int CO,
                                                                     int act, float alpha) {
    __shared__ float tile[TILE][TILE + 1];
    const int n = blockIdx.z, c0 = blockIdx.y * TILE;
    const int tx = threadIdx.x, ty = threadIdx.y;
    const long long image = static_cast<long long>(n) * CO * OHW;
    const float* src = dy + image;
    const float* gate = gate_y ? gate_y + image : nullptr;
    float* dst = dyT ? dyT + static_cast<long long>(n) * OHW * CO : nullptr;
    double acc[TILE / TROWS];
#pragma unroll
    for (int k = 0; k < TILE / TROWS; ++k) acc[k] = 0.0;
    for (int p0 = blockIdx.x * TILE; p0 < OHW; p0 += gridDim.x * TILE) {
#pragma unroll
        for (int k = 0; k < TILE / TROWS; ++k) {
            const int c = c0 + ty + k * TROWS, p = p0 + tx;
            float v = 0.0f;
            if (p < OHW && c < CO) {
                const int at = c * OHW + p;
                v = src[at];
                if (act == ACT_RELU) v = gate[at] > 0.0f ? v : 0.0f;
                else if (act == ACT_LEAKY_RELU) v = gate[at] > 0.0f ? v : alpha * v;
            }
            tile[ty + k * TROWS][tx] = v;
            acc[k] += static_cast<double>(v);
        }
        __syncthreads();
        if (dst) {
#pragma unroll
            for (int k = 0; k < TILE / TROWS; ++k) {
                const int p = p0 + ty + k * TROWS, c = c0 + tx;
                if (p < OHW && c < CO) dst[p * CO + c] = tile[tx][ty + k * TROWS];
            }
        }
        __syncthreads();
    }
    if (!partial) return;
#pragma unroll
    for (int k = 0; k < TILE / TROWS; ++k) {
        double s = acc[k];
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) s += __shfl_xor(s, offset, 64);
        const int c = c0 + ty + k * TROWS;
        if (tx == 0 && c < CO) partial[(static_cast<long long>(n) * gridDim.x + blockIdx.x) * CO + c] = s;
    }
}

constexpr int RP_COLS = 16, RP_LANES = 16;  // columns per workgroup, row lanes per column

// out[i] = (float) sum_{j = 0..count-1} partial[j * width + i] in FP64, in a fixed order: lane r of
// column i sums the rows j = r, r + 16, r + 32, ... in increasing j, then the 16 lane sums are added
// in lane order. Deterministic, and with 16 independent chains per column the loads overlap.
__global__ __launch_bounds__(RP_COLS* RP_LANES) void reduce_partials_kernel(const double* __restrict__ partial,
                                                                            float* __restrict__ out, int count,
                                                                            int width) {
    __shared__ double lane_sum[RP_LANES][RP_COLS];
    const int c = threadIdx.x % RP_COLS, r = threadIdx.x / RP_COLS;
    const int i = blockIdx.x * RP_COLS + c;
    double s = 0.0;
    if (i < width)
        for (int j = r; j < count; j += RP_LANES) s += partial[static_cast<long long>(j) * width + i];
    lane_sum[r][c] = s;
    __syncthreads();
    if (r == 0 && i < width) {
        double total = 0.0;
#pragma unroll
        for (int k = 0; k < RP_LANES; ++k) total += lane_sum[k][c];
        out[i] = static_cast<float>(total);
    }
}

__global__ __launch_bounds__(256) void add_bias_kernel(float* __restrict__ rows, const float* __restrict__ bias,
                                                       int total, FastDiv div_n) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    int col;
    div_n.divmod(idx, col);
    rows[idx] += bias[col];
}

// Window maximum in (kh, kw) row-major order with a strict '>' (the first maximum wins ties); a NaN
// takes over, so any NaN in the window gives a NaN output. argmax (optional: null when no backward
// will read it) is the flat index into x.
__global__ __launch_bounds__(256) void pool_forward_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                           int* __restrict__ argmax, int total, FastDiv div_ow,
                                                           FastDiv div_oh, int H, int W, int KH, int KW, int SH,
                                                           int SW) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    int ow, oh;
    const int t = div_ow.divmod(idx, ow);
    const int nc = div_oh.divmod(t, oh);
    const int first = (nc * H + oh * SH) * W + ow * SW;
    int best = first;
    float value = x[first];
    for (int kh = 0; kh < KH; ++kh) {
        const float* row = x + first + kh * W;
        for (int kw = 0; kw < KW; ++kw) {
            const float v = row[kw];
            if (v > value || v != v) {
                value = v;
                best = first + kh * W + kw;
            }
        }
    }
    y[idx] = value;
    if (argmax) argmax[idx] = best;
}

// dx[i] = sum of dy over the windows (visited in increasing oh, ow order) whose argmax is i.
__global__ __launch_bounds__(256) void pool_backward_kernel(const float* __restrict__ dy,
                                                            const int* __restrict__ argmax, float* __restrict__ dx,
                                                            int total, FastDiv div_w, FastDiv div_h, int OH, int OW,
                                                            int KH, int KW, FastDiv div_sh, FastDiv div_sw) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    int iw, ih;
    const int t = div_w.divmod(idx, iw);
    const int nc = div_h.divmod(t, ih);
    const int oh_lo = ih >= KH ? div_sh.div(ih - KH) + 1 : 0;
    const int oh_hi = min(OH - 1, div_sh.div(ih));
    const int ow_lo = iw >= KW ? div_sw.div(iw - KW) + 1 : 0;
    const int ow_hi = min(OW - 1, div_sw.div(iw));
    float sum = 0.0f;
    for (int oh = oh_lo; oh <= oh_hi; ++oh)
        for (int ow = ow_lo; ow <= ow_hi; ++ow) {
            const int out = (nc * OH + oh) * OW + ow;
            if (argmax[out] == idx) sum += dy[out];
        }
    dx[idx] = sum;
}

constexpr int PLANE_FLOATS = 16384;   // floats of one workgroup's LDS plane buffer (64 KB)
constexpr int ROW_AHEAD = 8;          // the span kernel's global loads per thread in flight while it stages
constexpr long long SPAN_RUNS = 4096;  // runs of output pixels the im2col span kernel aims for
constexpr int SPAN_AHEAD = 8;           // band floats per thread the span kernel reads ahead
constexpr int SPAN_PER_CU = 4;          // resident span workgroups per CU
constexpr long long SPAN_LDS_FLOATS = 16384;  // the span kernel's LDS (band and feature offsets, 64 KB)

// Workgroups are handed to the 8 XCDs of an MI355X round-robin by id, and each XCD has its own L2.
// Renumbering workgroup b of `total` gives XCD x one contiguous run of logical ids, so that the
// workgroups one XCD runs together are neighbours and meet in its L2 on the data they share.
__device__ __forceinline__ int xcd_contiguous(int b, int total) {
    constexpr int XCDS = 8;
    const int xcd = b % XCDS, position = b / XCDS;
    const int base = total / XCDS, extra = total % XCDS;
    return xcd * base + min(xcd, extra) + position;
}

// im2col in runs of `span` output pixels (n, oh, ow0 .. ow0 + span - 1), `items` runs in all, taken
// by a grid of resident workgroups in turn (workgroup L takes runs L, L + gridDim.x, ...). A run's
// input band (KH rows x bw = (span - 1) * SW + KW columns for every channel, padding as zeros) is
// staged in LDS; then the span x K block of cols that the run owns (contiguous in memory) is
// written in order, with no bounds tests: feature f of pixel p is band[offset[f] + p * SW], the
// offsets (ci * KH + kh) * bw + kw of the K features held in LDS too, so the writes decompose no
// index (four features per 16-byte store when K % 4 == 0). The first SPAN_AHEAD * 256 entries of
// the next run's band are read into registers before the current run is written, so the reads of
// one run overlap the writes of the other.
template <bool VEC>
__global__ __launch_bounds__(256) void im2col_span_kernel(const float* __restrict__ x, float* __restrict__ cols,
                                                          int CI, int H, int W, int KH, int KW, int OH, int OW, int SH,
                                                          int SW, int PH, int PW, int span, int bw, int items,
                                                          FastDiv div_k, FastDiv div_khkw, FastDiv div_kw,
                                                          FastDiv div_kh, FastDiv div_bw, FastDiv div_runs,
                                                          FastDiv div_oh) {
    extern __shared__ float band[];  // CI * KH * bw floats, then (16-byte aligned) the K feature offsets
    const int entries = CI * KH * bw, K = CI * KH * KW;
    int* offset = reinterpret_cast<int*>(band + (entries + 3) / 4 * 4);
    for (int f = threadIdx.x; f < K; f += 256) {
        int tap, kw;
        const int ci = div_khkw.divmod(f, tap);
        const int kh = div_kw.divmod(tap, kw);
        offset[f] = (ci * KH + kh) * bw + kw;
    }
    struct Run {
        const float* image;
        float* out;
        int ih0, iw0, pixels;
    };
    auto run_of = [&](int item) {
        int run, oh;
        const int n = div_oh.divmod(div_runs.divmod(item, run), oh);
        const int ow0 = run * span;
        return Run{x + static_cast<long long>(n) * CI * H * W, cols + ((static_cast<long long>(n) * OH + oh) * OW + ow0) * K,
                   oh * SH - PH, ow0 * SW - PW, min(span, OW - ow0)};
    };
    auto input = [&](const Run& r, int e) {
        int col, kh;
        const int ci = div_kh.divmod(div_bw.divmod(e, col), kh);  // band row ci * KH + kh
        const int ih = r.ih0 + kh, iw = r.iw0 + col;
        return static_cast<unsigned>(ih) < static_cast<unsigned>(H) && static_cast<unsigned>(iw) < static_cast<unsigned>(W)
                   ? r.image[(ci * H + ih) * W + iw]
                   : 0.0f;
    };
    float ahead[SPAN_AHEAD];
    auto read_ahead = [&](const Run& r) {
#pragma unroll
        for (int u = 0; u < SPAN_AHEAD; ++u) {
            const int e = threadIdx.x + u * 256;
            ahead[u] = e < entries ? input(r, e) : 0.0f;
        }
    };
    // Consecutive workgroups of one XCD take consecutive runs, which read input rows in common.
    int item = xcd_contiguous(blockIdx.x, gridDim.x);
    if (item >= items) return;
    Run r = run_of(item);
    read_ahead(r);
    constexpr int STEP = VEC ? 4 * 256 : 256;  // floats of cols a workgroup writes per round
    const int step_pixels = div_k.div(STEP), step_features = STEP - step_pixels * K;
    for (;;) {
#pragma unroll
        for (int u = 0; u < SPAN_AHEAD; ++u) {
            const int e = threadIdx.x + u * 256;
            if (e < entries) band[e] = ahead[u];
        }
        for (int e = threadIdx.x + SPAN_AHEAD * 256; e < entries; e += 256) band[e] = input(r, e);
        __syncthreads();
        const int next_item = item + gridDim.x;
        const bool more = next_item < items;
        Run next{};
        if (more) {
            next = run_of(next_item);
            read_ahead(next);
        }
        // Element j = p * K + f of the run's block; j advances by STEP, (p, f) with it.
        const int count = r.pixels * K;
        int j = VEC ? 4 * threadIdx.x : threadIdx.x, f;
        int p = div_k.divmod(j, f);
        for (; j < count; j += STEP) {
            const int base = p * SW;
            if constexpr (VEC) {
                const int4 o = *reinterpret_cast<const int4*>(offset + f);
                *reinterpret_cast<float4*>(r.out + j) =
                    make_float4(band[o.x + base], band[o.y + base], band[o.z + base], band[o.w + base]);
            } else {
                r.out[j] = band[offset[f] + base];
            }
            f += step_features;
            p += step_pixels;
            if (f >= K) {
                f -= K;
                ++p;
            }
        }
        __syncthreads();  // every read of the band is done before the next run overwrites it
        if (!more) break;
        item = next_item;
        r = next;
    }
}

constexpr int STAGE_AHEAD = 4;  // global loads per thread in flight while planes are staged in LDS

// Max-pool forward over `per` consecutive (n, c) planes per workgroup, each staged whole in LDS with
// coalesced reads; the window rule is pool_forward_kernel's.
__global__ __launch_bounds__(256) void pool_forward_plane_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                 int* __restrict__ argmax, int planes, int per, int H,
                                                                 int W, int OH, int OW, int KH, int KW, int SH, int SW,
                                                                 FastDiv div_ohw, FastDiv div_ow, int vec) {
    extern __shared__ float tile[];  // per * H * W floats
    const int first_plane = blockIdx.x * per;
    const int count = min(per, planes - first_plane);
    const int hw = H * W, ohw = OH * OW;
    const long long base = static_cast<long long>(first_plane) * hw;
    const int elems = count * hw;
    // The copy keeps STAGE_AHEAD loads per thread in flight: at most three 49 KB planes fit a CU's
    // LDS, too few waves to cover HBM latency one load at a time.
    if (vec) {  // x is 16-byte aligned and H*W % 4 == 0: every plane starts aligned, copy in float4s
        const float4* src = reinterpret_cast<const float4*>(x + base);
        float4* dst = reinterpret_cast<float4*>(tile);
        const int quads = elems / 4;
        int q = threadIdx.x;
        for (; q + (STAGE_AHEAD - 1) * 256 < quads; q += STAGE_AHEAD * 256) {
            float4 v[STAGE_AHEAD];
#pragma unroll
            for (int u = 0; u < STAGE_AHEAD; ++u) v[u] = src[q + u * 256];
#pragma unroll
            for (int u = 0; u < STAGE_AHEAD; ++u) dst[q + u * 256] = v[u];
        }
        for (; q < quads; q += 256) dst[q] = src[q];
    } else {
        int e = threadIdx.x;
        for (; e + (STAGE_AHEAD - 1) * 256 < elems; e += STAGE_AHEAD * 256) {
            float v[STAGE_AHEAD];
#pragma unroll
            for (int u = 0; u < STAGE_AHEAD; ++u) v[u] = x[base + e + u * 256];
#pragma unroll
            for (int u = 0; u < STAGE_AHEAD; ++u) tile[e + u * 256] = v[u];
        }
        for (; e < elems; e += 256) tile[e] = x[base + e];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < count * ohw; o += 256) {
        int within, ow;
        const int pl = div_ohw.divmod(o, within);
        const int oh = div_ow.divmod(within, ow);
        const int first = pl * hw + oh * SH * W + ow * SW;  // LDS index of the window's first element
        int best;
        const float value = window_max(tile, first, W, KH, KW, best);
        const long long out = static_cast<long long>(first_plane) * ohw + o;
        __builtin_nontemporal_store(value, y + out);
        if (argmax) __builtin_nontemporal_store(static_cast<int>(base + best), argmax + out);
    }
}

// 2x2 windows at stride 2 that tile the planes exactly (H = 2*OH, W = 2*OW, W a multiple of 4): each
// input pixel lies in one window, so no plane is staged. Thread q takes output row r = q / (W/4)
// (over all planes: input rows 2r and 2r + 1) and the output pair (2j, 2j + 1), j = q % (W/4): two
// float4 reads of columns 4j .. 4j + 3, the two windows scanned in window_max's (kh, kw) order with
// its comparison, so the values and indices are the staged kernels' bits.
__device__ __forceinline__ void window_take(float v, int at, float& value, int& best) {
    if (v > value || v != v) {
        value = v;
        best = at;
    }
}

__global__ __launch_bounds__(256) void pool_forward_2x2_kernel(const float4* __restrict__ x, float2* __restrict__ y,
                                                               int2* __restrict__ argmax, int total, FastDiv div_quads,
                                                               int quads) {
    const int q = blockIdx.x * 256 + threadIdx.x;
    if (q >= total) return;
    const int r = div_quads.div(q);
    const int top = q + r * quads;  // float4 index of columns 4j .. 4j+3 of input row 2r
    const float4 a = x[top], b = x[top + quads];
    const int at = 4 * top, below = 4 * (top + quads);
    float v0 = a.x, v1 = a.z;
    int i0 = at, i1 = at + 2;
    window_take(a.x, at, v0, i0);
    window_take(a.y, at + 1, v0, i0);
    window_take(b.x, below, v0, i0);
    window_take(b.y, below + 1, v0, i0);
    window_take(a.z, at + 2, v1, i1);
    window_take(a.w, at + 3, v1, i1);
    window_take(b.z, below + 2, v1, i1);
    window_take(b.w, below + 3, v1, i1);
    y[q] = make_float2(v0, v1);
    if (argmax) argmax[q] = make_int2(i0, i1);
}

// Its backward: every input pixel takes 0 + the dy of its window when the window's argmax is that
// pixel (the one window pool_pixel_grad would visit for it), else 0.
__global__ __launch_bounds__(256) void pool_backward_2x2_kernel(const float2* __restrict__ dy,
                                                                const int2* __restrict__ argmax,
                                                                float* __restrict__ dx, int total, FastDiv div_quads,
                                                                int quads) {
    const int q = blockIdx.x * 256 + threadIdx.x;
    if (q >= total) return;
    const int r = div_quads.div(q);
    const int top = q + r * quads;
    const float2 g = dy[q];
    const int2 w = argmax[q];
    const int at = 4 * top, below = 4 * (top + quads);
    auto pick = [](int where, int target, float grad) { return where == target ? 0.0f + grad : 0.0f; };
    store_streaming4(dx + at, pick(w.x, at, g.x), pick(w.x, at + 1, g.x), pick(w.y, at + 2, g.y),
                     pick(w.y, at + 3, g.y));
    store_streaming4(dx + below, pick(w.x, below, g.x), pick(w.x, below + 1, g.x), pick(w.y, below + 2, g.y),
                     pick(w.y, below + 3, g.y));
}

// Whether a pool takes the 2x2 kernels above: the window shape and stride, planes they tile exactly,
// and the alignment of their vector accesses.
bool pool_tiles_2x2(const void* x, const void* y, const void* argmax, int H, int W, int OH, int OW, int KH, int KW,
                    int SH, int SW) {
    const auto aligned = [](const void* p, std::uintptr_t bytes) {
        return (reinterpret_cast<std::uintptr_t>(p) & (bytes - 1)) == 0;
    };
    return KH == 2 && KW == 2 && SH == 2 && SW == 2 && H == 2 * OH && W == 2 * OW && W % 4 == 0 && aligned(x, 16) &&
           aligned(y, 8) && aligned(argmax, 8);
}

// Max-pool backward over `per` consecutive planes per workgroup: the planes' dy and argmax are
// staged in LDS, then every input pixel gathers the windows that cover it, in (oh, ow) order.
// div_plane and div_row divide by the units of a plane and of a row: pixels (H*W, W), or under VEC4
// (W a multiple of 4, dx 16-byte aligned) blocks of two rows by four columns ((H+1)/2 * W/4, W/4),
// whose gradients a thread forms together and writes with two non-temporal 16-byte stores.
template <bool VEC4>
__global__ __launch_bounds__(256) void pool_backward_plane_kernel(const float* __restrict__ dy,
                                                                  const int* __restrict__ argmax,
                                                                  float* __restrict__ dx, int planes, int per, int H,
                                                                  int W, int OH, int OW, int KH, int KW,
                                                                  FastDiv div_plane, FastDiv div_row, FastDiv div_sh,
                                                                  FastDiv div_sw) {
    extern __shared__ float staged[];  // per * OH * OW floats of dy, then as many int32 argmax
    const int first_plane = blockIdx.x * per;
    const int count = min(per, planes - first_plane);
    const int hw = H * W, ohw = OH * OW;
    float* grad = staged;
    int* where = reinterpret_cast<int*>(staged + per * ohw);
    const long long out_base = static_cast<long long>(first_plane) * ohw;
    const int staged_count = count * ohw;
    int o = threadIdx.x;
    for (; o + (STAGE_AHEAD - 1) * 256 < staged_count; o += STAGE_AHEAD * 256) {
        float g[STAGE_AHEAD];
        int a[STAGE_AHEAD];
#pragma unroll
        for (int u = 0; u < STAGE_AHEAD; ++u) {
            g[u] = dy[out_base + o + u * 256];
            a[u] = argmax[out_base + o + u * 256];
        }
#pragma unroll
        for (int u = 0; u < STAGE_AHEAD; ++u) {
            grad[o + u * 256] = g[u];
            where[o + u * 256] = a[u];
        }
    }
    for (; o < staged_count; o += 256) {
        grad[o] = dy[out_base + o];
        where[o] = argmax[out_base + o];
    }
    __syncthreads();
    const long long in_base = static_cast<long long>(first_plane) * hw;
    if constexpr (VEC4) {
        const int blocks = count * static_cast<int>(div_plane.d);
        for (int b = threadIdx.x; b < blocks; b += 256) {
            int within, col;
            const int pl = div_plane.divmod(b, within);
            const int ih = 2 * div_row.divmod(within, col);
            const int iw = 4 * col;
            const int rows = min(2, H - ih);
            const int target = static_cast<int>(in_base) + pl * hw + ih * W + iw;
            float sum[2][4];
            pool_rows_grad<2>(grad, where, pl, ih, rows, iw, target, W, OH, OW, KH, KW, div_sh, div_sw, sum);
            store_streaming4(dx + target, sum[0][0], sum[0][1], sum[0][2], sum[0][3]);
            if (rows > 1) store_streaming4(dx + target + W, sum[1][0], sum[1][1], sum[1][2], sum[1][3]);
        }
    } else {
        for (int e = threadIdx.x; e < count * hw; e += 256) {
            int within, iw;
            const int pl = div_plane.divmod(e, within);
            const int ih = div_row.divmod(within, iw);
            dx[in_base + e] = pool_pixel_grad(grad, where, pl, ih, iw, static_cast<int>(in_base + e), OH, OW, KH, KW,
                                              div_sh, div_sw);
        }
    }
}

}  // namespace

int launch_im2col(const float* x, float* cols, const ConvGeometry& g, hipStream_t stream) {
    const int K = g.features();
    const int total = g.rows() * K;
    // Runs of output pixels: several per resident workgroup (about SPAN_RUNS in all), each run's
    // band and the feature offsets within SPAN_LDS_FLOATS.
    const long long rows = static_cast<long long>(g.N) * g.OH;
    int runs = static_cast<int>(std::min<long long>(g.OW, std::max<long long>(1, (SPAN_RUNS + rows - 1) / rows)));
    int span = (g.OW + runs - 1) / runs;
    // LDS floats of a run of s pixels: its band, rounded up to whole 16 bytes, and the feature offsets.
    auto band_of = [&](int s) { return (static_cast<long long>(g.CI) * g.KH * ((s - 1) * g.SW + g.KW) + 3) / 4 * 4; };
    while (span > 1 && band_of(span) + K > SPAN_LDS_FLOATS) span = (span + 1) / 2;
    runs = (g.OW + span - 1) / span;
    if (band_of(span) + K <= SPAN_LDS_FLOATS && rows * runs <= INDEX_LIMIT) {
        const bool vec = K % 4 == 0 && (reinterpret_cast<std::uintptr_t>(cols) & 15) == 0;
        const int items = static_cast<int>(rows * runs);
        const unsigned blocks =
            static_cast<unsigned>(std::min<long long>(items, SPAN_PER_CU * std::max(1, device_cu_count())));
        const int bw = (span - 1) * g.SW + g.KW;
        const FastDiv dk(K), dkk(g.KH * g.KW), dkw(g.KW), dkh(g.KH), dbw(bw), druns(runs), doh(g.OH);
        const size_t lds = static_cast<size_t>(band_of(span) + K) * sizeof(float);
        if (vec)
            launch(im2col_span_kernel<true>, blocks, 256, lds, stream, x, cols, g.CI, g.H, g.W, g.KH, g.KW, g.OH, g.OW,
                   g.SH, g.SW, g.PH, g.PW, span, bw, items, dk, dkk, dkw, dkh, dbw, druns, doh);
        else
            launch(im2col_span_kernel<false>, blocks, 256, lds, stream, x, cols, g.CI, g.H, g.W, g.KH, g.KW, g.OH, g.OW,
                   g.SH, g.SW, g.PH, g.PW, span, bw, items, dk, dkk, dkw, dkh, dbw, druns, doh);
        return MFH_CHECK_LAUNCH("im2col_span", stream);
    }
    if (K % 4 == 0 && (reinterpret_cast<std::uintptr_t>(cols) & 15) == 0) {
        const int quads = total / 4;
        launch(im2col_vec4_kernel, blocks_for(quads, 256), 256, 0, stream, x, cols, quads, FastDiv(K), FastDiv(g.KW), FastDiv(g.KH), FastDiv(g.OW), FastDiv(g.OH), g.CI, g.KH, g.KW,
            g.H, g.W, g.SH, g.SW, g.PH, g.PW);
        return MFH_CHECK_LAUNCH("im2col_vec4", stream);
    }
    launch(im2col_kernel, blocks_for(total, 256), 256, 0, stream, x, cols, total, FastDiv(K), FastDiv(g.KW),
                                                                FastDiv(g.KH), FastDiv(g.OW), FastDiv(g.OH), g.CI,
                                                                g.H, g.W, g.SH, g.SW, g.PH, g.PW);
    return MFH_CHECK_LAUNCH("im2col", stream);
}

int launch_col2im_t(const float* gcT, float* dx, const ConvGeometry& g, bool per_image, bool accumulate,
                    hipStream_t stream) {
    const int total = g.N * g.CI * g.H * g.W;
    const long long ohw = g.ohw();
    const long long f_stride = per_image ? ohw : static_cast<long long>(g.rows());
    const long long n_stride = per_image ? ohw * g.features() : ohw;
    auto kernel = col2im_t_kernel<0, 0, 0, 0>;
    if (g.KH == 3 && g.KW == 3 && g.SH == 1 && g.SW == 1) kernel = col2im_t_kernel<3, 3, 1, 1>;
    else if (g.KH == 3 && g.KW == 3 && g.SH == 2 && g.SW == 2) kernel = col2im_t_kernel<3, 3, 2, 2>;
    launch(kernel, blocks_for(total, 256), 256, 0, stream, gcT, dx, total, FastDiv(g.W), FastDiv(g.H), FastDiv(g.CI),
           g.CI, g.KH, g.KW, g.OH, g.OW, g.SH, g.SW, FastDiv(g.SH), FastDiv(g.SW), g.PH, g.PW, f_stride, n_stride,
           accumulate ? 1 : 0);
    return MFH_CHECK_LAUNCH("col2im_t", stream);
}

int launch_conv_epilogue(const float* rows, const float* bias, float* y, int N, int OHW, int CO, int act,
                         float alpha, hipStream_t stream) {
    const dim3 grid(blocks_for(OHW, TILE), blocks_for(CO, TILE), N), block(TILE, TROWS);
    launch(conv_epilogue_kernel, grid, block, 0, stream, rows, bias, y, OHW, CO, act, alpha);
    return MFH_CHECK_LAUNCH("conv_epilogue", stream);
}

int conv_grad_tile() { return TILE; }

int launch_conv_grad_rows(const float* dy, const float* y, float* dyT, double* partial, int N, int OHW, int CO,
                          int grid_x, int act, float alpha, hipStream_t stream) {
    const dim3 grid(grid_x, blocks_for(CO, TILE), N), block(TILE, TROWS);
    launch(conv_grad_rows_kernel, grid, block, 0, stream, dy, y, dyT, partial, OHW, CO, act, alpha);
    return MFH_CHECK_LAUNCH("conv_grad_rows", stream);
}

int launch_reduce_partials(const double* partial, float* out, int count, int width, hipStream_t stream) {
    launch(reduce_partials_kernel, blocks_for(width, RP_COLS), RP_COLS * RP_LANES, 0, stream, partial, out, count, width);
    return MFH_CHECK_LAUNCH("reduce_partials", stream);
}

int launch_add_bias(float* rows, const float* bias, int M, int N, hipStream_t stream) {
    const int total = M * N;
    launch(add_bias_kernel, blocks_for(total, 256), 256, 0, stream, rows, bias, total, FastDiv(N));
    return MFH_CHECK_LAUNCH("add_bias", stream);
}

// Planes per workgroup for the LDS pooling kernels: about 2048 elements of work each, within the
// LDS plane buffer; 0 when one plane does not fit.
int pool_planes_per_block(int plane_floats, int capacity) {
    if (plane_floats > capacity) return 0;
    return std::max(1, std::min(2048 / plane_floats, capacity / plane_floats));
}

int launch_pool_forward(const float* x, float* y, int* argmax, int N, int C, int H, int W, int OH, int OW, int KH,
                        int KW, int SH, int SW, hipStream_t stream) {
    const int total = N * C * OH * OW;
    if (pool_tiles_2x2(x, y, argmax, H, W, OH, OW, KH, KW, SH, SW)) {
        const int quads = W / 4;
        launch(pool_forward_2x2_kernel, blocks_for(total / 2, 256), 256, 0, stream,
               reinterpret_cast<const float4*>(x), reinterpret_cast<float2*>(y), reinterpret_cast<int2*>(argmax),
               total / 2, FastDiv(quads), quads);
        return MFH_CHECK_LAUNCH("pool_forward_2x2", stream);
    }
    const int per = pool_planes_per_block(H * W, PLANE_FLOATS);
    if (per > 0) {
        const int planes = N * C;
        const size_t lds = static_cast<size_t>(per) * H * W * sizeof(float);
        launch(pool_forward_plane_kernel, blocks_for(planes, per), 256, lds, stream, x, y, argmax, planes, per, H, W, OH, OW, KH, KW, SH, SW, FastDiv(OH * OW), FastDiv(OW),
            (H * W) % 4 == 0 && (reinterpret_cast<std::uintptr_t>(x) & 15) == 0 ? 1 : 0);
        return MFH_CHECK_LAUNCH("pool_forward_plane", stream);
    }
    launch(pool_forward_kernel, blocks_for(total, 256), 256, 0, stream, x, y, argmax, total, FastDiv(OW), FastDiv(OH), H,
                                                                      W, KH, KW, SH, SW);
    return MFH_CHECK_LAUNCH("pool_forward", stream);
}

int launch_pool_backward(const float* dy, const int* argmax, float* dx, int N, int C, int H, int W, int OH, int OW,
                         int KH, int KW, int SH, int SW, hipStream_t stream) {
    const int total = N * C * H * W;
    if (pool_tiles_2x2(dx, dy, argmax, H, W, OH, OW, KH, KW, SH, SW)) {
        const int quads = W / 4, pairs = N * C * OH * OW / 2;
        launch(pool_backward_2x2_kernel, blocks_for(pairs, 256), 256, 0, stream, reinterpret_cast<const float2*>(dy),
               reinterpret_cast<const int2*>(argmax), dx, pairs, FastDiv(quads), quads);
        return MFH_CHECK_LAUNCH("pool_backward_2x2", stream);
    }
    const int per = std::min(pool_planes_per_block(OH * OW, PLANE_FLOATS / 2),
                             pool_planes_per_block(H * W, 1 << 30));
    if (per > 0) {
        const int planes = N * C;
        const size_t lds = static_cast<size_t>(per) * OH * OW * 2 * sizeof(float);
        const bool vec4 = W % 4 == 0 && (reinterpret_cast<std::uintptr_t>(dx) & 15) == 0;
        const int per_row = vec4 ? W / 4 : W, per_plane = vec4 ? (H + 1) / 2 * per_row : H * W;
        launch((vec4 ? pool_backward_plane_kernel<true> : pool_backward_plane_kernel<false>), blocks_for(planes, per), 256,
                                                                                       lds, stream, dy, argmax, dx, planes, per, H, W, OH, OW, KH, KW, FastDiv(per_plane), FastDiv(per_row), FastDiv(SH),
            FastDiv(SW));
        return MFH_CHECK_LAUNCH("pool_backward_plane", stream);
    }
    launch(pool_backward_kernel, blocks_for(total, 256), 256, 0, stream, dy, argmax, dx, total, FastDiv(W), FastDiv(H),
                                                                       OH, OW, KH, KW, FastDiv(SH), FastDiv(SW));
    return MFH_CHECK_LAUNCH("pool_backward", stream);
}

int probe_code_object() {
    hipFuncAttributes attributes;
    const hipError_t status = hipFuncGetAttributes(&attributes, reinterpret_cast<const void*>(&im2col_kernel));
    if (status != hipSuccess)
        return MFH_FAIL(ERR_INIT, std::string("no usable gfx950 code object: ") + hipGetErrorString(status));
    return OK;
}

}  // namespace mfh
