// The max-pool window rules, shared by the pooling kernels (conv.hip) and the batch-norm kernels
// that pool their own output (norm.hip), so that both give the same values, indices and gradients.
#pragma once

#include "common.h"
#include "fastdiv.h"

namespace mfh {

// Window maximum over a KH x KW window of a plane staged in LDS (row length W), starting at LDS
// index `first`: the first element wins ties, a NaN wins over every number (the first NaN once one
// is found). `best` receives the LDS index of the winner. Follows native_cublas.cpp:360-376.
__device__ __forceinline__ float window_max(const float* tile, int first, int W, int KH, int KW, int& best) {
    best = first;
    float value = tile[first];
    for (int kh = 0; kh < KH; ++kh)
        for (int kw = 0; kw < KW; ++kw) {
            const float v = tile[first + kh * W + kw];
            if (v > value || v != v) {
                value = v;
                best = first + kh * W + kw;
            }
        }
    return value;
}

// The gradient of input pixel (ih, iw) of staged plane pl: the dy of every window that covers the
// pixel and whose argmax (a flat index, `target` for this pixel) is it, added in (oh, ow) order.
// Follows native_cublas.cpp:378-393.
__device__ __forceinline__ float pool_pixel_grad(const float* grad, const int* where, int pl, int ih, int iw,
                                                 int target, int OH, int OW, int KH, int KW, const FastDiv& div_sh,
                                                 const FastDiv& div_sw) {
    const int ohw = OH * OW;
    const int oh_lo = ih >= KH ? div_sh.div(ih - KH) + 1 : 0;
    const int oh_hi = min(OH - 1, div_sh.div(ih));
    const int ow_lo = iw >= KW ? div_sw.div(iw - KW) + 1 : 0;
    const int ow_hi = min(OW - 1, div_sw.div(iw));
    float sum = 0.0f;
    for (int oh = oh_lo; oh <= oh_hi; ++oh)
        for (int ow = ow_lo; ow <= ow_hi; ++ow) {
            const int o = pl * ohw + oh * OW + ow;
            if (where[o] == target) sum += grad[o];
        }
    return sum;
}

// The gradients of four adjacent pixels (ih, iw .. iw + 3) of one row of staged plane pl, the first
// at flat index `target`: each window that covers any of them is visited once, in (oh, ow) order,
// and adds its dy to the one of the four pixels its argmax names (if any). Per pixel that is the
// windows of pool_pixel_grad in the same order, so the four sums are its bits; the window range
// and the LDS reads are shared by the four pixels.
__device__ __forceinline__ float4 pool_quad_grad(const float* grad, const int* where, int pl, int ih, int iw,
                                                 int target, int OH, int OW, int KH, int KW, const FastDiv& div_sh,
                                                 const FastDiv& div_sw) {
    const int ohw = OH * OW;
    const int oh_lo = ih >= KH ? div_sh.div(ih - KH) + 1 : 0;
    const int oh_hi = min(OH - 1, div_sh.div(ih));
    const int ow_lo = iw >= KW ? div_sw.div(iw - KW) + 1 : 0;
    const int ow_hi = min(OW - 1, div_sw.div(iw + 3));
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int oh = oh_lo; oh <= oh_hi; ++oh)
        for (int ow = ow_lo; ow <= ow_hi; ++ow) {
            const int o = pl * ohw + oh * OW + ow;
            const unsigned u = static_cast<unsigned>(where[o] - target);
            if (u < 4u) {
                const float g = grad[o];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (u == static_cast<unsigned>(k)) sum[k] += g;
            }
        }
    return make_float4(sum[0], sum[1], sum[2], sum[3]);
}

// A 16-byte store marked non-temporal: the line goes out to memory without displacing what the
// caches hold for the rest of the kernel (a pass's output that the pass itself never reads).
__device__ __forceinline__ void store_streaming4(float* p, float a, float b, float c, float d) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    const v4f v = {a, b, c, d};
    __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(p));
}

// The gradients of a block of `rows` (at most R) rows by four columns of staged plane pl: rows ih ..
// ih + rows - 1, columns iw .. iw + 3, pixel (ih, iw) at flat index `target`. Every window that covers
// any of them is visited once, in (oh, ow) order; a window whose argmax names a pixel of the block
// covers that pixel, so per pixel the visits that add are pool_pixel_grad's windows in its order and
// the sums are its bits. Rows ih and ih + 1 of a 3x3 stride-2 pool share two of their three window
// rows, so a two-row block reads 6 windows for 8 pixels where two quads read 9.
template <int R>
__device__ __forceinline__ void pool_rows_grad(const float* grad, const int* where, int pl, int ih, int rows, int iw,
                                               int target, int W, int OH, int OW, int KH, int KW,
                                               const FastDiv& div_sh, const FastDiv& div_sw, float (&sum)[R][4]) {
    const int ohw = OH * OW;
    const int oh_lo = ih >= KH ? div_sh.div(ih - KH) + 1 : 0;
    const int oh_hi = min(OH - 1, div_sh.div(ih + rows - 1));
    const int ow_lo = iw >= KW ? div_sw.div(iw - KW) + 1 : 0;
    const int ow_hi = min(OW - 1, div_sw.div(iw + 3));
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int k = 0; k < 4; ++k) sum[r][k] = 0.0f;
    for (int oh = oh_lo; oh <= oh_hi; ++oh)
        for (int ow = ow_lo; ow <= ow_hi; ++ow) {
            const int o = pl * ohw + oh * OW + ow;
            const int d = where[o] - target;
            const float g = grad[o];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const unsigned u = static_cast<unsigned>(d - r * W);
                if (u < 4u) {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (u == static_cast<unsigned>(k)) sum[r][k] += g;
                }
            }
        }
}

}  // namespace mfh
