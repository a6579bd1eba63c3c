// Implicit-GEMM convolution: the im2col matrix is never written to HBM. The GEMM's operand loads
// gather it from the NCHW tensor instead, so a convolution reads its input once from HBM (the 9x
// reuse of a 3x3 window is served by L2/L1) instead of writing and re-reading an M x K matrix.
//
// The gathered view. For an NCHW source of C channels and H x W pixels, a KH x KW window with stride
// (SH, SW) and padding (PH, PW), and an OH x OW output grid:
//   view[k][q] = src[n, c, oh*SH - PH + kh, ow*SW - PW + kw]   (0 outside the source)
// with feature k = (c*KH + kh)*KW + kw and output pixel q = (n*OH + oh)*OW + ow. This is the
// transpose of the im2col matrix of conv.hip, element for element.
//
// The three products of a convolution (M = N*OH*OW pixels, K = CI*KH*KW features):
//   * forward:  Y (CO x M) = W (CO x K) . view (K x M), stored into NCHW y by the segmented
//     epilogue with the bias per row and the activation fused;
//   * dW:       dW (CO x K) = dy (CO x M) . view^T (M x K), reduced over the pixels, usually split;
//     dy is read in place from NCHW (image n's rows are CO x OH*OW);
//   * dX (stride 1): a forward convolution of dy with the kernel flipped and transposed,
//     wflip[ci][co][kh][kw] = W[co][ci][KH-1-kh][KW-1-kw], padding KH-1-PH / KW-1-PW, written
//     straight into NCHW dx: no column gradient and no col2im pass.
// Feature order. When the source has a multiple of 32 channels the features are taken in chunked
// order k = ((c / 32)*KH*KW + tap)*32 + c % 32 (tap = kh*KW + kw), so a 32-deep stage of the
// forward product covers 32 channels at one window tap: the tap is decomposed once per stage (a
// scalar), each thread tests its pixel's window bounds once per stage and then reads 32/RSTEP
// channels at a fixed stride. The kernel is reordered to match by weight_order_kernel (with the
// dX flip folded in; one launch can reorder every kernel of a network), and dW's output columns
// are mapped back to natural order by the epilogue.
// Other channel counts (the 3-channel stem) take the natural order k = c*KH*KW + tap, decomposed
// per feature row (a wave-uniform scalar computation).
// Both gather loaders keep one pixel per thread column so that the pixel's decomposition
// (n, oh, ow) is done once per stage (dW) or once per kernel (forward).
#include <algorithm>
#include <type_traits>
#include <vector>

#include "common.h"
#include "gemm_core.h"

namespace mfh {
namespace {

constexpr int BK = 32;     // stage depth of the forward / dX products (one channel chunk)
constexpr int BK_WG = 16;  // stage depth of the dW products (a run of pixels)
constexpr int GROUPED_REDUCE_SLICES = 16;  // dW splits from which the partials take the grouped reduction
constexpr int FAR = -(1 << 24);  // window offset of a feature row past the end: every pixel is out of bounds

// Forward orientation: a BK x BN tile of the view, rows = features [kt, kt + BK), columns = pixels
// [n0, n0 + BN), stored mn-contiguous ([BK][BN + 4]). Thread t always loads pixel n0 + t % BN.
template <int BN, int THREADS>
struct GatherFeatureRows {
    static_assert(BN % 64 == 0 && THREADS % BN == 0, "each wave must read a single feature row");
    static constexpr int RSTEP = THREADS / BN, PER = BK / RSTEP;
    static_assert(BK % RSTEP == 0, "rows split evenly over the threads");
    int origin;  // offset of window position (0, 0) of this thread's pixel in src (may be negative)
    int ih0, iw0;
    bool valid;
    float v[PER];

    __device__ __forceinline__ void init(const ConvGather& g, int n0, int tid) {
        const int q = n0 + tid % BN;
        valid = q < g.pixels;
        int rem, ow;
        const int n = g.div_ohw.divmod(valid ? q : 0, rem);
        const int oh = g.div_ow.divmod(rem, ow);
        ih0 = oh * g.SH - g.PH;
        iw0 = ow * g.SW - g.PW;
        origin = n * g.chw + ih0 * g.W + iw0;
    }

    __device__ __forceinline__ void load(const ConvGather& g, int kt, int k_end, int tid) {
        const int r0 = tid / BN;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int k = __builtin_amdgcn_readfirstlane(kt + r0 + i * RSTEP);
            int rem, kw;
            const int c = g.div_khkw.divmod(k, rem);
            const int kh = g.div_kw.divmod(rem, kw);
            const int ih = ih0 + kh, iw = iw0 + kw;
            const bool ok = valid && k < k_end && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                            static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
            v[i] = ok ? g.src[origin + c * g.hw + kh * g.W + kw] : 0.0f;
        }
    }

    template <int LD>
    __device__ __forceinline__ void store(float* lds, int tid) const {
        const int r0 = tid / BN, col = tid % BN;
#pragma unroll
        for (int i = 0; i < PER; ++i) lds[(r0 + i * RSTEP) * LD + col] = v[i];
    }
};

// Most features a natural-order product may have to read its padded source (the LDS table of their
// offsets below).
constexpr int PADDED_TABLE_MAX = 1024;

// The natural-order tile read from the zero-padded copy of the source (ConvGather::padded) and stored
// pixel-major like GatherChunkRows' ([BN][BK + 4]): thread t takes pixel n0 + t % BN and the PER
// consecutive features (t / BN) * PER + i of the stage. The byte offset of every feature inside an
// image's padded planes is read from a table in LDS (PER / 4 16-byte reads per stage, the same
// address for a whole wave), so a load costs one add, with no window bounds test and no division. A feature
// past the last (table entry BUFFER_OOB), or a pixel past the last, reads zero; both at once read
// the tensor's first element, which only reaches an output column past the last pixel, never
// stored.
template <int BN, int THREADS>
struct GatherPaddedRows {
    static_assert(BN % 64 == 0 && THREADS % BN == 0, "each wave must read features of a single row group");
    static constexpr int RSTEP = THREADS / BN, PER = BK / RSTEP;
    static_assert(BK % RSTEP == 0 && PER % 4 == 0, "runs of whole float4s per thread");
    __amdgpu_buffer_rsrc_t rsrc;
    unsigned lane;  // byte offset of this thread's window origin in the padded source
    float v[PER];

    __device__ __forceinline__ void init(const ConvGather& g, int n0, int tid) {
        rsrc = buffer_of(g.padded, g.padded_floats);
        const int q = n0 + tid % BN;
        int rem, ow;
        const int n = g.div_ohw.divmod(q < g.pixels ? q : 0, rem);
        const int oh = g.div_ow.divmod(rem, ow);
        lane = q < g.pixels ? static_cast<unsigned>(n * g.C * g.phw + oh * g.SH * g.pw + ow * g.SW) * 4u : BUFFER_OOB;
    }

    __device__ __forceinline__ void load(const unsigned* table, int kt, int tid) {
        const unsigned* at = table + kt + (tid / BN) * PER;
#pragma unroll
        for (int q = 0; q < PER / 4; ++q) {
            const uint4 o = *reinterpret_cast<const uint4*>(at + 4 * q);
            v[4 * q] = buffer_load(rsrc, lane + o.x, 0);
            v[4 * q + 1] = buffer_load(rsrc, lane + o.y, 0);
            v[4 * q + 2] = buffer_load(rsrc, lane + o.z, 0);
            v[4 * q + 3] = buffer_load(rsrc, lane + o.w, 0);
        }
    }

    template <int LD>
    __device__ __forceinline__ void store(float* lds, int tid) const {
        float* row = lds + (tid % BN) * LD + (tid / BN) * PER;
#pragma unroll
        for (int q = 0; q < PER / 4; ++q)
            *reinterpret_cast<float4*>(row + 4 * q) = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    }
};

// The same tile in chunked feature order: stage kt covers channels [c0, c0 + 32) at one tap. The
// tap is uniform over the stage, so a wave may span two rows (BN a multiple of 32). The loads are
// buffer loads: a lane's offset is its pixel's window origin plus the stage's (uniform) channel
// chunk and tap, or BUFFER_OOB when the tap falls outside the image, and the PER channels of a
// thread (a contiguous run of the chunk) are one plane apart. A stage then costs a handful of vector
// instructions besides its loads, and the loads need no branches (the matrix cores and the vector
// ALU of a SIMD do not run at the same time, so every vector instruction of the loop is time the
// MFMAs lose). The tile is stored pixel-major ([BN][BK + 4]): a thread writes its channel run with
// 16-byte stores, and the MFMA loop reads four channels of a pixel with one 16-byte read, as it
// reads the kernel operand.
template <int BN, int THREADS>
struct GatherChunkRows {
    static_assert(BN % 32 == 0 && THREADS % BN == 0, "whole rows per thread group");
    static constexpr int RSTEP = THREADS / BN, PER = BK / RSTEP;
    static_assert(BK == CHANNEL_CHUNK && BK % RSTEP == 0 && PER % 4 == 0,
                  "one stage is one channel chunk, in runs of whole float4s per thread");
    __amdgpu_buffer_rsrc_t rsrc;
    int origin, ih0, iw0;  // origin: offset of channel (tid / BN) * PER at window position (0, 0) (may be negative)
    bool valid;
    float v[PER];

    __device__ __forceinline__ void init(const ConvGather& g, int n0, int tid) {
        rsrc = buffer_of(g.src, g.src_floats);
        const int q = n0 + tid % BN;
        valid = q < g.pixels;
        int rem, ow;
        const int n = g.div_ohw.divmod(valid ? q : 0, rem);
        const int oh = g.div_ow.divmod(rem, ow);
        ih0 = oh * g.SH - g.PH;
        iw0 = ow * g.SW - g.PW;
        origin = n * g.chw + (tid / BN) * PER * g.hw + ih0 * g.W + iw0;
    }

    __device__ __forceinline__ void load(const ConvGather& g, int kt, int k_end, int tid) {
        int tap, kw;
        const int chunk = g.div_khkw.divmod(kt / CHANNEL_CHUNK, tap);
        const int kh = g.div_kw.divmod(tap, kw);
        const int ih = ih0 + kh, iw = iw0 + kw;
        const bool ok = valid && kt < k_end && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                        static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
        const int uniform = chunk * CHANNEL_CHUNK * g.hw + kh * g.W + kw;
        const unsigned lane_bytes = ok ? static_cast<unsigned>(origin + uniform) * 4u : BUFFER_OOB;
        const int step_bytes = g.hw * 4;
#pragma unroll
        for (int i = 0; i < PER; ++i) v[i] = buffer_load(rsrc, lane_bytes, i * step_bytes);
    }

    template <int LD>
    __device__ __forceinline__ void store(float* lds, int tid) const {
        float* row = lds + (tid % BN) * LD + (tid / BN) * PER;
#pragma unroll
        for (int q = 0; q < PER / 4; ++q)
            *reinterpret_cast<float4*>(row + 4 * q) = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    }
};

// (c, kh, kw) of feature k in the gather's feature order.
__device__ __forceinline__ void feature_of(const ConvGather& g, int k, int& c, int& kh, int& kw) {
    int tap;
    if (g.chunked) {
        const int chunk = g.div_khkw.divmod(k / CHANNEL_CHUNK, tap);
        c = chunk * CHANNEL_CHUNK + k % CHANNEL_CHUNK;
    } else {
        c = g.div_khkw.divmod(k, tap);
    }
    kh = g.div_kw.divmod(tap, kw);
}

// Fills the LDS table of GatherPaddedRows: entry k < K is the byte offset of feature k = (c, kh, kw)
// inside an image's padded planes, entries K .. features_padded - 1 are BUFFER_OOB.
template <int THREADS>
__device__ __forceinline__ void fill_padded_table(unsigned* table, const ConvGather& g, int features_padded, int tid) {
    for (int k = tid; k < features_padded; k += THREADS) {
        int c = 0, kh = 0, kw = 0;
        if (k < g.features) feature_of(g, k, c, kh, kw);
        table[k] = k < g.features ? static_cast<unsigned>(c * g.phw + kh * g.pw + kw) * 4u : BUFFER_OOB;
    }
}

// The decomposition of one output pixel q (dW orientation: thread t handles pixel kt + t % BK_WG).
struct PixelAt {
    bool valid;
    int n, p;       // image and pixel within the image (p = oh*OW + ow)
    int ih0, iw0;   // window origin in the source
};

__device__ __forceinline__ PixelAt pixel_at(const ConvGather& g, int q, int q_end) {
    PixelAt at;
    at.valid = q < q_end;
    at.n = g.div_ohw.divmod(at.valid ? q : 0, at.p);
    int ow;
    const int oh = g.div_ow.divmod(at.p, ow);
    at.ih0 = oh * g.SH - g.PH;
    at.iw0 = ow * g.SW - g.PW;
    return at;
}

// dW orientation: a BN x BK_WG tile of the transposed view, rows = features [n0, n0 + BN), columns =
// pixels [kt, kt + BK_WG), stored k-contiguous ([BN][BK_WG + 4]). A thread's feature rows are fixed for
// the whole kernel, so their (c, kh, kw) offsets are decomposed once.
template <int BN, int THREADS>
struct GatherPixelColumns {
    static_assert(THREADS % BK_WG == 0 && BN % (THREADS / BK_WG) == 0, "rows split evenly over the threads");
    static constexpr int RSTEP = THREADS / BK_WG, PER = BN / RSTEP;
    int offset[PER], kh[PER], kw[PER];
    float v[PER];

    __device__ __forceinline__ void init(const ConvGather& g, int n0, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int k = n0 + tid / BK_WG + i * RSTEP;
            if (k < g.features) {
                int c, h, w;
                feature_of(g, k, c, h, w);
                offset[i] = c * g.hw + h * g.W + w;
                kh[i] = h;
                kw[i] = w;
            } else {
                offset[i] = 0;
                kh[i] = FAR;
                kw[i] = 0;
            }
        }
    }

    __device__ __forceinline__ void load(const ConvGather& g, const PixelAt& at) {
        const int origin = at.n * g.chw + at.ih0 * g.W + at.iw0;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int ih = at.ih0 + kh[i], iw = at.iw0 + kw[i];
            const bool ok = at.valid && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                            static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
            v[i] = ok ? g.src[origin + offset[i]] : 0.0f;
        }
    }

    template <int LD>
    __device__ __forceinline__ void store(float* lds, int tid) const {
        const int r0 = tid / BK_WG, col = tid % BK_WG;
#pragma unroll
        for (int i = 0; i < PER; ++i) lds[(r0 + i * RSTEP) * LD + col] = v[i];
    }
};

// dW's A operand: dy read in place, A[co][q] = dy[n, co, p] for pixel q = (n, p), as a BM x BK_WG
// k-contiguous tile (rows = output channels, columns = the same pixels as the gathered tile).
template <int BM, int THREADS>
struct GradRowsInPlace {
    static constexpr int RSTEP = THREADS / BK_WG, PER = BM / RSTEP;
    static_assert(BM % RSTEP == 0, "rows split evenly over the threads");
    float v[PER];

    __device__ __forceinline__ void load(const float* __restrict__ dy, int CO, int ohw, int m0, const PixelAt& at,
                                         int tid) {
        const int base = (at.n * CO + m0 + tid / BK_WG) * ohw + at.p;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int row = m0 + tid / BK_WG + i * RSTEP;
            v[i] = at.valid && row < CO ? dy[base + i * RSTEP * ohw] : 0.0f;
        }
    }

    template <int LD>
    __device__ __forceinline__ void store(float* lds, int tid) const {
        const int r0 = tid / BK_WG, col = tid % BK_WG;
#pragma unroll
        for (int i = 0; i < PER; ++i) lds[(r0 + i * RSTEP) * LD + col] = v[i];
    }

    // Adds the loaded values (0 outside the pixel range) to the thread's FP64 row sums.
    __device__ __forceinline__ void add_to(double (&sums)[PER]) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) sums[i] += static_cast<double>(v[i]);
    }

    // The row sums over this workgroup's pixels: the BK_WG threads of a row (adjacent lanes)
    // combine their sums with a fixed butterfly, then the first of them stores the FP64 sum to
    // out[row], or, when the workgroup covers every pixel, its float rounding to final[row].
    __device__ __forceinline__ static void store_sums(double (&sums)[PER], double* out, float* final, int CO, int m0,
                                               int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            double s = sums[i];
#pragma unroll
            for (int offset = BK_WG / 2; offset > 0; offset >>= 1) s += __shfl_xor(s, offset, BK_WG);
            const int row = m0 + tid / BK_WG + i * RSTEP;
            if (tid % BK_WG == 0 && row < CO) {
                if (final) final[row] = static_cast<float>(s);
                else out[row] = s;
            }
        }
    }
};

// One BM x BN tile (tile_m, tile_n) of Y (M x pixels) = A (M x K, row-major, lda) . view (K x
// pixels), K slice z. Split-K writes dense partials (z-th slice at C + z * c_batch); otherwise the
// epilogue of p (segmented NCHW, bias, activation).
template <int BM, int BN, int WM, int WN, bool VA, bool CHUNKED, bool PADDED = false>
__device__ __forceinline__ void implicit_forward_tile(const GemmParams& p, const ConvGather& g, int tile_m, int tile_n,
                                                      int z) {
    // The chunked and padded gathers store their tile pixel-major (TB), the natural-order one
    // feature-major.
    constexpr bool AHEAD = CHUNKED || PADDED;
    using S = MfmaShape<BM, BN, BK, WM, WN, false, AHEAD>;
    __shared__ __attribute__((aligned(16))) float smem[2 * S::STAGE];
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm0 = (wave / S::WGN) * WM, wn0 = (wave % S::WGN) * WN;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int k_begin = p.split ? z * p.k_chunk : 0;
    const int k_end = p.split ? min(p.K, k_begin + p.k_chunk) : p.K;
    float* __restrict__ C = p.C + (p.split ? z * p.c_batch : 0);

    // Chunked products (K a multiple of BK) read the kernel order with buffer loads too, two stages
    // ahead (two register slots of loaders); so do padded natural-order products, whose kernel is
    // a copy with its rows padded to whole stages (lda a multiple of BK, zeros past K).
    using LoadA = std::conditional_t<AHEAD, BufferRowTile<BM, BK, S::THREADS>, TileLoader<BM, BK, S::THREADS, VA>>;
    using LoadB = std::conditional_t<CHUNKED, GatherChunkRows<BN, S::THREADS>,
                                     std::conditional_t<PADDED, GatherPaddedRows<BN, S::THREADS>,
                                                        GatherFeatureRows<BN, S::THREADS>>>;
    LoadA la[AHEAD ? 2 : 1];
    LoadB lb[AHEAD ? 2 : 1];
#pragma unroll
    for (int i = 0; i < (AHEAD ? 2 : 1); ++i) {
        if constexpr (AHEAD) la[i].init(p.A, p.lda, p.M, m0, tid);
        lb[i].init(g, n0, tid);
    }
    __shared__ unsigned table[PADDED ? PADDED_TABLE_MAX : 1];
    if constexpr (PADDED) {
        fill_padded_table<S::THREADS>(table, g, p.lda, tid);
        __syncthreads();
    }
    v16f acc[S::TM][S::TN];
    zero_acc<S>(acc);
    // Two-level FP32 sum: 32-term stage sums on the matrix cores, added in FP32. Measured on the
    // batch-64 ResNet18 products, it brings the normwise error of the forward and dX products 4-7x
    // below one 576-4608-term chain (below the NumPy float32 path's) for 2 % of their time; FP64
    // totals were 3x more accurate still but cost 7 % (registers: one workgroup less per CU).
    StageSums<S, float> sums;
    if constexpr (AHEAD) {
        // The loop also fetches the two stages past the last (into slots no MFMA reads): the kernel
        // operand then re-reads the last stage, since its column offset is a scalar offset, which
        // the buffer range check does not cover (and the padded gather's table ends there).
        const int k_last = max(k_begin, k_end - BK);
        auto fetch = [&](auto slot, int kt) {
            la[decltype(slot)::value].load(min(kt, k_last));
            if constexpr (CHUNKED) lb[decltype(slot)::value].load(g, kt, k_end, tid);
            else lb[decltype(slot)::value].load(table, min(kt, k_last), tid);
        };
        auto store = [&](auto slot, float* a_lds, float* b_lds) {
            la[decltype(slot)::value].template store<S::LDA_S>(a_lds, tid);
            lb[decltype(slot)::value].template store<S::LDB_S>(b_lds, tid);
        };
        // The next stage's operands are in registers when a stage starts (read two stages ahead),
        // so they go to LDS after the first quarter of the stage's MFMAs.
        mfma_k_loop_ahead<S, STAGE_EARLY_STORE>(smem, k_begin, k_end, fetch, store, acc, wm0, wn0, lane, sums);
    } else {
        auto fetch = [&](int kt) {
            la[0].load(p.A, p.lda, m0, p.M, kt, k_end, tid);
            lb[0].load(g, kt, k_end, tid);
        };
        auto store = [&](float* a_lds, float* b_lds) {
            la[0].template store<S::LDA_S>(a_lds, tid);
            lb[0].template store<S::LDB_S>(b_lds, tid);
        };
        mfma_k_loop<S>(smem, k_begin, k_end, fetch, store, acc, wm0, wn0, lane, sums);
    }
    sums.rounded(acc);
    store_acc<S>(p, C, acc, m0, n0, wm0, wn0, lane);
}

template <int BM, int BN, int WM, int WN, bool VA, bool CHUNKED, bool PADDED>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv_implicit_forward_kernel(GemmParams p,
                                                                                          ConvGather g) {
    int tile_m, tile_n, z;
    tile_of_workgroup(tile_m, tile_n, z);
    implicit_forward_tile<BM, BN, WM, WN, VA, CHUNKED, PADDED>(p, g, tile_m, tile_n, z);
}

// Several implicit products of one tile shape in one launch (the phases of a strided dX): product
// j owns the workgroups [first[j], first[j + 1]), its tiles taken column-fastest; no K split.
constexpr int GROUPED_PRODUCTS = 4;
struct GroupedProducts {
    GemmParams p[GROUPED_PRODUCTS];
    ConvGather g[GROUPED_PRODUCTS];
    int first[GROUPED_PRODUCTS + 1];
    int tiles_n[GROUPED_PRODUCTS];
    int count;
};
static_assert(sizeof(GroupedProducts) <= 4096, "the grouped products travel in the kernel arguments");

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv_implicit_grouped_kernel(GroupedProducts batch) {
    const int block = static_cast<int>(blockIdx.x);
    int j = 0;
    while (j + 1 < batch.count && block >= batch.first[j + 1]) ++j;
    const int local = block - batch.first[j];
    implicit_forward_tile<BM, BN, WM, WN, true, true>(batch.p[j], batch.g[j], local / batch.tiles_n[j],
                                                      local % batch.tiles_n[j], 0);
}

// Both operand loads of one dW stage in chunked feature order: BK_WG pixels [kt, kt + BK_WG) of
// dy's rows (A, BM x BK_WG) and of the gathered view's feature rows (B, BN x BK_WG), all with buffer
// loads. Thread t owns pixel column kt + t % BK_WG and, with r = t / BK_WG (R threads per column),
// the A rows r, r + R, ... The tile's BN feature rows are BN / 32 groups of 32 channels at one
// (chunk, tap); thread r takes group r % G and the channels r / G + i * (R / G) of it, so its B_PER
// features share a tap: one bounds test per stage, then loads a uniform channel stride apart. A
// lane's offsets into dy and x are 32-bit and the row / channel steps wave-uniform (scalar
// offsets), so a stage's loads need no 64-bit address arithmetic and no branches. A lane past the
// pixel range, or whose window tap falls outside the image, reads zero.
// Rows of A past CO (the last row tile) read zero.
template <int BM, int BN, int THREADS, bool CHECK_ROWS>
struct WgradChunkStage {
    static constexpr int R = THREADS / BK_WG, A_PER = BM / R;
    static constexpr int G = BN / 32, SPAN = R / G, B_PER = 32 / SPAN;
    static_assert(BM % R == 0 && BN % 32 == 0 && R % G == 0 && 32 % SPAN == 0,
                  "a pixel column's threads split the rows and the groups evenly");
    __amdgpu_buffer_rsrc_t dy_rsrc, x_rsrc;
    int lo, a_row, kh, kw, b_offset, b_row0;
    float a[A_PER], b[B_PER];

    __device__ __forceinline__ void init(const ConvGather& g, const float* dy, int CO, int m0, int n0, int tid) {
        dy_rsrc = buffer_of(dy, static_cast<long long>(g.pixels) * CO);
        x_rsrc = buffer_of(g.src, g.src_floats);
        lo = tid % BK_WG;
        const int r = tid / BK_WG, group = r % G, sub = r / G;
        a_row = m0 + r;
        b_row0 = group * 32 + sub;
        const int k = n0 + group * 32;  // the group's first feature
        if (k < g.features) {
            int tap;
            const int chunk = g.div_khkw.divmod(k / CHANNEL_CHUNK, tap);
            kh = g.div_kw.divmod(tap, kw);
            b_offset = (chunk * CHANNEL_CHUNK + sub) * g.hw + kh * g.W + kw;
        } else {  // past the last feature: every pixel is out of bounds
            kh = FAR;
            kw = 0;
            b_offset = 0;
        }
    }

    __device__ __forceinline__ void load(const ConvGather& g, int CO, int kt, int k_end) {
        const int ohw = g.OH * g.OW;
        const int q = kt + lo;
        const bool valid = q < k_end;
        int pix, ow;
        const int n = g.div_ohw.divmod(valid ? q : 0, pix);
        const int oh = g.div_ow.divmod(pix, ow);
        const int ih0 = oh * g.SH - g.PH, iw0 = ow * g.SW - g.PW;
        const int ih = ih0 + kh, iw = iw0 + kw;
        const bool ok = valid && static_cast<unsigned>(ih) < static_cast<unsigned>(g.H) &&
                        static_cast<unsigned>(iw) < static_cast<unsigned>(g.W);
        // Both lane offsets first (selects, no branch around the loads), then the loads.
        const unsigned a_at = static_cast<unsigned>((n * CO + a_row) * ohw + pix) * 4u;
        const unsigned b_at = static_cast<unsigned>(n * g.chw + ih0 * g.W + iw0 + b_offset) * 4u;
        const unsigned a_lane = valid ? a_at : BUFFER_OOB;
        const unsigned b_lane = ok ? b_at : BUFFER_OOB;
        const int a_step = R * ohw * 4, b_step = SPAN * g.hw * 4;
        load_rows(CO, a_lane, a_step);
#pragma unroll
        for (int i = 0; i < B_PER; ++i) b[i] = buffer_load(x_rsrc, b_lane, i * b_step);
    }

    // dy's rows a_row + i R at this lane's pixel (lane offset a_lane of row a_row). The row steps
    // are scalar offsets, which the buffer range check does not cover; CHECK_ROWS (the last row
    // tile of an output whose rows end inside it) adds them to the lane offset instead, and its
    // rows past CO read zero.
    __device__ __forceinline__ void load_rows(int CO, unsigned a_lane, int a_step) {
        if constexpr (CHECK_ROWS) {
#pragma unroll
            for (int i = 0; i < A_PER; ++i)
                a[i] = buffer_load(dy_rsrc, a_row + i * R < CO ? a_lane + i * a_step : BUFFER_OOB, 0);
        } else {
#pragma unroll
            for (int i = 0; i < A_PER; ++i) a[i] = buffer_load(dy_rsrc, a_lane, i * a_step);
        }
    }

    template <int LDA, int LDB>
    __device__ __forceinline__ void store(float* a_lds, float* b_lds, int tid) const {
        const int r = tid / BK_WG;
#pragma unroll
        for (int i = 0; i < A_PER; ++i) a_lds[(r + i * R) * LDA + lo] = a[i];
#pragma unroll
        for (int i = 0; i < B_PER; ++i) b_lds[(b_row0 + i * SPAN) * LDB + lo] = b[i];
    }

    // Adds this thread's A values (0 past the pixel range) to its FP64 row sums.
    __device__ __forceinline__ void add_to(double (&sums)[A_PER]) const {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) sums[i] += static_cast<double>(a[i]);
    }
};

// Both operand loads of one dW stage in natural feature order from the zero-padded source
// (ConvGather::padded): dy's rows as in WgradChunkStage, and the thread's feature rows r, r + R, ...
// at one byte offset each into an image's padded planes, so a load costs one add and no window
// bounds test. A feature row past the last, or a pixel past the range, reads zero (an offset beyond
// the extent); both at once read the tensor's first element, which only reaches an output column
// past the last feature, never stored.
template <int BM, int BN, int THREADS, bool CHECK_ROWS>
struct WgradPaddedStage {
    static constexpr int R = THREADS / BK_WG, A_PER = BM / R, B_PER = BN / R;
    static_assert(BM % R == 0 && BN % R == 0, "a pixel column's threads split the rows evenly");
    __amdgpu_buffer_rsrc_t dy_rsrc, x_rsrc;
    int lo, a_row, b_row0;
    unsigned b_offset[B_PER];
    float a[A_PER], b[B_PER];

    __device__ __forceinline__ void init(const ConvGather& g, const float* dy, int CO, int m0, int n0, int tid) {
        dy_rsrc = buffer_of(dy, static_cast<long long>(g.pixels) * CO);
        x_rsrc = buffer_of(g.padded, g.padded_floats);
        lo = tid % BK_WG;
        const int r = tid / BK_WG;
        a_row = m0 + r;
        b_row0 = r;
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int k = n0 + r + i * R;
            int c = 0, kh = 0, kw = 0;
            if (k < g.features) feature_of(g, k, c, kh, kw);
            b_offset[i] = k < g.features ? static_cast<unsigned>(c * g.phw + kh * g.pw + kw) * 4u : BUFFER_OOB;
        }
    }

    __device__ __forceinline__ void load(const ConvGather& g, int CO, int kt, int k_end) {
        const int ohw = g.OH * g.OW;
        const int q = kt + lo;
        const bool valid = q < k_end;
        int pix, ow;
        const int n = g.div_ohw.divmod(valid ? q : 0, pix);
        const int oh = g.div_ow.divmod(pix, ow);
        const unsigned a_at = static_cast<unsigned>((n * CO + a_row) * ohw + pix) * 4u;
        const unsigned b_at = static_cast<unsigned>(n * g.C * g.phw + oh * g.SH * g.pw + ow * g.SW) * 4u;
        const unsigned a_lane = valid ? a_at : BUFFER_OOB;
        const unsigned b_lane = valid ? b_at : BUFFER_OOB;
        const int a_step = R * ohw * 4;
        if constexpr (CHECK_ROWS) {  // dy's rows as in WgradChunkStage::load_rows
#pragma unroll
            for (int i = 0; i < A_PER; ++i)
                a[i] = buffer_load(dy_rsrc, a_row + i * R < CO ? a_lane + i * a_step : BUFFER_OOB, 0);
        } else {
#pragma unroll
            for (int i = 0; i < A_PER; ++i) a[i] = buffer_load(dy_rsrc, a_lane, i * a_step);
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) b[i] = buffer_load(x_rsrc, b_lane + b_offset[i], 0);
    }

    template <int LDA, int LDB>
    __device__ __forceinline__ void store(float* a_lds, float* b_lds, int tid) const {
        const int r = tid / BK_WG;
#pragma unroll
        for (int i = 0; i < A_PER; ++i) a_lds[(r + i * R) * LDA + lo] = a[i];
#pragma unroll
        for (int i = 0; i < B_PER; ++i) b_lds[(b_row0 + i * R) * LDB + lo] = b[i];
    }

    __device__ __forceinline__ void add_to(double (&sums)[A_PER]) const {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) sums[i] += static_cast<double>(a[i]);
    }
};

// dW (CO x K) = dy (CO x pixels) . view^T (pixels x K), the pixel range split over z when p.split.
// SUMS: the workgroups of feature tile 0 also sum each dy row over their pixel range in FP64, the
// conv bias gradient: db[co] directly when unsplit, else sums[z * CO + co] for the reduction.
template <int BM, int BN, int WM, int WN, bool SUMS, bool CHUNKED, bool PADDED>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv_implicit_wgrad_kernel(GemmParams p, ConvGather g,
                                                                                        double* sums, float* db) {
    using S = MfmaShape<BM, BN, BK_WG, WM, WN, false, true>;
    __shared__ __attribute__((aligned(16))) float smem[2 * S::STAGE];
    int tile_m, tile_n, z;
    tile_of_workgroup(tile_m, tile_n, z);
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm0 = (wave / S::WGN) * WM, wn0 = (wave % S::WGN) * WN;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int k_begin = p.split ? z * p.k_chunk : 0;
    const int k_end = p.split ? min(p.K, k_begin + p.k_chunk) : p.K;
    float* __restrict__ C = p.C + (p.split ? z * p.c_batch : 0);
    const int ohw = g.OH * g.OW;
    v16f acc[S::TM][S::TN];
    zero_acc<S>(acc);
    using RowLoader = GradRowsInPlace<BM, S::THREADS>;
    double row_sums[RowLoader::PER];
#pragma unroll
    for (int i = 0; i < RowLoader::PER; ++i) row_sums[i] = 0.0;
    const bool summing = SUMS && tile_n == 0;

    if constexpr (CHUNKED || PADDED) {
        // Two register slots of loads, two stages ahead; the row sums as a separate loop body, so
        // that the other feature tiles' stages carry no FP64 work.
        auto run = [&](auto check_rows) {
            constexpr bool CHECK = decltype(check_rows)::value;
            using Stage = std::conditional_t<CHUNKED, WgradChunkStage<BM, BN, S::THREADS, CHECK>,
                                             WgradPaddedStage<BM, BN, S::THREADS, CHECK>>;
            static_assert(Stage::A_PER == RowLoader::PER, "the row sums follow the A rows");
            Stage st[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) st[i].init(g, p.A, p.M, m0, n0, tid);
            auto fetch = [&](auto slot, int kt) { st[decltype(slot)::value].load(g, p.M, kt, k_end); };
            if (summing) {
                auto store = [&](auto slot, float* a_lds, float* b_lds) {
                    st[decltype(slot)::value].template store<S::LDA_S, S::LDB_S>(a_lds, b_lds, tid);
                    st[decltype(slot)::value].add_to(row_sums);
                };
                mfma_k_loop_ahead<S, STAGE_MID_STORE>(smem, k_begin, k_end, fetch, store, acc, wm0, wn0, lane);
            } else {
                auto store = [&](auto slot, float* a_lds, float* b_lds) {
                    st[decltype(slot)::value].template store<S::LDA_S, S::LDB_S>(a_lds, b_lds, tid);
                };
                mfma_k_loop_ahead<S, STAGE_MID_STORE>(smem, k_begin, k_end, fetch, store, acc, wm0, wn0, lane);
            }
        };
        // Only the last row tile of an output whose rows end inside it reads dy's rows with
        // range-checked offsets.
        if (m0 + BM <= p.M) run(std::false_type{});
        else run(std::true_type{});
    } else {
        RowLoader la;
        GatherPixelColumns<BN, S::THREADS> lb;
        lb.init(g, n0, tid);
        auto fetch = [&](int kt) {
            const PixelAt at = pixel_at(g, kt + tid % BK_WG, k_end);
            la.load(p.A, p.M, ohw, m0, at, tid);
            lb.load(g, at);
        };
        auto store = [&](float* a_lds, float* b_lds) {
            la.template store<S::LDA_S>(a_lds, tid);
            lb.template store<S::LDB_S>(b_lds, tid);
            if constexpr (SUMS)
                if (summing) la.add_to(row_sums);
        };
        mfma_k_loop<S, STAGE_MID_STORE>(smem, k_begin, k_end, fetch, store, acc, wm0, wn0, lane);
    }
    store_acc<S>(p, C, acc, m0, n0, wm0, wn0, lane);
    if constexpr (SUMS)
        if (summing)
            RowLoader::store_sums(row_sums, sums + static_cast<long long>(z) * p.M, p.split ? nullptr : db, p.M, m0,
                                  tid);
}

// The kernel as the A operand of an implicit product: out[o][k] for O rows and features k over C
// channels and T = KH*KW taps, in chunked order when `chunked` (else natural order c*T + tap).
// Forward (flip = 0): O = CO, C = CI, out[co][(c, tap)] = w[co][c][tap]. dX (flip = 1): O = CI,
// C = CO, out[ci][(co, tap)] = w[co][ci][T - 1 - tap], the flipped and transposed kernel.
// One launch writes up to ORDER_BATCH orders: order i owns the workgroups [first_block[i],
// first_block[i + 1]).
//   * Chunked orders with at most TILE_TAPS taps go through LDS, one workgroup per TILE_ROWS output
//     rows x one chunk of 32 channels: the reads and the writes are contiguous runs (forward: each
//     row's 32*T source floats of that chunk; dX: for each of the chunk's 32 output channels, the
//     TILE_ROWS*T floats of the rows' input channels; writes: each row's 32*T floats).
//   * Other orders (natural channel counts, wider windows) take one output element per thread.
constexpr int ORDER_BATCH = 32;
constexpr int TILE_TAPS = 9;
constexpr int TILE_ROWS = 8;
constexpr int TILE_STRIDE = TILE_ROWS * TILE_TAPS + 1;  // floats per channel-within-chunk slab of the LDS tile
struct OrderJob {
    const float* w;
    float* out;
    int O, C, T, chunked, flip, total;
    int tiled;               // LDS path: blocks are (row block, chunk), chunk fastest
    // A phase of a strided dX (flip 1): T = th * tw sub-kernel taps; sub-tap (t, u) reads tap
    // (rh + sh * (th - 1 - t), rw + sw * (tw - 1 - u)) of the source kernel's src_T = KH * KW taps.
    int phase, src_T, src_kw, rh, rw, sh, sw, th, tw;
    FastDiv div_tw;
    FastDiv div_row, div_t;  // by C * T, by T
    FastDiv div_panel;       // by 32 * T (a destination run)
    FastDiv div_run;         // by the length of a source run: 32 * T (forward) or TILE_ROWS * T (dX)
    FastDiv div_chunks;      // by C / 32
};
struct OrderBatch {
    OrderJob job[ORDER_BATCH];
    int first_block[ORDER_BATCH + 1];
    int count;
};

// Elements a thread moves per batch of the tiled path (TILE_ROWS * 32 * T / 256 = T at most 9):
// all of its loads are issued before the first LDS store.
constexpr int ORDER_UNROLL = 12;
static_assert(TILE_ROWS * 32 * TILE_TAPS <= 256 * ORDER_UNROLL, "one batch covers a workgroup's tile");

__device__ __forceinline__ void order_tiled(const OrderJob& job, int block, float* tile) {
    const int T = job.T, panel = 32 * T, per_thread = TILE_ROWS * T / 8;  // TILE_ROWS*32*T / 256
    int chunk;
    const int ob = job.div_chunks.divmod(block, chunk);
    const int rows = min(TILE_ROWS, job.O - ob * TILE_ROWS);
    const long long row_len = static_cast<long long>(job.C) * T;
    // Source run s (flip: output channel co = chunk*32 + s of W over the rows' input channels and all
    // taps, TILE_ROWS*T floats; forward: output row ob*TILE_ROWS + s over the chunk's 32 input
    // channels and all taps, 32*T floats).
    const float* src =
        job.flip ? job.w + static_cast<long long>(chunk) * 32 * job.O * T + static_cast<long long>(ob) * TILE_ROWS * T
                 : job.w + static_cast<long long>(ob) * TILE_ROWS * row_len + static_cast<long long>(chunk) * panel;
    const long long run_stride = job.flip ? static_cast<long long>(job.O) * T : row_len;
    float v[ORDER_UNROLL];
    int slot[ORDER_UNROLL];
#pragma unroll
    for (int u = 0; u < ORDER_UNROLL; ++u) {
        const int idx = threadIdx.x + u * 256;
        slot[u] = -1;
        v[u] = 0.0f;
        if (u < per_thread) {
            int e;
            const int run = job.div_run.divmod(idx, e);
            int tap;
            const int q = job.div_t.divmod(e, tap);  // flip: row r = q; forward: channel j = q
            const int r = job.flip ? q : run, j = job.flip ? run : q;
            if (r < rows) {
                v[u] = src[run * run_stride + e];
                slot[u] = j * TILE_STRIDE + r * T + (job.flip ? T - 1 - tap : tap);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < ORDER_UNROLL; ++u)
        if (slot[u] >= 0) tile[slot[u]] = v[u];
    __syncthreads();
    // Destination run r: row ob*TILE_ROWS + r, features (chunk, tap, j) = tap*32 + j within the chunk.
    float* dst = job.out + static_cast<long long>(ob) * TILE_ROWS * row_len + static_cast<long long>(chunk) * panel;
#pragma unroll
    for (int u = 0; u < ORDER_UNROLL; ++u) {
        const int idx = threadIdx.x + u * 256;
        if (u < per_thread) {
            int d;
            const int r = job.div_panel.divmod(idx, d);
            const int tap = d / 32, j = d % 32;
            if (r < rows) dst[r * row_len + d] = tile[j * TILE_STRIDE + r * T + tap];
        }
    }
}

__global__ __launch_bounds__(256) void weight_order_kernel(OrderBatch batch) {
    __shared__ float tile[CHANNEL_CHUNK * TILE_STRIDE];
    int j = 0;
    while (j + 1 < batch.count && static_cast<int>(blockIdx.x) >= batch.first_block[j + 1]) ++j;
    const OrderJob& job = batch.job[j];
    const int block = static_cast<int>(blockIdx.x) - batch.first_block[j];
    if (job.tiled) {
        order_tiled(job, block, tile);
        return;
    }
    const int idx = block * 256 + threadIdx.x;
    if (idx >= job.total) return;
    int k, c, tap;
    const int o = job.div_row.divmod(idx, k);
    if (job.chunked) {
        const int group = k / CHANNEL_CHUNK;
        const int chunk = job.div_t.divmod(group, tap);
        c = chunk * CHANNEL_CHUNK + k % CHANNEL_CHUNK;
    } else {
        c = job.div_t.divmod(k, tap);
    }
    if (job.phase) {
        int u;
        const int t = job.div_tw.divmod(tap, u);
        const int kh = job.rh + job.sh * (job.th - 1 - t), kw = job.rw + job.sw * (job.tw - 1 - u);
        job.out[idx] = job.w[(c * job.O + o) * job.src_T + kh * job.src_kw + kw];
        return;
    }
    job.out[idx] = job.flip ? job.w[(c * job.O + o) * job.T + (job.T - 1 - tap)] : job.w[(o * job.C + c) * job.T + tap];
}

// partial[row] = sum of the row's `length` floats in FP64 (rows are the (n, co) planes of dy). One
// wave per row: lane l runs four chains over elements l + 64 (4 t + u), u = 0..3 (four loads in
// flight), adds the chains in order, then a fixed butterfly adds the lanes.
__global__ __launch_bounds__(256) void row_sums_kernel(const float* __restrict__ src, double* __restrict__ partial,
                                                       int rows, int length) {
    const int row = blockIdx.x * 4 + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= rows) return;
    const float* r = src + static_cast<long long>(row) * length;
    double chain[4] = {0.0, 0.0, 0.0, 0.0};
    for (int i = lane; i < length; i += 256) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = i + 64 * u < length ? r[i + 64 * u] : 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) chain[u] += static_cast<double>(v[u]);
    }
    double s = (chain[0] + chain[1]) + (chain[2] + chain[3]);
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) s += __shfl_xor(s, offset, 64);
    if (lane == 0) partial[row] = s;
}

// The padded operands of a natural-order product, one launch: the first plane_blocks workgroups
// write the source planes with PH / PW zero rows / columns on each side ((H + 2 PH) x (W + 2 PW),
// pw columns; planes_total floats, four consecutive ones per thread, stored as one float4 when all
// four exist), the others the forward kernel's rows (K floats of w) padded with zeros to kp columns
// (kernel_total floats, one per thread).
__global__ __launch_bounds__(256) void pad_operands_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                           int planes_total, int plane_blocks, FastDiv div_pw,
                                                           FastDiv div_ph, int H, int W, int PH, int PW,
                                                           const float* __restrict__ w, float* __restrict__ w_dst,
                                                           int kernel_total, FastDiv div_kp, int K) {
    if (static_cast<int>(blockIdx.x) < plane_blocks) {
        const int i0 = (blockIdx.x * 256 + threadIdx.x) * 4;
        if (i0 >= planes_total) return;
        const int pw = W + 2 * PW, ph = H + 2 * PH;
        int col, row;
        const int t = div_pw.divmod(i0, col);
        int plane = div_ph.divmod(t, row);
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int h = row - PH, x = col - PW;
            const bool inside = i0 + u < planes_total && static_cast<unsigned>(h) < static_cast<unsigned>(H) &&
                                static_cast<unsigned>(x) < static_cast<unsigned>(W);
            v[u] = inside ? src[static_cast<long long>(plane) * H * W + h * W + x] : 0.0f;
            if (++col == pw) {
                col = 0;
                if (++row == ph) {
                    row = 0;
                    ++plane;
                }
            }
        }
        if (i0 + 4 <= planes_total) {
            *reinterpret_cast<float4*>(dst + i0) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            for (int u = 0; i0 + u < planes_total; ++u) dst[i0 + u] = v[u];
        }
        return;
    }
    const int i = (blockIdx.x - plane_blocks) * 256 + threadIdx.x;
    if (i >= kernel_total) return;
    int col;
    const int row = div_kp.divmod(i, col);
    w_dst[i] = col < K ? w[static_cast<long long>(row) * K + col] : 0.0f;
}

using ConvFn = void (*)(GemmParams, ConvGather);

// Tile catalogue of the implicit products: block tile BM x BN, wave tile WM x WN. The 64 x 64 wave
// tiles keep four independent MFMA accumulators per wave and read half as much LDS per MFMA as
// 32 x 32 ones; the tiles of 32 x 32 (or 32 x 64) waves serve the batch-64 products, whose outputs
// are too small to fill the GPU with large waves. Tile 11's 96-pixel columns exist only for the
// chunked forward orientation.
struct ImplicitTile {
    int bm, bn, wm, wn;
};
constexpr ImplicitTile TILE_TABLE[] = {
    {64, 64, 64, 64},    // 0: one wave
    {64, 128, 64, 64},   // 1: two waves
    {128, 64, 64, 64},   // 2: two waves
    {128, 128, 64, 64},  // 3: four waves
    {64, 256, 64, 64},   // 4: four waves
    {256, 64, 64, 64},   // 5: four waves
    {64, 64, 32, 32},    // 6: four 32 x 32 waves
    {32, 64, 32, 32},    // 7: two 32 x 32 waves
    {64, 128, 32, 32},   // 8: eight 32 x 32 waves
    {128, 64, 32, 32},   // 9: eight 32 x 32 waves
    {128, 128, 32, 64},  // 10: eight 32 x 64 waves
    {128, 96, 32, 32},   // 11: twelve 32 x 32 waves (chunked forward only)
};
constexpr int TILE_COUNT = sizeof(TILE_TABLE) / sizeof(TILE_TABLE[0]);
constexpr int threads_of(const ImplicitTile& t) { return (t.bm / t.wm) * (t.bn / t.wn) * 64; }
// Which kernels a tile has: the natural-order forward loader reads whole waves of one feature row
// (BN a multiple of 64); the dW loaders split BM and BN rows evenly over THREADS / BK_WG threads.
constexpr bool has_natural(const ImplicitTile& t) { return t.bn % 64 == 0; }
constexpr bool has_wgrad(const ImplicitTile& t) {
    return t.bn % 64 == 0 && t.bm % (threads_of(t) / BK_WG) == 0 && t.bn % (threads_of(t) / BK_WG) == 0;
}

template <int T, bool VA, bool CHUNKED, bool PADDED = false>
constexpr ConvFn forward_of() {
    constexpr ImplicitTile t = TILE_TABLE[T];
    return conv_implicit_forward_kernel<t.bm, t.bn, t.wm, t.wn, VA, CHUNKED, PADDED>;
}

using WgradFn = void (*)(GemmParams, ConvGather, double*, float*);
using GroupedFn = void (*)(GroupedProducts);

template <int T, bool SUMS, bool CHUNKED, bool PADDED = false>
constexpr WgradFn wgrad_of() {
    constexpr ImplicitTile t = TILE_TABLE[T];
    return conv_implicit_wgrad_kernel<t.bm, t.bn, t.wm, t.wn, SUMS, CHUNKED, PADDED>;
}

// forward[tile][0 | 1 | 2 | 3]: natural feature order with scalar / float4 A loads, chunked order,
// natural order from the padded operands;
// wgrad[tile][0 | 1][0 | 1 | 2]: without / with the FP64 row sums of dy; natural / chunked feature
// order / natural order from the padded source.
struct ConvKernels {
    ConvFn forward[TILE_COUNT][4] = {};
    WgradFn wgrad[TILE_COUNT][2][3] = {};
    GroupedFn grouped[TILE_COUNT] = {};  // chunked products only, tile 6 (the strided dX phases)
    template <int T>
    void fill() {
        if constexpr (has_natural(TILE_TABLE[T])) {
            forward[T][0] = forward_of<T, false, false>();
            forward[T][1] = forward_of<T, true, false>();
            forward[T][3] = forward_of<T, true, false, true>();
        }
        forward[T][2] = forward_of<T, true, true>();
        if constexpr (has_wgrad(TILE_TABLE[T])) {
            wgrad[T][0][0] = wgrad_of<T, false, false>();
            wgrad[T][1][0] = wgrad_of<T, true, false>();
            wgrad[T][0][1] = wgrad_of<T, false, true>();
            wgrad[T][1][1] = wgrad_of<T, true, true>();
            wgrad[T][0][2] = wgrad_of<T, false, false, true>();
            wgrad[T][1][2] = wgrad_of<T, true, false, true>();
        }
    }
    ConvKernels() {
        fill<0>();
        fill<1>();
        fill<2>();
        fill<3>();
        fill<4>();
        fill<5>();
        fill<6>();
        fill<7>();
        fill<8>();
        fill<9>();
        fill<10>();
        fill<11>();
        grouped[6] = conv_implicit_grouped_kernel<64, 64, 32, 32>;
    }
};
static_assert(TILE_COUNT == 12, "ConvKernels fills every tile");

// Whether tile `tile` has a kernel for this product (dW, or the forward orientation in chunked or
// natural feature order).
bool tile_available(int tile, bool wgrad, bool chunked) {
    const ImplicitTile& t = TILE_TABLE[tile];
    return wgrad ? has_wgrad(t) : (chunked || has_natural(t));
}

const ConvKernels& conv_kernels() {
    static const ConvKernels table;
    return table;
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15) == 0; }

ConvGather gather_of(const float* src, int C, int H, int W, int KH, int KW, int SH, int SW, int PH, int PW, int N,
                     int OH, int OW) {
    ConvGather g{};
    g.src = src;
    g.C = C;
    g.H = H;
    g.W = W;
    g.KH = KH;
    g.KW = KW;
    g.SH = SH;
    g.SW = SW;
    g.PH = PH;
    g.PW = PW;
    g.OH = OH;
    g.OW = OW;
    g.pixels = N * OH * OW;
    g.features = C * KH * KW;
    g.src_floats = static_cast<long long>(N) * C * H * W;
    g.hw = H * W;
    g.chw = C * H * W;
    g.chunked = implicit_chunked(C) ? 1 : 0;
    g.div_ohw = FastDiv(OH * OW);
    g.div_ow = FastDiv(OW);
    g.div_khkw = FastDiv(KH * KW);
    g.div_kw = FastDiv(KW);
    return g;
}

// Planner model. Each tile runs at a fraction `efficiency` of the matrix peak once the GPU is
// full; a launch of W waves occupies each of the 4 * CUs SIMDs for ceil(W / SIMDs) wave-times (the
// last, partial round costs a whole one). A split over K adds its partials' HBM round trip and the
// reduction launch. The constants are fitted to a sweep of every tile and split on MI355X over
// ResNet18's batch-64 convolutions (forward, dW and dX).
struct PlannerModel {
    double efficiency[TILE_COUNT];
    double hbm_bytes_per_s;  // achieved rate of the split-K partial traffic
    double launch_s;         // cost of the extra reduction launch
};
// Tiles 8-11 have no fitted efficiency (0): the model leaves them to the measured plans below.
constexpr PlannerModel FORWARD_MODEL = {{0.49, 0.53, 0.54, 0.43, 0.32, 0.49, 0.56, 0.42, 0, 0, 0, 0}, 6.0e12, 2.0e-6};
constexpr PlannerModel WGRAD_MODEL = {{0.57, 0.37, 0.49, 0.72, 0.56, 0.34, 0.55, 0.32, 0, 0, 0, 0}, 3.0e12, 2.0e-6};
constexpr double SIMD_MACS_PER_S = 157.3e12 / 2 / 1024;  // FP32 multiply-adds per second per SIMD
constexpr int SPLIT_CHOICES[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96, 128};

double implicit_cost(bool wgrad, int tile, int M, int N, int slices, int chunk) {
    const ImplicitTile& t = TILE_TABLE[tile];
    const int waves = (t.bm / t.wm) * (t.bn / t.wn);
    const std::int64_t tiles = static_cast<std::int64_t>(blocks_for(M, t.bm)) * blocks_for(N, t.bn);
    const int simds = 4 * std::max(1, device_cu_count());
    const std::int64_t rounds = (tiles * slices * waves + simds - 1) / simds;
    const double wave_macs = static_cast<double>(t.wm) * t.wn * chunk;
    const PlannerModel& model = wgrad ? WGRAD_MODEL : FORWARD_MODEL;
    double cost = rounds * wave_macs / (SIMD_MACS_PER_S * model.efficiency[tile]);
    if (slices > 1) cost += 4.0 * (2.0 * slices + 1.0) * M * N / model.hbm_bytes_per_s + model.launch_s;
    return cost;
}

// A plan's K slices as whole stages of depth bk.
GemmPlan whole_stages(int tile, int K, int requested, int bk) {
    const int chunk = (static_cast<int>((static_cast<std::int64_t>(K) + requested - 1) / requested) + bk - 1) / bk * bk;
    const int slices = (K + chunk - 1) / chunk;
    return slices > 1 ? GemmPlan{tile, slices, chunk} : GemmPlan{tile, 1, K};
}

bool tile_fits(int tile, int M) { return blocks_for(M, TILE_TABLE[tile].bm) <= GRID_YZ_LIMIT; }

// dW products reduce over the pixels into a small output, so they are split over K. The rule below
// reproduces the fastest plan of a sweep over every tile and split on MI355X for ResNet18's batch-64
// dW products: four 64 x 64 waves per tile (tile 3) for outputs of at least 128 x 1024, else four
// 32 x 32 waves (tile 6); the K split brings the launch to about 432 (tile 3) or 1000 (tile 6)
// workgroups, with slices of at least 160 pixels.
constexpr int WGRAD_MIN_SLICE = 160;

GemmPlan wgrad_plan(int M, int N, int K) {
    const int tile = (M >= 128 && N >= 1024) ? 3 : 6;
    const ImplicitTile& t = TILE_TABLE[tile];
    const std::int64_t tiles = static_cast<std::int64_t>(blocks_for(M, t.bm)) * blocks_for(N, t.bn);
    const std::int64_t target = tile == 3 ? 432 : 1000;
    const int most = std::max(1, std::min(WGRAD_MAX_SLICES, K / WGRAD_MIN_SLICE));
    int wanted = static_cast<int>(std::max<std::int64_t>(1, (target + tiles / 2) / tiles));
    wanted = std::min(wanted, most);
    int requested = 1;
    for (const int choice : SPLIT_CHOICES)
        if (choice <= wanted) requested = choice;
    return whole_stages(tile, K, requested, BK_WG);
}

// Measured plans: products whose best tile and split, in a sweep of every tile and split on MI355X,
// beat the automatic plan below by at least 2 % (ResNet18's batch-64 convolutions at 3x120x160, and
// its batch-256 inference forwards at 224x224). The forward-orientation entries were re-measured for
// the two-level stage sums, whose extra registers cost tiles 8, 10 and 11 a resident workgroup; the
// dW entries for the chunked dW loads of WgradChunkStage (layer2 to layer4 moved to tile 6 with
// fewer slices, 5-8 % faster than their previous plans).
// Key: orientation (0 forward / dX, 1 dW), M, N, K; value: tile and requested K split.
struct MeasuredPlan {
    int wgrad, M, N, K, tile, requested;
};
constexpr MeasuredPlan MEASURED_PLANS[] = {
    {0, 64, 307200, 147, 6, 1},    // stem forward
    {0, 128, 19200, 576, 11, 1},   // layer2.0 conv1 forward (stride 2)
    {0, 128, 19200, 1152, 11, 1},  // layer2 3x3 forward and dX
    {0, 128, 19200, 64, 11, 1},    // layer2 1x1 downsample forward
    {0, 256, 5120, 1152, 9, 3},    // layer3.0 conv1 forward
    {0, 256, 5120, 2304, 9, 3},    // layer3 3x3 forward and dX
    {0, 256, 5120, 128, 9, 1},     // layer3 1x1 downsample forward
    {0, 512, 1280, 2304, 9, 6},    // layer4.0 conv1 forward
    {0, 512, 1280, 4608, 9, 6},    // layer4 3x3 forward and dX
    // ResNet18 inference forward, batch 256 at 224 x 224 (split 1 where within 1 % of the best)
    {0, 64, 3211264, 147, 6, 1},   // stem
    {0, 64, 774400, 576, 8, 1},    // layer1 3x3 (55 x 55 after the stem's unpadded 3 x 3 / 2 pool)
    {0, 128, 200704, 576, 9, 1},   // layer2.0 conv1 (stride 2)
    {0, 128, 200704, 1152, 9, 1},  // layer2 3x3
    {0, 128, 200704, 64, 6, 1},    // layer2 1x1 downsample
    {0, 256, 50176, 1152, 9, 1},   // layer3.0 conv1
    {0, 256, 50176, 2304, 6, 1},   // layer3 3x3
    {0, 256, 50176, 128, 6, 1},    // layer3 1x1 downsample
    {0, 512, 12544, 2304, 9, 4},   // layer4.0 conv1
    {0, 512, 12544, 4608, 9, 4},   // layer4 3x3
    {1, 64, 147, 307200, 6, 256},  // stem dW (more slices than the dW rule makes: its gathers need the waves)
    {1, 64, 576, 72384, 8, 96},    // layer1 dW
    {1, 128, 576, 19200, 8, 48},   // layer2.0 conv1 dW
    {1, 128, 1152, 19200, 6, 48},  // layer2 3x3 dW
    {1, 128, 64, 19200, 6, 128},   // layer2 1x1 downsample dW
    {1, 256, 1152, 5120, 8, 12},   // layer3.0 conv1 dW
    {1, 256, 2304, 5120, 6, 12},   // layer3 3x3 dW
    {1, 256, 128, 5120, 6, 32},    // layer3 1x1 downsample dW
    {1, 512, 2304, 1280, 6, 4},    // layer4.0 conv1 dW
    {1, 512, 256, 1280, 6, 8},     // layer4 1x1 downsample dW
    {1, 512, 4608, 1280, 6, 4},    // layer4 3x3 dW
};

// The plan of a product: a measured plan when one matches, else the dW rule, else the plan of least
// estimated cost (forward orientation).
GemmPlan implicit_auto_plan(bool wgrad, int M, int N, int K, bool chunked) {
    for (const MeasuredPlan& m : MEASURED_PLANS)
        if (m.wgrad == (wgrad ? 1 : 0) && m.M == M && m.N == N && m.K == K && tile_available(m.tile, wgrad, chunked) &&
            tile_fits(m.tile, M))
            return whole_stages(m.tile, K, m.requested, wgrad ? BK_WG : BK);
    if (wgrad && tile_fits(3, M) && tile_fits(6, M)) return wgrad_plan(M, N, K);
    const int bk = wgrad ? BK_WG : BK;
    const PlannerModel& model = wgrad ? WGRAD_MODEL : FORWARD_MODEL;
    GemmPlan best{-1, 1, K};
    double best_cost = 0.0;
    for (int tile = 0; tile < TILE_COUNT; ++tile) {
        if (!tile_fits(tile, M) || model.efficiency[tile] <= 0.0 || !tile_available(tile, wgrad, chunked)) continue;
        for (const int requested : SPLIT_CHOICES) {
            if (requested > 1 && K / requested < bk) break;
            const GemmPlan plan = whole_stages(tile, K, requested, bk);
            if (plan.slices > static_cast<int>(GRID_YZ_LIMIT)) continue;
            const double cost = implicit_cost(wgrad, tile, M, N, plan.slices, plan.slices > 1 ? plan.k_chunk : K);
            if (best.tile < 0 || cost < best_cost) {
                best = plan;
                best_cost = cost;
            }
        }
    }
    return best;
}

// The plan of a product from an engine code (1 = automatic; 16 + tile * 128 + slices - 1 names a
// tile of TILE_TABLE and a requested K split); the split is dropped when the workspace cannot hold
// it.
int implicit_plan(bool wgrad, bool chunked, int engine, int M, int N, int K, float* workspace,
                  std::int64_t workspace_floats, GemmPlan* plan) {
    if (engine == 1) {
        *plan = implicit_auto_plan(wgrad, M, N, K, chunked);
    } else {
        const int code = engine - 16;
        const int tile = code / 128, requested = code % 128 + 1;
        if (code < 0 || tile >= TILE_COUNT) return MFH_FAIL(ERR_ARG, "unknown implicit convolution plan code");
        if (!tile_available(tile, wgrad, chunked))
            return MFH_FAIL(ERR_ARG, "this implicit convolution tile has no kernel for this product");
        *plan = whole_stages(tile, K, requested, wgrad ? BK_WG : BK);
    }
    if (plan->tile < 0 || !tile_fits(plan->tile, M))
        return MFH_FAIL(ERR_ARG, "this tile cannot run the implicit convolution");
    if (plan->slices > 1 && (!workspace || workspace_floats < gemm_workspace_floats(*plan, M, N)))
        *plan = GemmPlan{plan->tile, 1, K};
    const ImplicitTile& t = TILE_TABLE[plan->tile];
    if (static_cast<unsigned>(plan->slices) > GRID_YZ_LIMIT ||
        static_cast<std::int64_t>(blocks_for(M, t.bm)) * blocks_for(N, t.bn) * plan->slices > INDEX_LIMIT)
        return MFH_FAIL(ERR_ARG, "implicit convolution grid exceeds the launch limits");
    return OK;
}

// The output fields of an unsplit product: C (ldc) and the epilogue e.
void set_epilogue(GemmParams& p, float* c, int ldc, const GemmEpilogue& e) {
    p.C = c;
    p.ldc = ldc;
    p.bias = e.bias;
    p.bias_mode = e.bias_mode;
    p.act = e.act;
    p.alpha = e.alpha;
    p.segment = e.segment;
    if (e.segment > 0) p.segment_div = FastDiv(e.segment);
    p.segment_stride = e.segment_stride;
    p.taps = e.taps;
    if (e.taps > 0) p.taps_div = FastDiv(e.taps);
    p.accumulate = e.accumulate ? 1 : 0;
    p.residual = e.residual;
    p.lattice_w = e.lattice_w;
    if (e.lattice_w > 0) p.lattice_div = FastDiv(e.lattice_w);
    p.lattice_row = e.lattice_row;
    p.lattice_col = e.lattice_col;
    p.lattice_offset = e.lattice_offset;
    p.cell_h = e.cell_h;
    p.cell_w = e.cell_w;
    p.plane_h = e.plane_h;
    p.plane_w = e.plane_w;
}

// Whether the operands of a chunked forward-orientation product fit the buffer loads' 31-bit
// byte extents: the gathered source and the M x lda kernel order (a chunked dW product gathers
// its source with buffer loads too).
bool buffer_extents_fit(const ConvGather& g, int M, int lda) {
    return g.src_floats <= BUFFER_LIMIT_FLOATS && static_cast<std::int64_t>(M) * lda <= BUFFER_LIMIT_FLOATS;
}

// Where a natural-order product's padded operands live in its workspace, past the split-K partials:
// the zero-padded source copy ((H + 2 PH) x (W + 2 PW) planes; none for an unpadded source, read in
// place) and, for a forward product, the kernel's rows padded with zeros to whole stages. `usable`
// is false where the product keeps the bounds-tested gather: chunked sources, operands past the
// buffer loads' extent, forward products with more features than the offset table holds.
struct PaddedLayout {
    bool usable = false;
    std::int64_t source_at = 0, source_floats = 0, kernel_at = 0, kernel_floats = 0, total = 0;
    int kp = 0;
};

std::int64_t aligned64(std::int64_t floats) { return (floats + 63) / 64 * 64; }

PaddedLayout padded_layout(const ConvGather& g, int images, std::int64_t partial_floats, bool forward, int M) {
    PaddedLayout l;
    l.total = partial_floats;
    const std::int64_t all = static_cast<std::int64_t>(images) * g.C * (g.H + 2 * g.PH) * (g.W + 2 * g.PW);
    l.kp = (g.features + BK - 1) / BK * BK;
    if (g.chunked || all > BUFFER_LIMIT_FLOATS) return l;
    if (forward && (l.kp > PADDED_TABLE_MAX || static_cast<std::int64_t>(M) * l.kp > BUFFER_LIMIT_FLOATS)) return l;
    l.usable = true;
    l.source_at = aligned64(partial_floats);
    l.source_floats = g.PH || g.PW ? all : 0;
    l.kernel_at = aligned64(l.source_at + l.source_floats);
    l.kernel_floats = forward ? static_cast<std::int64_t>(M) * l.kp : 0;
    l.total = l.kernel_at + l.kernel_floats;
    return l;
}

// Sets up a natural-order product to read padded operands without window bounds tests
// (ConvGather::padded): the source itself when it has no padding, else a zero-padded copy made here
// in the workspace; a forward product also gets its kernel with rows padded to whole stages
// (*kernel, *kp columns). Where the layout is not usable or the workspace cannot hold it, the gather
// keeps its bounds tests (g.padded stays null).
int pad_operands(ConvGather& g, int images, const GemmPlan& plan, int M, int N, float* workspace,
                 std::int64_t workspace_floats, hipStream_t stream, const float** kernel = nullptr, int* kp = nullptr) {
    const bool forward = kernel != nullptr;
    const PaddedLayout l =
        padded_layout(g, images, plan.slices > 1 ? gemm_workspace_floats(plan, M, N) : 0, forward, M);
    if (!l.usable || (l.total > 0 && (!workspace || workspace_floats < l.total))) return OK;
    const int ph = g.H + 2 * g.PH, pw = g.W + 2 * g.PW;
    float* source = l.source_floats ? workspace + l.source_at : nullptr;
    float* kernel_copy = forward ? workspace + l.kernel_at : nullptr;
    // The padded planes are written and the padded kernel read with 16-byte accesses.
    if ((source && !aligned16(source)) || (forward && !aligned16(kernel_copy))) return OK;
    const int plane_blocks = blocks_for((l.source_floats + 3) / 4, 256);
    const int blocks = plane_blocks + blocks_for(l.kernel_floats, 256);
    if (blocks > 0) {
        launch(pad_operands_kernel, blocks, 256, 0, stream, g.src, source, static_cast<int>(l.source_floats),
               plane_blocks, FastDiv(pw), FastDiv(ph), g.H, g.W, g.PH, g.PW, forward ? *kernel : nullptr,
               kernel_copy, static_cast<int>(l.kernel_floats), FastDiv(l.kp), g.features);
        MFH_TRY(MFH_CHECK_LAUNCH("pad_operands", stream));
    }
    g.padded = source ? source : g.src;
    g.pw = pw;
    g.phw = ph * pw;
    g.padded_floats = static_cast<long long>(images) * g.C * ph * pw;
    if (forward) {
        *kernel = kernel_copy;
        *kp = l.kp;
    }
    return OK;
}

// Runs one implicit product with the epilogue e (directly, or through split-K partials and the
// FP64 slice reduction).
int run_implicit(bool wgrad, const GemmPlan& plan, const float* a, int lda, int M, int N, int K, const ConvGather& g,
                 float* c, int ldc, GemmEpilogue e, float* workspace, hipStream_t stream,
                 double* row_sums = nullptr, float* row_out = nullptr, bool defer_reduce = false) {
    const bool split = plan.slices > 1;
    GemmParams p{};
    p.A = a;
    p.lda = lda;
    p.M = M;
    p.N = N;
    p.K = K;
    p.split = split ? 1 : 0;
    p.k_chunk = split ? plan.k_chunk : K;
    if (split) {
        p.C = workspace;
        p.ldc = N;
        p.c_batch = static_cast<long long>(M) * N;
    } else {
        set_epilogue(p, c, ldc, e);
    }
    const ImplicitTile& t = TILE_TABLE[plan.tile];
    const dim3 grid(blocks_for(N, t.bn), blocks_for(M, t.bm), static_cast<unsigned>(plan.slices));
    const dim3 block(threads_of(t));
    const bool vec_a = K % 4 == 0 && lda % 4 == 0 && aligned16(a);
    const int variant = g.chunked ? 2 : g.padded ? 3 : vec_a ? 1 : 0;
    const int order = g.chunked ? 1 : g.padded ? 2 : 0;
    if (!wgrad && (g.chunked || g.padded) && !vec_a)
        return MFH_FAIL(ERR_ARG, "the reordered kernel buffer must be 16-byte aligned");
    if (g.chunked && (wgrad ? g.src_floats > BUFFER_LIMIT_FLOATS || static_cast<std::int64_t>(g.pixels) * M >
                                                                       BUFFER_LIMIT_FLOATS
                            : !buffer_extents_fit(g, M, lda)))
        return MFH_FAIL(ERR_ARG, "a chunked implicit convolution reads tensors of at most 2 GiB");
    if (wgrad)
        launch(conv_kernels().wgrad[plan.tile][row_out ? 1 : 0][order], grid, block, 0, stream,
                           p, g, row_sums,
                           row_out);
    else
        launch(conv_kernels().forward[plan.tile][variant], grid, block, 0, stream, p, g);
    MFH_TRY(MFH_CHECK_LAUNCH(wgrad ? "conv_implicit_wgrad" : "conv_implicit_forward", stream));
    if (!split || defer_reduce) return OK;
    if (row_out) {  // the row sums' slice partials are finished by the same reduction launch
        e.row_partial = row_sums;
        e.row_out = row_out;
        e.row_count = M;
    }
    // dW products split into many pixel slices over a small output: a grouped reduction keeps the
    // whole GPU busy (one thread per output would leave most CUs idle).
    if (wgrad && plan.slices >= GROUPED_REDUCE_SLICES)
        return split_reduce_grouped(workspace, c, e, M, N, ldc, plan.slices, stream);
    return split_reduce_epilogue(workspace, c, e, M, N, ldc, plan.slices, stream);
}

}  // namespace

bool implicit_engine_valid(int engine) { return engine == 1 || (engine >= 16 && engine < 16 + TILE_COUNT * 128); }

std::int64_t implicit_workspace_floats(const ConvGeometry& g, int pass) {
    if (pass == IMPLICIT_DGRAD && (g.SH > 1 || g.SW > 1)) {
        // Phase products, or the column gradient's one product (MFH_CONV_COLUMN_ORDER).
        std::int64_t most = implicit_chunked(g.CO) ? implicit_workspace_floats(column_geometry(g), pass) : 0;
        for (int a = 0; a < g.SH; ++a)
            for (int b = 0; b < g.SW; ++b) {
                const DgradPhase ph = dgrad_phase(g, a, b);
                if (ph.th * ph.tw == 0 || ph.hp == 0 || ph.wp == 0) continue;
                const int M = g.CI, N = g.N * ph.hp * ph.wp, K = g.CO * ph.th * ph.tw;
                const GemmPlan plan = implicit_auto_plan(false, M, N, K, implicit_chunked(g.CO));
                most = std::max(most, gemm_workspace_floats(plan, M, N));
            }
        return most;
    }
    GemmPlan plan;
    if (pass == IMPLICIT_FORWARD) plan = implicit_auto_plan(false, g.CO, g.rows(), g.features(), implicit_chunked(g.CI));
    else if (pass == IMPLICIT_WGRAD) plan = implicit_auto_plan(true, g.CO, g.features(), g.rows(), implicit_chunked(g.CI));
    else plan = implicit_auto_plan(false, g.CI, g.N * g.H * g.W, g.CO * g.KH * g.KW, implicit_chunked(g.CO));
    const std::int64_t partials = pass == IMPLICIT_WGRAD
                                      ? gemm_workspace_floats(plan, g.CO, g.features())
                                      : gemm_workspace_floats(plan, pass == IMPLICIT_FORWARD ? g.CO : g.CI,
                                                              pass == IMPLICIT_FORWARD ? g.rows() : g.N * g.H * g.W);
    if (pass == IMPLICIT_DGRAD) return partials;
    // The forward and dW products of a natural-order convolution also hold its padded operands.
    const ConvGather gather = gather_of(nullptr, g.CI, g.H, g.W, g.KH, g.KW, g.SH, g.SW, g.PH, g.PW, g.N, g.OH, g.OW);
    return padded_layout(gather, g.N, partials, pass == IMPLICIT_FORWARD, g.CO).total;
}

// The jobs of one order: one, or one per non-empty phase of a strided dX (sub-kernels back to back).
void order_jobs(const WeightOrder& o, std::vector<OrderJob>& jobs) {
    const int rows = o.flip ? o.CI : o.CO, channels = o.flip ? o.CO : o.CI;
    auto base = [&](OrderJob& job, float* out, int taps) {
        job.w = o.w;
        job.out = out;
        job.O = rows;
        job.C = channels;
        job.T = taps;
        job.chunked = implicit_chunked(channels) ? 1 : 0;
        job.flip = o.flip;
        job.total = rows * channels * taps;
        job.div_row = FastDiv(channels * taps);
        job.div_t = FastDiv(taps);
        job.div_panel = FastDiv(32 * taps);
        job.div_run = FastDiv((o.flip ? TILE_ROWS : 32) * taps);
        job.div_chunks = FastDiv(std::max(1, channels / CHANNEL_CHUNK));
    };
    if (!o.flip || (o.SH == 1 && o.SW == 1)) {
        OrderJob job{};
        base(job, o.out, o.KH * o.KW);
        job.tiled = job.chunked && job.T <= TILE_TAPS ? 1 : 0;
        jobs.push_back(job);
        return;
    }
    const ConvGeometry g{1, o.CI, 1, 1, o.CO, o.KH, o.KW, 1, 1, o.SH, o.SW, o.PH, o.PW};
    long long offset = 0;
    for (int a = 0; a < o.SH; ++a)
        for (int b = 0; b < o.SW; ++b) {
            const DgradPhase ph = dgrad_phase(g, a, b);
            const int taps = ph.th * ph.tw;
            if (taps == 0) continue;
            OrderJob job{};
            base(job, o.out + offset, taps);
            job.tiled = 0;
            job.phase = 1;
            job.src_T = o.KH * o.KW;
            job.src_kw = o.KW;
            job.rh = ph.rh;
            job.rw = ph.rw;
            job.sh = o.SH;
            job.sw = o.SW;
            job.th = ph.th;
            job.tw = ph.tw;
            job.div_tw = FastDiv(ph.tw);
            jobs.push_back(job);
            offset += static_cast<long long>(rows) * channels * taps;
        }
}

int launch_weight_orders(const WeightOrder* orders, int count, hipStream_t stream) {
    std::vector<OrderJob> jobs;
    for (int i = 0; i < count; ++i) order_jobs(orders[i], jobs);
    const int total = static_cast<int>(jobs.size());
    for (int first = 0; first < total; first += ORDER_BATCH) {
        OrderBatch batch{};
        batch.count = std::min(ORDER_BATCH, total - first);
        int blocks = 0;
        for (int i = 0; i < batch.count; ++i) {
            const OrderJob& job = batch.job[i] = jobs[first + i];
            batch.first_block[i] = blocks;
            blocks += static_cast<int>(job.tiled ? blocks_for(job.O, TILE_ROWS) * (job.C / CHANNEL_CHUNK)
                                                 : blocks_for(job.total, 256));
        }
        batch.first_block[batch.count] = blocks;
        if (blocks == 0) continue;
        launch(weight_order_kernel, blocks, 256, 0, stream, batch);
        MFH_TRY(MFH_CHECK_LAUNCH("weight_order", stream));
    }
    return OK;
}

int conv_implicit_forward(const ConvGeometry& g, const float* x, const float* w, float* wt, bool prepared,
                          const float* bias, const float* residual, float* y, int act, float alpha, int engine,
                          float* workspace, std::int64_t workspace_floats, hipStream_t stream, int* deferred) {
    const int M = g.CO, N = g.rows(), K = g.features();
    GemmPlan plan;
    MFH_TRY(implicit_plan(false, implicit_chunked(g.CI), engine, M, N, K, workspace, workspace_floats, &plan));
    ConvGather gather = gather_of(x, g.CI, g.H, g.W, g.KH, g.KW, g.SH, g.SW, g.PH, g.PW, g.N, g.OH, g.OW);
    if (gather.chunked) {
        if (!prepared) {
            const WeightOrder order{w, wt, g.CO, g.CI, g.KH, g.KW, 0};
            MFH_TRY(launch_weight_orders(&order, 1, stream));
        }
        w = wt;
    }
    int lda = K;
    if (!gather.chunked) MFH_TRY(pad_operands(gather, g.N, plan, M, N, workspace, workspace_floats, stream, &w, &lda));
    GemmEpilogue e;
    e.bias = bias;
    e.bias_mode = bias ? BIAS_ROW : BIAS_NONE;
    e.act = act;
    e.alpha = alpha;
    e.segment = g.ohw();
    e.segment_stride = static_cast<long long>(g.CO) * g.ohw();
    e.residual = residual;
    // A split product without residual or activation may leave its slices in the workspace for the
    // caller to reduce and add the bias to (the slice count goes to *deferred; 1 when y was written
    // here).
    const bool defer = deferred && plan.slices > 1 && !residual && act == ACT_NONE;
    if (deferred) *deferred = defer ? plan.slices : 1;
    // A padded product runs over the padded kernel's whole stages (features past K read zeros).
    return run_implicit(false, plan, w, lda, M, N, gather.padded ? lda : K, gather, y, g.ohw(), e, workspace, stream,
                        nullptr, nullptr, defer);
}

int conv_implicit_wgrad(const ConvGeometry& g, const float* x, const float* dy, float* dw, double* bias_partial,
                        float* db, int engine, float* workspace, std::int64_t workspace_floats, hipStream_t stream) {
    const int M = g.CO, N = g.features(), K = g.rows();
    GemmPlan plan;
    MFH_TRY(implicit_plan(true, implicit_chunked(g.CI), engine, M, N, K, workspace, workspace_floats, &plan));
    if (db && (!bias_partial || plan.slices > WGRAD_MAX_SLICES))
        return MFH_FAIL(ERR_ARG, "the dW plan's bias partials need bias_partial rows for every pixel slice");
    ConvGather gather = gather_of(x, g.CI, g.H, g.W, g.KH, g.KW, g.SH, g.SW, g.PH, g.PW, g.N, g.OH, g.OW);
    MFH_TRY(pad_operands(gather, g.N, plan, M, N, workspace, workspace_floats, stream));
    GemmEpilogue e;
    if (gather.chunked) e.taps = g.KH * g.KW;
    return run_implicit(true, plan, dy, g.ohw(), M, N, K, gather, dw, N, e, workspace, stream, bias_partial, db);
}

int conv_implicit_dgrad(const ConvGeometry& g, const float* dy, const float* w, float* wflip, bool prepared, float* dx,
                        bool accumulate, int engine, float* workspace, std::int64_t workspace_floats,
                        hipStream_t stream, int* deferred) {
    const int khw = g.KH * g.KW;
    const int M = g.CI, N = g.N * g.H * g.W, K = g.CO * khw;
    GemmPlan plan;
    MFH_TRY(implicit_plan(false, implicit_chunked(g.CO), engine, M, N, K, workspace, workspace_floats, &plan));
    if (!prepared) {
        const WeightOrder order{w, wflip, g.CO, g.CI, g.KH, g.KW, 1};
        MFH_TRY(launch_weight_orders(&order, 1, stream));
    }
    // dy as the source of a stride-1 convolution with padding KH-1-PH whose output grid is H x W.
    const ConvGather gather =
        gather_of(dy, g.CO, g.OH, g.OW, g.KH, g.KW, 1, 1, g.KH - 1 - g.PH, g.KW - 1 - g.PW, g.N, g.H, g.W);
    GemmEpilogue e;
    e.segment = g.H * g.W;
    e.segment_stride = static_cast<long long>(g.CI) * g.H * g.W;
    e.accumulate = accumulate;
    const bool defer = deferred && plan.slices > 1 && !accumulate;
    if (deferred) *deferred = defer ? plan.slices : 1;
    return run_implicit(false, plan, wflip, K, M, N, K, gather, dx, g.H * g.W, e, workspace, stream, nullptr, nullptr,
                        defer);
}

int conv_implicit_dgrad_phases(const ConvGeometry& g, const float* dy, const float* w, float* wphase, bool prepared,
                               float* dx, bool accumulate, int engine, float* workspace,
                               std::int64_t workspace_floats, hipStream_t stream) {
    if (!prepared) {
        const WeightOrder order{w, wphase, g.CO, g.CI, g.KH, g.KW, 1, g.SH, g.SW, g.PH, g.PW};
        MFH_TRY(launch_weight_orders(&order, 1, stream));
    }
    bool gaps = false;    // input positions that no tap reaches (a phase without taps)
    int with_taps = 0;    // phases that have taps
    for (int a = 0; a < g.SH; ++a)
        for (int b = 0; b < g.SW; ++b) {
            const DgradPhase ph = dgrad_phase(g, a, b);
            gaps = gaps || (ph.th * ph.tw == 0 && ph.hp > 0 && ph.wp > 0);
            with_taps += ph.th * ph.tw > 0 ? 1 : 0;
        }
    // When phase (0, 0) alone has taps (a 1x1 kernel without padding), its product zeroes the rest
    // of each cell itself; other gaps are cleared by a fill first.
    const bool cells = gaps && !accumulate && with_taps == 1 && dgrad_phase(g, 0, 0).th * dgrad_phase(g, 0, 0).tw > 0;
    if (gaps && !accumulate && !cells) {
        MFH_TRY(launch_fill_zero(dx, static_cast<std::int64_t>(g.N) * g.CI * g.H * g.W, stream));
        accumulate = true;
    }
    if (engine == 1 && with_taps > 1 && implicit_chunked(g.CO)) {
        // Every phase in one launch (64 x 64 tiles of four 32 x 32 waves, the fastest of the
        // sweep on MI355X; no K split), the phase with the most taps first so that its longer
        // tiles start first. The choice depends on the geometry only, so a dX written fresh and
        // one added to a gradient run the same products.
        const int tile = 6;
        const ImplicitTile& t = TILE_TABLE[tile];
        GroupedProducts batch{};
        struct Entry { DgradPhase ph; long long offset; };
        Entry entries[GROUPED_PRODUCTS];
        int count = 0;
        long long offset = 0;
        bool fits = true;
        for (int a = 0; a < g.SH; ++a)
            for (int b = 0; b < g.SW; ++b) {
                const DgradPhase ph = dgrad_phase(g, a, b);
                const int taps = ph.th * ph.tw;
                if (taps == 0) continue;
                if (ph.hp > 0 && ph.wp > 0) {
                    if (count == GROUPED_PRODUCTS) fits = false;
                    else entries[count++] = Entry{ph, offset};
                }
                offset += static_cast<long long>(g.CI) * g.CO * taps;
            }
        std::stable_sort(entries, entries + (fits ? count : 0), [](const Entry& x, const Entry& y) {
            return x.ph.th * x.ph.tw > y.ph.th * y.ph.tw;
        });
        std::int64_t blocks = 0;
        for (int i = 0; fits && i < count; ++i) {
            const DgradPhase& ph = entries[i].ph;
            const int M = g.CI, N = g.N * ph.hp * ph.wp, K = g.CO * ph.th * ph.tw;
            GemmParams& p = batch.p[i];
            p.A = wphase + entries[i].offset;
            p.lda = K;
            p.M = M;
            p.N = N;
            p.K = K;
            p.k_chunk = K;
            GemmEpilogue e;
            e.segment = ph.hp * ph.wp;
            e.segment_stride = static_cast<long long>(g.CI) * g.H * g.W;
            e.accumulate = accumulate;
            e.lattice_w = ph.wp;
            e.lattice_row = g.SH * g.W;
            e.lattice_col = g.SW;
            e.lattice_offset = ph.a * g.W + ph.b;
            set_epilogue(p, dx, g.H * g.W, e);
            batch.g[i] = gather_of(dy, g.CO, g.OH, g.OW, ph.th, ph.tw, 1, 1, ph.pad_h, ph.pad_w, g.N, ph.hp, ph.wp);
            batch.tiles_n[i] = static_cast<int>(blocks_for(N, t.bn));
            batch.first[i] = static_cast<int>(blocks);
            blocks += static_cast<std::int64_t>(blocks_for(M, t.bm)) * batch.tiles_n[i];
            fits = fits && aligned16(p.A) && blocks <= INDEX_LIMIT && buffer_extents_fit(batch.g[i], M, K);
        }
        if (fits && count > 0) {
            batch.first[count] = static_cast<int>(blocks);
            batch.count = count;
            launch(conv_kernels().grouped[tile], dim3(static_cast<unsigned>(blocks)), dim3(threads_of(t)),
                               0, stream, batch);
            return MFH_CHECK_LAUNCH("conv_implicit_grouped", stream);
        }
    }
    long long offset = 0;
    for (int a = 0; a < g.SH; ++a)
        for (int b = 0; b < g.SW; ++b) {
            const DgradPhase ph = dgrad_phase(g, a, b);
            const int taps = ph.th * ph.tw;
            if (taps == 0) continue;
            const float* sub = wphase + offset;
            offset += static_cast<long long>(g.CI) * g.CO * taps;
            if (ph.hp == 0 || ph.wp == 0) continue;
            const int M = g.CI, N = g.N * ph.hp * ph.wp, K = g.CO * taps;
            GemmPlan plan;
            MFH_TRY(implicit_plan(false, implicit_chunked(g.CO), engine, M, N, K, workspace, workspace_floats, &plan));
            const ConvGather gather =
                gather_of(dy, g.CO, g.OH, g.OW, ph.th, ph.tw, 1, 1, ph.pad_h, ph.pad_w, g.N, ph.hp, ph.wp);
            GemmEpilogue e;
            e.segment = ph.hp * ph.wp;
            e.segment_stride = static_cast<long long>(g.CI) * g.H * g.W;
            e.accumulate = accumulate;
            e.lattice_w = ph.wp;
            e.lattice_row = g.SH * g.W;
            e.lattice_col = g.SW;
            e.lattice_offset = a * g.W + b;
            if (cells) {
                e.cell_h = g.SH;
                e.cell_w = g.SW;
                e.plane_h = g.H;
                e.plane_w = g.W;
            }
            MFH_TRY(run_implicit(false, plan, sub, K, M, N, K, gather, dx, g.H * g.W, e, workspace, stream));
        }
    return OK;
}

int launch_row_sums(const float* src, double* partial, int rows, int length, hipStream_t stream) {
    launch(row_sums_kernel, blocks_for(rows, 4), 256, 0, stream, src, partial, rows, length);
    return MFH_CHECK_LAUNCH("row_sums", stream);
}

}  // namespace mfh
