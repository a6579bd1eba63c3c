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
// Both gather loaders keep one pixel per thread column so that the pixel's decomposition
// (n, oh, ow) is done once per stage (dW) or once per kernel (forward); in the forward loader every
// wave reads one feature row k, so k's decomposition is a wave-uniform scalar computation.
#include "common.h"
#include "gemm_core.h"

namespace mfh {
namespace {

constexpr int BK = 16;
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

// The decomposition of one output pixel q (dW orientation: thread t handles pixel kt + t % BK).
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

// dW orientation: a BN x BK tile of the transposed view, rows = features [n0, n0 + BN), columns =
// pixels [kt, kt + BK), stored k-contiguous ([BN][BK + 4]). A thread's feature rows are fixed for
// the whole kernel, so their (c, kh, kw) offsets are decomposed once.
template <int BN, int THREADS>
struct GatherPixelColumns {
    static_assert(THREADS % BK == 0 && BN % (THREADS / BK) == 0, "rows split evenly over the threads");
    static constexpr int RSTEP = THREADS / BK, PER = BN / RSTEP;
    int offset[PER], kh[PER], kw[PER];
    float v[PER];

    __device__ __forceinline__ void init(const ConvGather& g, int n0, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int k = n0 + tid / BK + i * RSTEP;
            if (k < g.features) {
                int rem, w;
                const int c = g.div_khkw.divmod(k, rem);
                const int h = g.div_kw.divmod(rem, w);
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
        const int r0 = tid / BK, col = tid % BK;
#pragma unroll
        for (int i = 0; i < PER; ++i) lds[(r0 + i * RSTEP) * LD + col] = v[i];
    }
};

// dW's A operand: dy read in place, A[co][q] = dy[n, co, p] for pixel q = (n, p), as a BM x BK
// k-contiguous tile (rows = output channels, columns = the same pixels as the gathered tile).
template <int BM, int THREADS>
struct GradRowsInPlace {
    static constexpr int RSTEP = THREADS / BK, PER = BM / RSTEP;
    static_assert(BM % RSTEP == 0, "rows split evenly over the threads");
    float v[PER];

    __device__ __forceinline__ void load(const float* __restrict__ dy, int CO, int ohw, int m0, const PixelAt& at,
                                         int tid) {
        const int base = (at.n * CO + m0 + tid / BK) * ohw + at.p;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int row = m0 + tid / BK + i * RSTEP;
            v[i] = at.valid && row < CO ? dy[base + i * RSTEP * ohw] : 0.0f;
        }
    }

    template <int LD>
    __device__ __forceinline__ void store(float* lds, int tid) const {
        const int r0 = tid / BK, col = tid % BK;
#pragma unroll
        for (int i = 0; i < PER; ++i) lds[(r0 + i * RSTEP) * LD + col] = v[i];
    }
};

// Y (M x pixels) = A (M x K, row-major, lda) . view (K x pixels). Split-K writes dense partials
// (z-th slice at C + z * c_batch); otherwise the epilogue of p (segmented NCHW, bias, activation).
template <int BM, int BN, int WM, int WN, bool VA>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv_implicit_forward_kernel(GemmParams p,
                                                                                          ConvGather g) {
    using S = MfmaShape<BM, BN, BK, WM, WN, false, false>;
    __shared__ __attribute__((aligned(16))) float smem[2 * S::STAGE];
    int tile_m, tile_n, z;
    tile_of_workgroup(tile_m, tile_n, z);
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm0 = (wave / S::WGN) * WM, wn0 = (wave % S::WGN) * WN;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int k_begin = p.split ? z * p.k_chunk : 0;
    const int k_end = p.split ? min(p.K, k_begin + p.k_chunk) : p.K;
    float* __restrict__ C = p.C + (p.split ? z * p.c_batch : 0);

    TileLoader<BM, BK, S::THREADS, VA> la;
    GatherFeatureRows<BN, S::THREADS> lb;
    lb.init(g, n0, tid);
    auto fetch = [&](int kt) {
        la.load(p.A, p.lda, m0, p.M, kt, k_end, tid);
        lb.load(g, kt, k_end, tid);
    };
    auto store = [&](float* a_lds, float* b_lds) {
        la.template store<S::LDA_S>(a_lds, tid);
        lb.template store<S::LDB_S>(b_lds, tid);
    };
    v16f acc[S::TM][S::TN];
    zero_acc<S>(acc);
    mfma_k_loop<S>(smem, k_begin, k_end, fetch, store, acc, wm0, wn0, lane);
    store_acc<S>(p, C, acc, m0, n0, wm0, wn0, lane);
}

// dW (CO x K) = dy (CO x pixels) . view^T (pixels x K), the pixel range split over z when p.split.
template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void conv_implicit_wgrad_kernel(GemmParams p,
                                                                                        ConvGather g) {
    using S = MfmaShape<BM, BN, BK, WM, WN, false, true>;
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

    GradRowsInPlace<BM, S::THREADS> la;
    GatherPixelColumns<BN, S::THREADS> lb;
    lb.init(g, n0, tid);
    auto fetch = [&](int kt) {
        const PixelAt at = pixel_at(g, kt + tid % BK, k_end);
        la.load(p.A, p.M, ohw, m0, at, tid);
        lb.load(g, at);
    };
    auto store = [&](float* a_lds, float* b_lds) {
        la.template store<S::LDA_S>(a_lds, tid);
        lb.template store<S::LDB_S>(b_lds, tid);
    };
    v16f acc[S::TM][S::TN];
    zero_acc<S>(acc);
    mfma_k_loop<S>(smem, k_begin, k_end, fetch, store, acc, wm0, wn0, lane);
    store_acc<S>(p, C, acc, m0, n0, wm0, wn0, lane);
}

// wflip[ci][co][kh][kw] = w[co][ci][KH-1-kh][KW-1-kw]: the kernel of dX as a forward convolution.
__global__ __launch_bounds__(256) void weight_flip_kernel(const float* __restrict__ w, float* __restrict__ wflip,
                                                          int total, int CO, int CI, int KHW) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int tap = idx % KHW;
    const int co = (idx / KHW) % CO;
    const int ci = idx / (KHW * CO);
    wflip[idx] = w[(co * CI + ci) * KHW + (KHW - 1 - tap)];
}

// partial[row] = sum of the row's `length` floats in FP64 (rows are the (n, co) planes of dy). One
// wave per row: lane l adds elements l, l + 64, ... in order, then a fixed butterfly adds the lanes.
__global__ __launch_bounds__(256) void row_sums_kernel(const float* __restrict__ src, double* __restrict__ partial,
                                                       int rows, int length) {
    const int row = blockIdx.x * 4 + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= rows) return;
    const float* r = src + static_cast<long long>(row) * length;
    double s = 0.0;
    for (int i = lane; i < length; i += 64) s += static_cast<double>(r[i]);
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) s += __shfl_xor(s, offset, 64);
    if (lane == 0) partial[row] = s;
}

using ConvFn = void (*)(GemmParams, ConvGather);

// Forward tiles need BN to be a multiple of 64 (one feature row per wave); every tile serves dW.
constexpr unsigned FORWARD_TILES = (1u << 0) | (1u << 1) | (1u << 2) | (1u << 3) | (1u << 6) | (1u << 7);

template <int T, bool VA>
constexpr ConvFn forward_of() {
    constexpr GemmTile t = gemm_tile_constexpr(T);
    return conv_implicit_forward_kernel<t.bm, t.bn, t.wm, t.wn, VA>;
}

template <int T>
constexpr ConvFn wgrad_of() {
    constexpr GemmTile t = gemm_tile_constexpr(T);
    return conv_implicit_wgrad_kernel<t.bm, t.bn, t.wm, t.wn>;
}

struct ConvKernels {
    ConvFn forward[8][2] = {};
    ConvFn wgrad[8] = {};
    ConvKernels() {
        forward[0][0] = forward_of<0, false>();
        forward[0][1] = forward_of<0, true>();
        forward[1][0] = forward_of<1, false>();
        forward[1][1] = forward_of<1, true>();
        forward[2][0] = forward_of<2, false>();
        forward[2][1] = forward_of<2, true>();
        forward[3][0] = forward_of<3, false>();
        forward[3][1] = forward_of<3, true>();
        forward[6][0] = forward_of<6, false>();
        forward[6][1] = forward_of<6, true>();
        forward[7][0] = forward_of<7, false>();
        forward[7][1] = forward_of<7, true>();
        wgrad[0] = wgrad_of<0>();
        wgrad[1] = wgrad_of<1>();
        wgrad[2] = wgrad_of<2>();
        wgrad[3] = wgrad_of<3>();
        wgrad[4] = wgrad_of<4>();
        wgrad[5] = wgrad_of<5>();
        wgrad[6] = wgrad_of<6>();
        wgrad[7] = wgrad_of<7>();
    }
};

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
    g.hw = H * W;
    g.chw = C * H * W;
    g.div_ohw = FastDiv(OH * OW);
    g.div_ow = FastDiv(OW);
    g.div_khkw = FastDiv(KH * KW);
    g.div_kw = FastDiv(KW);
    return g;
}

// The plan of a product: tile and K split, from an engine code, limited to the tiles a kernel
// family has; the split is dropped when the workspace cannot hold it.
int implicit_plan(int engine, int M, int N, int K, unsigned tiles, float* workspace, std::int64_t workspace_floats,
                  GemmPlan* plan) {
    if (engine == 1) *plan = gemm_auto_plan(M, N, K, 1, tiles);
    else MFH_TRY(gemm_plan_from_engine(engine, M, N, K, plan));
    if (!(tiles & (1u << plan->tile))) return MFH_FAIL(ERR_ARG, "this GEMM tile cannot run the implicit convolution");
    if (plan->slices > 1 && (!workspace || workspace_floats < gemm_workspace_floats(*plan, M, N)))
        *plan = GemmPlan{plan->tile, 1, K};
    const GemmTile& t = gemm_tile(plan->tile);
    if (blocks_for(M, t.bm) > GRID_YZ_LIMIT || static_cast<unsigned>(plan->slices) > GRID_YZ_LIMIT ||
        static_cast<std::int64_t>(blocks_for(M, t.bm)) * blocks_for(N, t.bn) * plan->slices > INDEX_LIMIT)
        return MFH_FAIL(ERR_ARG, "implicit convolution grid exceeds the launch limits");
    return OK;
}

// Runs one implicit product with the epilogue e (directly, or through split-K partials and the
// FP64 slice reduction).
int run_implicit(bool wgrad, const GemmPlan& plan, const float* a, int lda, int M, int N, int K, const ConvGather& g,
                 float* c, int ldc, const GemmEpilogue& e, float* workspace, hipStream_t stream) {
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
        p.C = c;
        p.ldc = ldc;
        p.bias = e.bias;
        p.bias_mode = e.bias_mode;
        p.act = e.act;
        p.alpha = e.alpha;
        p.segment = e.segment;
        if (e.segment > 0) p.segment_div = FastDiv(e.segment);
        p.segment_stride = e.segment_stride;
    }
    const GemmTile& t = gemm_tile(plan.tile);
    const dim3 grid(blocks_for(N, t.bn), blocks_for(M, t.bm), static_cast<unsigned>(plan.slices));
    const dim3 block((t.bm / t.wm) * (t.bn / t.wn) * 64);
    const bool vec_a = K % 4 == 0 && lda % 4 == 0 && aligned16(a);
    const ConvFn fn = wgrad ? conv_kernels().wgrad[plan.tile] : conv_kernels().forward[plan.tile][vec_a ? 1 : 0];
    hipLaunchKernelGGL(fn, grid, block, 0, stream, p, g);
    MFH_TRY(MFH_CHECK_LAUNCH(wgrad ? "conv_implicit_wgrad" : "conv_implicit_forward", stream));
    if (!split) return OK;
    return split_reduce_epilogue(workspace, c, e, M, N, ldc, plan.slices, stream);
}

}  // namespace

unsigned implicit_forward_tiles() { return FORWARD_TILES; }

std::int64_t implicit_workspace_floats(const ConvGeometry& g, int pass) {
    GemmPlan plan;
    if (pass == IMPLICIT_FORWARD) plan = gemm_auto_plan(g.CO, g.rows(), g.features(), 1, FORWARD_TILES);
    else if (pass == IMPLICIT_WGRAD) plan = gemm_auto_plan(g.CO, g.features(), g.rows(), 1, ALL_TILES);
    else plan = gemm_auto_plan(g.CI, g.N * g.H * g.W, g.CO * g.KH * g.KW, 1, FORWARD_TILES);
    return pass == IMPLICIT_WGRAD ? gemm_workspace_floats(plan, g.CO, g.features())
                                  : gemm_workspace_floats(plan, pass == IMPLICIT_FORWARD ? g.CO : g.CI,
                                                          pass == IMPLICIT_FORWARD ? g.rows() : g.N * g.H * g.W);
}

int conv_implicit_forward(const ConvGeometry& g, const float* x, const float* w, const float* bias, float* y, int act,
                          float alpha, int engine, float* workspace, std::int64_t workspace_floats,
                          hipStream_t stream) {
    const int M = g.CO, N = g.rows(), K = g.features();
    GemmPlan plan;
    MFH_TRY(implicit_plan(engine, M, N, K, FORWARD_TILES, workspace, workspace_floats, &plan));
    const ConvGather gather = gather_of(x, g.CI, g.H, g.W, g.KH, g.KW, g.SH, g.SW, g.PH, g.PW, g.N, g.OH, g.OW);
    GemmEpilogue e;
    e.bias = bias;
    e.bias_mode = bias ? BIAS_ROW : BIAS_NONE;
    e.act = act;
    e.alpha = alpha;
    e.segment = g.ohw();
    e.segment_stride = static_cast<long long>(g.CO) * g.ohw();
    return run_implicit(false, plan, w, K, M, N, K, gather, y, g.ohw(), e, workspace, stream);
}

int conv_implicit_wgrad(const ConvGeometry& g, const float* x, const float* dy, float* dw, int engine,
                        float* workspace, std::int64_t workspace_floats, hipStream_t stream) {
    const int M = g.CO, N = g.features(), K = g.rows();
    GemmPlan plan;
    MFH_TRY(implicit_plan(engine, M, N, K, ALL_TILES, workspace, workspace_floats, &plan));
    const ConvGather gather = gather_of(x, g.CI, g.H, g.W, g.KH, g.KW, g.SH, g.SW, g.PH, g.PW, g.N, g.OH, g.OW);
    return run_implicit(true, plan, dy, g.ohw(), M, N, K, gather, dw, N, GemmEpilogue{}, workspace, stream);
}

int conv_implicit_dgrad(const ConvGeometry& g, const float* dy, const float* w, float* wflip, float* dx, int engine,
                        float* workspace, std::int64_t workspace_floats, hipStream_t stream) {
    const int khw = g.KH * g.KW;
    const int M = g.CI, N = g.N * g.H * g.W, K = g.CO * khw;
    const int total = g.CI * K;
    weight_flip_kernel<<<blocks_for(total, 256), 256, 0, stream>>>(w, wflip, total, g.CO, g.CI, khw);
    MFH_TRY(MFH_CHECK_LAUNCH("weight_flip", stream));
    GemmPlan plan;
    MFH_TRY(implicit_plan(engine, M, N, K, FORWARD_TILES, workspace, workspace_floats, &plan));
    // dy as the source of a stride-1 convolution with padding KH-1-PH whose output grid is H x W.
    const ConvGather gather =
        gather_of(dy, g.CO, g.OH, g.OW, g.KH, g.KW, 1, 1, g.KH - 1 - g.PH, g.KW - 1 - g.PW, g.N, g.H, g.W);
    GemmEpilogue e;
    e.segment = g.H * g.W;
    e.segment_stride = static_cast<long long>(g.CI) * g.H * g.W;
    return run_implicit(false, plan, wflip, K, M, N, K, gather, dx, g.H * g.W, e, workspace, stream);
}

int launch_row_sums(const float* src, double* partial, int rows, int length, hipStream_t stream) {
    row_sums_kernel<<<blocks_for(rows, 4), 256, 0, stream>>>(src, partial, rows, length);
    return MFH_CHECK_LAUNCH("row_sums", stream);
}

}  // namespace mfh
