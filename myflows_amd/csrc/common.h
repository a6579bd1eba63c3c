// Host-side plumbing shared by the translation units of libmfhip: status codes, the thread-local
// error text, launch checks, and the internal interfaces through which the C ABI (api.hip) reaches
// the kernels of conv.hip, gemm.hip, matmul.hip, norm.hip and pointwise.hip. Every kernel indexes
// its buffers with int32 offsets; the entry points reject larger problems before launching anything.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "fastdiv.h"
#include "launch.h"

namespace mfh {

enum Status : int {
    OK = 0,
    ERR_INIT = 1,
    ERR_ARG = 2,
    ERR_HIP = 3,
    ERR_UNUSED = 4,  // kept free so that status numbers line up with the reference's codes
    ERR_DEVICE = 5,
};

// Activation codes of the C ABI.
constexpr int ACT_NONE = 0, ACT_RELU = 1, ACT_LEAKY_RELU = 2;

constexpr std::int64_t INDEX_LIMIT = 2147483647;  // int32 element offsets inside every kernel
constexpr unsigned GRID_YZ_LIMIT = 65535;         // hardware limit of gridDim.y and gridDim.z

// Records "file:line: what" as this thread's last error and returns status.
int fail(int status, const char* file, int line, const std::string& what);

// Checks the launch that was just issued (and, in debug-sync mode, the stream) and names the kernel.
int after_launch(const char* kernel, hipStream_t stream, const char* file, int line);

bool debug_sync_enabled();
int device_cu_count();

inline unsigned blocks_for(std::int64_t total, unsigned threads) {
    return static_cast<unsigned>((total + threads - 1) / threads);
}

inline bool fits_index(std::int64_t value) { return value >= 0 && value <= INDEX_LIMIT; }

#define MFH_FAIL(status, what) ::mfh::fail((status), __FILE_NAME__, __LINE__, (what))
#define MFH_TRY(call)                             \
    do {                                          \
        const int mfh_rc_ = (call);               \
        if (mfh_rc_ != ::mfh::OK) return mfh_rc_; \
    } while (0)
#define MFH_REQUIRE(condition, message)                               \
    do {                                                              \
        if (!(condition)) return MFH_FAIL(::mfh::ERR_ARG, (message)); \
    } while (0)
#define MFH_CHECK_LAUNCH(name, stream) ::mfh::after_launch((name), (stream), __FILE_NAME__, __LINE__)

// Geometry of one 2-D convolution (NCHW input, OIHW weight).
struct ConvGeometry {
    int N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW;
    int ohw() const { return OH * OW; }
    int rows() const { return N * OH * OW; }     // M of the im2col matrix
    int features() const { return CI * KH * KW; }  // K of the im2col matrix
};

// The column gradient of a convolution's dX as a convolution: the dX of a 1x1 convolution from
// CI*KH*KW channels to CO channels on the OH x OW output grid (whose input is the per-image column
// gradient [n][CI*KH*KW][OH*OW]).
inline ConvGeometry column_geometry(const ConvGeometry& g) {
    return ConvGeometry{g.N, g.CI * g.KH * g.KW, g.OH, g.OW, g.CO, 1, 1, g.OH, g.OW, 1, 1, 0, 0};
}

// ---- conv.hip ---------------------------------------------------------------------------------
int launch_im2col(const float* x, float* cols, const ConvGeometry& g, hipStream_t stream);
// dx from the feature-major column gradient: gcT[n][CI*KH*KW][OH*OW] when per_image, else
// gcT[CI*KH*KW][N*OH*OW]. With accumulate, dx += the gathered sums instead of dx = them.
int launch_col2im_t(const float* gcT, float* dx, const ConvGeometry& g, bool per_image, bool accumulate,
                    hipStream_t stream);
int launch_conv_epilogue(const float* rows, const float* bias, float* y, int N, int OHW, int CO, int act,
                         float alpha, hipStream_t stream);
int conv_grad_tile();  // pixels per conv_grad_rows tile (grid_x counts these tiles)
int launch_conv_grad_rows(const float* dy, const float* y, float* dyT, double* partial, int N, int OHW, int CO,
                          int grid_x, int act, float alpha, hipStream_t stream);
int launch_reduce_partials(const double* partial, float* out, int count, int width, hipStream_t stream);
int launch_add_bias(float* rows, const float* bias, int M, int N, hipStream_t stream);
int launch_pool_forward(const float* x, float* y, int* argmax, int N, int C, int H, int W, int OH, int OW,
                        int KH, int KW, int SH, int SW, hipStream_t stream);
int launch_pool_backward(const float* dy, const int* argmax, float* dx, int N, int C, int H, int W, int OH,
                         int OW, int KH, int KW, int SH, int SW, hipStream_t stream);

// Loads the code object of this library's kernels (fails when the device has no gfx950 binary).
int probe_code_object();

// The bandwidth kernels on a training step's critical path (every batch-norm kernel, the plain
// split-K reductions) run their waves at a raised issue priority (s_setprio 2: the priority of a
// wave within its CU, not of a stream). In the backward they run on the main stream beside the
// weight-gradient products of the other stream, whose waves share their SIMDs: issued first, their
// loads and sums no longer wait behind the products' MFMAs, and the main stream's chain of
// dependent kernels moves on sooner (the batch-64 step 3.754 -> 3.615 ms on MI355X, the same bits).
// The products themselves keep the default: raising the forward / dX products over the dW products
// was slower.
__device__ __forceinline__ void raise_wave_priority() { __builtin_amdgcn_s_setprio(2); }

// ---- gemm.hip ---------------------------------------------------------------------------------
struct GemmTile {
    int bm, bn, bk, wm, wn;  // block tile, reduction depth per LDS stage, wave tile
    int kg = 1;              // K groups: sets of (BM/WM) x (BN/WN) waves that share the tile's K range
};
// Tile catalogue of the MFMA kernels: block tile BM x BN, stage depth BK, wave tile WM x WN
// (multiples of 32).
inline constexpr GemmTile GEMM_TILES[] = {
    {128, 128, 16, 64, 64},  // 0: general
    {256, 64, 16, 64, 64},   // 1: tall outputs, N <= 64
    {64, 128, 16, 32, 64},   // 2: short outputs, M <= 64
    {64, 64, 16, 32, 32},    // 3: small outputs
    {128, 32, 16, 32, 32},   // 4: N <= 32
    {32, 128, 16, 32, 32},   // 5: M <= 32
    {256, 128, 16, 64, 64},  // 6: large outputs, 8 waves
    {128, 256, 16, 64, 64},  // 7: large outputs, 8 waves
    {64, 64, 16, 32, 32, 2},  // 8: small outputs: two groups of four waves share the K range
    {256, 256, 32, 64, 64},  // 9: large outputs, 16 waves, 32-deep stages (one workgroup per CU)
};
constexpr int GEMM_TILE_COUNT = sizeof(GEMM_TILES) / sizeof(GEMM_TILES[0]);
constexpr unsigned ALL_TILES = (1u << GEMM_TILE_COUNT) - 1;
constexpr GemmTile gemm_tile_constexpr(int index) { return GEMM_TILES[index]; }
int gemm_tile_count();
const GemmTile& gemm_tile(int index);

struct GemmPlan {
    int tile, slices, k_chunk;
};
// Tile and split-K choice for C(M, N) over K, or for `batch` such problems at once (never split),
// among the tiles whose bits are set in `tiles`.
GemmPlan gemm_auto_plan(int M, int N, int K, int batch = 1, unsigned tiles = ALL_TILES);
// Plan from an engine code: 1 = automatic, 16 + tile * 128 + (slices - 1) = explicit.
int gemm_plan_from_engine(int engine, int M, int N, int K, GemmPlan* plan, int batch = 1);
bool gemm_engine_valid(int engine);
std::int64_t gemm_workspace_floats(const GemmPlan& plan, int M, int N);

constexpr int BIAS_NONE = 0, BIAS_COLUMN = 1, BIAS_ROW = 2;

// Kernel argument block of the MFMA GEMM (see gemm.hip for the meaning of split, the batches and
// the segmented output).
struct GemmParams {
    const float* A;
    const float* B;
    float* C;
    const float* bias;
    int M, N, K, lda, ldb, ldc;
    int k_chunk, split;
    long long a_batch, b_batch, c_batch;
    int bias_mode, act;
    float alpha;
    int segment;               // 0: C is dense; > 0: output column j is (j / segment, j % segment)
    FastDiv segment_div;       // division by segment
    long long segment_stride;  // distance between consecutive segments of C
    int taps;                  // > 0: columns are convolution features in chunked order (see ConvGather)
    FastDiv taps_div;          // division by taps
    int accumulate;            // 1: each output is added to what C holds (C = C + result)
    const float* residual;     // non-null: added to (product + bias) before the activation, C's layout
    // > 0: a segment is a lattice_w-wide grid of a larger plane, element (i, j) of the segment at
    // i * lattice_row + j * lattice_col + lattice_offset (the phases of a strided dX).
    int lattice_w;
    FastDiv lattice_div;       // division by lattice_w
    int lattice_row, lattice_col, lattice_offset;
    // > 0 (lattice of phase (0, 0) only): element (i, j) also zeroes the other positions of its
    // cell_h x cell_w cell (rows cell_h * i + a, columns cell_w * j + b of a plane_h x plane_w
    // plane), which no product writes (the other phases of a strided dX have no taps).
    int cell_h, cell_w, plane_h, plane_w;
    // Split-K reduction only: also row_out[r] = (float) sum over z of row_partial[z * row_count + r]
    // (FP64, in z order) for r < row_count, with row_slices values of z.
    const double* row_partial;
    float* row_out;
    int row_count, row_slices;
};

// One GEMM problem, or `batch` of them at constant strides: C(M x N) = op(A) op(B), row-major;
// A is stored K x M when trans_a, B is stored N x K when trans_b.
struct GemmOperands {
    bool trans_a, trans_b;
    int M, N, K;
    const float* a;
    int lda;
    const float* b;
    int ldb;
    float* c;
    int ldc;
    int batch = 1;
    long long a_batch = 0, b_batch = 0, c_batch = 0;
};

// What happens to each output after the product: + bias (per column or per row), activation, and
// where it goes. With segment > 0 output (i, j) is stored at
// c + (j / segment) * segment_stride + i * ldc + j % segment: one GEMM over all images writes an
// NCHW tensor (segment = OH*OW, segment_stride = C*OH*OW, ldc = OH*OW).
struct GemmEpilogue {
    const float* bias = nullptr;
    int bias_mode = BIAS_NONE;
    int act = ACT_NONE;
    float alpha = 0.0f;
    int segment = 0;
    long long segment_stride = 0;
    int taps = 0;  // KH*KW when the output columns are features in chunked order; stored in natural order
    bool accumulate = false;  // C = C + result: a gradient added to one already there, in one pass
    const float* residual = nullptr;  // act(product + bias + residual), residual laid out as C
    // Segments spread over a lattice of a larger plane (see GemmParams::lattice_w); 0: contiguous.
    int lattice_w = 0, lattice_row = 0, lattice_col = 0, lattice_offset = 0;
    int cell_h = 0, cell_w = 0, plane_h = 0, plane_w = 0;  // see GemmParams::cell_h
    // With a split-K reduction: row sums of FP64 slice partials finished in the same launch
    // (row_out[r] = sum over the slices of row_partial[z * row_count + r]).
    const double* row_partial = nullptr;
    float* row_out = nullptr;
    int row_count = 0;
};

// Runs the engine; splits K through the workspace (never for batches) only when it holds the
// plan's slices * M * N floats.
int gemm_launch(int engine, hipStream_t stream, const GemmOperands& operands, const GemmEpilogue& epilogue,
                float* workspace, std::int64_t workspace_floats);
// Workspace floats gemm_launch uses for one problem with a plain epilogue (bias per column at
// most) when it is given all it asks for: the plan's slices * M * N, or 0 (no split, or an output
// of at most 8 columns under the automatic plan, which takes the one-wave-per-row kernel).
std::int64_t gemm_launch_workspace(int engine, int M, int N, int K);
int split_reduce(const float* partial, float* c, int slices, int M, int N, int ldc, bool reference,
                 hipStream_t stream);
// The FP64 slice-order reduction of split-K partials (slices x M x N, dense) followed by the
// epilogue e (bias, activation, dense rows of ldc or segmented output).
int split_reduce_epilogue(const float* partial, float* c, const GemmEpilogue& e, int M, int N, int ldc, int slices,
                          hipStream_t stream);
// The same reduction for many slices over few outputs: the slices in 8 contiguous groups, each
// summed in slice order in FP64, then the groups added in order (a fixed regrouping of the sum).
int split_reduce_grouped(const float* partial, float* c, const GemmEpilogue& e, int M, int N, int ldc, int slices,
                         hipStream_t stream);

// ---- implicit.hip -----------------------------------------------------------------------------
// The im2col view of an NCHW source read in place: view[k][q] = src[n, c, oh*SH - PH + kh,
// ow*SW - PW + kw] (0 outside), pixel q = (n*OH + oh)*OW + ow. Feature k is (c, tap = kh*KW + kw)
// in natural order, k = c*KH*KW + tap, or, when `chunked` (C a multiple of 32), in chunked order
// k = ((c / 32)*KH*KW + tap)*32 + c % 32: every run of 32 features then shares one window tap.
constexpr int CHANNEL_CHUNK = 32;
struct ConvGather {
    const float* src;
    int C, H, W;
    int KH, KW, SH, SW, PH, PW;
    int OH, OW;
    int pixels;    // N * OH * OW
    int features;  // C * KH * KW
    int hw, chw;   // H * W, C * H * W
    int chunked;
    FastDiv div_ohw, div_ow, div_khkw, div_kw;
    long long src_floats;  // N * C * H * W: the extent of src that the buffer loads may read
    // Natural feature order only: when non-null, src with PH / PW zero rows / columns on each side
    // ((H + 2 PH) x (W + 2 PW) planes of pw columns, phw floats each, padded_floats in all), which the
    // products read without window bounds tests.
    const float* padded;
    int pw, phw;
    long long padded_floats;
};
// The chunked implicit products read their operands with buffer loads, whose byte offsets are 32-bit:
// each operand tensor they read must hold at most this many floats.
constexpr std::int64_t BUFFER_LIMIT_FLOATS = 2147483647 / 4;
constexpr int IMPLICIT_FORWARD = 0, IMPLICIT_WGRAD = 1, IMPLICIT_DGRAD = 2;
// Split-K workspace floats of one pass of the implicit convolution under the automatic plan.
std::int64_t implicit_workspace_floats(const ConvGeometry& g, int pass);
// Whether an engine code names the automatic plan or a tile and split of the implicit products.
bool implicit_engine_valid(int engine);
// Whether the implicit kernels take a convolution over C input channels in chunked feature order.
inline bool implicit_chunked(int C) { return C % CHANNEL_CHUNK == 0; }
// y = act(conv(x, w) + bias), NCHW, without an im2col buffer. When C is chunked the product reads
// the kernel in the order launch_weight_orders writes (flip 0): from wt, which this call fills
// from w unless `prepared` says that it holds that order already.
int conv_implicit_forward(const ConvGeometry& g, const float* x, const float* w, float* wt, bool prepared,
                          const float* bias, const float* residual, float* y, int act, float alpha, int engine,
                          float* workspace, std::int64_t workspace_floats, hipStream_t stream,
                          int* deferred = nullptr);
// dW = dy . im2col(x), with dy read in place from NCHW. With db, the workgroups of the first
// feature tile also sum dy over their pixel slice in FP64; an unsplit product writes db itself, a
// split one leaves bias_partial[z * CO + co] for slice z (at most WGRAD_MAX_SLICES) and its
// reduction finishes db in slice order.
int conv_implicit_wgrad(const ConvGeometry& g, const float* x, const float* dy, float* dw, double* bias_partial,
                        float* db, int engine, float* workspace, std::int64_t workspace_floats, hipStream_t stream);
// dX of a stride-1 convolution as a forward convolution of dy with the flipped kernel, read from
// wflip (CI x CO*KH*KW floats in the order launch_weight_orders writes with flip 1), which this call
// fills from w unless `prepared`. With accumulate, dx += the result. With `deferred`, a product
// split over K that writes dx fresh may leave its FP32 slices in the workspace for the caller to
// reduce (slice z of CI x N*H*W floats at workspace + z * CI * N*H*W; dx unwritten): *deferred
// receives the slice count, or 1 when dx was written here.
int conv_implicit_dgrad(const ConvGeometry& g, const float* dy, const float* w, float* wflip, bool prepared, float* dx,
                        bool accumulate, int engine, float* workspace, std::int64_t workspace_floats,
                        hipStream_t stream, int* deferred = nullptr);
// dX of a strided convolution as SH*SW phase products (see DgradPhase), each a stride-1 implicit
// convolution of dy with its flipped sub-kernel whose epilogue writes the phase's lattice of dx.
// The sub-kernels are read from wphase (CI*CO*KH*KW floats in the order launch_weight_orders
// writes with flip 1 for this geometry), which this call fills from w unless `prepared`. Input
// positions that no tap reaches are zeroed (or left as they are with accumulate).
int conv_implicit_dgrad_phases(const ConvGeometry& g, const float* dy, const float* w, float* wphase, bool prepared,
                               float* dx, bool accumulate, int engine, float* workspace,
                               std::int64_t workspace_floats, hipStream_t stream);
// One phase of the dX of a strided convolution (sub-pixel decomposition). The input positions
// (ih, iw) = (SH*i + a, SW*j + b) receive dy only through the taps kh = rh + SH*t, kw = rw + SW*u
// (t < th, u < tw), from dy[oh = i + ch - t][ow = j + cw - u]: a stride-1 convolution of dy with
// that sub-kernel, flipped, under padding (pad_h, pad_w), over an hp x wp output grid. The phases
// (a, b) in [0, SH) x [0, SW) partition both the input positions and the taps; stride 1 has the
// single phase (0, 0), the whole kernel flipped under padding KH-1-PH.
struct DgradPhase {
    int a, b, rh, rw, th, tw, hp, wp, pad_h, pad_w;
};
inline DgradPhase dgrad_phase(const ConvGeometry& g, int a, int b) {
    DgradPhase p{};
    p.a = a;
    p.b = b;
    p.rh = (a + g.PH) % g.SH;
    p.rw = (b + g.PW) % g.SW;
    p.th = p.rh < g.KH ? (g.KH - p.rh + g.SH - 1) / g.SH : 0;
    p.tw = p.rw < g.KW ? (g.KW - p.rw + g.SW - 1) / g.SW : 0;
    p.hp = a < g.H ? (g.H - a + g.SH - 1) / g.SH : 0;
    p.wp = b < g.W ? (g.W - b + g.SW - 1) / g.SW : 0;
    p.pad_h = p.th - 1 - (a + g.PH - p.rh) / g.SH;
    p.pad_w = p.tw - 1 - (b + g.PW - p.rw) / g.SW;
    return p;
}

// The kernel W (CO, CI, KH, KW) in the order an implicit product reads it: flip 0 for the forward
// (CO rows over (ci, tap) features), flip 1 for the dX (CI rows over (co, flipped tap) features;
// for a stride above 1, the flipped sub-kernel of each dX phase in turn, phases in (a, b) order),
// each in chunked feature order when its channel count is chunked. SH, SW, PH, PW matter for the
// strided dX order only.
struct WeightOrder {
    const float* w;
    float* out;
    int CO, CI, KH, KW, flip, SH = 1, SW = 1, PH = 0, PW = 0;
};
constexpr int WEIGHT_ORDER_DIMS = 9;  // ints per kernel in mfh_conv_weight_orders' dims
// All `count` orders in as few launches as the kernel arguments allow.
int launch_weight_orders(const WeightOrder* orders, int count, hipStream_t stream);
// Largest number of pixel slices the dW plan makes (rows of conv_implicit_wgrad's bias_partial).
constexpr int WGRAD_MAX_SLICES = 256;
// partial[r] = FP64 sum of row r (rows x length floats).
int launch_row_sums(const float* src, double* partial, int rows, int length, hipStream_t stream);

// ---- matmul.hip -------------------------------------------------------------------------------
// variant 0 basic, 1 tiled, 2 shared, 4 register (compensated modes); see matmul.hip.
int launch_matmul(int variant, int tile, int accumulate, const float* a, const float* b, float* c, int M, int N,
                  int K, hipStream_t stream);

// ---- norm.hip ---------------------------------------------------------------------------------
// Batch normalisation over the (N, H*W) positions of each channel of an NCHW tensor.
struct NormShape {
    int N, C, HW;
};
// Per-channel slices of the FP64 partial-sum pass and the workspace doubles they need.
int norm_slices(const NormShape& s);
std::int64_t norm_workspace_doubles(const NormShape& s);

struct NormForward {
    const float* x;
    const float* gamma;
    const float* beta;
    float* running_mean;  // updated in place when training
    float* running_var;
    const float* residual;  // optional same-shape tensor added after the affine transform
    float* y;
    float* mean;     // 2 x C: FP64 mean split into hi + lo floats
    float* inv_std;  // C
    double* partial;
    bool training, relu;
    double momentum, eps, var_scale;
};
int norm_forward(const NormShape& s, const NormForward& f, hipStream_t stream);
// Training forward of a one-launch shape whose x is formed first from `slices` split-K slices of a
// convolution product (partial: slices x C x N*HW floats) plus the convolution's bias (optional),
// and stored into x.
int norm_forward_split(const NormShape& s, const NormForward& f, const float* partial, int slices, const float* bias,
                       float* x, hipStream_t stream);

struct NormBackward {
    const float* x;
    const float* dy;
    const float* gate;  // optional forward output of a fused ReLU: dy counts only where gate > 0
    const float* gamma;
    const float* mean;
    const float* inv_std;
    float* x_grad;
    float* gamma_grad;
    float* beta_grad;
    float* residual_grad;  // optional: receives the gated dy (the residual branch of a fused Add)
    double* partial;
    bool training, add_x, add_gamma, add_beta, add_residual;
};
int norm_backward(const NormShape& s, const NormBackward& b, hipStream_t stream);
// Backward of a one-launch shape (a pass with sums) whose dy is formed first from `slices` split-K
// slices of a convolution's dX product (partial: slices x C x N*HW floats) and stored into dy,
// which must be b.dy.
int norm_backward_split(const NormShape& s, const NormBackward& b, const float* partial, int slices, float* dy,
                        hipStream_t stream);

// Batch norm + ReLU + max-pool (no padding) as one unit; the ReLU output is never stored. The
// forward writes the pooled values and their int32 flat argmax into the N x C x H x W tensor, the
// backward takes the pooled gradient and that argmax (NormBackward's dy, gate and residual fields
// are unused). Same bits as norm_forward with relu, the max-pool, and their backward passes.
struct PoolDims {
    int H, W, OH, OW, KH, KW, SH, SW;
};
bool norm_pool_supported(const NormShape& s, const PoolDims& d);
int norm_relu_pool_forward(const NormShape& s, const NormForward& f, const PoolDims& d, float* pooled, int* argmax,
                           hipStream_t stream);
int norm_relu_pool_backward(const NormShape& s, const NormBackward& b, const PoolDims& d, const float* pooled_grad,
                            const int* argmax, const float* beta, hipStream_t stream);

// ---- pointwise.hip ----------------------------------------------------------------------------
int launch_relu_forward(const float* x, float* y, std::int64_t count, hipStream_t stream);
// p[0 .. count) = 0 (a kernel, not a memset, so that it may sit in a captured graph)
int launch_fill(float* p, std::int64_t count, float value, hipStream_t stream);
int launch_fill_zero(float* p, std::int64_t count, hipStream_t stream);
// out (+)= x > 0 ? g : alpha * g   (alpha = 0 for ReLU)
int launch_relu_backward(const float* x, const float* g, float* out, std::int64_t count, float alpha, bool add,
                         hipStream_t stream);

// One tensor of a multi-tensor Adam step.
struct AdamTensor {
    float* param;
    const float* grad;
    float* m;
    float* v;
    std::int64_t size;
    float lr, decay, bc1, bc2;  // learning rate, weight decay, bias corrections 1 - beta^step (float32)
};
struct AdamScalars {
    float grad_scale, b1, omb1, b2, omb2, eps;
};
int launch_adam(const AdamTensor* tensors, int count, const AdamScalars& s, hipStream_t stream);

// ---- head.hip -------------------------------------------------------------------------------
// y[p] = float(FP64 mean of x[p * hw .. p * hw + hw))
int launch_plane_mean(const float* x, float* y, std::int64_t planes, int hw, hipStream_t stream);
// dx[p * hw + i] (+)= dy[p] / float(hw)
int launch_plane_mean_backward(const float* dy, float* dx, std::int64_t planes, int hw, bool add, hipStream_t stream);
// loss[0] = float(FP64 sum of float32 (pred - target)^2 / count), NaN when count is 0
int launch_mse_loss(const float* pred, const float* target, float* loss, std::int64_t count, hipStream_t stream);
// grad (+)= seed[0] * ((2 * (pred - target)) / float(count)), float32 in that order
int launch_mse_grad(const float* pred, const float* target, const float* seed, float* grad, std::int64_t count,
                    bool add, hipStream_t stream);
// out[j] = float(FP64 sum over r of src[r * cols + j])
int launch_column_sums(const float* src, float* out, std::int64_t rows, std::int64_t cols, hipStream_t stream);

}  // namespace mfh
