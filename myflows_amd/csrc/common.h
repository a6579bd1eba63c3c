// Shared host-side plumbing of libmfhip: status codes, the thread-local error text, launch checks
// and the declarations through which the C-ABI translation unit (api.hip) reaches the kernels of
// conv.hip, gemm.hip and matmul.hip. Every kernel indexes its buffers with int32 offsets; the
// entry points reject larger problems before launching anything.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace mfh {

enum Status : int {
    OK = 0,
    ERR_INIT = 1,
    ERR_ARG = 2,
    ERR_HIP = 3,
    ERR_UNUSED = 4,  // kept free so that status numbers line up with the reference's codes
    ERR_DEVICE = 5,
};

enum Activation : int { ACT_NONE = 0, ACT_RELU = 1, ACT_LEAKY_RELU = 2 };

constexpr std::int64_t INDEX_LIMIT = 2147483647;  // int32 element offsets inside every kernel
constexpr unsigned GRID_YZ_LIMIT = 65535;

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
#define MFH_TRY(call)                           \
    do {                                        \
        const int mfh_rc_ = (call);             \
        if (mfh_rc_ != ::mfh::OK) return mfh_rc_; \
    } while (0)
#define MFH_REQUIRE(condition, message)                                   \
    do {                                                                  \
        if (!(condition)) return MFH_FAIL(::mfh::ERR_ARG, (message));     \
    } while (0)
#define MFH_CHECK_LAUNCH(name, stream) ::mfh::after_launch((name), (stream), __FILE_NAME__, __LINE__)

struct ConvDims {
    int N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW;
};

// ---- conv.hip ---------------------------------------------------------------------------------
int launch_im2col(const float* x, float* cols, const ConvDims& d, hipStream_t stream);
int launch_col2im(const float* grad_cols, float* dx, const ConvDims& d, hipStream_t stream);
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

// Loads the code object of this file's kernels (fails when the device has no gfx950 binary).
int conv_probe_kernels();

// ---- gemm.hip ---------------------------------------------------------------------------------
struct GemmTile {
    int bm, bn, bk, wm, wn;  // block tile, reduction depth per LDS stage, wave tile
};
int gemm_tile_count();
const GemmTile& gemm_tile(int index);

struct GemmPlan {
    int tile, slices, k_chunk;
};
// Tile and split-K choice for C(M, N) over K (the engine's automatic plan).
GemmPlan gemm_auto_plan(int M, int N, int K);
// Plan from an engine code: 1 = automatic, 16 + tile * 128 + (slices - 1) = explicit.
int gemm_plan_from_engine(int engine, int M, int N, int K, GemmPlan* plan);
bool gemm_engine_valid(int engine);
std::int64_t gemm_workspace_floats(const GemmPlan& plan, int M, int N);

// Row-major C(M x N) = op(A) op(B); A stored K x M when trans_a, B stored N x K when trans_b.
// Splits K through the workspace only when it holds the plan's slices * M * N floats.
int gemm_rows(int engine, hipStream_t stream, bool trans_a, bool trans_b, int M, int N, int K, const float* a,
              int lda, const float* b, int ldb, float* c, int ldc, float* workspace, std::int64_t workspace_floats);
int gemm_rows_bias(int engine, hipStream_t stream, bool trans_a, bool trans_b, int M, int N, int K, const float* a,
                   int lda, const float* b, int ldb, float* c, int ldc, const float* bias, float* workspace,
                   std::int64_t workspace_floats);
int split_reduce(const float* partial, float* c, int slices, int M, int N, int ldc, bool reference,
                 hipStream_t stream);

// ---- matmul.hip -------------------------------------------------------------------------------
// variant 0 basic, 1 tiled, 2 shared, 4 register (kahan / dot2 accumulation only); see matmul.hip.
int launch_matmul(int variant, int tile, int accumulate, const float* a, const float* b, float* c, int M, int N,
                  int K, hipStream_t stream);

}  // namespace mfh
