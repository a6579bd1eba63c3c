// The C ABI of libmfhip (declared in include/mfhip.h): initialisation, error reporting, argument
// validation and the launch sequences of the convolution, pooling, GEMM and matmul entry points.
// Validation follows the reference scheduler (ops/cuda_native/native_cublas.cpp:1379-1409 and the
// MF_REQUIRE checks of its entry points) so that the same bad calls fail with status 2 and a message
// naming the reason.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "../../include/mfhip.h"
#include "common.h"

namespace mfh {
namespace {

std::mutex init_mutex;
bool initialized = false;
bool debug_sync = false;
int init_device = -1;
int cu_count = 0;
std::string info_text = "{}";
thread_local std::string last_error;

int check_ready() {
    if (!initialized) return MFH_FAIL(ERR_INIT, "mfh_init has not succeeded");
    int device = -1;
    const hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess) return MFH_FAIL(ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(status));
    if (device != init_device) return MFH_FAIL(ERR_DEVICE, "called on a different HIP device than the one used by mfh_init");
    return OK;
}

int check_conv(const ConvDims& d) {
    const bool positive = d.N > 0 && d.CI > 0 && d.H > 0 && d.W > 0 && d.CO > 0 && d.KH > 0 && d.KW > 0 && d.OH > 0 &&
                          d.OW > 0 && d.SH > 0 && d.SW > 0 && d.PH >= 0 && d.PW >= 0;
    if (!positive) return MFH_FAIL(ERR_ARG, "convolution dimensions must be positive");
    if (d.OH != (d.H + 2 * d.PH - d.KH) / d.SH + 1 || d.OW != (d.W + 2 * d.PW - d.KW) / d.SW + 1)
        return MFH_FAIL(ERR_ARG, "convolution output size does not match input, kernel, stride and padding");
    const std::int64_t rows = static_cast<std::int64_t>(d.N) * d.OH * d.OW;
    const std::int64_t features = static_cast<std::int64_t>(d.CI) * d.KH * d.KW;
    if (!fits_index(rows * features) || !fits_index(rows * d.CO) ||
        !fits_index(static_cast<std::int64_t>(d.N) * d.CI * d.H * d.W) || !fits_index(features * d.CO))
        return MFH_FAIL(ERR_ARG, "convolution buffers exceed the int32 indexing limit");
    if (static_cast<unsigned>(d.N) > GRID_YZ_LIMIT || blocks_for(d.CO, conv_grad_tile()) > GRID_YZ_LIMIT)
        return MFH_FAIL(ERR_ARG, "batch or channel count exceeds the grid limit");
    return OK;
}

int check_activation(int activation, float alpha) {
    if (activation != ACT_NONE && activation != ACT_RELU && activation != ACT_LEAKY_RELU)
        return MFH_FAIL(ERR_ARG, "unknown activation code");
    if (activation == ACT_LEAKY_RELU && !(alpha > 0.0f)) return MFH_FAIL(ERR_ARG, "fused LeakyReLU requires alpha > 0");
    return OK;
}

int check_engine(int engine) {
    if (!gemm_engine_valid(engine)) return MFH_FAIL(ERR_ARG, "unknown GEMM engine or plan code");
    return OK;
}

int check_pool(int N, int C, int H, int W, int OH, int OW, int KH, int KW, int SH, int SW) {
    MFH_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0 && OH > 0 && OW > 0 && KH > 0 && KW > 0 && SH > 0 && SW > 0,
                "pooling dimensions must be positive");
    MFH_REQUIRE(OH == (H - KH) / SH + 1 && OW == (W - KW) / SW + 1, "pooling output size does not match the input");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(N) * C * H * W), "pooling input exceeds int32 indexing");
    return OK;
}

template <typename T>
T* ptr(std::uint64_t address) {
    return reinterpret_cast<T*>(static_cast<std::uintptr_t>(address));
}

hipStream_t as_stream(std::uint64_t handle) { return reinterpret_cast<hipStream_t>(static_cast<std::uintptr_t>(handle)); }

}  // namespace

int fail(int status, const char* file, int line, const std::string& what) {
    last_error = std::string(file) + ":" + std::to_string(line) + ": " + what;
    return status;
}

int after_launch(const char* kernel, hipStream_t stream, const char* file, int line) {
    const hipError_t launched = hipGetLastError();
    if (launched != hipSuccess)
        return fail(ERR_HIP, file, line, std::string("launch ") + kernel + ": " + hipGetErrorString(launched));
    if (debug_sync) {
        const hipError_t synced = hipStreamSynchronize(stream);
        if (synced != hipSuccess)
            return fail(ERR_HIP, file, line, std::string("after kernel ") + kernel + ": " + hipGetErrorString(synced));
    }
    return OK;
}

bool debug_sync_enabled() { return debug_sync; }
int device_cu_count() { return cu_count; }

}  // namespace mfh

using namespace mfh;

extern "C" {

MFH_API const char* mfh_last_error(void) { return last_error.c_str(); }

MFH_API const char* mfh_info(void) { return info_text.c_str(); }

MFH_API void mfh_set_debug_sync(int enabled) { debug_sync = enabled != 0; }

MFH_API int mfh_init(void) {
    std::lock_guard<std::mutex> lock(init_mutex);
    if (initialized) return OK;
    const auto start = std::chrono::steady_clock::now();
    int device = -1;
    hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess) return MFH_FAIL(ERR_INIT, std::string("hipGetDevice: ") + hipGetErrorString(status));
    hipDeviceProp_t props;
    status = hipGetDeviceProperties(&props, device);
    if (status != hipSuccess)
        return MFH_FAIL(ERR_INIT, std::string("hipGetDeviceProperties: ") + hipGetErrorString(status));
    const std::string arch = props.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return MFH_FAIL(ERR_INIT, "libmfhip is built for gfx950 only; the current device is " + arch);
    MFH_TRY(conv_probe_kernels());
    const char* sync_flag = std::getenv("MFHIP_SYNC");
    if (sync_flag && sync_flag[0] && sync_flag[0] != '0') debug_sync = true;
    int runtime = 0;
    hipRuntimeGetVersion(&runtime);
    cu_count = props.multiProcessorCount;
    init_device = device;
    const double load_ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
    char info[512];
    std::snprintf(info, sizeof(info),
                  "{\"device_arch\": \"%s\", \"device_name\": \"%s\", \"device\": %d, \"cu_count\": %d, "
                  "\"binary\": \"hsaco\", \"offload_arch\": \"gfx950\", \"hip_runtime\": %d, \"load_ms\": %.3f, "
                  "\"lds_bytes_per_block\": %zu}",
                  arch.c_str(), props.name, device, cu_count, runtime, load_ms, props.sharedMemPerBlock);
    info_text = info;
    initialized = true;
    return OK;
}

MFH_API int mfh_conv_im2col(std::uint64_t x, std::uint64_t cols, int N, int CI, int H, int W, int CO, int KH, int KW,
                            int OH, int OW, int SH, int SW, int PH, int PW, std::uint64_t stream) {
    MFH_TRY(check_ready());
    const ConvDims d{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(check_conv(d));
    MFH_REQUIRE(x && cols, "im2col requires input and output buffers");
    return launch_im2col(ptr<const float>(x), ptr<float>(cols), d, as_stream(stream));
}

MFH_API int mfh_conv_forward(std::uint64_t x, std::uint64_t weight, std::uint64_t bias, std::uint64_t cols,
                             std::uint64_t rows, std::uint64_t y, int N, int CI, int H, int W, int CO, int KH, int KW,
                             int OH, int OW, int SH, int SW, int PH, int PW, int activation, float alpha, int engine,
                             std::uint64_t workspace, std::int64_t workspace_floats, std::uint64_t stream) {
    MFH_TRY(check_ready());
    const ConvDims d{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(check_conv(d));
    MFH_TRY(check_activation(activation, alpha));
    MFH_TRY(check_engine(engine));
    MFH_REQUIRE(x && weight && cols && rows && y, "conv forward received a null buffer");
    MFH_REQUIRE(workspace_floats >= 0, "workspace size must be non-negative");
    const hipStream_t s = as_stream(stream);
    const int M = N * OH * OW, K = CI * KH * KW;
    MFH_TRY(launch_im2col(ptr<const float>(x), ptr<float>(cols), d, s));
    MFH_TRY(gemm_rows(engine, s, false, true, M, CO, K, ptr<const float>(cols), K, ptr<const float>(weight), K,
                      ptr<float>(rows), CO, ptr<float>(workspace), workspace_floats));
    return launch_conv_epilogue(ptr<const float>(rows), ptr<const float>(bias), ptr<float>(y), N, OH * OW, CO,
                                activation, alpha, s);
}

MFH_API int mfh_conv_backward(std::uint64_t weight, std::uint64_t dy, std::uint64_t y, std::uint64_t cols,
                              std::uint64_t dyT, std::uint64_t dw, std::uint64_t grad_cols, std::uint64_t dx,
                              std::uint64_t partial, std::uint64_t db, int N, int CI, int H, int W, int CO, int KH,
                              int KW, int OH, int OW, int SH, int SW, int PH, int PW, int grid_x, int activation,
                              float alpha, int dw_engine, int dx_engine, std::uint64_t workspace,
                              std::int64_t workspace_floats, std::uint64_t stream) {
    MFH_TRY(check_ready());
    const ConvDims d{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(check_conv(d));
    MFH_TRY(check_activation(activation, alpha));
    MFH_TRY(check_engine(dw_engine));
    MFH_TRY(check_engine(dx_engine));
    const bool direct_dx = dx && !dw && !db;
    MFH_REQUIRE(weight && dy, "conv backward requires weight and dy");
    MFH_REQUIRE(!dw || (cols && dyT), "dW requires cols and transposed dy");
    MFH_REQUIRE(!dx || direct_dx || dyT, "dX requires a gradient matrix");
    MFH_REQUIRE(!direct_dx || activation == ACT_NONE, "dX-only expects the gated NCHW gradient");
    MFH_REQUIRE(activation == ACT_NONE || y, "a fused activation needs the forward output");
    MFH_REQUIRE((grad_cols == 0) == (dx == 0), "grad_cols and dx must be given together");
    MFH_REQUIRE((partial == 0) == (db == 0), "partial and db must be given together");
    MFH_REQUIRE(workspace_floats >= 0, "workspace size must be non-negative");
    const int OHW = OH * OW;
    const int tiles = (OHW + conv_grad_tile() - 1) / conv_grad_tile();
    MFH_REQUIRE(grid_x > 0 && grid_x <= tiles, "grid_x must be in [1, spatial tiles]");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(N) * grid_x * CO), "bias partial buffer exceeds int32 indexing");
    const hipStream_t s = as_stream(stream);
    const int M = N * OHW, K = CI * KH * KW;
    float* ws = ptr<float>(workspace);
    if (dw || db)
        MFH_TRY(launch_conv_grad_rows(ptr<const float>(dy), ptr<const float>(y), ptr<float>(dyT), ptr<double>(partial), N,
                                      OHW, CO, grid_x, activation, alpha, s));
    if (db) MFH_TRY(launch_reduce_partials(ptr<const double>(partial), ptr<float>(db), N * grid_x, CO, s));
    // dW (CO x K) = dyT^T cols; grad_cols (M x K) = dyT W. Both reuse the workspace in stream order.
    if (dw)
        MFH_TRY(gemm_rows(dw_engine, s, true, false, CO, K, M, ptr<const float>(dyT), CO, ptr<const float>(cols), K,
                          ptr<float>(dw), K, ws, workspace_floats));
    if (!dx) return OK;
    if (direct_dx) {
        // Each NCHW image of dy is a contiguous CO x OHW matrix: read it transposed straight into the
        // image's slab of grad_cols, without an NHWC copy of dy.
        for (int n = 0; n < N; ++n) {
            const float* image = ptr<const float>(dy) + static_cast<std::int64_t>(n) * CO * OHW;
            float* grad_image = ptr<float>(grad_cols) + static_cast<std::int64_t>(n) * OHW * K;
            MFH_TRY(gemm_rows(dx_engine, s, true, false, OHW, K, CO, image, OHW, ptr<const float>(weight), K, grad_image,
                              K, ws, workspace_floats));
        }
    } else {
        MFH_TRY(gemm_rows(dx_engine, s, false, false, M, K, CO, ptr<const float>(dyT), CO, ptr<const float>(weight), K,
                          ptr<float>(grad_cols), K, ws, workspace_floats));
    }
    return launch_col2im(ptr<const float>(grad_cols), ptr<float>(dx), d, s);
}

MFH_API int mfh_pool_forward(std::uint64_t x, std::uint64_t y, std::uint64_t argmax, int N, int C, int H, int W,
                             int OH, int OW, int KH, int KW, int SH, int SW, std::uint64_t stream) {
    MFH_TRY(check_ready());
    MFH_TRY(check_pool(N, C, H, W, OH, OW, KH, KW, SH, SW));
    MFH_REQUIRE(x && y && argmax, "pool forward received a null buffer");
    return launch_pool_forward(ptr<const float>(x), ptr<float>(y), ptr<int>(argmax), N, C, H, W, OH, OW, KH, KW, SH, SW,
                               as_stream(stream));
}

MFH_API int mfh_pool_backward(std::uint64_t dy, std::uint64_t argmax, std::uint64_t dx, int N, int C, int H, int W,
                              int OH, int OW, int KH, int KW, int SH, int SW, std::uint64_t stream) {
    MFH_TRY(check_ready());
    MFH_TRY(check_pool(N, C, H, W, OH, OW, KH, KW, SH, SW));
    MFH_REQUIRE(dy && argmax && dx, "pool backward received a null buffer");
    return launch_pool_backward(ptr<const float>(dy), ptr<const int>(argmax), ptr<float>(dx), N, C, H, W, OH, OW, KH, KW,
                                SH, SW, as_stream(stream));
}

MFH_API int mfh_matmul(int variant, int tile, int accumulate, std::uint64_t a, std::uint64_t b, std::uint64_t bias,
                       std::uint64_t c, int M, int N, int K, std::uint64_t stream) {
    MFH_TRY(check_ready());
    MFH_REQUIRE(M > 0 && N > 0 && K > 0, "matmul dimensions must be positive");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(M) * K) && fits_index(static_cast<std::int64_t>(K) * N) &&
                    fits_index(static_cast<std::int64_t>(M) * N),
                "matmul operands exceed int32 indexing");
    MFH_REQUIRE(a && b && c, "matmul received a null buffer");
    MFH_REQUIRE(variant == 0 || variant == 1 || variant == 2 || variant == 4,
                "matmul variant must be 0 (basic), 1 (tiled), 2 (shared) or 4 (register); there is no cuBLAS variant");
    MFH_REQUIRE(accumulate >= 0 && accumulate <= 2, "accumulate must be 0, 1 or 2");
    if (variant == 1 || variant == 2) MFH_REQUIRE(tile == 16 || tile == 32, "tile must be 16 or 32");
    const hipStream_t s = as_stream(stream);
    if (variant == 4 && accumulate == 0) {
        // The fp32 register variant is the GEMM engine in one pass over K (no workspace, so no split;
        // the bias is fused in the epilogue).
        return gemm_rows_bias(1, s, false, false, M, N, K, ptr<const float>(a), K, ptr<const float>(b), N,
                              ptr<float>(c), N, ptr<const float>(bias), nullptr, 0);
    }
    MFH_TRY(launch_matmul(variant, tile, accumulate, ptr<const float>(a), ptr<const float>(b), ptr<float>(c), M, N, K, s));
    if (!bias) return OK;
    return launch_add_bias(ptr<float>(c), ptr<const float>(bias), M, N, s);
}

MFH_API int mfh_gemm_tile_count(void) { return gemm_tile_count(); }

MFH_API int mfh_gemm_tile_info(int index, int* values) {
    MFH_REQUIRE(values && index >= 0 && index < gemm_tile_count(), "unknown GEMM tile");
    const GemmTile& t = gemm_tile(index);
    values[0] = t.bm;
    values[1] = t.bn;
    values[2] = t.wm;
    values[3] = t.wn;
    values[4] = t.bk;
    return OK;
}

MFH_API int mfh_gemm_plan(int M, int N, int K, int* tile, int* slices) {
    MFH_TRY(check_ready());
    MFH_REQUIRE(M > 0 && N > 0 && K > 0, "GEMM dimensions must be positive");
    MFH_REQUIRE(tile && slices, "mfh_gemm_plan received a null output");
    const GemmPlan plan = gemm_auto_plan(M, N, K);
    *tile = plan.tile;
    *slices = plan.slices;
    return OK;
}

MFH_API std::int64_t mfh_gemm_workspace(int M, int N, int K) {
    if (check_ready() != OK) return -1;
    if (M <= 0 || N <= 0 || K <= 0) {
        MFH_FAIL(ERR_ARG, "GEMM dimensions must be positive");
        return -1;
    }
    return gemm_workspace_floats(gemm_auto_plan(M, N, K), M, N);
}

MFH_API int mfh_split_reduce(std::uint64_t partial, std::uint64_t c, int slices, int M, int N, int ldc, int reference,
                             std::uint64_t stream) {
    MFH_TRY(check_ready());
    MFH_REQUIRE(partial && c, "the split-K reduction requires partial and output buffers");
    MFH_REQUIRE(slices >= 2 && M > 0 && N > 0 && ldc >= N, "the split-K reduction needs two or more slices and ldc >= N");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(slices) * M * N) &&
                    fits_index(static_cast<std::int64_t>(M - 1) * ldc + N),
                "split-K buffers exceed the int32 indexing limit");
    return split_reduce(ptr<const float>(partial), ptr<float>(c), slices, M, N, ldc, reference != 0, as_stream(stream));
}

MFH_API int mfh_gemm(int engine, int trans_a, int trans_b, std::uint64_t a, std::uint64_t b, std::uint64_t bias,
                     std::uint64_t c, int M, int N, int K, int lda, int ldb, int ldc, std::uint64_t workspace,
                     std::int64_t workspace_floats, std::uint64_t stream) {
    MFH_TRY(check_ready());
    MFH_TRY(check_engine(engine));
    MFH_REQUIRE(M > 0 && N > 0 && K > 0, "GEMM dimensions must be positive");
    MFH_REQUIRE(!(trans_a && trans_b), "GEMM supports A^T B and A B^T but not A^T B^T");
    MFH_REQUIRE(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N) && ldc >= N,
                "GEMM leading dimensions are smaller than the rows");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(M) * K) && fits_index(static_cast<std::int64_t>(K) * N) &&
                    fits_index(static_cast<std::int64_t>(M) * N),
                "GEMM operands exceed int32 indexing");
    MFH_REQUIRE(a && b && c, "GEMM received a null buffer");
    MFH_REQUIRE(!bias || ldc == N, "GEMM bias needs ldc == N");
    MFH_REQUIRE(workspace_floats >= 0, "workspace size must be non-negative");
    return gemm_rows_bias(engine, as_stream(stream), trans_a != 0, trans_b != 0, M, N, K, ptr<const float>(a), lda,
                          ptr<const float>(b), ldb, ptr<float>(c), ldc, ptr<const float>(bias), ptr<float>(workspace),
                          workspace_floats);
}

}  // extern "C"
