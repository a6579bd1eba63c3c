// The C ABI of libmfhip (declared in include/mfhip.h): initialisation, error reporting, argument
// validation, and the launch sequences behind each entry point. Invalid calls return status 2 with
// a message naming the reason, before anything is launched.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "../../include/mfhip.h"
#include "common.h"

namespace mfh {
namespace {

struct LibraryState {
    std::mutex lock;
    bool ready = false;
    bool sync_each_launch = false;
    int device = -1;
    int cus = 0;
    std::string info = "{}";
    // Device address of `scratch` on each device that mfh_init has set up (index: device id).
    std::vector<float*> scratch_address;
    // Events of mfh_stream_wait, used in turn (a wait holds on to the record it was issued after).
    std::vector<hipEvent_t> order_events;
    unsigned next_order_event = 0;
};

constexpr int ORDER_EVENTS = 16;

LibraryState& state() {
    static LibraryState s;
    return s;
}

thread_local std::string error_text;
thread_local Program* recording_program = nullptr;

// The split-K workspace of mfh_gemm_noalloc: a fixed array in device memory, one copy per GPU that
// the library runs on, held until the process ends. Host code never passes its name to a kernel
// (on the host the name is only a stand-in); it uses the device address that mfh_init looks up
// with hipGetSymbolAddress. Every mfh_gemm_noalloc call on a GPU shares that GPU's copy, so calls
// that overlap in time on one GPU (other streams, other threads) race. A split-K slice writes its
// whole M x N partial before the reduction reads it, so nothing in it needs to start at zero.
__device__ __align__(256) float scratch[MFH_GEMM_NOALLOC_SCRATCH_FLOATS];

// Looks up this device's address of `scratch` (the current device must be `device`).
int set_up_scratch(LibraryState& s, int device) {
    void* address = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (rc != hipSuccess)
        return MFH_FAIL(ERR_INIT, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(rc));
    if (static_cast<int>(s.scratch_address.size()) <= device) s.scratch_address.resize(device + 1, nullptr);
    s.scratch_address[device] = static_cast<float*>(address);
    return OK;
}

template <typename T>
T* as_ptr(std::uint64_t address) {
    return reinterpret_cast<T*>(static_cast<std::uintptr_t>(address));
}

hipStream_t as_stream(std::uint64_t handle) { return reinterpret_cast<hipStream_t>(static_cast<std::uintptr_t>(handle)); }

int issue_order(hipStream_t waiting, hipStream_t signalling);

// A stream ordering of a recorded program (issued again, with the ring's next event, on replay).
struct OrderStep final : ProgramStep {
    hipStream_t waiting, signalling;
    OrderStep(hipStream_t w, hipStream_t s) : waiting(w), signalling(s) {}
    hipError_t issue() override { return issue_order(waiting, signalling) == OK ? hipSuccess : hipErrorUnknown; }
};

// Nothing issued on `waiting` from now on starts before the work issued so far on `signalling` has
// finished: an event of the ring recorded on one stream and waited for by the other.
int order_after(hipStream_t waiting, hipStream_t signalling) {
    if (waiting == signalling) return OK;
    if (Program* program = recording()) program->steps.push_back(std::make_unique<OrderStep>(waiting, signalling));
    return issue_order(waiting, signalling);
}

int issue_order(hipStream_t waiting, hipStream_t signalling) {
    LibraryState& s = state();
    std::lock_guard<std::mutex> guard(s.lock);
    hipEvent_t event = s.order_events[s.next_order_event++ % s.order_events.size()];
    hipError_t rc = hipEventRecord(event, signalling);
    if (rc != hipSuccess) return MFH_FAIL(ERR_HIP, std::string("hipEventRecord: ") + hipGetErrorString(rc));
    rc = hipStreamWaitEvent(waiting, event, 0);
    if (rc != hipSuccess) return MFH_FAIL(ERR_HIP, std::string("hipStreamWaitEvent: ") + hipGetErrorString(rc));
    return OK;
}

int require_ready() {
    LibraryState& s = state();
    if (!s.ready) return MFH_FAIL(ERR_INIT, "mfh_init has not succeeded");
    int device = -1;
    const hipError_t rc = hipGetDevice(&device);
    if (rc != hipSuccess) return MFH_FAIL(ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(rc));
    if (device != s.device) return MFH_FAIL(ERR_DEVICE, "called on a different HIP device than the one mfh_init used");
    return OK;
}

int validate(const ConvGeometry& g) {
    const bool positive = g.N > 0 && g.CI > 0 && g.H > 0 && g.W > 0 && g.CO > 0 && g.KH > 0 && g.KW > 0 && g.OH > 0 &&
                          g.OW > 0 && g.SH > 0 && g.SW > 0 && g.PH >= 0 && g.PW >= 0;
    MFH_REQUIRE(positive, "convolution dimensions must be positive");
    MFH_REQUIRE(g.OH == (g.H + 2 * g.PH - g.KH) / g.SH + 1 && g.OW == (g.W + 2 * g.PW - g.KW) / g.SW + 1,
                "convolution output size does not match input, kernel, stride and padding");
    const std::int64_t m = static_cast<std::int64_t>(g.N) * g.OH * g.OW;
    const std::int64_t k = static_cast<std::int64_t>(g.CI) * g.KH * g.KW;
    MFH_REQUIRE(fits_index(m * k) && fits_index(m * g.CO) && fits_index(static_cast<std::int64_t>(g.N) * g.CI * g.H * g.W) &&
                    fits_index(k * g.CO),
                "convolution buffers exceed the int32 indexing limit");
    MFH_REQUIRE(static_cast<unsigned>(g.N) <= GRID_YZ_LIMIT && blocks_for(g.CO, conv_grad_tile()) <= GRID_YZ_LIMIT,
                "batch or channel count exceeds the grid limit");
    return OK;
}

int validate_activation(int activation, float alpha) {
    MFH_REQUIRE(activation == ACT_NONE || activation == ACT_RELU || activation == ACT_LEAKY_RELU,
                "unknown activation code");
    MFH_REQUIRE(activation != ACT_LEAKY_RELU || alpha > 0.0f, "fused LeakyReLU requires alpha > 0");
    return OK;
}

int validate_engine(int engine) {
    MFH_REQUIRE(gemm_engine_valid(engine), "unknown GEMM engine or plan code");
    return OK;
}

int validate_pool(int N, int C, int H, int W, int OH, int OW, int KH, int KW, int SH, int SW) {
    MFH_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0 && OH > 0 && OW > 0 && KH > 0 && KW > 0 && SH > 0 && SW > 0,
                "pooling dimensions must be positive");
    MFH_REQUIRE(OH == (H - KH) / SH + 1 && OW == (W - KW) / SW + 1, "pooling output size does not match the input");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(N) * C * H * W), "pooling input exceeds int32 indexing");
    return OK;
}

int validate_norm(const NormShape& s) {
    MFH_REQUIRE(s.N > 0 && s.C > 0 && s.HW > 0, "batch-norm dimensions must be positive");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(s.N) * s.C * s.HW), "batch-norm tensor exceeds int32 indexing");
    MFH_REQUIRE(static_cast<unsigned>(s.C) <= GRID_YZ_LIMIT, "batch-norm channel count exceeds the grid limit");
    return OK;
}

// The column gradient of dX, feature-major: with the transposed rows dyT (M x CO) one GEMM
// gcT (K x M) = W^T dyT^T over every image; from the NCHW gradient alone one GEMM per image,
// gcT[n] (K x OHW) = W^T dy_n (dy_n is CO x OHW). Returns whether the layout is per image.
int column_gradient(int engine, const ConvGeometry& g, const float* weight, const float* dy_nchw, const float* dyT,
                    float* gcT, bool* per_image, hipStream_t stream) {
    const int K = g.features(), ohw = g.ohw();
    GemmOperands o{};
    o.trans_a = true;  // W stored CO x K
    o.M = K;
    o.K = g.CO;
    o.a = weight;
    o.lda = K;
    o.c = gcT;
    *per_image = dyT == nullptr;
    if (dyT) {
        o.trans_b = true;  // dyT stored M x CO
        o.N = g.rows();
        o.b = dyT;
        o.ldb = g.CO;
        o.ldc = g.rows();
    } else {
        o.trans_b = false;  // dy_n stored CO x OHW
        o.N = ohw;
        o.b = dy_nchw;
        o.ldb = ohw;
        o.ldc = ohw;
        o.batch = g.N;
        o.b_batch = static_cast<long long>(g.CO) * ohw;
        o.c_batch = static_cast<long long>(K) * ohw;
    }
    return gemm_launch(engine, stream, o, GemmEpilogue{}, nullptr, 0);
}

// The products of mfh_conv_backward_implicit: dW (and db) on dw_stream with the workspace
// [ws_dw, ws_dw + dw_floats), dX on `stream` with [ws_dx, ws_dx + dx_floats). With two streams the
// dW stream is first ordered after `stream` (after the gating of dy, when an activation is fused).
int conv_backward_implicit(std::uint64_t x, std::uint64_t weight, std::uint64_t dy, std::uint64_t y,
                           std::uint64_t gated, std::uint64_t dw, std::uint64_t dx, std::uint64_t wflip,
                           std::uint64_t grad_cols, std::uint64_t partial, std::uint64_t db, const ConvGeometry& g,
                           int activation, float alpha, int dw_engine, int dx_engine, int flags, float* ws_dw,
                           std::int64_t dw_floats, float* ws_dx, std::int64_t dx_floats, hipStream_t s,
                           hipStream_t dw_s, int* dx_slices = nullptr) {
    if (dx_slices) *dx_slices = 1;
    MFH_TRY(validate(g));
    MFH_TRY(validate_activation(activation, alpha));
    const bool gated_dy = activation != ACT_NONE;
    const bool unit_stride = g.SH == 1 && g.SW == 1;
    // dW and dX given wflip are implicit products (a strided dX as its phase products); a strided dX
    // given grad_cols goes through the column gradient and col2im: one implicit product with the
    // column order in wflip (MFH_CONV_COLUMN_ORDER), else a dense GEMM per image.
    const bool column_order = !unit_stride && (flags & MFH_CONV_COLUMN_ORDER) != 0;
    const bool phases = !unit_stride && wflip != 0 && !column_order;
    MFH_REQUIRE(implicit_engine_valid(dw_engine), "unknown implicit convolution engine or plan code");
    if (unit_stride || phases || column_order)
        MFH_REQUIRE(implicit_engine_valid(dx_engine), "unknown implicit convolution engine or plan code");
    else MFH_TRY(validate_engine(dx_engine));
    const bool prepared = (flags & MFH_CONV_WFLIP_READY) != 0, accumulate = (flags & MFH_CONV_ACCUMULATE_DX) != 0;
    MFH_REQUIRE((flags & ~(MFH_CONV_WFLIP_READY | MFH_CONV_ACCUMULATE_DX | MFH_CONV_COLUMN_ORDER)) == 0,
                "unknown conv backward flags");
    MFH_REQUIRE(!column_order || (!dx || (wflip && grad_cols && implicit_chunked(g.CO))),
                "the column order needs wflip, grad_cols and a multiple of 32 output channels");
    MFH_REQUIRE(dy && (weight || ((unit_stride || phases || column_order) && prepared)),
                "conv backward needs weight and dy");
    MFH_REQUIRE(!gated_dy || (y && gated), "a fused activation needs the forward output and the gated buffer");
    MFH_REQUIRE((partial == 0) == (db == 0), "partial and db must be given together");
    MFH_REQUIRE(!dw || x, "dW needs x");
    MFH_REQUIRE(!dx || wflip != 0 || (!unit_stride && grad_cols != 0),
                "dX needs wflip (any stride) or grad_cols (strides above 1)");
    MFH_REQUIRE(dw_floats >= 0 && dx_floats >= 0, "workspace size must be non-negative");
    const float* grad = as_ptr<const float>(dy);
    const std::int64_t count = static_cast<std::int64_t>(g.N) * g.CO * g.ohw();
    if (gated_dy) {
        MFH_TRY(launch_relu_backward(as_ptr<const float>(y), grad, as_ptr<float>(gated), count,
                                     activation == ACT_LEAKY_RELU ? alpha : 0.0f, false, s));
        grad = as_ptr<const float>(gated);
    }
    double* bias_rows = as_ptr<double>(partial);
    if (dw || db) MFH_TRY(order_after(dw_s, s));
    if (dw) {
        // db rides on the dW product: its first feature tile sums dy over each pixel slice, and
        // the split-K reduction (or the product itself, when unsplit) finishes it.
        MFH_TRY(conv_implicit_wgrad(g, as_ptr<const float>(x), grad, as_ptr<float>(dw), bias_rows, as_ptr<float>(db),
                                    dw_engine, ws_dw, dw_floats, dw_s));
    } else if (db) {
        MFH_TRY(launch_row_sums(grad, bias_rows, g.N * g.CO, g.ohw(), dw_s));
        MFH_TRY(launch_reduce_partials(bias_rows, as_ptr<float>(db), g.N, g.CO, dw_s));
    }
    if (!dx) return OK;
    if (unit_stride)
        return conv_implicit_dgrad(g, grad, as_ptr<const float>(weight), as_ptr<float>(wflip), prepared,
                                   as_ptr<float>(dx), accumulate, dx_engine, ws_dx, dx_floats, s, dx_slices);
    if (phases)
        return conv_implicit_dgrad_phases(g, grad, as_ptr<const float>(weight), as_ptr<float>(wflip), prepared,
                                          as_ptr<float>(dx), accumulate, dx_engine, ws_dx, dx_floats, s);
    if (column_order) {
        // The column gradient gcT[n][f][p] = sum_co W[co][f] dy[n][co][p] is the dX of a 1x1
        // convolution from CI*KH*KW channels to CO channels on the OH x OW grid: one implicit product
        // over every image, reading dy in place, with the 1x1 kernel's dX order of W in wflip.
        const ConvGeometry g1 = column_geometry(g);
        MFH_TRY(conv_implicit_dgrad(g1, grad, as_ptr<const float>(weight), as_ptr<float>(wflip), prepared,
                                    as_ptr<float>(grad_cols), false, dx_engine, ws_dx, dx_floats, s));
        return launch_col2im_t(as_ptr<const float>(grad_cols), as_ptr<float>(dx), g, true, accumulate, s);
    }
    bool per_image = false;
    MFH_TRY(column_gradient(dx_engine, g, as_ptr<const float>(weight), grad, nullptr, as_ptr<float>(grad_cols),
                            &per_image, s));
    return launch_col2im_t(as_ptr<const float>(grad_cols), as_ptr<float>(dx), g, per_image, accumulate, s);
}

}  // namespace

int fail(int status, const char* file, int line, const std::string& what) {
    error_text = std::string(file) + ":" + std::to_string(line) + ": " + what;
    return status;
}

int after_launch(const char* kernel, hipStream_t stream, const char* file, int line) {
    const hipError_t launched = hipGetLastError();
    if (launched != hipSuccess)
        return fail(ERR_HIP, file, line, std::string("launch ") + kernel + ": " + hipGetErrorString(launched));
    if (state().sync_each_launch) {
        const hipError_t synced = hipStreamSynchronize(stream);
        if (synced != hipSuccess)
            return fail(ERR_HIP, file, line, std::string("after kernel ") + kernel + ": " + hipGetErrorString(synced));
    }
    return OK;
}

bool debug_sync_enabled() { return state().sync_each_launch; }
int device_cu_count() { return state().cus; }

Program*& recording() { return recording_program; }

}  // namespace mfh

using namespace mfh;

extern "C" {

MFH_API const char* mfh_last_error(void) { return error_text.c_str(); }

MFH_API const char* mfh_info(void) { return state().info.c_str(); }

MFH_API void mfh_set_debug_sync(int enabled) { state().sync_each_launch = enabled != 0; }

MFH_API int mfh_init(void) {
    LibraryState& s = state();
    std::lock_guard<std::mutex> guard(s.lock);
    if (s.ready) return OK;
    const auto t0 = std::chrono::steady_clock::now();
    int device = -1;
    hipError_t rc = hipGetDevice(&device);
    if (rc != hipSuccess) return MFH_FAIL(ERR_INIT, std::string("hipGetDevice: ") + hipGetErrorString(rc));
    hipDeviceProp_t props;
    rc = hipGetDeviceProperties(&props, device);
    if (rc != hipSuccess) return MFH_FAIL(ERR_INIT, std::string("hipGetDeviceProperties: ") + hipGetErrorString(rc));
    const std::string arch = props.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return MFH_FAIL(ERR_INIT, "libmfhip is built for gfx950 only; the current device is " + arch);
    MFH_TRY(probe_code_object());
    MFH_TRY(set_up_scratch(s, device));
    // The ordering events only order one GPU's streams after each other, so they go without the
    // system-scope fence (the writeback that makes memory visible to the host and other devices):
    // the kernels' own completion releases at device scope order the two streams' memory. Each
    // record and wait of a system-fenced event left the waiting stream idle for about 6 us between
    // two dependent kernels (26 orderings per batch-64 training step). Host synchronisation
    // (hipStreamSynchronize, hipDeviceSynchronize, copies to the host) keeps its own fences.
    for (int i = static_cast<int>(s.order_events.size()); i < ORDER_EVENTS; ++i) {
        hipEvent_t event = nullptr;
        rc = hipEventCreateWithFlags(&event, hipEventDisableTiming | hipEventDisableSystemFence);
        if (rc != hipSuccess) return MFH_FAIL(ERR_INIT, std::string("hipEventCreateWithFlags: ") + hipGetErrorString(rc));
        s.order_events.push_back(event);
    }
    const char* flag = std::getenv("MFHIP_SYNC");
    if (flag && flag[0] && flag[0] != '0') s.sync_each_launch = true;
    int runtime = 0;
    if (hipRuntimeGetVersion(&runtime) != hipSuccess) runtime = 0;
    s.cus = props.multiProcessorCount;
    s.device = device;
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    char text[512];
    std::snprintf(text, sizeof(text),
                  "{\"device_arch\": \"%s\", \"device_name\": \"%s\", \"device\": %d, \"cu_count\": %d, "
                  "\"binary\": \"hsaco\", \"offload_arch\": \"gfx950\", \"hip_runtime\": %d, \"load_ms\": %.3f, "
                  "\"lds_bytes_per_block\": %zu}",
                  arch.c_str(), props.name, device, s.cus, runtime, ms, props.sharedMemPerBlock);
    s.info = text;
    s.ready = true;
    return OK;
}

MFH_API int mfh_stream_wait(std::uint64_t waiting, std::uint64_t signalling) {
    MFH_TRY(require_ready());
    return order_after(as_stream(waiting), as_stream(signalling));
}

MFH_API int mfh_program_begin(void) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(recording() == nullptr, "a program is already being recorded on this thread");
    recording() = new Program();
    return OK;
}

MFH_API int mfh_program_end(std::uint64_t* program, std::int64_t* launches) {
    Program* recorded = recording();
    MFH_REQUIRE(recorded != nullptr, "no program is being recorded on this thread");
    recording() = nullptr;
    if (!program) {
        delete recorded;
        return MFH_FAIL(ERR_ARG, "mfh_program_end needs somewhere to put the program");
    }
    *program = static_cast<std::uint64_t>(reinterpret_cast<std::uintptr_t>(recorded));
    if (launches) *launches = static_cast<std::int64_t>(recorded->launches);
    return OK;
}

MFH_API int mfh_program_run(std::uint64_t program) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(program != 0, "mfh_program_run received a null program");
    MFH_REQUIRE(recording() == nullptr, "a program cannot be replayed while one is being recorded");
    Program* p = as_ptr<Program>(program);
    for (std::size_t i = 0; i < p->steps.size(); ++i) {
        const hipError_t rc = p->steps[i]->issue();
        if (rc != hipSuccess)
            return MFH_FAIL(ERR_HIP, "program step " + std::to_string(i) + ": " + hipGetErrorString(rc));
    }
    if (state().sync_each_launch) {
        const hipError_t rc = hipDeviceSynchronize();
        if (rc != hipSuccess) return MFH_FAIL(ERR_HIP, std::string("program: ") + hipGetErrorString(rc));
    }
    return OK;
}

MFH_API void mfh_program_free(std::uint64_t program) { delete as_ptr<Program>(program); }

MFH_API int mfh_fill(std::uint64_t p, std::int64_t count, float value, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(count >= 0 && fits_index(count), "fill count must be non-negative and within int32 indexing");
    MFH_REQUIRE(p || count == 0, "fill received a null buffer");
    return launch_fill(as_ptr<float>(p), static_cast<int>(count), value, as_stream(stream));
}

MFH_API int mfh_conv_im2col(std::uint64_t x, std::uint64_t cols, int N, int CI, int H, int W, int CO, int KH, int KW,
                            int OH, int OW, int SH, int SW, int PH, int PW, std::uint64_t stream) {
    MFH_TRY(require_ready());
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(validate(g));
    MFH_REQUIRE(x && cols, "im2col needs input and output buffers");
    return launch_im2col(as_ptr<const float>(x), as_ptr<float>(cols), g, as_stream(stream));
}

MFH_API int mfh_conv_col2im(std::uint64_t grad_cols, std::uint64_t dx, int N, int CI, int H, int W, int CO, int KH,
                            int KW, int OH, int OW, int SH, int SW, int PH, int PW, int per_image, int accumulate,
                            std::uint64_t stream) {
    MFH_TRY(require_ready());
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(validate(g));
    MFH_REQUIRE(grad_cols && dx, "col2im needs input and output buffers");
    MFH_REQUIRE((per_image == 0 || per_image == 1) && (accumulate == 0 || accumulate == 1),
                "per_image and accumulate must be 0 or 1");
    return launch_col2im_t(as_ptr<const float>(grad_cols), as_ptr<float>(dx), g, per_image != 0, accumulate != 0,
                           as_stream(stream));
}

MFH_API int mfh_conv_forward(std::uint64_t x, std::uint64_t weight, std::uint64_t bias, std::uint64_t cols,
                             std::uint64_t rows, std::uint64_t y, int N, int CI, int H, int W, int CO, int KH, int KW,
                             int OH, int OW, int SH, int SW, int PH, int PW, int activation, float alpha, int engine,
                             std::uint64_t workspace, std::int64_t workspace_floats, std::uint64_t stream) {
    MFH_TRY(require_ready());
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(validate(g));
    MFH_TRY(validate_activation(activation, alpha));
    MFH_TRY(validate_engine(engine));
    MFH_REQUIRE(x && weight && cols && y, "conv forward received a null buffer");
    MFH_REQUIRE(workspace_floats >= 0, "workspace size must be non-negative");
    const hipStream_t s = as_stream(stream);
    const int M = g.rows(), K = g.features(), ohw = g.ohw();
    MFH_TRY(launch_im2col(as_ptr<const float>(x), as_ptr<float>(cols), g, s));
    GemmEpilogue e;
    e.bias = as_ptr<const float>(bias);
    e.act = activation;
    e.alpha = alpha;
    if (rows) {
        // rows (M x CO) = cols W^T, then the NCHW epilogue kernel (bias + activation).
        GemmOperands o{};
        o.trans_b = true;
        o.M = M;
        o.N = CO;
        o.K = K;
        o.a = as_ptr<const float>(cols);
        o.lda = K;
        o.b = as_ptr<const float>(weight);
        o.ldb = K;
        o.c = as_ptr<float>(rows);
        o.ldc = CO;
        MFH_TRY(gemm_launch(engine, s, o, GemmEpilogue{}, as_ptr<float>(workspace), workspace_floats));
        return launch_conv_epilogue(as_ptr<const float>(rows), e.bias, as_ptr<float>(y), N, ohw, CO, activation, alpha,
                                    s);
    }
    // One GEMM over every image: Y (CO x N*OH*OW) = W cols^T, with output column j = (n, p) stored at
    // y[n][co][p] (a segmented epilogue), bias per output row; the workspace lets it split K.
    GemmOperands o{};
    o.trans_b = true;  // cols stored M x K
    o.M = CO;
    o.N = M;
    o.K = K;
    o.a = as_ptr<const float>(weight);
    o.lda = K;
    o.b = as_ptr<const float>(cols);
    o.ldb = K;
    o.c = as_ptr<float>(y);
    o.ldc = ohw;
    e.bias_mode = bias ? BIAS_ROW : BIAS_NONE;
    e.segment = ohw;
    e.segment_stride = static_cast<long long>(CO) * ohw;
    return gemm_launch(engine, s, o, e, as_ptr<float>(workspace), workspace_floats);
}

MFH_API int mfh_conv_backward(std::uint64_t weight, std::uint64_t dy, std::uint64_t y, std::uint64_t cols,
                              std::uint64_t dyT, std::uint64_t dw, std::uint64_t grad_cols, std::uint64_t dx,
                              std::uint64_t partial, std::uint64_t db, int N, int CI, int H, int W, int CO, int KH,
                              int KW, int OH, int OW, int SH, int SW, int PH, int PW, int grid_x, int activation,
                              float alpha, int dw_engine, int dx_engine, std::uint64_t workspace,
                              std::int64_t workspace_floats, std::uint64_t stream) {
    MFH_TRY(require_ready());
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(validate(g));
    MFH_TRY(validate_activation(activation, alpha));
    MFH_TRY(validate_engine(dw_engine));
    MFH_TRY(validate_engine(dx_engine));
    const bool gated = activation != ACT_NONE;
    MFH_REQUIRE(weight && dy, "conv backward needs weight and dy");
    MFH_REQUIRE(!gated || y, "a fused activation needs the forward output");
    MFH_REQUIRE((grad_cols == 0) == (dx == 0), "grad_cols and dx must be given together");
    MFH_REQUIRE((partial == 0) == (db == 0), "partial and db must be given together");
    MFH_REQUIRE(!dw || (cols && dyT), "dW needs cols and the transposed dy buffer");
    MFH_REQUIRE(!(dx && gated) || dyT, "dX through a fused activation needs the transposed dy buffer");
    MFH_REQUIRE(workspace_floats >= 0, "workspace size must be non-negative");
    const int ohw = g.ohw();
    const int tiles = (ohw + conv_grad_tile() - 1) / conv_grad_tile();
    MFH_REQUIRE(grid_x > 0 && grid_x <= tiles, "grid_x must be in [1, spatial tiles]");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(N) * grid_x * CO), "bias partial buffer exceeds int32 indexing");
    const hipStream_t s = as_stream(stream);
    const int M = g.rows(), K = g.features();
    // Gated, transposed dy (for dW, and for dX through an activation) and the db partials: one pass.
    const bool need_rows = dw || (dx && gated);
    if (need_rows || db)
        MFH_TRY(launch_conv_grad_rows(as_ptr<const float>(dy), as_ptr<const float>(y),
                                      need_rows ? as_ptr<float>(dyT) : nullptr, as_ptr<double>(partial), N, ohw, CO,
                                      grid_x, activation, alpha, s));
    if (db) MFH_TRY(launch_reduce_partials(as_ptr<const double>(partial), as_ptr<float>(db), N * grid_x, CO, s));
    if (dw) {
        // dW (CO x K) = dyT^T cols, split over the M = N*OH*OW pixels.
        GemmOperands o{};
        o.trans_a = true;
        o.M = CO;
        o.N = K;
        o.K = M;
        o.a = as_ptr<const float>(dyT);
        o.lda = CO;
        o.b = as_ptr<const float>(cols);
        o.ldb = K;
        o.c = as_ptr<float>(dw);
        o.ldc = K;
        MFH_TRY(gemm_launch(dw_engine, s, o, GemmEpilogue{}, as_ptr<float>(workspace), workspace_floats));
    }
    if (!dx) return OK;
    // dX from the transposed rows when they were formed (one GEMM over all pixels), else per image
    // from the NCHW gradient.
    bool per_image = false;
    MFH_TRY(column_gradient(dx_engine, g, as_ptr<const float>(weight), as_ptr<const float>(dy),
                            need_rows ? as_ptr<const float>(dyT) : nullptr, as_ptr<float>(grad_cols), &per_image, s));
    return launch_col2im_t(as_ptr<const float>(grad_cols), as_ptr<float>(dx), g, per_image, false, s);
}

MFH_API int mfh_conv_backward_single(std::uint64_t weight, std::uint64_t dy, std::uint64_t y, std::uint64_t cols,
                                     std::uint64_t dyT, std::uint64_t dw, std::uint64_t grad_cols, std::uint64_t dx,
                                     std::uint64_t partial, std::uint64_t db, int N, int CI, int H, int W, int CO,
                                     int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW, int grid_x,
                                     int activation, float alpha, int engine, std::uint64_t workspace,
                                     std::int64_t workspace_floats, std::uint64_t stream) {
    return mfh_conv_backward(weight, dy, y, cols, dyT, dw, grad_cols, dx, partial, db, N, CI, H, W, CO, KH, KW, OH,
                             OW, SH, SW, PH, PW, grid_x, activation, alpha, engine, engine, workspace,
                             workspace_floats, stream);
}

MFH_API int mfh_conv_forward_implicit(std::uint64_t x, std::uint64_t weight, std::uint64_t wt, int prepared,
                                      std::uint64_t bias, std::uint64_t residual, std::uint64_t y, int N, int CI, int H, int W, int CO, int KH,
                                      int KW, int OH, int OW, int SH, int SW, int PH, int PW, int activation,
                                      float alpha, int engine, std::uint64_t workspace, std::int64_t workspace_floats,
                                      std::uint64_t stream) {
    MFH_TRY(require_ready());
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(validate(g));
    MFH_TRY(validate_activation(activation, alpha));
    MFH_REQUIRE(implicit_engine_valid(engine), "unknown implicit convolution engine or plan code");
    MFH_REQUIRE(x && y && (weight || (prepared && wt)), "conv forward received a null buffer");
    MFH_REQUIRE(wt || !implicit_chunked(CI), "the implicit forward needs the reordered-kernel buffer wt");
    MFH_REQUIRE(prepared == 0 || prepared == 1, "prepared must be 0 or 1");
    MFH_REQUIRE(workspace_floats >= 0, "workspace size must be non-negative");
    MFH_REQUIRE(residual != y || residual == 0, "the residual must not be the output buffer");
    return conv_implicit_forward(g, as_ptr<const float>(x), as_ptr<const float>(weight), as_ptr<float>(wt),
                                 prepared == 1, as_ptr<const float>(bias), as_ptr<const float>(residual),
                                 as_ptr<float>(y), activation, alpha, engine, as_ptr<float>(workspace),
                                 workspace_floats, as_stream(stream));
}

MFH_API int mfh_conv_forward_implicit_deferred(std::uint64_t x, std::uint64_t weight, std::uint64_t wt, int prepared,
                                               std::uint64_t bias, std::uint64_t y, int N, int CI, int H, int W, int CO, int KH, int KW,
                                               int OH, int OW, int SH, int SW, int PH, int PW, int engine,
                                               std::uint64_t workspace, std::int64_t workspace_floats,
                                               int* slices, std::uint64_t stream) {
    MFH_TRY(require_ready());
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_TRY(validate(g));
    MFH_REQUIRE(implicit_engine_valid(engine), "unknown implicit convolution engine or plan code");
    MFH_REQUIRE(x && y && slices && (weight || (prepared && wt)), "conv forward received a null buffer");
    MFH_REQUIRE(wt || !implicit_chunked(CI), "the implicit forward needs the reordered-kernel buffer wt");
    MFH_REQUIRE(prepared == 0 || prepared == 1, "prepared must be 0 or 1");
    MFH_REQUIRE(workspace_floats >= 0, "workspace size must be non-negative");
    return conv_implicit_forward(g, as_ptr<const float>(x), as_ptr<const float>(weight), as_ptr<float>(wt),
                                 prepared == 1, as_ptr<const float>(bias), nullptr, as_ptr<float>(y), ACT_NONE, 0.0f, engine,
                                 as_ptr<float>(workspace), workspace_floats, as_stream(stream), slices);
}

MFH_API int mfh_conv_weight_orders(const std::uint64_t* weights, const std::uint64_t* outs, const int* dims, int count,
                                   std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(count >= 0, "count must be non-negative");
    MFH_REQUIRE(count == 0 || (weights && outs && dims), "weight orders need the weights, outputs and dims arrays");
    std::vector<WeightOrder> orders(static_cast<size_t>(count));
    for (int i = 0; i < count; ++i) {
        const int* d = dims + WEIGHT_ORDER_DIMS * i;
        const int CO = d[0], CI = d[1], KH = d[2], KW = d[3], flip = d[4], SH = d[5], SW = d[6], PH = d[7], PW = d[8];
        MFH_REQUIRE(weights[i] && outs[i], "weight order received a null buffer");
        MFH_REQUIRE(CO > 0 && CI > 0 && KH > 0 && KW > 0, "kernel dimensions must be positive");
        MFH_REQUIRE(static_cast<std::int64_t>(CO) * CI * KH * KW <= INDEX_LIMIT, "kernel exceeds the int32 index range");
        MFH_REQUIRE(flip == 0 || flip == 1, "flip must be 0 or 1");
        MFH_REQUIRE(SH > 0 && SW > 0 && PH >= 0 && PW >= 0, "stride must be positive and padding non-negative");
        orders[i] = WeightOrder{as_ptr<const float>(weights[i]), as_ptr<float>(outs[i]), CO, CI, KH, KW, flip,
                                SH, SW, PH, PW};
    }
    return launch_weight_orders(orders.data(), count, as_stream(stream));
}

MFH_API std::int64_t mfh_conv_implicit_workspace(int N, int CI, int H, int W, int CO, int KH, int KW, int OH, int OW,
                                                 int SH, int SW, int PH, int PW, int pass) {
    if (require_ready() != OK) return -1;
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    if (validate(g) != OK) return -1;
    if (pass < IMPLICIT_FORWARD || pass > IMPLICIT_DGRAD) {
        MFH_FAIL(ERR_ARG, "pass must be 0 (forward), 1 (dW) or 2 (dX)");
        return -1;
    }
    return implicit_workspace_floats(g, pass);
}

MFH_API int mfh_conv_backward_implicit(std::uint64_t x, std::uint64_t weight, std::uint64_t dy, std::uint64_t y,
                                       std::uint64_t gated, std::uint64_t dw, std::uint64_t dx, std::uint64_t wflip,
                                       std::uint64_t grad_cols, std::uint64_t partial, std::uint64_t db, int N, int CI,
                                       int H, int W, int CO, int KH, int KW, int OH, int OW, int SH, int SW, int PH,
                                       int PW, int activation, float alpha, int dw_engine, int dx_engine, int flags,
                                       std::uint64_t workspace, std::int64_t workspace_floats, std::uint64_t stream) {
    MFH_TRY(require_ready());
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    float* ws = as_ptr<float>(workspace);
    return conv_backward_implicit(x, weight, dy, y, gated, dw, dx, wflip, grad_cols, partial, db, g, activation, alpha,
                                  dw_engine, dx_engine, flags, ws, workspace_floats, ws, workspace_floats,
                                  as_stream(stream), as_stream(stream));
}

MFH_API int mfh_conv_backward_implicit_streams(
    std::uint64_t x, std::uint64_t weight, std::uint64_t dy, std::uint64_t y, std::uint64_t gated, std::uint64_t dw,
    std::uint64_t dx, std::uint64_t wflip, std::uint64_t grad_cols, std::uint64_t partial, std::uint64_t db, int N,
    int CI, int H, int W, int CO, int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW, int activation,
    float alpha, int dw_engine, int dx_engine, int flags, std::uint64_t workspace, std::int64_t dw_workspace_floats,
    std::int64_t workspace_floats, std::uint64_t stream, std::uint64_t dw_stream) {
    MFH_TRY(require_ready());
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_REQUIRE(dw_workspace_floats >= 0 && dw_workspace_floats <= workspace_floats,
                "the dW part of the workspace must lie within it");
    float* ws = as_ptr<float>(workspace);
    float* ws_dx = ws ? ws + dw_workspace_floats : nullptr;
    return conv_backward_implicit(x, weight, dy, y, gated, dw, dx, wflip, grad_cols, partial, db, g, activation, alpha,
                                  dw_engine, dx_engine, flags, ws, dw_workspace_floats, ws_dx,
                                  workspace_floats - dw_workspace_floats, as_stream(stream), as_stream(dw_stream));
}

MFH_API int mfh_conv_backward_implicit_deferred(
    std::uint64_t x, std::uint64_t weight, std::uint64_t dy, std::uint64_t y, std::uint64_t gated, std::uint64_t dw,
    std::uint64_t dx, std::uint64_t wflip, std::uint64_t grad_cols, std::uint64_t partial, std::uint64_t db, int N,
    int CI, int H, int W, int CO, int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW, int activation,
    float alpha, int dw_engine, int dx_engine, int flags, std::uint64_t workspace, std::int64_t dw_workspace_floats,
    std::int64_t workspace_floats, int* dx_slices, std::uint64_t stream, std::uint64_t dw_stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(dx_slices, "the deferred conv backward needs the slice-count output");
    *dx_slices = 1;
    const ConvGeometry g{N, CI, H, W, CO, KH, KW, OH, OW, SH, SW, PH, PW};
    MFH_REQUIRE(dw_workspace_floats >= 0 && dw_workspace_floats <= workspace_floats,
                "the dW part of the workspace must lie within it");
    float* ws = as_ptr<float>(workspace);
    float* ws_dx = ws ? ws + dw_workspace_floats : nullptr;
    return conv_backward_implicit(x, weight, dy, y, gated, dw, dx, wflip, grad_cols, partial, db, g, activation, alpha,
                                  dw_engine, dx_engine, flags, ws, dw_workspace_floats, ws_dx,
                                  workspace_floats - dw_workspace_floats, as_stream(stream), as_stream(dw_stream),
                                  dx_slices);
}

MFH_API int mfh_pool_forward(std::uint64_t x, std::uint64_t y, std::uint64_t argmax, int N, int C, int H, int W,
                             int OH, int OW, int KH, int KW, int SH, int SW, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_TRY(validate_pool(N, C, H, W, OH, OW, KH, KW, SH, SW));
    MFH_REQUIRE(x && y, "pool forward received a null buffer");  // argmax is optional
    return launch_pool_forward(as_ptr<const float>(x), as_ptr<float>(y), as_ptr<int>(argmax), N, C, H, W, OH, OW, KH,
                               KW, SH, SW, as_stream(stream));
}

MFH_API int mfh_pool_backward(std::uint64_t dy, std::uint64_t argmax, std::uint64_t dx, int N, int C, int H, int W,
                              int OH, int OW, int KH, int KW, int SH, int SW, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_TRY(validate_pool(N, C, H, W, OH, OW, KH, KW, SH, SW));
    MFH_REQUIRE(dy && argmax && dx, "pool backward received a null buffer");
    return launch_pool_backward(as_ptr<const float>(dy), as_ptr<const int>(argmax), as_ptr<float>(dx), N, C, H, W, OH,
                                OW, KH, KW, SH, SW, as_stream(stream));
}

MFH_API int mfh_matmul(int variant, int tile, int accumulate, std::uint64_t a, std::uint64_t b, std::uint64_t bias,
                       std::uint64_t c, int M, int N, int K, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(M > 0 && N > 0 && K > 0, "matmul dimensions must be positive");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(M) * K) && fits_index(static_cast<std::int64_t>(K) * N) &&
                    fits_index(static_cast<std::int64_t>(M) * N),
                "matmul operands exceed int32 indexing");
    MFH_REQUIRE(a && b && c, "matmul received a null buffer");
    MFH_REQUIRE(variant == 0 || variant == 1 || variant == 2 || variant == 4,
                "matmul variant must be 0 (basic), 1 (tiled), 2 (shared) or 4 (register); there is no vendor-BLAS variant");
    MFH_REQUIRE(accumulate >= 0 && accumulate <= 2, "accumulate must be 0, 1 or 2");
    MFH_REQUIRE(!(variant == 1 || variant == 2) || tile == 16 || tile == 32, "tile must be 16 or 32");
    const hipStream_t s = as_stream(stream);
    if (variant == 4 && accumulate == 0) {
        // The fp32 register variant is the MFMA engine in one pass over K, bias fused.
        GemmOperands o{};
        o.M = M;
        o.N = N;
        o.K = K;
        o.a = as_ptr<const float>(a);
        o.lda = K;
        o.b = as_ptr<const float>(b);
        o.ldb = N;
        o.c = as_ptr<float>(c);
        o.ldc = N;
        GemmEpilogue e;
        e.bias = as_ptr<const float>(bias);
        e.bias_mode = bias ? BIAS_COLUMN : BIAS_NONE;
        return gemm_launch(1, s, o, e, nullptr, 0);
    }
    MFH_TRY(launch_matmul(variant, tile, accumulate, as_ptr<const float>(a), as_ptr<const float>(b), as_ptr<float>(c), M,
                          N, K, s));
    if (!bias) return OK;
    return launch_add_bias(as_ptr<float>(c), as_ptr<const float>(bias), M, N, s);
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

MFH_API int mfh_gemm_tile_groups(int index) {
    if (index < 0 || index >= gemm_tile_count()) {
        MFH_FAIL(ERR_ARG, "unknown GEMM tile");
        return -1;
    }
    return gemm_tile(index).kg;
}

MFH_API int mfh_gemm_tile_stages(int index) {
    if (index < 0 || index >= gemm_tile_count()) {
        MFH_FAIL(ERR_ARG, "unknown GEMM tile");
        return -1;
    }
    return 2;
}

MFH_API int mfh_gemm_plan(int M, int N, int K, int* tile, int* slices) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(M > 0 && N > 0 && K > 0, "GEMM dimensions must be positive");
    MFH_REQUIRE(tile && slices, "mfh_gemm_plan received a null output");
    const GemmPlan plan = gemm_auto_plan(M, N, K);
    *tile = plan.tile;
    *slices = plan.slices;
    return OK;
}

MFH_API std::int64_t mfh_gemm_workspace(int M, int N, int K) {
    if (require_ready() != OK) return -1;
    if (M <= 0 || N <= 0 || K <= 0) {
        MFH_FAIL(ERR_ARG, "GEMM dimensions must be positive");
        return -1;
    }
    return gemm_workspace_floats(gemm_auto_plan(M, N, K), M, N);
}

MFH_API int mfh_split_reduce(std::uint64_t partial, std::uint64_t c, int slices, int M, int N, int ldc, int reference,
                             std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(partial && c, "the split-K reduction needs partial and output buffers");
    MFH_REQUIRE(slices >= 2 && M > 0 && N > 0 && ldc >= N, "the split-K reduction needs two or more slices and ldc >= N");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(slices) * M * N) &&
                    fits_index(static_cast<std::int64_t>(M - 1) * ldc + N),
                "split-K buffers exceed the int32 indexing limit");
    return split_reduce(as_ptr<const float>(partial), as_ptr<float>(c), slices, M, N, ldc, reference != 0,
                        as_stream(stream));
}

MFH_API int mfh_gemm(int engine, int trans_a, int trans_b, std::uint64_t a, std::uint64_t b, std::uint64_t bias,
                     std::uint64_t c, int M, int N, int K, int lda, int ldb, int ldc, std::uint64_t workspace,
                     std::int64_t workspace_floats, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_TRY(validate_engine(engine));
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
    GemmOperands o{};
    o.trans_a = trans_a != 0;
    o.trans_b = trans_b != 0;
    o.M = M;
    o.N = N;
    o.K = K;
    o.a = as_ptr<const float>(a);
    o.lda = lda;
    o.b = as_ptr<const float>(b);
    o.ldb = ldb;
    o.c = as_ptr<float>(c);
    o.ldc = ldc;
    GemmEpilogue e;
    e.bias = as_ptr<const float>(bias);
    e.bias_mode = bias ? BIAS_COLUMN : BIAS_NONE;
    return gemm_launch(engine, as_stream(stream), o, e, as_ptr<float>(workspace), workspace_floats);
}

MFH_API int mfh_gemm_noalloc(int engine, int trans_a, int trans_b, std::uint64_t a, std::uint64_t b,
                             std::uint64_t bias, std::uint64_t c, int M, int N, int K, int lda, int ldb, int ldc,
                             std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_TRY(validate_engine(engine));
    MFH_REQUIRE(M > 0 && N > 0 && K > 0, "GEMM dimensions must be positive");
    const std::int64_t needed = gemm_launch_workspace(engine, M, N, K);
    if (needed < 0) return MFH_FAIL(ERR_ARG, "unknown GEMM engine or plan code");
    if (needed > MFH_GEMM_NOALLOC_SCRATCH_FLOATS)
        return MFH_FAIL(ERR_ARG, "mfh_gemm_noalloc: this plan's split-K workspace needs " + std::to_string(needed) +
                                     " floats, more than the " + std::to_string(MFH_GEMM_NOALLOC_SCRATCH_FLOATS) +
                                     " of the static scratch; use fewer K slices or mfh_gemm with a workspace");
    float* workspace = state().scratch_address[state().device];
    return mfh_gemm(engine, trans_a, trans_b, a, b, bias, c, M, N, K, lda, ldb, ldc,
                    static_cast<std::uint64_t>(reinterpret_cast<std::uintptr_t>(workspace)),
                    MFH_GEMM_NOALLOC_SCRATCH_FLOATS, stream);
}

MFH_API std::int64_t mfh_bn_workspace(int N, int C, int HW) {
    if (require_ready() != OK) return -1;
    const NormShape s{N, C, HW};
    if (validate_norm(s) != OK) return -1;
    return norm_workspace_doubles(s);
}

MFH_API int mfh_bn_forward(std::uint64_t x, std::uint64_t gamma, std::uint64_t beta, std::uint64_t running_mean,
                           std::uint64_t running_var, std::uint64_t residual, std::uint64_t y, std::uint64_t mean,
                           std::uint64_t inv_std, std::uint64_t workspace, std::int64_t workspace_doubles, int N, int C,
                           int HW, int training, int relu, double momentum, double eps, double var_scale,
                           std::uint64_t stream) {
    MFH_TRY(require_ready());
    const NormShape s{N, C, HW};
    MFH_TRY(validate_norm(s));
    MFH_REQUIRE(x && gamma && beta && running_mean && running_var && y && mean && inv_std,
                "batch-norm forward received a null buffer");
    MFH_REQUIRE(!training || (workspace && workspace_doubles >= norm_workspace_doubles(s)),
                "batch-norm workspace is smaller than mfh_bn_workspace");
    MFH_REQUIRE(!training || (workspace & 15) == 0, "batch-norm workspace must be 16-byte aligned");
    MFH_REQUIRE(eps >= 0.0 && momentum >= 0.0 && momentum <= 1.0, "batch-norm eps and momentum are out of range");
    NormForward f{};
    f.x = as_ptr<const float>(x);
    f.gamma = as_ptr<const float>(gamma);
    f.beta = as_ptr<const float>(beta);
    f.running_mean = as_ptr<float>(running_mean);
    f.running_var = as_ptr<float>(running_var);
    f.residual = as_ptr<const float>(residual);
    f.y = as_ptr<float>(y);
    f.mean = as_ptr<float>(mean);
    f.inv_std = as_ptr<float>(inv_std);
    f.partial = as_ptr<double>(workspace);
    f.training = training != 0;
    f.relu = relu != 0;
    f.momentum = momentum;
    f.eps = eps;
    f.var_scale = var_scale;
    return norm_forward(s, f, as_stream(stream));
}

MFH_API int mfh_bn_forward_split(std::uint64_t partial, int slices, std::uint64_t bias, std::uint64_t x,
                                 std::uint64_t gamma,
                                 std::uint64_t beta, std::uint64_t running_mean, std::uint64_t running_var,
                                 std::uint64_t residual, std::uint64_t y, std::uint64_t mean, std::uint64_t inv_std,
                                 int N, int C, int HW, int relu, double momentum, double eps, double var_scale,
                                 std::uint64_t stream) {
    MFH_TRY(require_ready());
    const NormShape s{N, C, HW};
    MFH_TRY(validate_norm(s));
    MFH_REQUIRE(partial && x && gamma && beta && running_mean && running_var && y && mean && inv_std,
                "batch-norm forward received a null buffer");
    MFH_REQUIRE(slices >= 1, "slices must be positive");
    MFH_REQUIRE(static_cast<std::int64_t>(slices) * N * C * HW <= INDEX_LIMIT, "the slices exceed the int32 index range");
    MFH_REQUIRE(eps >= 0.0 && momentum >= 0.0 && momentum <= 1.0, "batch-norm eps and momentum are out of range");
    NormForward f{};
    f.x = as_ptr<const float>(x);
    f.gamma = as_ptr<const float>(gamma);
    f.beta = as_ptr<const float>(beta);
    f.running_mean = as_ptr<float>(running_mean);
    f.running_var = as_ptr<float>(running_var);
    f.residual = as_ptr<const float>(residual);
    f.y = as_ptr<float>(y);
    f.mean = as_ptr<float>(mean);
    f.inv_std = as_ptr<float>(inv_std);
    f.training = true;
    f.relu = relu != 0;
    f.momentum = momentum;
    f.eps = eps;
    f.var_scale = var_scale;
    return norm_forward_split(s, f, as_ptr<const float>(partial), slices, as_ptr<const float>(bias), as_ptr<float>(x),
                              as_stream(stream));
}

namespace {

int bn_backward_of(std::uint64_t x, std::uint64_t dy, std::uint64_t gate, std::uint64_t gamma, std::uint64_t mean,
                   std::uint64_t inv_std, std::uint64_t x_grad, std::uint64_t gamma_grad, std::uint64_t beta_grad,
                   std::uint64_t residual_grad, std::uint64_t workspace, std::int64_t workspace_doubles,
                   const NormShape& s, int training, int add_x, int add_gamma, int add_beta, int add_residual,
                   NormBackward* b) {
    MFH_TRY(validate_norm(s));
    MFH_REQUIRE(x && dy && gamma && mean && inv_std, "batch-norm backward received a null buffer");
    MFH_REQUIRE(!residual_grad || gate, "a residual gradient comes from a fused ReLU: pass its output as gate");
    MFH_REQUIRE(workspace && workspace_doubles >= norm_workspace_doubles(s),
                "batch-norm workspace is smaller than mfh_bn_workspace");
    MFH_REQUIRE((workspace & 15) == 0, "batch-norm workspace must be 16-byte aligned");
    *b = NormBackward{};
    b->x = as_ptr<const float>(x);
    b->dy = as_ptr<const float>(dy);
    b->gate = as_ptr<const float>(gate);
    b->gamma = as_ptr<const float>(gamma);
    b->mean = as_ptr<const float>(mean);
    b->inv_std = as_ptr<const float>(inv_std);
    b->x_grad = as_ptr<float>(x_grad);
    b->gamma_grad = as_ptr<float>(gamma_grad);
    b->beta_grad = as_ptr<float>(beta_grad);
    b->residual_grad = as_ptr<float>(residual_grad);
    b->partial = as_ptr<double>(workspace);
    b->training = training != 0;
    b->add_x = add_x != 0;
    b->add_gamma = add_gamma != 0;
    b->add_beta = add_beta != 0;
    b->add_residual = add_residual != 0;
    return OK;
}

}  // namespace

MFH_API int mfh_bn_backward(std::uint64_t x, std::uint64_t dy, std::uint64_t gate, std::uint64_t gamma,
                            std::uint64_t mean, std::uint64_t inv_std, std::uint64_t x_grad, std::uint64_t gamma_grad,
                            std::uint64_t beta_grad, std::uint64_t residual_grad, std::uint64_t workspace,
                            std::int64_t workspace_doubles, int N, int C, int HW, int training, int add_x,
                            int add_gamma, int add_beta, int add_residual, std::uint64_t stream) {
    MFH_TRY(require_ready());
    const NormShape s{N, C, HW};
    NormBackward b;
    MFH_TRY(bn_backward_of(x, dy, gate, gamma, mean, inv_std, x_grad, gamma_grad, beta_grad, residual_grad, workspace,
                           workspace_doubles, s, training, add_x, add_gamma, add_beta, add_residual, &b));
    return norm_backward(s, b, as_stream(stream));
}

MFH_API int mfh_bn_backward_split(std::uint64_t partial, int slices, std::uint64_t x, std::uint64_t dy,
                                  std::uint64_t gate, std::uint64_t gamma, std::uint64_t mean, std::uint64_t inv_std,
                                  std::uint64_t x_grad, std::uint64_t gamma_grad, std::uint64_t beta_grad,
                                  std::uint64_t residual_grad, std::uint64_t workspace, std::int64_t workspace_doubles,
                                  int N, int C, int HW, int training, int add_x, int add_gamma, int add_beta,
                                  int add_residual, std::uint64_t stream) {
    MFH_TRY(require_ready());
    const NormShape s{N, C, HW};
    NormBackward b;
    MFH_TRY(bn_backward_of(x, dy, gate, gamma, mean, inv_std, x_grad, gamma_grad, beta_grad, residual_grad, workspace,
                           workspace_doubles, s, training, add_x, add_gamma, add_beta, add_residual, &b));
    MFH_REQUIRE(partial, "batch-norm backward received a null buffer");
    MFH_REQUIRE(slices >= 1, "slices must be positive");
    MFH_REQUIRE(static_cast<std::int64_t>(slices) * N * C * HW <= INDEX_LIMIT, "the slices exceed the int32 index range");
    return norm_backward_split(s, b, as_ptr<const float>(partial), slices, as_ptr<float>(dy), as_stream(stream));
}

namespace {

// The unit's shapes: a training or eval batch norm over N x C x H x W, then a KH x KW / (SH, SW)
// max-pool without padding.
int pool_unit_shapes(int N, int C, int H, int W, int KH, int KW, int SH, int SW, NormShape* s, PoolDims* d) {
    MFH_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0, "batch-norm + max-pool dimensions must be positive");
    MFH_REQUIRE(KH > 0 && KW > 0 && SH > 0 && SW > 0 && KH <= H && KW <= W,
                "max-pool window and stride must be positive and the window inside the input");
    MFH_REQUIRE(fits_index(static_cast<std::int64_t>(N) * C * H * W), "tensor exceeds int32 element offsets");
    *s = NormShape{N, C, H * W};
    *d = PoolDims{H, W, (H - KH) / SH + 1, (W - KW) / SW + 1, KH, KW, SH, SW};
    return validate_norm(*s);
}

}  // namespace

MFH_API int mfh_bn_relu_pool_supported(int N, int C, int H, int W, int KH, int KW, int SH, int SW) {
    NormShape s;
    PoolDims d;
    if (require_ready() != OK || pool_unit_shapes(N, C, H, W, KH, KW, SH, SW, &s, &d) != OK) return 0;
    return norm_pool_supported(s, d) ? 1 : 0;
}

MFH_API int mfh_bn_relu_pool_forward(std::uint64_t x, std::uint64_t gamma, std::uint64_t beta,
                                     std::uint64_t running_mean, std::uint64_t running_var, std::uint64_t pooled,
                                     std::uint64_t argmax, std::uint64_t mean, std::uint64_t inv_std,
                                     std::uint64_t workspace, std::int64_t workspace_doubles, int N, int C, int H, int W,
                                     int KH, int KW, int SH, int SW, int training, double momentum, double eps,
                                     double var_scale, std::uint64_t stream) {
    MFH_TRY(require_ready());
    NormShape s;
    PoolDims d;
    MFH_TRY(pool_unit_shapes(N, C, H, W, KH, KW, SH, SW, &s, &d));
    MFH_REQUIRE(x && gamma && beta && running_mean && running_var && pooled && argmax && mean && inv_std,
                "batch-norm + max-pool forward received a null buffer");
    MFH_REQUIRE(!training || (workspace && workspace_doubles >= norm_workspace_doubles(s)),
                "batch-norm workspace is smaller than mfh_bn_workspace");
    MFH_REQUIRE(!training || (workspace & 15) == 0, "batch-norm workspace must be 16-byte aligned");
    MFH_REQUIRE(eps >= 0.0 && momentum >= 0.0 && momentum <= 1.0, "batch-norm eps and momentum are out of range");
    NormForward f{};
    f.x = as_ptr<const float>(x);
    f.gamma = as_ptr<const float>(gamma);
    f.beta = as_ptr<const float>(beta);
    f.running_mean = as_ptr<float>(running_mean);
    f.running_var = as_ptr<float>(running_var);
    f.mean = as_ptr<float>(mean);
    f.inv_std = as_ptr<float>(inv_std);
    f.partial = as_ptr<double>(workspace);
    f.training = training != 0;
    f.relu = true;
    f.momentum = momentum;
    f.eps = eps;
    f.var_scale = var_scale;
    return norm_relu_pool_forward(s, f, d, as_ptr<float>(pooled), as_ptr<int>(argmax), as_stream(stream));
}

MFH_API int mfh_bn_relu_pool_backward(std::uint64_t x, std::uint64_t pooled_grad, std::uint64_t argmax,
                                      std::uint64_t gamma, std::uint64_t beta, std::uint64_t mean,
                                      std::uint64_t inv_std, std::uint64_t x_grad, std::uint64_t gamma_grad,
                                      std::uint64_t beta_grad, std::uint64_t workspace, std::int64_t workspace_doubles,
                                      int N, int C, int H, int W, int KH, int KW, int SH, int SW, int training,
                                      int add_x, int add_gamma, int add_beta, std::uint64_t stream) {
    MFH_TRY(require_ready());
    NormShape s;
    PoolDims d;
    MFH_TRY(pool_unit_shapes(N, C, H, W, KH, KW, SH, SW, &s, &d));
    MFH_REQUIRE(x && pooled_grad && argmax && gamma && beta && mean && inv_std,
                "batch-norm + max-pool backward received a null buffer");
    MFH_REQUIRE(workspace && workspace_doubles >= norm_workspace_doubles(s),
                "batch-norm workspace is smaller than mfh_bn_workspace");
    MFH_REQUIRE((workspace & 15) == 0, "batch-norm workspace must be 16-byte aligned");
    NormBackward b{};
    b.x = as_ptr<const float>(x);
    b.gamma = as_ptr<const float>(gamma);
    b.mean = as_ptr<const float>(mean);
    b.inv_std = as_ptr<const float>(inv_std);
    b.x_grad = as_ptr<float>(x_grad);
    b.gamma_grad = as_ptr<float>(gamma_grad);
    b.beta_grad = as_ptr<float>(beta_grad);
    b.partial = as_ptr<double>(workspace);
    b.training = training != 0;
    b.add_x = add_x != 0;
    b.add_gamma = add_gamma != 0;
    b.add_beta = add_beta != 0;
    return norm_relu_pool_backward(s, b, d, as_ptr<const float>(pooled_grad), as_ptr<const int>(argmax),
                                   as_ptr<const float>(beta), as_stream(stream));
}

MFH_API int mfh_relu_forward(std::uint64_t x, std::uint64_t y, std::int64_t count, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(count >= 0, "element count must be non-negative");
    MFH_REQUIRE(count == 0 || (x && y), "relu forward received a null buffer");
    return launch_relu_forward(as_ptr<const float>(x), as_ptr<float>(y), count, as_stream(stream));
}

MFH_API int mfh_relu_backward(std::uint64_t x, std::uint64_t grad, std::uint64_t out, std::int64_t count, float alpha,
                              int add, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(count >= 0, "element count must be non-negative");
    MFH_REQUIRE(count == 0 || (x && grad && out), "relu backward received a null buffer");
    return launch_relu_backward(as_ptr<const float>(x), as_ptr<const float>(grad), as_ptr<float>(out), count, alpha,
                                add != 0, as_stream(stream));
}

MFH_API int mfh_plane_mean(std::uint64_t x, std::uint64_t y, std::int64_t planes, int hw, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(planes >= 0 && hw > 0 && fits_index(planes * hw), "plane mean needs planes >= 0 and hw > 0 within the index range");
    MFH_REQUIRE(planes == 0 || (x && y), "plane mean received a null buffer");
    return launch_plane_mean(as_ptr<const float>(x), as_ptr<float>(y), planes, hw, as_stream(stream));
}

MFH_API int mfh_plane_mean_backward(std::uint64_t dy, std::uint64_t dx, std::int64_t planes, int hw, int add,
                                    std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(planes >= 0 && hw > 0 && fits_index(planes * hw), "plane mean backward needs planes >= 0 and hw > 0 within the index range");
    MFH_REQUIRE(planes == 0 || (dy && dx), "plane mean backward received a null buffer");
    return launch_plane_mean_backward(as_ptr<const float>(dy), as_ptr<float>(dx), planes, hw, add != 0,
                                      as_stream(stream));
}

MFH_API int mfh_mse_loss(std::uint64_t pred, std::uint64_t target, std::uint64_t loss, std::int64_t count,
                         std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(count >= 0 && fits_index(count), "mse element count out of range");
    MFH_REQUIRE(loss && (count == 0 || (pred && target)), "mse loss received a null buffer");
    return launch_mse_loss(as_ptr<const float>(pred), as_ptr<const float>(target), as_ptr<float>(loss), count,
                           as_stream(stream));
}

MFH_API int mfh_mse_loss_backward(std::uint64_t pred, std::uint64_t target, std::uint64_t seed, std::uint64_t grad,
                                  std::int64_t count, int add, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(count >= 0 && fits_index(count), "mse element count out of range");
    MFH_REQUIRE(count == 0 || (pred && target && seed && grad), "mse loss backward received a null buffer");
    return launch_mse_grad(as_ptr<const float>(pred), as_ptr<const float>(target), as_ptr<const float>(seed),
                           as_ptr<float>(grad), count, add != 0, as_stream(stream));
}

MFH_API int mfh_column_sums(std::uint64_t src, std::uint64_t out, std::int64_t rows, std::int64_t cols,
                            std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(rows >= 0 && cols >= 0 && fits_index(rows * cols), "column sums shape out of range");
    MFH_REQUIRE(cols == 0 || (out && (rows == 0 || src)), "column sums received a null buffer");
    return launch_column_sums(as_ptr<const float>(src), as_ptr<float>(out), rows, cols, as_stream(stream));
}

MFH_API int mfh_adam_step(const mfh_adam_tensor* tensors, int count, float grad_scale, float beta1,
                          float one_minus_beta1, float beta2, float one_minus_beta2, float eps, std::uint64_t stream) {
    MFH_TRY(require_ready());
    MFH_REQUIRE(count >= 0 && (count == 0 || tensors), "adam needs a tensor table");
    std::vector<AdamTensor> table(static_cast<std::size_t>(count));
    for (int i = 0; i < count; ++i) {
        const mfh_adam_tensor& t = tensors[i];
        MFH_REQUIRE(t.size >= 0, "adam tensor sizes must be non-negative");
        MFH_REQUIRE(t.size == 0 || (t.param && t.grad && t.m && t.v), "adam tensor received a null buffer");
        MFH_REQUIRE(t.size <= INDEX_LIMIT, "adam tensor exceeds int32 indexing");
        table[i] = AdamTensor{as_ptr<float>(t.param), as_ptr<const float>(t.grad), as_ptr<float>(t.m), as_ptr<float>(t.v),
                              t.size, t.lr, t.weight_decay, t.bias_correction1, t.bias_correction2};
    }
    const AdamScalars s{grad_scale, beta1, one_minus_beta1, beta2, one_minus_beta2, eps};
    return launch_adam(table.data(), count, s, as_stream(stream));
}

}  // extern "C"
