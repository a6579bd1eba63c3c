// Kernel launches of libmfhip, and the recording of a sequence of them as a program.
//
// Every kernel of the library is launched through launch(): hipLaunchKernel with an argument array
// built from the kernel's own parameter types (the conversions a <<<...>>> launch makes). While a
// program is being recorded on the calling thread (mfh_program_begin), each launch is also kept,
// with a copy of its arguments, as a step of that program, and so is each stream ordering
// (order_after). mfh_program_run issues the steps again in the recorded order on the recorded
// streams: the same kernels with the same arguments, without the host work (argument checks, plans,
// Python) that chose them. The recorded pass must therefore leave nothing to other libraries: every
// GPU write it relies on must be a library launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <memory>
#include <tuple>
#include <utility>
#include <vector>

namespace mfh {

struct ProgramStep {
    virtual ~ProgramStep() = default;
    virtual hipError_t issue() = 0;
};

struct Program {
    std::vector<std::unique_ptr<ProgramStep>> steps;
    std::size_t launches = 0;
};

// The program being recorded on this thread, or nullptr.
Program*& recording();

template <typename... Params>
struct KernelStep final : ProgramStep {
    const void* kernel;
    dim3 grid, block;
    unsigned shared;
    hipStream_t stream;
    std::tuple<Params...> args;

    KernelStep(const void* k, dim3 g, dim3 b, unsigned s, hipStream_t st, std::tuple<Params...>&& a)
        : kernel(k), grid(g), block(b), shared(s), stream(st), args(std::move(a)) {}

    hipError_t issue() override { return issue_with(std::index_sequence_for<Params...>{}); }

    template <std::size_t... I>
    hipError_t issue_with(std::index_sequence<I...>) {
        void* argv[] = {static_cast<void*>(&std::get<I>(args))..., nullptr};
        return hipLaunchKernel(kernel, grid, block, argv, shared, stream);
    }
};

template <typename... Params, std::size_t... I>
hipError_t launch_packed(const void* kernel, dim3 grid, dim3 block, unsigned shared, hipStream_t stream,
                         std::tuple<Params...>& args, std::index_sequence<I...>) {
    void* argv[] = {static_cast<void*>(&std::get<I>(args))..., nullptr};
    return hipLaunchKernel(kernel, grid, block, argv, shared, stream);
}

// Launches kernel<<<grid, block, shared, stream>>>(args...) (and records it while a program is
// being recorded). The launch's status is left for MFH_CHECK_LAUNCH, as for a <<<...>>> launch.
template <typename... Params, typename... Args>
void launch(void (*kernel)(Params...), dim3 grid, dim3 block, std::size_t shared, hipStream_t stream,
            Args&&... args) {
    static_assert(sizeof...(Params) == sizeof...(Args), "launch() takes one argument per kernel parameter");
    std::tuple<std::decay_t<Params>...> packed(static_cast<std::decay_t<Params>>(std::forward<Args>(args))...);
    const void* entry = reinterpret_cast<const void*>(kernel);
    (void)launch_packed(entry, grid, block, static_cast<unsigned>(shared), stream, packed,
                        std::index_sequence_for<Params...>{});
    if (Program* program = recording()) {
        program->steps.push_back(std::make_unique<KernelStep<std::decay_t<Params>...>>(
            entry, grid, block, static_cast<unsigned>(shared), stream, std::move(packed)));
        ++program->launches;
    }
}

}  // namespace mfh
