// Division of non-negative int32 values by a runtime divisor without the ~30-instruction integer
// divide sequence: q = (umulhi(n, magic) + n) >> shift with shift = ceil(log2 d) and
// magic = floor(2^32 (2^shift - d) / d) + 1 (Granlund & Montgomery, "Division by Invariant Integers
// using Multiplication", 1994, the round-up variant). Exact for 0 <= n < 2^31 and 1 <= d < 2^31.
// The host builds the constants once per launch; the device pays one mul_hi, one add and one shift.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mfh {

struct FastDiv {
    std::uint32_t d, magic, shift;

    FastDiv() = default;
    __host__ explicit FastDiv(int divisor) : d(static_cast<std::uint32_t>(divisor)), magic(0), shift(0) {
        while ((std::uint64_t(1) << shift) < d) ++shift;
        magic = static_cast<std::uint32_t>(((std::uint64_t(1) << 32) * ((std::uint64_t(1) << shift) - d)) / d + 1);
    }

    __device__ __forceinline__ int div(int n) const {
        const std::uint32_t u = static_cast<std::uint32_t>(n);
        return static_cast<int>((__umulhi(u, magic) + u) >> shift);
    }
    // Quotient and remainder of n / d.
    __device__ __forceinline__ int divmod(int n, int& rem) const {
        const int q = div(n);
        rem = n - q * static_cast<int>(d);
        return q;
    }
};

}  // namespace mfh
