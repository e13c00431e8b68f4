// Shader-clock sampler: a diagnostic with no counterpart in the reference.
//
// MI355X runs its shader clock below the 2.4 GHz the dense MFMA peak is
// quoted at whenever the board's power limit binds, and operand movement
// (global -> LDS fills, LDS fragment reads) costs power as well as the
// matrix cores do. To read the clock that a kernel actually ran at, this
// one-wave kernel runs on a side stream beside it and records, every `gap`
// ticks of the constant-rate wall clock (s_memrealtime, 100 MHz on gfx950),
// the pair (s_memtime, s_memrealtime); s_memtime counts shader clock cycles.
// The clock over an interval is d(memtime) / d(realtime) x the wall-clock
// rate. The wave occupies a few registers of one SIMD for its lifetime, so
// a kernel that needs every CU's whole register file loses that CU while
// the sampler runs: read clocks from it, not durations.
//
// The loop is bounded: n samples, and each wait ends once the monotonic
// wall clock passes the next sample time.
#include "common.hpp"
#include "kernels.hpp"

namespace miori {

namespace {

__global__ __launch_bounds__(64) void clock_sampler_kernel(uint64_t* __restrict__ out,
                                                           uint32_t n, uint32_t gap) {
    uint64_t next = __builtin_amdgcn_s_memrealtime();
    for (uint32_t i = 0; i < n; ++i) {
        while (__builtin_amdgcn_s_memrealtime() < next) __builtin_amdgcn_s_sleep(1);
        const uint64_t c = __builtin_amdgcn_s_memtime();
        const uint64_t r = __builtin_amdgcn_s_memrealtime();
        if (threadIdx.x == 0) {
            out[2 * i] = c;
            out[2 * i + 1] = r;
        }
        next = r + gap;
    }
}

}  // namespace

hipError_t launch_clock_sampler(uint64_t* out, uint32_t n, uint32_t gap, hipStream_t st) {
    hipLaunchKernelGGL(clock_sampler_kernel, dim3(1), dim3(64), 0, st, out, n, gap);
    return hipGetLastError();
}

}  // namespace miori
