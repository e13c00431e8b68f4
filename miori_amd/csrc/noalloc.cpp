// Allocation-free variant of the fused 4-bit GEMM (miori_gemm_q4_static).
//
// For callers that cannot call hipMalloc (code under graph capture, serving
// loops, harnesses that forbid allocation): the split-K partials live in a
// fixed file-scope device array instead of the library's growable
// workspace. Each GPU holds its own copy of the array (module globals are
// per device) from the library's first use on that GPU until the process
// ends. Every call on one GPU shares that GPU's copy and leaves the last
// call's partials in it; nothing in it needs to start at zero (a split-K
// launch overwrites every partial it later reads). Calls that overlap on one
// GPU (different streams, or different host threads without ordering) race
// on the array.
#include "../../include/miori_hip.h"
#include "kernels.hpp"

#include <hip/hip_runtime.h>

#include <mutex>

namespace {

constexpr size_t kScratchBytes = (size_t)MIORI_STATIC_SCRATCH_BYTES;

// In host code `scratch` is a host-side stand-in for the device array, not a
// device address: host code uses only the per-device address that
// hipGetSymbolAddress returns (g_scratch_ptr).
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`, looked up once
// per device with that device current (the set-up of the first call there).
hipError_t scratch_address(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace

extern "C" int miori_gemm_q4_static(const void* A, const void* q, const void* scales,
                                    const void* biases, void* C, uint32_t M, uint32_t N,
                                    uint32_t K, uint32_t group, int out_dtype,
                                    miori_stream stream) {
    float* ptr = nullptr;
    if (scratch_address(&ptr) != hipSuccess) return MIORI_E_HIP;
    const miori::Scratch fixed{ptr, kScratchBytes};
    miori::ScratchScope scope(&fixed);
    return miori::gemm_q4_entry(A, q, scales, biases, C, M, N, K, group, out_dtype,
                                (hipStream_t)stream);
}
