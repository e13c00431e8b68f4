// Device workspace for split-K partial sums, one per device.
//
// Lifetime: a workspace is never freed. When a larger request arrives, a new
// buffer is allocated and the old one is retained until the process ends,
// because a HIP graph captured earlier may still hold the old address and
// replay into it later. Growing allocates (hipMalloc), so it is refused while
// the stream is being captured into a graph; a first call of the same or
// larger size outside capture sizes the buffer.
//
// Concurrency: every split-K launch on a device uses this one buffer.
// Launches on one stream are ordered; split-K products that overlap on
// different streams of one device race on the partials. (One buffer per
// device, rather than per stream, is what lets a product be captured on a
// graph-capture stream after an eager call on another stream sized it.)
#include "kernels.hpp"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <vector>

namespace miori {

namespace {

struct Workspace {
    float* part = nullptr;
    size_t bytes = 0;
};

std::mutex g_mu;
std::map<int, Workspace> g_ws;
std::vector<float*> g_retired;  // superseded buffers, kept for captured graphs

}  // namespace

hipError_t workspace_get(hipStream_t st, size_t bytes, float** part) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_mu);
    Workspace& w = g_ws[dev];
    if (w.bytes < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        // Earlier launches on other streams may still read the old buffer;
        // it is retired, not freed, so they (and captured graphs) stay valid.
        float* p = nullptr;
        e = hipMalloc((void**)&p, bytes);
        if (e != hipSuccess) return e;
        if (w.part) g_retired.push_back(w.part);
        w.part = p;
        w.bytes = bytes;
    }
    *part = w.part;
    return hipSuccess;
}

thread_local const Scratch* ScratchScope::current_ = nullptr;

hipError_t scratch_get(hipStream_t st, size_t bytes, float** part) {
    if (const Scratch* fixed = ScratchScope::current()) {
        if (bytes > fixed->bytes) return hipErrorOutOfMemory;
        *part = fixed->ptr;
        return hipSuccess;
    }
    return workspace_get(st, bytes, part);
}

}  // namespace miori
