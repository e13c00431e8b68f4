// Device workspace for split-K partial sums: one per device, grown on demand
// and kept until the process ends. Growing allocates (hipMalloc), so it is
// refused while the stream is being captured into a graph; a first call of
// the same or larger size outside capture sizes it. Every split-K launch on
// a device uses this one workspace: launches on one stream are ordered,
// launches that overlap on different streams of one device race.
#include "kernels.hpp"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

namespace miori {

namespace {

struct Workspace {
    float* part = nullptr;
    size_t bytes = 0;
};

std::mutex g_mu;
std::map<int, Workspace> g_ws;

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
        e = hipStreamSynchronize(st);  // earlier launches may still read the old buffer
        if (e != hipSuccess) return e;
        if (w.part) (void)hipFree(w.part);
        w.part = nullptr;
        w.bytes = 0;
        e = hipMalloc((void**)&w.part, bytes);
        if (e != hipSuccess) return e;
        w.bytes = bytes;
    }
    *part = w.part;
    return hipSuccess;
}

}  // namespace miori
