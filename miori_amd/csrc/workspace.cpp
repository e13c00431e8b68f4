// Device workspace for split-K partial sums: one per device, grown on demand
// and kept until the process ends. Growing allocates (hipMalloc) and clears
// the completion counters, so it is refused while the stream is being
// captured into a graph; a first call of the same or larger size outside
// capture sizes it. Every split-K launch on a device uses this one
// workspace: launches on one stream are ordered, launches that overlap on
// different streams of one device race (a limit shared with a static scratch
// buffer).
#include "kernels.hpp"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

namespace miori {

namespace {

struct Workspace {
    float* part = nullptr;
    size_t part_bytes = 0;
    uint32_t* counters = nullptr;
    size_t n_counters = 0;
};

std::mutex g_mu;
std::map<int, Workspace> g_ws;

}  // namespace

hipError_t workspace_get(hipStream_t st, size_t part_bytes, size_t n_counters, float** part,
                         uint32_t** counters) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_mu);
    Workspace& w = g_ws[dev];
    if (w.part_bytes < part_bytes || w.n_counters < n_counters) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        e = hipStreamSynchronize(st);
        if (e != hipSuccess) return e;
        if (w.part_bytes < part_bytes) {
            if (w.part) (void)hipFree(w.part);
            w.part = nullptr;
            w.part_bytes = 0;
            e = hipMalloc((void**)&w.part, part_bytes);
            if (e != hipSuccess) return e;
            w.part_bytes = part_bytes;
        }
        if (w.n_counters < n_counters) {
            if (w.counters) (void)hipFree(w.counters);
            w.counters = nullptr;
            w.n_counters = 0;
            e = hipMalloc((void**)&w.counters, n_counters * sizeof(uint32_t));
            if (e != hipSuccess) return e;
            e = hipMemset(w.counters, 0, n_counters * sizeof(uint32_t));
            if (e != hipSuccess) return e;
            w.n_counters = n_counters;
        }
    }
    *part = w.part;
    *counters = w.counters;
    return hipSuccess;
}

}  // namespace miori
