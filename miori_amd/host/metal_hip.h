// HIP-backed stand-in for the reference's Metal device runtime on the
// quantized-matmul path (src/metal.h, src/metal.cpp), so that the op
// wrappers keep their src/ops.h signatures.
//
//   Metal::init          -> selects the HIP device and creates one stream
//                           (src/metal.cpp:10-24: device + one command queue)
//   Metal::new_buffer    -> device memory (src/metal.cpp:42-48); a "shared"
//                           buffer also gets a pinned host shadow that
//                           contents() returns, kept coherent at the
//                           boundaries (see Buffer)
//   Metal::begin/submit  -> command buffer = work enqueued on the stream;
//                           submit(cb, wait) = optional stream sync
//                           (src/metal.cpp:50-59)
//
// Errors throw std::runtime_error, as the reference does.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace miori {

struct Metal;

namespace MTL {

// One device allocation. For shared buffers contents() returns a host copy:
// host writes are uploaded before the buffer is next bound to a kernel, and
// a buffer written by a kernel is downloaded the next time contents() is
// called after the command buffer that wrote it has completed.
class Buffer {
public:
    void* contents();
    size_t length() const { return len_; }
    void* gpu() const { return dev_; }
    bool shared() const { return host_ != nullptr; }
    // Explicit copies (any buffer kind), synchronous.
    void upload(const void* src, size_t bytes, size_t offset = 0);
    void download(void* dst, size_t bytes, size_t offset = 0);
    void release();

private:
    friend struct ::miori::Metal;
    friend class ComputeCommandEncoder;
    Metal* m_ = nullptr;
    void* dev_ = nullptr;
    void* host_ = nullptr;
    size_t len_ = 0;
    bool host_dirty_ = false;  // host shadow modified since last upload
    bool dev_dirty_ = false;   // device copy written since last download
};

class CommandBuffer;

class ComputeCommandEncoder {
public:
    void endEncoding() {}
    hipStream_t stream() const;
    // Called by the op wrappers for every buffer they bind.
    void use_in(Buffer* b);
    void use_out(Buffer* b);

private:
    friend class CommandBuffer;
    friend struct ::miori::Metal;
    CommandBuffer* cb_ = nullptr;
};

class CommandBuffer {
public:
    ComputeCommandEncoder* computeCommandEncoder() { return &enc_; }
    void commit() {}
    void waitUntilCompleted();

private:
    friend struct ::miori::Metal;
    friend class ComputeCommandEncoder;
    Metal* m_ = nullptr;
    ComputeCommandEncoder enc_;
};

}  // namespace MTL

struct Metal {
    int device = 0;
    hipStream_t stream = nullptr;
    // Quantisation group size of the raw-buffer ops (gemv4_raw, gemv8_off),
    // which carry no scale-tensor shape to read it from. Default: the
    // reference's kGroup (config/m6.h:48). One value per device context, so
    // engines with different weight formats keep separate Metal objects.
    uint32_t raw_group = 32;

    bool init(const std::string& unused_library_path, std::string& err);
    MTL::Buffer* new_buffer(size_t bytes, bool shared = true);
    MTL::CommandBuffer* begin();
    void submit(MTL::CommandBuffer* cb, bool wait = true);
    void print_info() const;
    ~Metal();

private:
    std::vector<MTL::CommandBuffer*> cbs_;
};

// Throws std::runtime_error with the HIP error text when e != hipSuccess.
void hip_check(hipError_t e, const char* what);

}  // namespace miori
