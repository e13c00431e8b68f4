#include "metal_hip.h"

#include <cstdio>
#include <cstring>
#include <stdexcept>

namespace miori {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

namespace MTL {

void* Buffer::contents() {
    if (!host_) return nullptr;  // private (device-only) storage, as in Metal
    if (dev_dirty_) {
        hip_check(hipStreamSynchronize(m_->stream), "sync before contents()");
        hip_check(hipMemcpy(host_, dev_, len_, hipMemcpyDeviceToHost), "download");
        dev_dirty_ = false;
    }
    host_dirty_ = true;  // the caller may write through the pointer
    return host_;
}

void Buffer::upload(const void* src, size_t bytes, size_t offset) {
    if (offset + bytes > len_) throw std::runtime_error("upload past end of buffer");
    hip_check(hipStreamSynchronize(m_->stream), "sync before upload");
    hip_check(hipMemcpy((char*)dev_ + offset, src, bytes, hipMemcpyHostToDevice), "upload");
    if (host_) memcpy((char*)host_ + offset, src, bytes);
}

void Buffer::download(void* dst, size_t bytes, size_t offset) {
    if (offset + bytes > len_) throw std::runtime_error("download past end of buffer");
    hip_check(hipStreamSynchronize(m_->stream), "sync before download");
    hip_check(hipMemcpy(dst, (const char*)dev_ + offset, bytes, hipMemcpyDeviceToHost), "download");
}

void Buffer::release() {
    if (dev_) (void)hipFree(dev_);
    if (host_) (void)hipHostFree(host_);
    dev_ = host_ = nullptr;
    len_ = 0;
}

hipStream_t ComputeCommandEncoder::stream() const { return cb_->m_->stream; }

void ComputeCommandEncoder::use_in(Buffer* b) {
    if (b->host_ && b->host_dirty_) {
        hip_check(hipMemcpyAsync(b->dev_, b->host_, b->len_, hipMemcpyHostToDevice, stream()),
                  "upload shared buffer");
        b->host_dirty_ = false;
    }
}

void ComputeCommandEncoder::use_out(Buffer* b) {
    use_in(b);  // a kernel may write part of the buffer
    b->dev_dirty_ = true;
}

void CommandBuffer::waitUntilCompleted() {
    hip_check(hipStreamSynchronize(m_->stream), "waitUntilCompleted");
}

}  // namespace MTL

bool Metal::init(const std::string&, std::string& err) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        err = "no HIP device";
        return false;
    }
    if (hipSetDevice(device) != hipSuccess) {
        err = "hipSetDevice failed";
        return false;
    }
    if (hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess) {
        err = "hipStreamCreate failed";
        return false;
    }
    return true;
}

MTL::Buffer* Metal::new_buffer(size_t bytes, bool shared) {
    auto* b = new MTL::Buffer();
    b->m_ = this;
    b->len_ = bytes;
    if (hipMalloc(&b->dev_, bytes ? bytes : 1) != hipSuccess) {
        delete b;
        throw std::runtime_error("device buffer allocation failed");
    }
    if (shared) {
        if (hipHostMalloc(&b->host_, bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess) {
            (void)hipFree(b->dev_);
            delete b;
            throw std::runtime_error("host shadow allocation failed");
        }
        memset(b->host_, 0, bytes);
        hip_check(hipMemset(b->dev_, 0, bytes), "clear shared buffer");
    }
    return b;
}

MTL::CommandBuffer* Metal::begin() {
    auto* cb = new MTL::CommandBuffer();
    cb->m_ = this;
    cb->enc_.cb_ = cb;
    cbs_.push_back(cb);
    return cb;
}

void Metal::submit(MTL::CommandBuffer* cb, bool wait) {
    cb->commit();
    if (wait) cb->waitUntilCompleted();
}

void Metal::print_info() const {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) == hipSuccess)
        printf("device: %s (%s), %d CUs, %.1f GB\n", p.name, p.gcnArchName, p.multiProcessorCount,
               p.totalGlobalMem / 1e9);
}

Metal::~Metal() {
    for (auto* cb : cbs_) delete cb;
    if (stream) (void)hipStreamDestroy(stream);
}

}  // namespace miori
