// Weights / Tensor for the HIP path: the reference's byte-range view into
// one weights buffer (src/weights.h:10-41), loaded from a safetensors file
// (src/weights.cpp:14-66) into device memory.
//
// Tensor::begin/end are byte offsets into Weights::buffer(), exactly as in
// the reference, so the op wrappers bind (buffer, begin) pairs the same way.
// Tensor::ptr points at a host copy of the bytes (the reference's shared
// buffer is CPU-visible; here the host copy serves the CPU-side checks).
#pragma once
#include "metal_hip.h"

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace miori {

struct Tensor {
    std::string name;
    std::string dtype;
    std::vector<int64_t> shape;
    uint64_t begin = 0;
    uint64_t end = 0;
    const uint8_t* ptr = nullptr;

    int64_t rows() const { return shape.empty() ? 0 : shape[0]; }
    int64_t cols() const { return shape.size() < 2 ? 0 : shape[1]; }
    size_t bytes() const { return (size_t)(end - begin); }
};

class Weights {
public:
    ~Weights();
    // Reads a safetensors file: an 8-byte little-endian header length, a JSON
    // header {name: {dtype, shape, data_offsets}}, then the data block.
    bool load(Metal& m, const std::string& path, std::string& err);
    const Tensor& get(const std::string& name) const;
    const Tensor* find(const std::string& name) const;
    bool has(const std::string& name) const;
    MTL::Buffer* buffer() const { return buf_; }
    const uint8_t* data() const { return host_.data(); }
    size_t data_size() const { return host_.size(); }
    size_t tensor_count() const { return tensors_.size(); }
    const std::map<std::string, Tensor>& tensors() const { return tensors_; }

private:
    MTL::Buffer* buf_ = nullptr;
    std::vector<uint8_t> host_;
    std::map<std::string, Tensor> tensors_;
};

// Parse a safetensors JSON header into tensor descriptors (no data). Throws
// std::runtime_error on malformed input.
std::map<std::string, Tensor> parse_safetensors_header(const std::string& json);

}  // namespace miori
