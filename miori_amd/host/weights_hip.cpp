#include "weights_hip.h"

#include <cctype>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>

namespace miori {

namespace {

// Minimal reader for the safetensors header: objects, arrays, strings and
// integers; other JSON values (metadata) are skipped.
class HeaderReader {
public:
    explicit HeaderReader(const std::string& s) : s_(s) {}

    std::map<std::string, Tensor> tensors() {
        std::map<std::string, Tensor> out;
        ws();
        expect('{');
        ws();
        if (peek() == '}') { ++i_; return out; }
        for (;;) {
            ws();
            std::string key = str();
            ws();
            expect(':');
            ws();
            if (key == "__metadata__") {
                skip_value();
            } else {
                Tensor t = tensor_entry();
                t.name = key;
                out.emplace(key, std::move(t));
            }
            ws();
            if (peek() == ',') { ++i_; continue; }
            expect('}');
            break;
        }
        return out;
    }

private:
    const std::string& s_;
    size_t i_ = 0;

    [[noreturn]] void fail(const char* what) {
        throw std::runtime_error(std::string("safetensors header: ") + what + " at byte " +
                                 std::to_string(i_));
    }
    char peek() { return i_ < s_.size() ? s_[i_] : '\0'; }
    void ws() { while (i_ < s_.size() && isspace((unsigned char)s_[i_])) ++i_; }
    void expect(char c) { if (peek() != c) fail("unexpected character"); ++i_; }

    std::string str() {
        expect('"');
        std::string r;
        while (i_ < s_.size() && s_[i_] != '"') {
            if (s_[i_] == '\\') {
                ++i_;
                if (i_ >= s_.size()) fail("bad escape");
                const char e = s_[i_];
                if (e == 'u') {  // keep the escape verbatim; names are ASCII in practice
                    r += "\\u";
                } else {
                    r += (e == 'n') ? '\n' : (e == 't') ? '\t' : e;
                }
                ++i_;
                continue;
            }
            r += s_[i_++];
        }
        expect('"');
        return r;
    }

    int64_t integer() {
        ws();
        size_t st = i_;
        if (peek() == '-') ++i_;
        while (isdigit((unsigned char)peek())) ++i_;
        if (st == i_) fail("expected integer");
        return std::stoll(s_.substr(st, i_ - st));
    }

    std::vector<int64_t> int_array() {
        std::vector<int64_t> v;
        expect('[');
        ws();
        if (peek() == ']') { ++i_; return v; }
        for (;;) {
            v.push_back(integer());
            ws();
            if (peek() == ',') { ++i_; continue; }
            expect(']');
            return v;
        }
    }

    void skip_value() {
        ws();
        const char c = peek();
        if (c == '"') { str(); return; }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++i_;
            ws();
            if (peek() == close) { ++i_; return; }
            for (;;) {
                ws();
                if (c == '{') { str(); ws(); expect(':'); }
                skip_value();
                ws();
                if (peek() == ',') { ++i_; continue; }
                expect(close);
                return;
            }
        }
        while (i_ < s_.size() && s_[i_] != ',' && s_[i_] != '}' && s_[i_] != ']') ++i_;
    }

    Tensor tensor_entry() {
        Tensor t;
        bool have_off = false;
        expect('{');
        for (;;) {
            ws();
            std::string k = str();
            ws();
            expect(':');
            ws();
            if (k == "dtype") {
                t.dtype = str();
            } else if (k == "shape") {
                t.shape = int_array();
            } else if (k == "data_offsets") {
                auto o = int_array();
                if (o.size() != 2 || o[0] < 0 || o[1] < o[0]) fail("bad data_offsets");
                t.begin = (uint64_t)o[0];
                t.end = (uint64_t)o[1];
                have_off = true;
            } else {
                skip_value();
            }
            ws();
            if (peek() == ',') { ++i_; continue; }
            expect('}');
            break;
        }
        if (!have_off || t.dtype.empty()) fail("tensor entry without dtype/data_offsets");
        return t;
    }
};

}  // namespace

std::map<std::string, Tensor> parse_safetensors_header(const std::string& json) {
    return HeaderReader(json).tensors();
}

Weights::~Weights() {
    if (buf_) {
        buf_->release();
        delete buf_;
    }
}

namespace {

// The safetensors format bounds its JSON header at 100 MB.
constexpr uint64_t kHeaderCap = 100ull << 20;

struct CloseFile {
    void operator()(FILE* f) const {
        if (f) fclose(f);
    }
};
using File = std::unique_ptr<FILE, CloseFile>;

bool read_all(FILE* f, void* dst, uint64_t n) {
    return n == 0 || fread(dst, 1, (size_t)n, f) == (size_t)n;
}

}  // namespace

// A safetensors file is <u64 little-endian header size><JSON header><data>.
// Everything is validated (header bounds, every tensor's byte range) before
// the data block is read and before any device memory is touched; the
// object is only modified once the device copy exists.
bool Weights::load(Metal& m, const std::string& path, std::string& err) {
    auto reject = [&](const std::string& why) {
        err = path + ": " + why;
        return false;
    };
    File f(fopen(path.c_str(), "rb"));
    if (!f) return reject(std::string("open failed: ") + strerror(errno));
    if (fseeko(f.get(), 0, SEEK_END) != 0) return reject("not a seekable file");
    const off_t end = ftello(f.get());
    if (end < 0) return reject("size unknown");
    const uint64_t total = (uint64_t)end;
    rewind(f.get());

    uint8_t prefix[8];
    if (total < 8 || !read_all(f.get(), prefix, 8)) return reject("no 8-byte header size");
    uint64_t hsize = 0;
    for (int i = 7; i >= 0; --i) hsize = (hsize << 8) | prefix[i];
    if (hsize == 0 || hsize > kHeaderCap || hsize > total - 8)
        return reject("header size " + std::to_string(hsize) + " does not fit a " +
                      std::to_string(total) + "-byte file");
    std::string json((size_t)hsize, '\0');
    if (!read_all(f.get(), &json[0], hsize)) return reject("header cut short");

    std::map<std::string, Tensor> table;
    try {
        table = parse_safetensors_header(json);
    } catch (const std::exception& e) {
        return reject(e.what());
    }
    const uint64_t data_bytes = total - 8 - hsize;
    for (const auto& kv : table)
        if (kv.second.end > data_bytes)
            return reject("tensor " + kv.first + " ends at byte " + std::to_string(kv.second.end) +
                          " of a " + std::to_string(data_bytes) + "-byte data block");

    std::vector<uint8_t> data((size_t)data_bytes);
    if (!read_all(f.get(), data.data(), data_bytes)) return reject("data block cut short");
    MTL::Buffer* dev = nullptr;
    try {
        dev = m.new_buffer(data.empty() ? 1 : data.size(), /*shared=*/false);
        dev->upload(data.data(), data.size());
    } catch (const std::exception& e) {
        if (dev) {
            dev->release();
            delete dev;
        }
        return reject(std::string("device copy failed: ") + e.what());
    }
    if (buf_) {
        buf_->release();
        delete buf_;
    }
    buf_ = dev;
    host_ = std::move(data);
    tensors_ = std::move(table);
    for (auto& kv : tensors_) kv.second.ptr = host_.data() + kv.second.begin;
    return true;
}

const Tensor* Weights::find(const std::string& name) const {
    const auto it = tensors_.find(name);
    return it != tensors_.end() ? &it->second : nullptr;
}

const Tensor& Weights::get(const std::string& name) const {
    if (const Tensor* t = find(name)) return *t;
    throw std::runtime_error("weights: no tensor named '" + name + "'");
}

bool Weights::has(const std::string& name) const { return find(name) != nullptr; }

}  // namespace miori
