#include "weights_hip.h"

#include <cctype>
#include <cstdio>
#include <cstring>
#include <fstream>
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

bool Weights::load(Metal& m, const std::string& path, std::string& err) {
    std::ifstream f(path, std::ios::binary);
    if (!f) { err = "cannot open " + path; return false; }
    f.seekg(0, std::ios::end);
    const size_t file_size = (size_t)f.tellg();
    f.seekg(0, std::ios::beg);
    uint64_t header_len = 0;
    f.read((char*)&header_len, 8);
    if (!f || header_len == 0 || header_len > 16 * 1024 * 1024 || 8 + header_len > file_size) {
        err = "bad safetensors header length";
        return false;
    }
    std::string header(header_len, '\0');
    f.read(header.data(), (std::streamsize)header_len);
    if (!f) { err = "truncated header"; return false; }
    const size_t data_start = 8 + (size_t)header_len;
    try {
        tensors_ = parse_safetensors_header(header);
    } catch (const std::exception& e) {
        err = e.what();
        return false;
    }
    host_.resize(file_size - data_start);
    f.read((char*)host_.data(), (std::streamsize)host_.size());
    if (!f) { err = "truncated data"; return false; }
    for (auto& kv : tensors_) {
        Tensor& t = kv.second;
        if (t.end > host_.size()) { err = "tensor out of range: " + t.name; return false; }
        t.ptr = host_.data() + t.begin;
    }
    try {
        buf_ = m.new_buffer(host_.size(), /*shared=*/false);
        buf_->upload(host_.data(), host_.size());
    } catch (const std::exception& e) {
        err = e.what();
        return false;
    }
    return true;
}

const Tensor& Weights::get(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("missing tensor: " + name);
    return it->second;
}

const Tensor* Weights::find(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

bool Weights::has(const std::string& name) const { return tensors_.count(name) != 0; }

}  // namespace miori
