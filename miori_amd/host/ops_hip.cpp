// src/ops.h hot-path wrappers over the C ABI. Each wrapper checks that every
// (buffer, offset) range it binds lies inside its buffer, so a wrong shape
// is an exception on the host, never an out-of-bounds access on the device.
#include "ops_hip.h"

#include "../../include/miori_hip.h"

#include <stdexcept>
#include <string>

namespace miori {

namespace {

void check(int st, const char* fn) {
    if (st != MIORI_OK)
        throw std::runtime_error(std::string(fn) + ": " + miori_status_string(st));
}

void need(const MTL::Buffer* b, uint64_t off, uint64_t bytes, const char* what) {
    if (!b) throw std::runtime_error(std::string(what) + ": null buffer");
    if (off + bytes > b->length())
        throw std::runtime_error(std::string(what) + ": range [" + std::to_string(off) + ", " +
                                 std::to_string(off + bytes) + ") exceeds buffer of " +
                                 std::to_string(b->length()) + " bytes");
}

void need_tensor(const Tensor& t, uint64_t bytes, const char* what) {
    if (t.bytes() < bytes)
        throw std::runtime_error(std::string(what) + ": tensor " + t.name + " holds " +
                                 std::to_string(t.bytes()) + " bytes, the shape needs " +
                                 std::to_string(bytes));
}

const char* at(const MTL::Buffer* b, uint64_t off) { return (const char*)b->gpu() + off; }
char* at_w(MTL::Buffer* b, uint64_t off) { return (char*)b->gpu() + off; }

// group = K / scales.cols() (scales are [N][K/group]).
uint32_t group_of(const Tensor& s, uint32_t K) {
    const int64_t c = s.cols();
    if (c <= 0 || K % c) throw std::runtime_error("cannot infer group size from " + s.name);
    return K / (uint32_t)c;
}

struct QArgs {
    const void* q;
    const void* s;
    const void* b;
    uint32_t G;
};

QArgs qargs(MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q, const Tensor& s,
            const Tensor& b, uint32_t N, uint32_t K, int bits) {
    const uint32_t G = group_of(s, K);
    need_tensor(q, (uint64_t)N * K * bits / 8, "weights");
    need_tensor(s, (uint64_t)N * (K / G) * 2, "scales");
    need_tensor(b, (uint64_t)N * (K / G) * 2, "biases");
    MTL::Buffer* wb = w.buffer();
    need(wb, q.end, 0, "weights buffer");
    e->use_in(wb);
    return {at(wb, q.begin), at(wb, s.begin), at(wb, b.begin), G};
}

void gemv_t(int bits, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
            const Tensor& s, const Tensor& b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
            uint32_t K, uint32_t B, uint32_t xoff, uint32_t yoff, bool batched) {
    QArgs a = qargs(e, w, q, s, b, N, K, bits);
    need(x, xoff, (uint64_t)B * K * 2, "x");
    need(y, yoff, (uint64_t)B * N * 4, "y");
    e->use_in(x);
    e->use_out(y);
    const char* fn;
    int st;
    if (!batched) {
        fn = bits == 4 ? "gemv4" : "gemv8";
        st = (bits == 4 ? miori_gemv_q4 : miori_gemv_q8)(a.q, a.s, a.b, at(x, xoff), at_w(y, yoff), N,
                                                         K, a.G, MIORI_F32, e->stream());
    } else {
        fn = bits == 4 ? "gemv4_b" : "gemv8_b";
        st = (bits == 4 ? miori_gemv_q4_batched : miori_gemv_q8_batched)(
            a.q, a.s, a.b, at(x, xoff), at_w(y, yoff), B, N, K, a.G, MIORI_F32, e->stream());
    }
    check(st, fn);
}

void dequant_t(int bits, bool tile, MTL::ComputeCommandEncoder* e, const Weights& w,
               const Tensor& q, const Tensor& s, const Tensor& b, MTL::Buffer* out, uint32_t N,
               uint32_t K, uint32_t boff) {
    QArgs a = qargs(e, w, q, s, b, N, K, bits);
    need(out, boff, (uint64_t)N * K * 2, "dequant out");
    e->use_out(out);
    int st;
    if (bits == 8)
        st = miori_dequant_q8(a.q, a.s, a.b, at_w(out, boff), N, K, a.G, e->stream());
    else if (tile)
        st = miori_dequant_q4_tile(a.q, a.s, a.b, at_w(out, boff), N, K, a.G, e->stream());
    else
        st = miori_dequant_q4(a.q, a.s, a.b, at_w(out, boff), N, K, a.G, e->stream());
    check(st, bits == 8 ? "dequant8" : tile ? "dequant_tile" : "dequant4");
}

}  // namespace

void gemv4(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
           const Tensor& s, const Tensor& b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
           uint32_t K) {
    gemv_t(4, e, w, q, s, b, x, y, N, K, 1, 0, 0, false);
}

void rmsnorm_gemv4(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
                   const Tensor& s, const Tensor& b, MTL::Buffer* x, const Tensor& norm_w,
                   MTL::Buffer* y, uint32_t N, uint32_t K, float eps) {
    QArgs a = qargs(e, w, q, s, b, N, K, 4);
    need_tensor(norm_w, (uint64_t)K * 2, "norm weight");
    need(x, 0, (uint64_t)K * 4, "x");
    need(y, 0, (uint64_t)N * 4, "y");
    e->use_in(x);
    e->use_out(y);
    check(miori_rmsnorm_gemv_q4((const float*)x->gpu(), at(w.buffer(), norm_w.begin), eps, a.q,
                                a.s, a.b, y->gpu(), N, K, a.G, MIORI_F32, e->stream()),
          "rmsnorm_gemv4");
}

void silu_mul_gemv4(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
                    const Tensor& s, const Tensor& b, MTL::Buffer* gate, MTL::Buffer* up,
                    MTL::Buffer* y, uint32_t N, uint32_t K) {
    QArgs a = qargs(e, w, q, s, b, N, K, 4);
    need(gate, 0, (uint64_t)K * 4, "gate");
    need(up, 0, (uint64_t)K * 4, "up");
    need(y, 0, (uint64_t)N * 4, "y");
    e->use_in(gate); e->use_in(up);
    e->use_out(y);
    check(miori_silu_mul_gemv_q4((const float*)gate->gpu(), (const float*)up->gpu(), a.q, a.s,
                                 a.b, y->gpu(), N, K, a.G, MIORI_F32, e->stream()),
          "silu_mul_gemv4");
}

void gemv8(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
           const Tensor& s, const Tensor& b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
           uint32_t K) {
    gemv_t(8, e, w, q, s, b, x, y, N, K, 1, 0, 0, false);
}

void gemv4x4(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
             const Tensor& s, const Tensor& b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
             uint32_t K) {
    gemv4(m, e, w, q, s, b, x, y, N, K);
}

void gemv4x2(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
             const Tensor& s, const Tensor& b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
             uint32_t K) {
    gemv4(m, e, w, q, s, b, x, y, N, K);
}

void gemv4_raw(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* q, MTL::Buffer* s,
               MTL::Buffer* b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N, uint32_t K) {
    gemv4_raw(m, e, q, s, b, x, y, N, K, m.raw_group);
}

void gemv4_raw(Metal&, MTL::ComputeCommandEncoder* e, MTL::Buffer* q, MTL::Buffer* s,
               MTL::Buffer* b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N, uint32_t K,
               uint32_t G) {
    if (G == 0 || K % G) throw std::runtime_error("gemv4_raw: K is not a multiple of the group");
    need(q, 0, (uint64_t)N * K / 2, "q");
    need(s, 0, (uint64_t)N * (K / G) * 2, "s");
    need(b, 0, (uint64_t)N * (K / G) * 2, "b");
    need(x, 0, (uint64_t)K * 2, "x");
    need(y, 0, (uint64_t)N * 4, "y");
    e->use_in(q); e->use_in(s); e->use_in(b); e->use_in(x);
    e->use_out(y);
    check(miori_gemv_q4(q->gpu(), s->gpu(), b->gpu(), x->gpu(), y->gpu(), N, K, G, MIORI_F32,
                        e->stream()),
          "gemv4_raw");
}

void gemv8_off(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* wbuf, uint32_t qoff,
               uint32_t soff, uint32_t boff, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
               uint32_t K, uint32_t xoff, uint32_t yoff) {
    gemv8_off(m, e, wbuf, qoff, soff, boff, x, y, N, K, xoff, yoff, m.raw_group);
}

void gemv8_off(Metal&, MTL::ComputeCommandEncoder* e, MTL::Buffer* wbuf, uint32_t qoff,
               uint32_t soff, uint32_t boff, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
               uint32_t K, uint32_t xoff, uint32_t yoff, uint32_t G) {
    if (G == 0 || K % G) throw std::runtime_error("gemv8_off: K is not a multiple of the group");
    need(wbuf, qoff, (uint64_t)N * K, "q");
    need(wbuf, soff, (uint64_t)N * (K / G) * 2, "s");
    need(wbuf, boff, (uint64_t)N * (K / G) * 2, "b");
    need(x, xoff, (uint64_t)K * 2, "x");
    need(y, yoff, (uint64_t)N * 4, "y");
    e->use_in(wbuf); e->use_in(x);
    e->use_out(y);
    check(miori_gemv_q8(at(wbuf, qoff), at(wbuf, soff), at(wbuf, boff), at(x, xoff),
                        at_w(y, yoff), N, K, G, MIORI_F32, e->stream()),
          "gemv8_off");
}

void gemv4_b(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
             const Tensor& s, const Tensor& b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
             uint32_t K, uint32_t B) {
    gemv_t(4, e, w, q, s, b, x, y, N, K, B, 0, 0, true);
}

void gemv8_b(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
             const Tensor& s, const Tensor& b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
             uint32_t K, uint32_t B) {
    gemv_t(8, e, w, q, s, b, x, y, N, K, B, 0, 0, true);
}

void gemv8_b_off(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
                 const Tensor& s, const Tensor& b, MTL::Buffer* x, MTL::Buffer* y, uint32_t N,
                 uint32_t K, uint32_t B, uint32_t xoff, uint32_t yoff) {
    gemv_t(8, e, w, q, s, b, x, y, N, K, B, xoff, yoff, true);
}

void dequant4(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
              const Tensor& s, const Tensor& b, MTL::Buffer* out, uint32_t N, uint32_t K,
              uint32_t boff) {
    dequant_t(4, false, e, w, q, s, b, out, N, K, boff);
}

void dequant_tile(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
                  const Tensor& s, const Tensor& b, MTL::Buffer* out, uint32_t N, uint32_t K,
                  uint32_t boff) {
    dequant_t(4, true, e, w, q, s, b, out, N, K, boff);
}

void dequant8(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
              const Tensor& s, const Tensor& b, MTL::Buffer* out, uint32_t N, uint32_t K) {
    dequant_t(8, false, e, w, q, s, b, out, N, K, 0);
}

void gemm_mpp_off(Metal&, MTL::ComputeCommandEncoder* e, MTL::Buffer* A, MTL::Buffer* B,
                  MTL::Buffer* C, uint32_t M, uint32_t N, uint32_t K, uint32_t aoff,
                  uint32_t boff, uint32_t coff) {
    need(A, aoff, (uint64_t)M * K * 2, "A");
    need(B, boff, (uint64_t)N * K * 2, "B");
    need(C, coff, (uint64_t)M * N * 4, "C");
    e->use_in(A); e->use_in(B);
    e->use_out(C);
    check(miori_gemm_bf16(at(A, aoff), at(B, boff), at_w(C, coff), M, N, K, MIORI_F32,
                          e->stream()),
          "gemm_mpp");
}

void gemm_naive(Metal&, MTL::ComputeCommandEncoder* e, MTL::Buffer* A, MTL::Buffer* B,
                MTL::Buffer* C, uint32_t M, uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb,
                uint32_t ldc, uint32_t aoff, uint32_t boff, uint32_t coff) {
    if (M == 0 || N == 0 || K == 0) throw std::runtime_error("gemm_naive: empty shape");
    need(A, aoff, ((uint64_t)(M - 1) * lda + K) * 2, "A");
    need(B, boff, ((uint64_t)(N - 1) * ldb + K) * 2, "B");
    need(C, coff, ((uint64_t)(M - 1) * ldc + N) * 4, "C");
    e->use_in(A); e->use_in(B);
    e->use_out(C);
    check(miori_gemm_naive(at(A, aoff), at(B, boff), (float*)at_w(C, coff), M, N, K, lda, ldb,
                           ldc, e->stream()),
          "gemm_naive");
}

void gemm_mpp(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* A, MTL::Buffer* B,
              MTL::Buffer* C, uint32_t M, uint32_t N, uint32_t K, uint32_t boff) {
    gemm_mpp_off(m, e, A, B, C, M, N, K, 0, boff, 0);
}

void gemm_mpp32(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* A, MTL::Buffer* B,
                MTL::Buffer* C, uint32_t M, uint32_t N, uint32_t K, uint32_t boff) {
    gemm_mpp_off(m, e, A, B, C, M, N, K, 0, boff, 0);
}

void linear(Metal&, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
            const Tensor& s, const Tensor& b, MTL::Buffer* A, MTL::Buffer* C, uint32_t N,
            uint32_t K, uint32_t B, MTL::Buffer* bf16_cache, uint32_t cache_off) {
    QArgs a = qargs(e, w, q, s, b, N, K, 4);
    need(A, 0, (uint64_t)B * K * 2, "A");
    need(C, 0, (uint64_t)B * N * 4, "C");
    const void* cache = nullptr;
    if (bf16_cache) {
        need(bf16_cache, cache_off, (uint64_t)N * K * 2, "bf16 cache");
        e->use_in(bf16_cache);
        cache = at(bf16_cache, cache_off);
    }
    e->use_in(A);
    e->use_out(C);
    check(miori_linear_q4(A->gpu(), a.q, a.s, a.b, cache, C->gpu(), B, N, K, a.G, MIORI_F32,
                          e->stream()),
          "linear");
}

void gemm_q4(Metal&, MTL::ComputeCommandEncoder* e, MTL::Buffer* A, const Weights& w,
             const Tensor& q, const Tensor& s, const Tensor& b, MTL::Buffer* C, uint32_t M,
             uint32_t N, uint32_t K) {
    QArgs a = qargs(e, w, q, s, b, N, K, 4);
    need(A, 0, (uint64_t)M * K * 2, "A");
    need(C, 0, (uint64_t)M * N * 4, "C");
    e->use_in(A);
    e->use_out(C);
    check(miori_gemm_q4(A->gpu(), a.q, a.s, a.b, C->gpu(), M, N, K, a.G, MIORI_F32, e->stream()),
          "gemm_q4");
}

}  // namespace miori
