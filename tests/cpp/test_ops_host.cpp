// C++ host test of the src/ops.h-signature wrappers (miori_amd/host):
// a synthetic MLX-4bit safetensors file is written, loaded with Weights, and
// the hot-path ops are called exactly as src/engine.cpp / src/main.cpp call
// them (Metal&, encoder, Weights&, Tensor&, MTL::Buffer*). Results are
// checked against the CPU oracle (oracle/cpu_ref.c) like the reference's
// test_gemv (src/main.cpp:44-87), with the benchmark tolerance.
//
// Usage: test_ops_host <scratch-dir>     exit status 0 = all checks passed
#include "../../miori_amd/host/ops_hip.h"
#include "../../oracle/cpu_ref.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

using namespace miori;

namespace {

int g_fail = 0;

void expect(bool ok, const std::string& what) {
    printf("%s %s\n", ok ? "PASS" : "FAIL", what.c_str());
    if (!ok) ++g_fail;
}

uint64_t g_state = 0x4D494F52ull;
uint64_t next64() {
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
double uni() { return (double)(next64() >> 11) * (1.0 / 9007199254740992.0); }

struct Entry {
    std::string name, dtype;
    std::vector<int64_t> shape;
    std::vector<uint8_t> bytes;
};

void write_safetensors(const std::string& path, const std::vector<Entry>& es) {
    std::string h = "{\"__metadata__\":{\"format\":\"mlx\"}";
    uint64_t off = 0;
    for (const auto& e : es) {
        h += ",\"" + e.name + "\":{\"dtype\":\"" + e.dtype + "\",\"shape\":[";
        for (size_t i = 0; i < e.shape.size(); ++i) h += (i ? "," : "") + std::to_string(e.shape[i]);
        h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + e.bytes.size()) + "]}";
        off += e.bytes.size();
    }
    h += "}";
    while (h.size() % 8) h += ' ';
    std::ofstream f(path, std::ios::binary);
    const uint64_t n = h.size();
    f.write((const char*)&n, 8);
    f.write(h.data(), (std::streamsize)h.size());
    for (const auto& e : es) f.write((const char*)e.bytes.data(), (std::streamsize)e.bytes.size());
}

// MLX-affine weights with the benchmark distributions.
void quant(const std::string& base, int bits, int64_t N, int64_t K, int64_t G,
           std::vector<Entry>& out) {
    Entry q{base + ".weight", "U32", {N, K * bits / 32}, {}};
    q.bytes.resize((size_t)N * K * bits / 8);
    for (size_t i = 0; i < q.bytes.size(); i += 4) {
        const uint32_t w = (uint32_t)(next64() >> 32);
        memcpy(&q.bytes[i], &w, 4);
    }
    Entry s{base + ".scales", "BF16", {N, K / G}, {}}, b{base + ".biases", "BF16", {N, K / G}, {}};
    s.bytes.resize((size_t)N * (K / G) * 2);
    b.bytes.resize(s.bytes.size());
    for (size_t i = 0; i < (size_t)N * (K / G); ++i) {
        const float sc = bits == 4 ? (float)(0.001 + 0.009 * uni()) : (float)(1e-4 + 9e-4 * uni());
        const uint16_t sb = orc_f32_to_bf16(sc);
        const float sf = orc_bf16_to_f32(sb);
        const float bi = bits == 4 ? (float)(-8.0 * sf + 1e-3 * (uni() - 0.5) * 3.4) : -128.f * sf;
        const uint16_t bb = orc_f32_to_bf16(bi);
        memcpy(&s.bytes[2 * i], &sb, 2);
        memcpy(&b.bytes[2 * i], &bb, 2);
    }
    out.push_back(std::move(q));
    out.push_back(std::move(s));
    out.push_back(std::move(b));
}

// x[k] = ((37k mod 101) - 50) / 50, the reference test input (src/main.cpp:28)
float xfn(size_t k) { return ((float)((k * 37) % 101) - 50.0f) / 50.0f; }

bool close_enough(const float* got, const double* ref, size_t n, const char* what) {
    double mref = 0, md = 0;
    size_t ok2 = 0;
    for (size_t i = 0; i < n; ++i) {
        mref = std::max(mref, std::fabs(ref[i]));
        const double d = std::fabs((double)got[i] - ref[i]);
        md = std::max(md, d);
        const double a = std::max(std::fabs(ref[i]), 1.1754943508222875e-38);
        const double ulp = std::ldexp(1.0, (int)std::floor(std::log2(a)) - 7);
        ok2 += d <= 2 * ulp;
    }
    const bool ok = md <= 1e-4 * mref && ok2 >= (size_t)std::ceil(0.999 * n);
    printf("  %s: max|d|=%.3g max|ref|=%.3g within-2ulp=%.5f\n", what, md, mref, (double)ok2 / n);
    return ok;
}

}  // namespace

int main(int argc, char** argv) {
    const std::string dir = argc > 1 ? argv[1] : ".";
    const std::string path = dir + "/test_ops_host.safetensors";
    const int64_t N = 2048, K = 2048, G = 64, NV = 4096;
    std::vector<Entry> es;
    quant("layers.2.self_attn.q_proj", 4, N, K, G, es);
    quant("embed_tokens", 8, NV, K, G, es);
    {
        Entry nw{"layers.2.input_layernorm.weight", "BF16", {K}, {}};
        nw.bytes.resize((size_t)K * 2);
        for (int64_t k = 0; k < K; ++k) {
            const uint16_t v = orc_f32_to_bf16((float)(0.8 + 0.4 * uni()));
            memcpy(&nw.bytes[2 * k], &v, 2);
        }
        es.push_back(std::move(nw));
    }
    write_safetensors(path, es);

    Metal m;
    std::string err;
    if (!m.init("", err)) { printf("FAIL init: %s\n", err.c_str()); return 2; }
    m.print_info();
    Weights w;
    if (!w.load(m, path, err)) { printf("FAIL load: %s\n", err.c_str()); return 2; }
    expect(w.tensor_count() == 7, "safetensors loader: 7 tensors");
    const Tensor& q = w.get("layers.2.self_attn.q_proj.weight");
    const Tensor& s = w.get("layers.2.self_attn.q_proj.scales");
    const Tensor& b = w.get("layers.2.self_attn.q_proj.biases");
    expect(q.rows() == N && q.cols() * 8 == K && s.cols() == K / G, "tensor shapes");

    // ---- gemv4, as test-gemv4 (src/main.cpp:44-87)
    const int B = 16;
    MTL::Buffer* x = m.new_buffer((size_t)B * K * 2);
    MTL::Buffer* y = m.new_buffer((size_t)B * N * 4);
    uint16_t* xp = (uint16_t*)x->contents();
    for (int r = 0; r < B; ++r)
        for (int64_t k = 0; k < K; ++k) xp[r * K + k] = orc_f32_to_bf16(xfn(k + 7 * r));
    {
        auto cb = m.begin();
        auto e = cb->computeCommandEncoder();
        gemv4(m, e, w, q, s, b, x, y, (uint32_t)N, (uint32_t)K);
        e->endEncoding();
        m.submit(cb, true);
    }
    std::vector<double> ref((size_t)B * N);
    orc_gemv4_f64((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr, xp,
                  ref.data(), 1, N, K, G, 8);
    expect(close_enough((const float*)y->contents(), ref.data(), N, "gemv4"), "gemv4 vs oracle");

    // ---- gemv4_b with B = 4 (the reference's batch) and B = 16
    for (int bb : {4, 16}) {
        auto cb = m.begin();
        auto e = cb->computeCommandEncoder();
        gemv4_b(m, e, w, q, s, b, x, y, (uint32_t)N, (uint32_t)K, (uint32_t)bb);
        m.submit(cb, true);
        xp = (uint16_t*)x->contents();
        orc_gemv4_f64((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr, xp,
                      ref.data(), bb, N, K, G, 8);
        expect(close_enough((const float*)y->contents(), ref.data(), (size_t)bb * N, "gemv4_b"),
               "gemv4_b B=" + std::to_string(bb));
    }

    // ---- gemv8 lm_head and gemv8_b_off on 4 rows at an offset
    {
        const Tensor& eq = w.get("embed_tokens.weight");
        const Tensor& esc = w.get("embed_tokens.scales");
        const Tensor& ebi = w.get("embed_tokens.biases");
        MTL::Buffer* logits = m.new_buffer((size_t)8 * NV * 4);
        auto cb = m.begin();
        auto e = cb->computeCommandEncoder();
        gemv8(m, e, w, eq, esc, ebi, x, logits, (uint32_t)NV, (uint32_t)K);
        m.submit(cb, true);
        xp = (uint16_t*)x->contents();
        std::vector<double> r8((size_t)8 * NV);
        orc_gemv8_f64((const uint32_t*)eq.ptr, (const uint16_t*)esc.ptr, (const uint16_t*)ebi.ptr,
                      xp, r8.data(), 1, NV, K, G, 8);
        expect(close_enough((const float*)logits->contents(), r8.data(), NV, "gemv8"), "gemv8 vs oracle");
        cb = m.begin();
        e = cb->computeCommandEncoder();
        gemv8_b_off(m, e, w, eq, esc, ebi, x, logits, (uint32_t)NV, (uint32_t)K, 4,
                    (uint32_t)(4 * K * 2), (uint32_t)(4 * NV * 4));
        m.submit(cb, true);
        xp = (uint16_t*)x->contents();
        orc_gemv8_f64((const uint32_t*)eq.ptr, (const uint16_t*)esc.ptr, (const uint16_t*)ebi.ptr,
                      xp + 4 * K, r8.data(), 4, NV, K, G, 8);
        expect(close_enough((const float*)logits->contents() + 4 * NV, r8.data(), 4 * (size_t)NV,
                            "gemv8_b_off"),
               "gemv8_b_off rows 4..7");
        logits->release();
        delete logits;
    }

    // ---- weight cache + prefill GEMM, and the fused GEMM on the same operands
    {
        const uint32_t M = 96;
        MTL::Buffer* cache = m.new_buffer((size_t)N * K * 2, false);
        MTL::Buffer* A = m.new_buffer((size_t)M * K * 2);
        MTL::Buffer* C1 = m.new_buffer((size_t)M * N * 4);
        MTL::Buffer* C2 = m.new_buffer((size_t)M * N * 4);
        uint16_t* ap = (uint16_t*)A->contents();
        for (size_t i = 0; i < (size_t)M * K; ++i) ap[i] = orc_f32_to_bf16(sinf(0.13f * (float)i));
        auto cb = m.begin();
        auto e = cb->computeCommandEncoder();
        dequant_tile(m, e, w, q, s, b, cache, (uint32_t)N, (uint32_t)K);
        gemm_mpp(m, e, A, cache, C1, M, (uint32_t)N, (uint32_t)K);
        gemm_q4(m, e, A, w, q, s, b, C2, M, (uint32_t)N, (uint32_t)K);
        m.submit(cb, true);
        std::vector<uint16_t> cache_host((size_t)N * K), cache_ref((size_t)N * K);
        cache->download(cache_host.data(), cache_host.size() * 2);
        orc_dequant4_bf16((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr,
                          cache_ref.data(), N, K, G);
        expect(cache_host == cache_ref, "dequant_tile bit-exact vs oracle");
        std::vector<int64_t> rows;
        for (uint32_t r = 0; r < M; ++r) rows.push_back(r);
        std::vector<double> cref((size_t)M * N);
        ap = (uint16_t*)A->contents();
        orc_gemm_bf16_f64(ap, cache_ref.data(), cref.data(), M, N, K, rows.data(), M, 8);
        const float* c1 = (const float*)C1->contents();
        const float* c2 = (const float*)C2->contents();
        expect(close_enough(c1, cref.data(), (size_t)M * N, "gemm_mpp"), "gemm_mpp vs oracle");
        expect(memcmp(c1, c2, (size_t)M * N * 4) == 0, "gemm_q4 bit-identical to dequant_tile + gemm_mpp");
    }

    // ---- fused decode steps: rmsnorm -> gemv4 and silu_mul -> gemv4
    {
        const Tensor& nw = w.get("layers.2.input_layernorm.weight");
        MTL::Buffer* xf = m.new_buffer((size_t)K * 4);
        MTL::Buffer* uf = m.new_buffer((size_t)K * 4);
        float* xfp = (float*)xf->contents();
        float* ufp = (float*)uf->contents();
        for (int64_t k = 0; k < K; ++k) {
            xfp[k] = (float)(3.0 * (uni() - 0.5));
            ufp[k] = (float)(2.0 * (uni() - 0.5));
        }
        auto cb = m.begin();
        auto e = cb->computeCommandEncoder();
        rmsnorm_gemv4(m, e, w, q, s, b, xf, nw, y, (uint32_t)N, (uint32_t)K, 1e-5f);
        m.submit(cb, true);
        std::vector<uint16_t> h((size_t)K);
        xfp = (float*)xf->contents();
        orc_rmsnorm_bf16(xfp, (const uint16_t*)nw.ptr, h.data(), K, 1e-5f);
        orc_gemv4_f64((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr,
                      h.data(), ref.data(), 1, N, K, G, 8);
        expect(close_enough((const float*)y->contents(), ref.data(), N, "rmsnorm_gemv4"),
               "rmsnorm_gemv4 vs oracle");
        cb = m.begin();
        e = cb->computeCommandEncoder();
        silu_mul_gemv4(m, e, w, q, s, b, xf, uf, y, (uint32_t)N, (uint32_t)K);
        m.submit(cb, true);
        xfp = (float*)xf->contents();
        ufp = (float*)uf->contents();
        orc_silu_mul_bf16(xfp, ufp, h.data(), K);
        orc_gemv4_f64((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr,
                      h.data(), ref.data(), 1, N, K, G, 8);
        expect(close_enough((const float*)y->contents(), ref.data(), N, "silu_mul_gemv4"),
               "silu_mul_gemv4 vs oracle");
        xf->release(); delete xf;
        uf->release(); delete uf;
    }

    // ---- gemm_naive: the reference's test-gemm case (src/main.cpp:578-602),
    // M=4 N=8 K=32 with lda=64 ldb=32 ldc=16, bit-exact against the
    // sequential fp32 FMA chain
    {
        const uint32_t M = 4, NN = 8, KK = 32, lda = 64, ldb = 32, ldc = 16;
        MTL::Buffer* A = m.new_buffer((size_t)M * lda * 2);
        MTL::Buffer* Bm = m.new_buffer((size_t)NN * ldb * 2);
        MTL::Buffer* C = m.new_buffer((size_t)M * ldc * 4);
        uint16_t* ap = (uint16_t*)A->contents();
        uint16_t* bp = (uint16_t*)Bm->contents();
        for (uint32_t i = 0; i < M * lda; ++i) ap[i] = orc_f32_to_bf16((float)(2.0 * uni() - 1.0));
        for (uint32_t i = 0; i < NN * ldb; ++i) bp[i] = orc_f32_to_bf16((float)(2.0 * uni() - 1.0));
        float* cp = (float*)C->contents();
        for (uint32_t i = 0; i < M * ldc; ++i) cp[i] = -7.f;   // untouched padding columns
        auto cb = m.begin();
        auto e = cb->computeCommandEncoder();
        gemm_naive(m, e, A, Bm, C, M, NN, KK, lda, ldb, ldc);
        m.submit(cb, true);
        std::vector<float> cref((size_t)M * ldc, -7.f);
        ap = (uint16_t*)A->contents();
        bp = (uint16_t*)Bm->contents();
        orc_gemm_naive_f32(ap, bp, cref.data(), M, NN, KK, lda, ldb, ldc);
        expect(memcmp(C->contents(), cref.data(), cref.size() * 4) == 0,
               "gemm_naive bit-exact vs sequential fp32 chain (padding untouched)");
        A->release(); delete A;
        Bm->release(); delete Bm;
        C->release(); delete C;
    }

    // ---- raw-buffer and offset entries the engines use: gemv8_off (batched
    // lm_head, src/batch.cpp:596-600) at group 64 through the Metal's
    // raw_group and through the explicit-group overload, gemv4_raw on its own
    // buffers, gemv8_b on 8 rows, dequant4 / dequant8 bit-exact
    {
        const Tensor& eq = w.get("embed_tokens.weight");
        const Tensor& esc = w.get("embed_tokens.scales");
        const Tensor& ebi = w.get("embed_tokens.biases");
        MTL::Buffer* logits = m.new_buffer((size_t)8 * NV * 4);
        std::vector<double> r8((size_t)8 * NV);
        xp = (uint16_t*)x->contents();
        // rows 2 and 5 of x, written at output rows 1 and 6
        m.raw_group = (uint32_t)G;
        auto cb = m.begin();
        auto e = cb->computeCommandEncoder();
        gemv8_off(m, e, w.buffer(), (uint32_t)eq.begin, (uint32_t)esc.begin, (uint32_t)ebi.begin, x,
                  logits, (uint32_t)NV, (uint32_t)K, (uint32_t)(2 * K * 2), (uint32_t)(1 * NV * 4));
        m.raw_group = 32;
        gemv8_off(m, e, w.buffer(), (uint32_t)eq.begin, (uint32_t)esc.begin, (uint32_t)ebi.begin, x,
                  logits, (uint32_t)NV, (uint32_t)K, (uint32_t)(5 * K * 2), (uint32_t)(6 * NV * 4),
                  (uint32_t)G);
        m.submit(cb, true);
        const float* lg = (const float*)logits->contents();
        xp = (uint16_t*)x->contents();
        orc_gemv8_f64((const uint32_t*)eq.ptr, (const uint16_t*)esc.ptr, (const uint16_t*)ebi.ptr,
                      xp + 2 * K, r8.data(), 1, NV, K, G, 8);
        expect(close_enough(lg + NV, r8.data(), NV, "gemv8_off raw_group=64"),
               "gemv8_off (Metal::raw_group = 64) vs oracle");
        orc_gemv8_f64((const uint32_t*)eq.ptr, (const uint16_t*)esc.ptr, (const uint16_t*)ebi.ptr,
                      xp + 5 * K, r8.data(), 1, NV, K, G, 8);
        expect(close_enough(lg + 6 * NV, r8.data(), NV, "gemv8_off group=64"),
               "gemv8_off (explicit group 64) vs oracle");

        cb = m.begin();
        e = cb->computeCommandEncoder();
        gemv8_b(m, e, w, eq, esc, ebi, x, logits, (uint32_t)NV, (uint32_t)K, 8);
        m.submit(cb, true);
        xp = (uint16_t*)x->contents();
        orc_gemv8_f64((const uint32_t*)eq.ptr, (const uint16_t*)esc.ptr, (const uint16_t*)ebi.ptr,
                      xp, r8.data(), 8, NV, K, G, 8);
        expect(close_enough((const float*)logits->contents(), r8.data(), 8 * (size_t)NV, "gemv8_b"),
               "gemv8_b B=8 vs oracle");

        // gemv4_raw: q / scales / biases in buffers of their own
        MTL::Buffer* rq = m.new_buffer(q.bytes(), false);
        MTL::Buffer* rs = m.new_buffer(s.bytes(), false);
        MTL::Buffer* rb = m.new_buffer(b.bytes(), false);
        rq->upload(q.ptr, q.bytes());
        rs->upload(s.ptr, s.bytes());
        rb->upload(b.ptr, b.bytes());
        cb = m.begin();
        e = cb->computeCommandEncoder();
        gemv4_raw(m, e, rq, rs, rb, x, y, (uint32_t)N, (uint32_t)K, (uint32_t)G);
        m.submit(cb, true);
        xp = (uint16_t*)x->contents();
        orc_gemv4_f64((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr, xp,
                      ref.data(), 1, N, K, G, 8);
        expect(close_enough((const float*)y->contents(), ref.data(), N, "gemv4_raw"),
               "gemv4_raw (group 64) vs oracle");
        rq->release(); delete rq;
        rs->release(); delete rs;
        rb->release(); delete rb;

        MTL::Buffer* d4 = m.new_buffer((size_t)N * K * 2, false);
        MTL::Buffer* d8 = m.new_buffer((size_t)NV * K * 2, false);
        cb = m.begin();
        e = cb->computeCommandEncoder();
        dequant4(m, e, w, q, s, b, d4, (uint32_t)N, (uint32_t)K);
        dequant8(m, e, w, eq, esc, ebi, d8, (uint32_t)NV, (uint32_t)K);
        m.submit(cb, true);
        std::vector<uint16_t> got4((size_t)N * K), ref4((size_t)N * K);
        std::vector<uint16_t> got8((size_t)NV * K), ref8((size_t)NV * K);
        d4->download(got4.data(), got4.size() * 2);
        d8->download(got8.data(), got8.size() * 2);
        orc_dequant4_bf16((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr,
                          ref4.data(), N, K, G);
        orc_dequant8_bf16((const uint32_t*)eq.ptr, (const uint16_t*)esc.ptr,
                          (const uint16_t*)ebi.ptr, ref8.data(), NV, K, G);
        expect(got4 == ref4, "dequant4 bit-exact vs oracle");
        expect(got8 == ref8, "dequant8 bit-exact vs oracle");
        d4->release(); delete d4;
        d8->release(); delete d8;
        logits->release(); delete logits;
    }

    // ---- gemm_mpp_off with non-zero A / B / C offsets (src/engine.cpp:508-518),
    // gemm_mpp32 on 32 rows, and the batch-engine linear policy
    // (src/batch.cpp:223-230) at 8 rows (exact GEMV) and 96 rows (cache GEMM,
    // and the fused GEMM without a cache)
    {
        const uint32_t M = 96, aoff = 3 * K * 2, boff = 4096, coff = 5 * N * 4;
        MTL::Buffer* cache = m.new_buffer(boff + (size_t)N * K * 2, false);
        MTL::Buffer* A = m.new_buffer(aoff + (size_t)M * K * 2);
        MTL::Buffer* C = m.new_buffer(coff + (size_t)M * N * 4);
        MTL::Buffer* C2 = m.new_buffer((size_t)M * N * 4);
        uint16_t* ap = (uint16_t*)A->contents();
        for (size_t i = 0; i < aoff / 2 + (size_t)M * K; ++i)
            ap[i] = orc_f32_to_bf16(cosf(0.07f * (float)i));
        auto cb = m.begin();
        auto e = cb->computeCommandEncoder();
        dequant_tile(m, e, w, q, s, b, cache, (uint32_t)N, (uint32_t)K, boff);
        gemm_mpp_off(m, e, A, cache, C, M, (uint32_t)N, (uint32_t)K, aoff, boff, coff);
        m.submit(cb, true);
        std::vector<uint16_t> cref16((size_t)N * K);
        orc_dequant4_bf16((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr,
                          cref16.data(), N, K, G);
        std::vector<int64_t> rows;
        for (uint32_t r = 0; r < M; ++r) rows.push_back(r);
        std::vector<double> cref((size_t)M * N);
        ap = (uint16_t*)A->contents();
        orc_gemm_bf16_f64(ap + aoff / 2, cref16.data(), cref.data(), M, N, K, rows.data(), M, 8);
        const float* cp = (const float*)((const char*)C->contents() + coff);
        expect(close_enough(cp, cref.data(), (size_t)M * N, "gemm_mpp_off"),
               "gemm_mpp_off (aoff, boff, coff != 0) vs oracle");

        // gemm_mpp32: rows 0..31 of the same product
        cb = m.begin();
        e = cb->computeCommandEncoder();
        gemm_mpp32(m, e, A, cache, C2, 32, (uint32_t)N, (uint32_t)K, boff);
        m.submit(cb, true);
        ap = (uint16_t*)A->contents();
        orc_gemm_bf16_f64(ap, cref16.data(), cref.data(), 32, N, K, rows.data(), 32, 8);
        expect(close_enough((const float*)C2->contents(), cref.data(), (size_t)32 * N, "gemm_mpp32"),
               "gemm_mpp32 vs oracle");

        // linear: 8 rows take the exact 4-bit GEMV (fp64-of-fp32-dequant oracle)
        cb = m.begin();
        e = cb->computeCommandEncoder();
        linear(m, e, w, q, s, b, x, C2, (uint32_t)N, (uint32_t)K, 8, cache, boff);
        m.submit(cb, true);
        xp = (uint16_t*)x->contents();
        std::vector<double> rl((size_t)8 * N);
        orc_gemv4_f64((const uint32_t*)q.ptr, (const uint16_t*)s.ptr, (const uint16_t*)b.ptr, xp,
                      rl.data(), 8, N, K, G, 8);
        expect(close_enough((const float*)C2->contents(), rl.data(), (size_t)8 * N, "linear B=8"),
               "linear B=8 (exact 4-bit) vs oracle");
        // 96 rows with the cache: the bf16 GEMM; without: the fused GEMM, same values
        cb = m.begin();
        e = cb->computeCommandEncoder();
        linear(m, e, w, q, s, b, A, C2, (uint32_t)N, (uint32_t)K, M, cache, boff);
        m.submit(cb, true);
        ap = (uint16_t*)A->contents();
        orc_gemm_bf16_f64(ap, cref16.data(), cref.data(), M, N, K, rows.data(), M, 8);
        std::vector<float> lc((size_t)M * N);
        memcpy(lc.data(), C2->contents(), lc.size() * 4);
        expect(close_enough(lc.data(), cref.data(), (size_t)M * N, "linear B=96 cache"),
               "linear B=96 (bf16 cache GEMM) vs oracle");
        cb = m.begin();
        e = cb->computeCommandEncoder();
        linear(m, e, w, q, s, b, A, C2, (uint32_t)N, (uint32_t)K, M);
        m.submit(cb, true);
        expect(memcmp(lc.data(), C2->contents(), lc.size() * 4) == 0,
               "linear B=96 without cache (fused GEMM) bit-identical to the cache GEMM");
        cache->release(); delete cache;
        A->release(); delete A;
        C->release(); delete C;
        C2->release(); delete C2;
    }

    // ---- errors surface as exceptions, as the reference's Metal::pso does
    {
        bool threw = false;
        try {
            auto cb = m.begin();
            auto e = cb->computeCommandEncoder();
            gemv4(m, e, w, q, s, b, x, y, (uint32_t)N * 2, (uint32_t)K);  // tensor too small
        } catch (const std::runtime_error&) { threw = true; }
        expect(threw, "out-of-range shape throws before launch");
        threw = false;
        try {
            auto cb = m.begin();
            auto e = cb->computeCommandEncoder();
            gemv4_b(m, e, w, q, s, b, x, y, (uint32_t)N, (uint32_t)K, 40);  // B > 32
        } catch (const std::runtime_error&) { threw = true; }
        expect(threw, "batch of 40 rows is rejected");
    }

    x->release(); delete x;
    y->release(); delete y;
    std::remove(path.c_str());
    printf("%s (%d failed)\n", g_fail ? "FAILED" : "ALL PASSED", g_fail);
    return g_fail ? 1 : 0;
}
