// Host-side robustness test, built with AddressSanitizer and
// UndefinedBehaviorSanitizer (tests/test_host_sanitize.py builds and runs it
// on the CPU; no GPU is touched):
//  * the safetensors header parser on valid headers, on every truncation of
//    one, and on thousands of random byte mutations: it must parse or throw,
//    never read out of bounds;
//  * Weights::load on malformed files (bad size prefix, oversize header,
//    tensor ranges past the data block, truncated data): it must reject them
//    with an error before any device call;
//  * the CPU oracle (oracle/cpu_ref.c) on small and ragged shapes, so every
//    index it computes stays inside its arrays.
#include "../../miori_amd/host/weights_hip.h"
#include "../../oracle/cpu_ref.h"

#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

using namespace miori;

namespace {

int g_fail = 0;
void expect(bool ok, const std::string& what) {
    if (!ok) {
        printf("FAIL %s\n", what.c_str());
        ++g_fail;
    }
}

const char* kHeader =
    "{\"__metadata__\":{\"format\":\"mlx\",\"nested\":{\"a\":[1,2,{\"b\":\"c\"}]}},"
    "\"w.weight\":{\"dtype\":\"U32\",\"shape\":[4,2],\"data_offsets\":[0,32]},"
    "\"w.scales\":{\"dtype\":\"BF16\",\"shape\":[4,1],\"data_offsets\":[32,40]},"
    "\"w.biases\":{\"dtype\":\"BF16\",\"shape\":[4,1],\"data_offsets\":[40,48]}}";

void write_file(const std::string& path, const std::string& header, size_t data_bytes,
                uint64_t size_field) {
    FILE* f = fopen(path.c_str(), "wb");
    uint8_t p[8];
    for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(size_field >> (8 * i));
    fwrite(p, 1, 8, f);
    fwrite(header.data(), 1, header.size(), f);
    std::vector<uint8_t> d(data_bytes, 0x5A);
    if (!d.empty()) fwrite(d.data(), 1, d.size(), f);
    fclose(f);
}

void parser_cases() {
    auto t = parse_safetensors_header(kHeader);
    expect(t.size() == 3 && t["w.weight"].end == 32 && t["w.scales"].shape[0] == 4, "valid header");
    const std::string h(kHeader);
    int threw = 0;
    for (size_t n = 0; n < h.size(); ++n) {
        try {
            parse_safetensors_header(h.substr(0, n));
        } catch (const std::runtime_error&) {
            ++threw;
        }
    }
    expect(threw == (int)h.size(), "every truncation is rejected");
    std::mt19937 rng(7);
    for (int i = 0; i < 20000; ++i) {
        std::string m = h;
        const int edits = 1 + (int)(rng() % 4);
        for (int e = 0; e < edits; ++e) m[rng() % m.size()] = (char)(rng() % 128);
        try {
            parse_safetensors_header(m);
        } catch (const std::exception&) {
        }
    }
    for (const char* bad : {"", "{", "{\"a\":", "{\"a\":{\"dtype\":\"U8\"}}",
                            "{\"a\":{\"dtype\":\"U8\",\"data_offsets\":[4,2]}}",
                            "{\"a\":{\"dtype\":\"U8\",\"data_offsets\":[0]}}", "[1,2]", "\"\\"}) {
        bool rejected = false;
        try {
            parse_safetensors_header(bad);
        } catch (const std::runtime_error&) {
            rejected = true;
        }
        expect(rejected, std::string("malformed header rejected: ") + bad);
    }
}

void loader_cases(const std::string& dir) {
    Metal m;  // never initialised: every case below must fail before a device call
    const std::string p = dir + "/sanitize.safetensors";
    const std::string h(kHeader);
    struct Case {
        const char* what;
        std::string header;
        size_t data;
        uint64_t size_field;
    } cases[] = {
        {"size prefix zero", h, 48, 0},
        {"size prefix past the file", h, 48, h.size() + 100},
        {"size prefix beyond the cap", h, 48, 1ull << 40},
        {"tensor past the data block", h, 40, h.size()},
        {"data block empty", h, 0, h.size()},
        {"header not JSON", std::string(64, 'x'), 48, 64},
    };
    for (const Case& c : cases) {
        write_file(p, c.header, c.data, c.size_field);
        Weights w;
        std::string err;
        const bool ok = w.load(m, p, err);
        expect(!ok && !err.empty() && w.tensor_count() == 0, std::string("loader rejects: ") + c.what);
    }
    {
        FILE* f = fopen(p.c_str(), "wb");
        fwrite("abc", 1, 3, f);
        fclose(f);
        Weights w;
        std::string err;
        expect(!w.load(m, p, err), "loader rejects a 3-byte file");
    }
    Weights w;
    std::string err;
    expect(!w.load(m, dir + "/does-not-exist.safetensors", err) && !err.empty(),
           "loader reports a missing file");
    expect(w.find("w.weight") == nullptr && !w.has("w.weight"), "empty weights find nothing");
    bool threw = false;
    try {
        w.get("w.weight");
    } catch (const std::runtime_error&) {
        threw = true;
    }
    expect(threw, "get() of a missing tensor throws");
    std::remove(p.c_str());
}

void oracle_cases() {
    std::mt19937 rng(11);
    for (int bits : {4, 8}) {
        for (int64_t N : {1, 3, 17}) {
            for (int64_t K : {32, 96, 256}) {
                for (int64_t G : {32, 64}) {
                    if (K % G) continue;
                    const int64_t words = N * K * bits / 32, ng = N * (K / G);
                    std::vector<uint32_t> q(words);
                    std::vector<uint16_t> s(ng), b(ng), x(2 * K), out((size_t)(N * K));
                    for (auto& v : q) v = rng();
                    for (int64_t i = 0; i < ng; ++i) {
                        s[i] = orc_f32_to_bf16(0.01f);
                        b[i] = orc_f32_to_bf16(-0.08f);
                    }
                    for (auto& v : x) v = orc_f32_to_bf16((float)(rng() % 200) / 100.f - 1.f);
                    std::vector<double> y(2 * N);
                    std::vector<float> f((size_t)(N * K));
                    if (bits == 4) {
                        orc_gemv4_f64(q.data(), s.data(), b.data(), x.data(), y.data(), 2, N, K, G, 1);
                        orc_gemv4_rows_f64(q.data(), s.data(), b.data(), x.data(), y.data(), 2, N, K, G,
                                           0, N, 1);
                        orc_dequant4_bf16(q.data(), s.data(), b.data(), out.data(), N, K, G);
                        orc_dequant4_f32(q.data(), s.data(), b.data(), f.data(), N, K, G);
                    } else {
                        orc_gemv8_f64(q.data(), s.data(), b.data(), x.data(), y.data(), 2, N, K, G, 1);
                        orc_gemv8_rows_f64(q.data(), s.data(), b.data(), x.data(), y.data(), 2, N, K, G,
                                           0, N, 1);
                        orc_dequant8_bf16(q.data(), s.data(), b.data(), out.data(), N, K, G);
                        orc_dequant8_f32(q.data(), s.data(), b.data(), f.data(), N, K, G);
                    }
                }
            }
        }
    }
    // GEMMs with row strides and a row subset
    const int64_t M = 5, N = 7, K = 40, lda = 48, ldb = 41, ldc = 9;
    std::vector<uint16_t> A(M * lda), B(N * ldb);
    for (auto& v : A) v = orc_f32_to_bf16((float)(rng() % 100) / 50.f - 1.f);
    for (auto& v : B) v = orc_f32_to_bf16((float)(rng() % 100) / 50.f - 1.f);
    std::vector<float> C(M * ldc, 0.f);
    orc_gemm_naive_f32(A.data(), B.data(), C.data(), M, N, K, lda, ldb, ldc);
    std::vector<uint16_t> Ad(M * K), Bd(N * K);
    for (int64_t i = 0; i < M * K; ++i) Ad[i] = A[i];
    for (int64_t i = 0; i < N * K; ++i) Bd[i] = B[i];
    const int64_t rows[2] = {4, 1};
    std::vector<double> Cd(2 * N);
    orc_gemm_bf16_f64(Ad.data(), Bd.data(), Cd.data(), M, N, K, rows, 2, 1);
    std::vector<float> xf(K), uf(K);
    std::vector<uint16_t> w(K), h(K);
    for (int64_t k = 0; k < K; ++k) {
        xf[k] = (float)k / K - 0.5f;
        uf[k] = 0.25f;
        w[k] = orc_f32_to_bf16(1.f);
    }
    orc_rmsnorm_bf16(xf.data(), w.data(), h.data(), K, 1e-5f);
    orc_silu_mul_bf16(xf.data(), uf.data(), h.data(), K);
}

}  // namespace

int main(int argc, char** argv) {
    const std::string dir = argc > 1 ? argv[1] : ".";
    parser_cases();
    loader_cases(dir);
    oracle_cases();
    printf("%s (%d failed)\n", g_fail ? "FAILED" : "ALL PASSED", g_fail);
    return g_fail ? 1 : 0;
}
