/*
 * TEST INFRASTRUCTURE ONLY -- see cpu_ref.h. Plain C restatement of the
 * reference dequant oracle (src/cpu_ref.h:9-45) and of the reference's
 * kernel-check loops (src/main.cpp:73-84 GEMV, src/main.cpp:594-601 GEMM).
 */
#include "cpu_ref.h"
#include <math.h>
#include <string.h>

float orc_bf16_to_f32(uint16_t v) {
    /* src/cpu_ref.h:9-14: the bf16 bits are the upper half of the fp32. */
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    /* src/cpu_ref.h:16-23: add 0x7FFF plus the kept LSB, truncate. */
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

void orc_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

float orc_dequant4_elem(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        int64_t n, int64_t k, int64_t K, int64_t G) {
    /* src/cpu_ref.h:25-34. Row n holds K/8 words (q.cols() == K/8). */
    const uint32_t* qrow = q + n * (K / 8);
    const uint32_t word = qrow[k / 8];
    const uint32_t qv = (word >> (4 * (k % 8))) & 0xFu;
    const int64_t g = k / G;
    const float sc = orc_bf16_to_f32(s[n * (K / G) + g]);
    const float bi = orc_bf16_to_f32(b[n * (K / G) + g]);
    return (float)qv * sc + bi;
}

float orc_dequant8_elem(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        int64_t n, int64_t k, int64_t K, int64_t G) {
    /* src/cpu_ref.h:36-45. Row n holds K/4 words. */
    const uint32_t* qrow = q + n * (K / 4);
    const uint32_t word = qrow[k / 4];
    const uint32_t qv = (word >> (8 * (k % 4))) & 0xFFu;
    const int64_t g = k / G;
    const float sc = orc_bf16_to_f32(s[n * (K / G) + g]);
    const float bi = orc_bf16_to_f32(b[n * (K / G) + g]);
    return (float)qv * sc + bi;
}

void orc_dequant4_f32(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                      float* out, int64_t N, int64_t K, int64_t G) {
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            out[n * K + k] = orc_dequant4_elem(q, s, b, n, k, K, G);
}

void orc_dequant8_f32(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                      float* out, int64_t N, int64_t K, int64_t G) {
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            out[n * K + k] = orc_dequant8_elem(q, s, b, n, k, K, G);
}

void orc_dequant4_bf16(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                       uint16_t* out, int64_t N, int64_t K, int64_t G) {
    /* shaders/ops.metal:142-166: out = bfloat(float(q)*sc + bi). */
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            out[n * K + k] = orc_f32_to_bf16(orc_dequant4_elem(q, s, b, n, k, K, G));
}

void orc_dequant8_bf16(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                       uint16_t* out, int64_t N, int64_t K, int64_t G) {
    /* shaders/ops.metal:754-779. */
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            out[n * K + k] = orc_f32_to_bf16(orc_dequant8_elem(q, s, b, n, k, K, G));
}

typedef float (*elem_fn)(const uint32_t*, const uint16_t*, const uint16_t*,
                         int64_t, int64_t, int64_t, int64_t);

static void gemv_rows(elem_fn fn, const uint32_t* q, const uint16_t* s,
                      const uint16_t* b, const uint16_t* x, double* y, int64_t M,
                      int64_t N, int64_t K, int64_t G, int64_t n0, int64_t n1,
                      int nthreads) {
    /* src/main.cpp:73-84: ref += (double)dequant_elem(n,k) * gx[k], with
     * gx[k] = bf16_to_float(x[k]). One sum per (activation row, output row). */
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads) if (nthreads > 1)
    for (int64_t n = n0; n < n1; ++n) {
        for (int64_t m = 0; m < M; ++m) {
            const uint16_t* xr = x + m * K;
            double ref = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                const float wv = fn(q, s, b, n, k, K, G);
                ref += (double)wv * (double)orc_bf16_to_f32(xr[k]);
            }
            y[m * N + n] = ref;
        }
    }
}

void orc_gemv4_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                   const uint16_t* x, double* y, int64_t M, int64_t N, int64_t K,
                   int64_t G, int nthreads) {
    gemv_rows(orc_dequant4_elem, q, s, b, x, y, M, N, K, G, 0, N, nthreads);
}

void orc_gemv8_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                   const uint16_t* x, double* y, int64_t M, int64_t N, int64_t K,
                   int64_t G, int nthreads) {
    gemv_rows(orc_dequant8_elem, q, s, b, x, y, M, N, K, G, 0, N, nthreads);
}

void orc_gemv4_rows_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        const uint16_t* x, double* y, int64_t M, int64_t N,
                        int64_t K, int64_t G, int64_t n0, int64_t n1, int nthreads) {
    gemv_rows(orc_dequant4_elem, q, s, b, x, y, M, N, K, G, n0, n1, nthreads);
}

void orc_gemv8_rows_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        const uint16_t* x, double* y, int64_t M, int64_t N,
                        int64_t K, int64_t G, int64_t n0, int64_t n1, int nthreads) {
    gemv_rows(orc_dequant8_elem, q, s, b, x, y, M, N, K, G, n0, n1, nthreads);
}

void orc_gemm_bf16_f64(const uint16_t* A, const uint16_t* B, double* C,
                       int64_t M, int64_t N, int64_t K, const int64_t* rows,
                       int64_t nrows, int nthreads) {
    /* src/main.cpp:594-601: ref += bf16_to_float(a[m][k]) * bf16_to_float(b[n][k]).
     * Products of two bf16 values are exact in fp64, so only the summation
     * order differs from any other correct evaluation. */
    (void)M;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads) if (nthreads > 1)
    for (int64_t r = 0; r < nrows; ++r) {
        const uint16_t* ar = A + rows[r] * K;
        for (int64_t n = 0; n < N; ++n) {
            const uint16_t* br = B + n * K;
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k)
                acc += (double)orc_bf16_to_f32(ar[k]) * (double)orc_bf16_to_f32(br[k]);
            C[r * N + n] = acc;
        }
    }
}

void orc_gemm_naive_f32(const uint16_t* A, const uint16_t* B, float* C, int64_t M, int64_t N,
                        int64_t K, int64_t lda, int64_t ldb, int64_t ldc) {
    /* shaders/ops.metal:199-251 (gemm_naive): each output is one fp32 FMA
     * chain acc = fma(A[m][k], B[n][k], acc) over k = 0..K-1 from +0, checked by
     * src/main.cpp:578-602. A product of two bf16 values is exact in fp32, so
     * the chain equals sequential multiply-then-add; the k order is the whole
     * definition. */
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            for (int64_t k = 0; k < K; ++k)
                acc = fmaf(orc_bf16_to_f32(A[m * lda + k]), orc_bf16_to_f32(B[n * ldb + k]), acc);
            C[m * ldc + n] = acc;
        }
}

void orc_rmsnorm_bf16(const float* x, const uint16_t* w, uint16_t* h, int64_t K, float eps) {
    /* shaders/ops.metal:86-114 (rmsnorm, one row): inv = rsqrt(sum(x^2)/n + eps),
     * y = bfloat(x * inv * float(w)). The sum runs in k order here; the GPU
     * sums in another fixed order, which moves inv by at most a few ulp. */
    float ss = 0.0f;
    for (int64_t k = 0; k < K; ++k) ss = fmaf(x[k], x[k], ss);
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
    for (int64_t k = 0; k < K; ++k) h[k] = orc_f32_to_bf16((x[k] * inv) * orc_bf16_to_f32(w[k]));
}

void orc_silu_mul_bf16(const float* g, const float* u, uint16_t* a, int64_t K) {
    /* shaders/ops.metal:129-139 (silu_mul): out = bfloat(g / (1 + exp(-g)) * up). */
    for (int64_t k = 0; k < K; ++k) a[k] = orc_f32_to_bf16((g[k] / (1.0f + expf(-g[k]))) * u[k]);
}
