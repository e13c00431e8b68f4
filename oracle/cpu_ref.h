/*
 * TEST INFRASTRUCTURE ONLY -- never linked into libmiori_hip.so.
 *
 * CPU restatement of the reference's dequant oracle and of its kernel check
 * loops, used by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg as the checker. The product path never calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root). The reference header src/cpu_ref.h cannot be
 * compiled here: it includes weights.h -> <Metal/Metal.hpp> (Apple metal-cpp,
 * Objective-C runtime headers), so the formulas are restated in plain C with
 * the quantisation group size G made a parameter (the reference hard-codes 32,
 * config/m6.h:48).
 *
 * Pinning (what makes this oracle trustworthy without the reference binary)
 * lives in tests/test_oracle.py: RNE against torch's bf16 cast, one-hot and
 * brute-force code enumeration for the unpacking, the exactness invariant of
 * q*s (<= 12 significant bits) for the dequant, closed-form sums and a torch
 * fp64 matmul cross-check for the GEMV/GEMM values.
 */
#ifndef MIORI_ORACLE_CPU_REF_H
#define MIORI_ORACLE_CPU_REF_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/cpu_ref.h:9-14 */
float orc_bf16_to_f32(uint16_t v);
/* src/cpu_ref.h:16-23 (round to nearest even, no NaN special case) */
uint16_t orc_f32_to_bf16(float f);
void orc_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n);

/* src/cpu_ref.h:25-34 with group size G: nibble k of row n sits in word k/8,
 * bits 4*(k%8); value = float(q)*scale + bias, scale/bias at [n][k/G]. */
float orc_dequant4_elem(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        int64_t n, int64_t k, int64_t K, int64_t G);
/* src/cpu_ref.h:36-45 with group size G: code k in word k/4, bits 8*(k%4). */
float orc_dequant8_elem(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        int64_t n, int64_t k, int64_t K, int64_t G);

/* Whole-matrix dequant to fp32 [N][K] (element formula above). */
void orc_dequant4_f32(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                      float* out, int64_t N, int64_t K, int64_t G);
void orc_dequant8_f32(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                      float* out, int64_t N, int64_t K, int64_t G);
/* Dequant to bf16 [N][K] row-major: bfloat(q*s+b) with RNE, as
 * shaders/ops.metal:142-166 (dequant4) and :754-779 (dequant8). */
void orc_dequant4_bf16(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                       uint16_t* out, int64_t N, int64_t K, int64_t G);
void orc_dequant8_bf16(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                       uint16_t* out, int64_t N, int64_t K, int64_t G);

/* Reference GEMV check, src/main.cpp:73-84: for every activation row m and
 * output row n, y[m][n] = sum_k (double)dequant_elem(n,k) * (float)x[m][k]
 * accumulated in fp64. x is bf16 [M][K]; y is fp64 [M][N].
 * nthreads <= 1 runs the faithful single-thread loop; > 1 splits output rows
 * over OpenMP threads (same per-row arithmetic, same result). */
void orc_gemv4_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                   const uint16_t* x, double* y, int64_t M, int64_t N, int64_t K,
                   int64_t G, int nthreads);
void orc_gemv8_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                   const uint16_t* x, double* y, int64_t M, int64_t N, int64_t K,
                   int64_t G, int nthreads);
/* Same sums restricted to output rows [n0, n1) (bounded CPU-baseline sample). */
void orc_gemv4_rows_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        const uint16_t* x, double* y, int64_t M, int64_t N,
                        int64_t K, int64_t G, int64_t n0, int64_t n1, int nthreads);
void orc_gemv8_rows_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        const uint16_t* x, double* y, int64_t M, int64_t N,
                        int64_t K, int64_t G, int64_t n0, int64_t n1, int nthreads);

/* GEMM check, src/main.cpp:594-601 (there fp32 accumulate; here fp64):
 * C[r][n] = sum_k (double)bf16(A[rows[r]][k]) * bf16(B[n][k]), B row-major
 * [N][K] bf16, for the nrows selected activation rows. C is fp64 [nrows][N]. */
void orc_gemm_bf16_f64(const uint16_t* A, const uint16_t* B, double* C,
                       int64_t M, int64_t N, int64_t K, const int64_t* rows,
                       int64_t nrows, int nthreads);

/* shaders/ops.metal:199-251 (gemm_naive), check src/main.cpp:578-602:
 * C[m*ldc+n] = fp32 FMA chain over k = 0..K-1 of A[m*lda+k] * B[n*ldb+k]. */
void orc_gemm_naive_f32(const uint16_t* A, const uint16_t* B, float* C, int64_t M, int64_t N,
                        int64_t K, int64_t lda, int64_t ldb, int64_t ldc);

/* shaders/ops.metal:86-114: h = bf16(x * rsqrt(sum(x^2)/K + eps) * w), one row. */
void orc_rmsnorm_bf16(const float* x, const uint16_t* w, uint16_t* h, int64_t K, float eps);
/* shaders/ops.metal:129-139: a = bf16(g / (1 + exp(-g)) * u). */
void orc_silu_mul_bf16(const float* g, const float* u, uint16_t* a, int64_t K);

#ifdef __cplusplus
}
#endif
#endif
