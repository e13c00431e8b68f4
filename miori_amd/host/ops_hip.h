// The quantized-matmul entry points of the reference's src/ops.h, with the
// same signatures, implemented over libmiori_hip.so (include/miori_hip.h).
// A C++ host written against src/ops.h (src/engine.cpp, src/batch.cpp) calls
// these unchanged once it includes this header and links libmiori_host.so.
//
// Semantics follow the reference wrappers (src/ops.cpp): they enqueue work
// on the encoder's stream and return; outputs are fp32 (`device float* y`);
// a failed call throws std::runtime_error. Differences, all widenings:
//  * the quantisation group size is read from the scale tensor's shape
//    (group = K / scales.cols()); the raw-buffer entries, which carry no
//    shapes, take it from Metal::raw_group (32 by default, the reference's
//    kGroup, config/m6.h:48) or from an explicit `group` argument;
//  * gemv4_b / gemv8_b / gemv8_b_off take any 1 <= B <= 32 and write B rows
//    (the reference returns early for B > 4 and always writes 4 rows,
//    shaders/batch.metal:156, :203);
//  * gemm_mpp's B operand is the bf16 cache written by this dequant_tile,
//    row-major [N][K] (the reference's MPP layout is [N/64][K][64]); N need
//    only be a multiple of 16 (the reference needs 64).
#pragma once
#include "metal_hip.h"
#include "weights_hip.h"

#include <cstdint>

namespace miori {

// src/ops.h:8-10
void gemv4(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
           const Tensor& q, const Tensor& s, const Tensor& b,
           MTL::Buffer* x, MTL::Buffer* y, uint32_t N, uint32_t K);
// src/ops.h:12-14
void gemv8(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
           const Tensor& q, const Tensor& s, const Tensor& b,
           MTL::Buffer* x, MTL::Buffer* y, uint32_t N, uint32_t K);
// src/ops.h:26-28
void dequant4(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
              const Tensor& q, const Tensor& s, const Tensor& b,
              MTL::Buffer* out, uint32_t N, uint32_t K, uint32_t boff = 0);
// src/ops.h:90-92
void dequant_tile(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
                  const Tensor& q, const Tensor& s, const Tensor& b,
                  MTL::Buffer* out, uint32_t N, uint32_t K, uint32_t boff = 0);
// Fused decode steps (no single reference function: the reference runs
// rmsnorm then gemv4, and silu_mul then gemv4, src/engine.cpp:388-400).
// norm_w is the bf16 norm weight tensor; x, gate and up are fp32 [K].
void rmsnorm_gemv4(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
                   const Tensor& q, const Tensor& s, const Tensor& b, MTL::Buffer* x,
                   const Tensor& norm_w, MTL::Buffer* y, uint32_t N, uint32_t K,
                   float eps = 1e-5f);
void silu_mul_gemv4(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
                    const Tensor& q, const Tensor& s, const Tensor& b, MTL::Buffer* gate,
                    MTL::Buffer* up, MTL::Buffer* y, uint32_t N, uint32_t K);
// src/ops.h:30-32 (fallback GEMM for any shape; fp32 C, strided operands)
void gemm_naive(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* A,
                MTL::Buffer* B, MTL::Buffer* C, uint32_t M, uint32_t N, uint32_t K,
                uint32_t lda, uint32_t ldb, uint32_t ldc,
                uint32_t aoff = 0, uint32_t boff = 0, uint32_t coff = 0);
// src/ops.h:94-96
void gemm_mpp(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* A,
              MTL::Buffer* B, MTL::Buffer* C, uint32_t M, uint32_t N, uint32_t K,
              uint32_t boff = 0);
// src/ops.h:101-103
void gemm_mpp_off(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* A,
                  MTL::Buffer* B, MTL::Buffer* C, uint32_t M, uint32_t N, uint32_t K,
                  uint32_t aoff, uint32_t boff, uint32_t coff);
// src/ops.h:105-107
void gemv4x4(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
             const Tensor& q, const Tensor& s, const Tensor& b,
             MTL::Buffer* x, MTL::Buffer* y, uint32_t N, uint32_t K);
// src/ops.h:113-115
void gemv4_raw(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* q,
               MTL::Buffer* s, MTL::Buffer* b, MTL::Buffer* x, MTL::Buffer* y,
               uint32_t N, uint32_t K);
// gemv4_raw with an explicit group size (no reference counterpart).
void gemv4_raw(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* q,
               MTL::Buffer* s, MTL::Buffer* b, MTL::Buffer* x, MTL::Buffer* y,
               uint32_t N, uint32_t K, uint32_t group);
// src/ops.h:126-128
void gemv4x2(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
             const Tensor& q, const Tensor& s, const Tensor& b,
             MTL::Buffer* x, MTL::Buffer* y, uint32_t N, uint32_t K);
// src/ops.h:135-138
void gemv8_off(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* wbuf,
               uint32_t qoff, uint32_t soff, uint32_t boff, MTL::Buffer* x,
               MTL::Buffer* y, uint32_t N, uint32_t K, uint32_t xoff,
               uint32_t yoff);
// gemv8_off with an explicit group size (no reference counterpart).
void gemv8_off(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* wbuf,
               uint32_t qoff, uint32_t soff, uint32_t boff, MTL::Buffer* x,
               MTL::Buffer* y, uint32_t N, uint32_t K, uint32_t xoff,
               uint32_t yoff, uint32_t group);
// src/ops.h:164-166
void gemv4_b(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
             const Tensor& q, const Tensor& s, const Tensor& b, MTL::Buffer* x,
             MTL::Buffer* y, uint32_t N, uint32_t K, uint32_t B);
// src/ops.h:168-171
void gemv8_b(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
             const Tensor& q, const Tensor& s, const Tensor& b, MTL::Buffer* x,
             MTL::Buffer* y, uint32_t N, uint32_t K, uint32_t B);
// src/ops.h:176-179
void gemv8_b_off(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
                 const Tensor& q, const Tensor& s, const Tensor& b, MTL::Buffer* x,
                 MTL::Buffer* y, uint32_t N, uint32_t K, uint32_t B, uint32_t xoff,
                 uint32_t yoff);
// src/ops.h:203-205
void dequant8(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w,
              const Tensor& q, const Tensor& s, const Tensor& b,
              MTL::Buffer* out, uint32_t N, uint32_t K);
// src/ops.h:207-209
void gemm_mpp32(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* A,
                MTL::Buffer* B, MTL::Buffer* C, uint32_t M, uint32_t N, uint32_t K,
                uint32_t boff = 0);

// BatchEngine::linear (src/batch.cpp:223-230) as a free function: C[B][N] =
// A[B][K] . W^T, the exact 4-bit batched GEMV for B <= 32, else the bf16
// cache GEMM when `bf16_cache` is given (the cache tensor starts at byte
// `cache_off`, row-major [N][K]), else the fused 4-bit GEMM.
void linear(Metal& m, MTL::ComputeCommandEncoder* e, const Weights& w, const Tensor& q,
            const Tensor& s, const Tensor& b, MTL::Buffer* A, MTL::Buffer* C, uint32_t N,
            uint32_t K, uint32_t B, MTL::Buffer* bf16_cache = nullptr, uint32_t cache_off = 0);

// No reference counterpart: the fused 4-bit GEMM (the weights dequantised
// inside the GEMM, never written as bf16), replacing the reference's dequant_tile + gemm_mpp
// pair (src/engine.cpp:144-146, 508-518) without the bf16 cache.
void gemm_q4(Metal& m, MTL::ComputeCommandEncoder* e, MTL::Buffer* A, const Weights& w,
             const Tensor& q, const Tensor& s, const Tensor& b, MTL::Buffer* C,
             uint32_t M, uint32_t N, uint32_t K);

}  // namespace miori
