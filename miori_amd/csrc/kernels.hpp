// Internal launchers behind the C ABI (no argument checking here; capi.cpp
// validates shapes, pointers and alignment before calling them).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace miori {

// y[M][N] = x[M][K] . dequant(W)^T on the VALU path (any M; M is split into
// launches of at most 4 activation rows).
hipError_t launch_gemv_valu(int bits, const void* q, const void* s, const void* b,
                            const void* x, void* y, uint32_t M, uint32_t N, uint32_t K,
                            uint32_t G, int out_bf16, hipStream_t st);
void gemv_split(int bits, uint32_t K, uint32_t* S, int* cpl);
// The 4-bit M = 1 GEMV (K <= 2048) with per-wave wall-clock stamps (4 per
// wave into stamps, at most cap values; *nwaves = waves launched).
hipError_t launch_gemv_q4_timeline(const void* q, const void* s, const void* b, const void* x,
                                   void* y, uint32_t N, uint32_t K, uint32_t G, int out_bf16,
                                   uint64_t* stamps, uint32_t cap, uint32_t* nwaves,
                                   hipStream_t st);
// Fused decode ops on the 4-bit GEMV (one activation row, K <= 8192):
// xm = 1: y = W . bf16(rmsnorm(x fp32) * w_norm bf16); xm = 2: y = W . bf16(silu(x) * x2)
hipError_t launch_gemv_fused(int xm, const void* q, const void* s, const void* b, const void* x,
                             const void* x2, float eps, void* y, uint32_t N, uint32_t K,
                             uint32_t G, int out_bf16, hipStream_t st);


// bf16 -> row-major bf16 dequant.
hipError_t launch_dequant(int bits, const void* q, const void* s, const void* b, void* out,
                          uint32_t N, uint32_t K, uint32_t G, hipStream_t st);

// C = A . B^T on MFMA, B bf16 row-major [N][K] (q == nullptr) or 4-bit
// (q/s/b given, B = bf16(dequant4)).
hipError_t launch_gemm(const void* A, const void* B, const void* q, const void* s,
                       const void* b, void* C, uint32_t M, uint32_t N, uint32_t K,
                       uint32_t G, int out_bf16, hipStream_t st);

// One-wave sampler of (shader clock, wall clock) pairs, `gap` wall-clock
// ticks apart, into out[2n].
hipError_t launch_clock_sampler(uint64_t* out, uint32_t n, uint32_t gap, hipStream_t st);

// C (fp32, row stride ldc) = A . B^T for any shape, bf16 operands with row
// strides lda / ldb; one sequential fp32 FMA chain over k per output.
hipError_t launch_gemm_naive(const void* A, const void* B, float* C, uint32_t M, uint32_t N,
                             uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc,
                             hipStream_t st);

// Skinny MFMA kernel (M <= 32), weight modes: 0 = 4-bit exact affine,
// 1 = 8-bit exact affine, 2 = 4-bit dequantised to bf16 (fused GEMM),
// 3 = bf16 weights.
bool skinny_supported(int mode, uint32_t M, uint32_t N, uint32_t K, uint32_t G);
hipError_t launch_skinny(int mode, const void* X, const void* W, const void* S, const void* B,
                         void* Y, uint32_t M, uint32_t N, uint32_t K, uint32_t G, int out_bf16,
                         hipStream_t st);

// Split-K partials workspace of the current device: grown outside graph
// capture only (st is the stream checked for capture), superseded buffers
// kept until the process ends.
hipError_t workspace_get(hipStream_t st, size_t bytes, float** part);

// A caller-provided fixed scratch buffer (device memory the library does not
// allocate). While a ScratchScope is alive on a host thread, every split-K
// launch that thread makes takes its partials from that buffer instead of
// the per-stream workspace, and fails with hipErrorOutOfMemory, before
// anything is enqueued, when the partials do not fit.
struct Scratch {
    float* ptr;
    size_t bytes;
};
class ScratchScope {
public:
    explicit ScratchScope(const Scratch* s) : prev_(current_) { current_ = s; }
    ~ScratchScope() { current_ = prev_; }
    ScratchScope(const ScratchScope&) = delete;
    ScratchScope& operator=(const ScratchScope&) = delete;
    static const Scratch* current() { return current_; }

private:
    const Scratch* prev_;
    static thread_local const Scratch* current_;
};
// Checked fused 4-bit GEMM behind miori_gemm_q4 (returns a MIORI_* status).
int gemm_q4_entry(const void* A, const void* q, const void* scales, const void* biases, void* C,
                  uint32_t M, uint32_t N, uint32_t K, uint32_t group, int out_dtype,
                  hipStream_t stream);
// Partials buffer for a split-K launch: the scoped fixed scratch if one is
// active on this thread, else workspace_get.
hipError_t scratch_get(hipStream_t st, size_t bytes, float** part);
// C[i] = sum over k = 0..SK-1 of part[k * MN + i], in that order, as fp32 or
// bf16 (MN a multiple of 8).
hipError_t launch_splitk_reduce(const float* part, void* C, size_t MN, uint32_t SK, int out_bf16,
                                hipStream_t st);

}  // namespace miori
