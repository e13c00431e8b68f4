// C ABI of libmiori_hip.so (declared in include/miori_hip.h): argument
// checking, then the internal launchers. Nothing is enqueued when a check
// fails. The reference kernels (shaders/*.metal) have no error path and skip
// unsupported shapes silently; this layer reports them instead, and the C++
// shim above it turns a non-zero status into std::runtime_error, the error
// convention of the reference's Metal::pso (src/metal.cpp:31-37).
#include "../../include/miori_hip.h"
#include "common.hpp"
#include "kernels.hpp"

#include <hip/hip_runtime.h>

using namespace miori;

namespace {

constexpr uint64_t kMaxBytes = 0xFFFFFFF0ull;
// Clock sampler bounds: at most 2^20 samples and 2 s of wall clock (the tick
// limit follows from the device's wall-clock rate).
constexpr uint32_t kClockMaxSamples = 1u << 20;
constexpr uint64_t kClockMaxMs = 2000;
// miori_linear_q4 takes the exact 4-bit batched GEMV up to this many rows.
constexpr uint32_t kLinearExactMaxM = 32;

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

inline int hip_status(hipError_t e) { return e == hipSuccess ? MIORI_OK : MIORI_E_HIP; }

int check_gemv(int bits, const void* q, const void* s, const void* b, const void* x,
               const void* y, uint32_t M, uint32_t N, uint32_t K, uint32_t G, int out_dtype) {
    if (!q || !s || !b || !x || !y) return MIORI_E_NULL;
    if (out_dtype != MIORI_F32 && out_dtype != MIORI_BF16) return MIORI_E_DTYPE;
    const uint32_t E = bits == 4 ? 32u : 16u;         // elements per 16-byte chunk
    const uint32_t kmax = bits == 4 ? 32768u : 16384u; // 4 waves x 64 lanes x 4 chunks
    if (M == 0 || N == 0 || K == 0 || K % E != 0 || K > kmax) return MIORI_E_SHAPE;
    if (!(G == 16 || G == 32 || G == 64 || G == 128) || G < E || K % G != 0) return MIORI_E_SHAPE;
    // Kernels address each operand with 32-bit byte offsets.
    if ((uint64_t)N * K * bits / 8 > kMaxBytes || (uint64_t)M * K * 2 > kMaxBytes ||
        (uint64_t)M * N * 4 > kMaxBytes)
        return MIORI_E_SHAPE;
    if (!aligned(q, 16) || !aligned(x, 16) || !aligned(s, 2) || !aligned(b, 2) ||
        !aligned(y, out_dtype == MIORI_F32 ? 4 : 2))
        return MIORI_E_ALIGN;
    return MIORI_OK;
}

// The skinny kernel DMAs each workgroup's scale / bias rows as 16-byte chunks.
bool skinny_ok(int mode, uint32_t M, uint32_t N, uint32_t K, uint32_t G, const void* s,
               const void* b) {
    return skinny_supported(mode, M, N, K, G) && aligned(s, 16) && aligned(b, 16);
}

// Batched GEMV: the VALU kernel up to 4 rows (bit-identical to the single-row
// product, as the reference's gemv4_b is), the MFMA kernel beyond.
hipError_t launch_batched(int bits, const void* q, const void* s, const void* b,
                          const void* x, void* y, uint32_t M, uint32_t N, uint32_t K,
                          uint32_t G, int out_bf16, hipStream_t st) {
    const int mode = bits == 4 ? 0 : 1;
    // MIORI_BATCH_MFMA_MIN_M overrides the first M served by the MFMA kernel
    // (tuning sweeps; default 5)
    static const uint32_t min_m = (uint32_t)tuning_env("MIORI_BATCH_MFMA_MIN_M", 5);
    if (M >= min_m && skinny_ok(mode, M, N, K, G, s, b))
        return launch_skinny(mode, x, q, s, b, y, M, N, K, G, out_bf16, st);
    return launch_gemv_valu(bits, q, s, b, x, y, M, N, K, G, out_bf16, st);
}

int check_gemm(const void* A, const void* C, uint32_t M, uint32_t N, uint32_t K,
               int out_dtype) {
    if (!A || !C) return MIORI_E_NULL;
    if (out_dtype != MIORI_F32 && out_dtype != MIORI_BF16) return MIORI_E_DTYPE;
    if (M == 0 || N == 0 || K == 0 || K % 64 != 0 || N % 16 != 0) return MIORI_E_SHAPE;
    // The GEMM addresses A and B rows with 32-bit byte offsets.
    if ((uint64_t)M * K * 2 > kMaxBytes || (uint64_t)N * K * 2 > kMaxBytes) return MIORI_E_SHAPE;
    if (!aligned(A, 16) || !aligned(C, 16)) return MIORI_E_ALIGN;
    return MIORI_OK;
}

}  // namespace

extern "C" {

int miori_abi_version(void) { return MIORI_HIP_ABI_VERSION; }

const char* miori_status_string(int status) {
    switch (status) {
        case MIORI_OK: return "ok";
        case MIORI_E_NULL: return "null pointer argument";
        case MIORI_E_SHAPE: return "unsupported shape (M/N/K/group)";
        case MIORI_E_ALIGN: return "misaligned pointer";
        case MIORI_E_DTYPE: return "unknown output dtype";
        case MIORI_E_HIP: return "HIP runtime error";
        case MIORI_E_SCRATCH: return "split-K partials exceed the fixed scratch buffer";
    }
    return "unknown status";
}

int miori_sync(miori_stream stream) {
    return hip_status(hipStreamSynchronize((hipStream_t)stream));
}

int miori_gemv_q4(const void* q, const void* scales, const void* biases, const void* x,
                  void* y, uint32_t N, uint32_t K, uint32_t group, int out_dtype,
                  miori_stream stream) {
    int st = check_gemv(4, q, scales, biases, x, y, 1, N, K, group, out_dtype);
    if (st) return st;
    return hip_status(launch_gemv_valu(4, q, scales, biases, x, y, 1, N, K, group,
                                       out_dtype == MIORI_BF16, (hipStream_t)stream));
}

int miori_rmsnorm_gemv_q4(const float* x, const void* norm_weight, float eps, const void* q,
                          const void* scales, const void* biases, void* y, uint32_t N,
                          uint32_t K, uint32_t group, int out_dtype, miori_stream stream) {
    int st = check_gemv(4, q, scales, biases, x, y, 1, N, K, group, out_dtype);
    if (st) return st;
    if (!norm_weight) return MIORI_E_NULL;
    if (K > 8192 || !(eps >= 0.f)) return MIORI_E_SHAPE;
    if (!aligned(norm_weight, 16)) return MIORI_E_ALIGN;
    return hip_status(launch_gemv_fused(1, q, scales, biases, x, norm_weight, eps, y, N, K, group,
                                        out_dtype == MIORI_BF16, (hipStream_t)stream));
}

int miori_silu_mul_gemv_q4(const float* gate, const float* up, const void* q,
                           const void* scales, const void* biases, void* y, uint32_t N,
                           uint32_t K, uint32_t group, int out_dtype, miori_stream stream) {
    int st = check_gemv(4, q, scales, biases, gate, y, 1, N, K, group, out_dtype);
    if (st) return st;
    if (!up) return MIORI_E_NULL;
    if (K > 8192) return MIORI_E_SHAPE;
    if (!aligned(up, 16)) return MIORI_E_ALIGN;
    return hip_status(launch_gemv_fused(2, q, scales, biases, gate, up, 0.f, y, N, K, group,
                                        out_dtype == MIORI_BF16, (hipStream_t)stream));
}

int miori_gemv_q8(const void* q, const void* scales, const void* biases, const void* x,
                  void* y, uint32_t N, uint32_t K, uint32_t group, int out_dtype,
                  miori_stream stream) {
    int st = check_gemv(8, q, scales, biases, x, y, 1, N, K, group, out_dtype);
    if (st) return st;
    return hip_status(launch_gemv_valu(8, q, scales, biases, x, y, 1, N, K, group,
                                       out_dtype == MIORI_BF16, (hipStream_t)stream));
}

int miori_gemv_q4_batched(const void* q, const void* scales, const void* biases,
                          const void* x, void* y, uint32_t M, uint32_t N, uint32_t K,
                          uint32_t group, int out_dtype, miori_stream stream) {
    int st = check_gemv(4, q, scales, biases, x, y, M, N, K, group, out_dtype);
    if (st) return st;
    if (M > 32) return MIORI_E_SHAPE;
    return hip_status(launch_batched(4, q, scales, biases, x, y, M, N, K, group,
                                       out_dtype == MIORI_BF16, (hipStream_t)stream));
}

int miori_gemv_q8_batched(const void* q, const void* scales, const void* biases,
                          const void* x, void* y, uint32_t M, uint32_t N, uint32_t K,
                          uint32_t group, int out_dtype, miori_stream stream) {
    int st = check_gemv(8, q, scales, biases, x, y, M, N, K, group, out_dtype);
    if (st) return st;
    if (M > 32) return MIORI_E_SHAPE;
    return hip_status(launch_batched(8, q, scales, biases, x, y, M, N, K, group,
                                       out_dtype == MIORI_BF16, (hipStream_t)stream));
}

int miori_gemm_bf16(const void* A, const void* B, void* C, uint32_t M, uint32_t N,
                    uint32_t K, int out_dtype, miori_stream stream) {
    int st = check_gemm(A, C, M, N, K, out_dtype);
    if (st) return st;
    if (!B) return MIORI_E_NULL;
    if (!aligned(B, 16)) return MIORI_E_ALIGN;
    if (M <= 32 && skinny_supported(3, M, N, K, 64))
        return hip_status(launch_skinny(3, A, B, nullptr, nullptr, C, M, N, K, 64,
                                        out_dtype == MIORI_BF16, (hipStream_t)stream));
    return hip_status(launch_gemm(A, B, nullptr, nullptr, nullptr, C, M, N, K, 0,
                                  out_dtype == MIORI_BF16, (hipStream_t)stream));
}

}  // extern "C"

// miori_gemm_q4 with the stream already cast; under a ScratchScope a split
// whose partials do not fit the fixed buffer returns MIORI_E_SCRATCH.
int miori::gemm_q4_entry(const void* A, const void* q, const void* scales, const void* biases,
                         void* C, uint32_t M, uint32_t N, uint32_t K, uint32_t group,
                         int out_dtype, hipStream_t stream) {
    int st = check_gemm(A, C, M, N, K, out_dtype);
    if (st) return st;
    if (!q || !scales || !biases) return MIORI_E_NULL;
    if (!(group == 32 || group == 64 || group == 128) || K % group != 0) return MIORI_E_SHAPE;
    if (!aligned(q, 16) || !aligned(scales, 2) || !aligned(biases, 2)) return MIORI_E_ALIGN;
    hipError_t e;
    // Small M runs on the skinny kernel, with the bf16 GEMM's routing (so the
    // fused product stays bit-identical to dequant + bf16 GEMM; that needs
    // K / group to be a multiple of 8 and 16-byte aligned scales / biases).
    if (M <= 32 && skinny_ok(2, M, N, K, group, scales, biases) && skinny_supported(3, M, N, K, 64))
        e = launch_skinny(2, A, q, scales, biases, C, M, N, K, group, out_dtype == MIORI_BF16,
                          stream);
    else
        e = launch_gemm(A, nullptr, q, scales, biases, C, M, N, K, group,
                        out_dtype == MIORI_BF16, stream);
    if (e == hipErrorOutOfMemory && ScratchScope::current()) return MIORI_E_SCRATCH;
    return hip_status(e);
}

extern "C" {

int miori_gemm_q4(const void* A, const void* q, const void* scales, const void* biases,
                  void* C, uint32_t M, uint32_t N, uint32_t K, uint32_t group,
                  int out_dtype, miori_stream stream) {
    return gemm_q4_entry(A, q, scales, biases, C, M, N, K, group, out_dtype, (hipStream_t)stream);
}

int miori_linear_q4(const void* A, const void* q, const void* scales, const void* biases,
                    const void* bf16_cache, void* C, uint32_t M, uint32_t N, uint32_t K,
                    uint32_t group, int out_dtype, miori_stream stream) {
    if (M <= kLinearExactMaxM)
        return miori_gemv_q4_batched(q, scales, biases, A, C, M, N, K, group, out_dtype, stream);
    if (bf16_cache) return miori_gemm_bf16(A, bf16_cache, C, M, N, K, out_dtype, stream);
    return miori_gemm_q4(A, q, scales, biases, C, M, N, K, group, out_dtype, stream);
}

int miori_gemm_naive(const void* A, const void* B, float* C, uint32_t M, uint32_t N,
                     uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc, miori_stream stream) {
    if (!A || !B || !C) return MIORI_E_NULL;
    if (M == 0 || N == 0 || K == 0 || lda < K || ldb < K || ldc < N) return MIORI_E_SHAPE;
    if (!aligned(A, 2) || !aligned(B, 2) || !aligned(C, 4)) return MIORI_E_ALIGN;
    return hip_status(launch_gemm_naive(A, B, C, M, N, K, lda, ldb, ldc, (hipStream_t)stream));
}

static int dequant_common(int bits, const void* q, const void* s, const void* b, void* out,
                          uint32_t N, uint32_t K, uint32_t G, hipStream_t st) {
    if (!q || !s || !b || !out) return MIORI_E_NULL;
    const uint32_t E = bits == 4 ? 32u : 16u;
    if (N == 0 || K == 0 || K % E != 0) return MIORI_E_SHAPE;
    if (!(G == 16 || G == 32 || G == 64 || G == 128) || G < E || K % G != 0) return MIORI_E_SHAPE;
    if (!aligned(q, 16) || !aligned(out, 16) || !aligned(s, 2) || !aligned(b, 2))
        return MIORI_E_ALIGN;
    return hip_status(launch_dequant(bits, q, s, b, out, N, K, G, st));
}

int miori_dequant_q4_tile(const void* q, const void* scales, const void* biases, void* out,
                          uint32_t N, uint32_t K, uint32_t group, miori_stream stream) {
    return dequant_common(4, q, scales, biases, out, N, K, group, (hipStream_t)stream);
}

int miori_dequant_q4(const void* q, const void* scales, const void* biases, void* out,
                     uint32_t N, uint32_t K, uint32_t group, miori_stream stream) {
    return dequant_common(4, q, scales, biases, out, N, K, group, (hipStream_t)stream);
}

int miori_dequant_q8(const void* q, const void* scales, const void* biases, void* out,
                     uint32_t N, uint32_t K, uint32_t group, miori_stream stream) {
    return dequant_common(8, q, scales, biases, out, N, K, group, (hipStream_t)stream);
}

int miori_diag_clock_sample(uint64_t* samples, uint32_t n, uint32_t gap_ticks,
                            uint32_t* wall_khz, miori_stream stream) {
    if (!samples || !wall_khz) return MIORI_E_NULL;
    if (n == 0 || gap_ticks == 0 || n > kClockMaxSamples) return MIORI_E_SHAPE;
    if (!aligned(samples, 8)) return MIORI_E_ALIGN;
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
        return MIORI_E_HIP;
    // ticks in 2 s at this device's wall-clock rate (kHz = ticks per ms)
    if ((uint64_t)n * gap_ticks > kClockMaxMs * (uint64_t)khz) return MIORI_E_SHAPE;
    *wall_khz = (uint32_t)khz;
    return hip_status(launch_clock_sampler(samples, n, gap_ticks, (hipStream_t)stream));
}

int miori_diag_gemv_q4_timeline(const void* q, const void* scales, const void* biases,
                                const void* x, void* y, uint32_t N, uint32_t K, uint32_t group,
                                int out_dtype, uint64_t* stamps, uint32_t cap,
                                uint32_t* nwaves, miori_stream stream) {
    int st = check_gemv(4, q, scales, biases, x, y, 1, N, K, group, out_dtype);
    if (st) return st;
    if (!stamps || !nwaves) return MIORI_E_NULL;
    if (K > 2048) return MIORI_E_SHAPE;
    if (!aligned(stamps, 8)) return MIORI_E_ALIGN;
    const uint64_t need = ((uint64_t)N + 15u) / 16u * 16u;
    *nwaves = (uint32_t)(need / 4u);
    if (cap < need) return MIORI_E_SHAPE;
    return hip_status(launch_gemv_q4_timeline(q, scales, biases, x, y, N, K, group,
                                              out_dtype == MIORI_BF16, stamps, cap, nwaves,
                                              (hipStream_t)stream));
}

}  // extern "C"
