/*
 * miori_hip.h -- C ABI of libmiori_hip.so, the MI355X (gfx950) implementation
 * of Miori's quantized-matmul hot path.
 *
 * This ABI replaces, for this path, the reference's Metal device runtime
 * (src/metal.cpp) and the Metal kernels shaders/ops.metal (gemv4, gemv8,
 * dequant4, dequant8), shaders/batch.metal (gemv4_b, gemv8_b) and
 * shaders/gemm_mpp.metal (dequant_tile, gemm_mpp, gemm_mpp32). The C++ shim in
 * miori_amd/host/ keeps the reference's src/ops.h signatures on top of it.
 *
 * Conventions (all entry points):
 *  - Plain device pointers. The caller owns every buffer. Where the reference
 *    binds (buffer, byte offset) pairs, the caller passes base + offset.
 *  - Non-blocking: work is enqueued on `stream` (a hipStream_t; NULL = the
 *    legacy default stream). miori_sync() waits, like the reference's
 *    Metal::submit(cb, wait=true) (src/metal.cpp:56-59).
 *  - Return 0 on success, a negative MIORI_E_* code otherwise; nothing is
 *    enqueued when a check fails. The reference kernels have no error path
 *    (unsupported shapes are silently skipped, shaders/batch.metal:156);
 *    here they are rejected.
 *  - Calls on one stream are ordered. The split-K GEMMs and the batched
 *    GEMV at M > 8 with K >= 8192 keep fp32 partials in one workspace per
 *    device: such calls that overlap on different streams of one device
 *    race, so a caller that uses several streams per device must order them
 *    (events) or serialise the calls. Every other entry point only touches
 *    its arguments and may overlap freely. The workspace grows (hipMalloc) on
 *    the first split-K call that needs more than it holds, which is refused
 *    while the stream is being captured into a graph (MIORI_E_HIP): run each
 *    shape once eagerly before capturing it. Superseded workspaces are never
 *    freed, so a captured graph stays valid for the life of the process.
 *    The reference drives one encoder per engine from one host thread
 *    (src/engine.h:176-177).
 *
 * Weight format (MLX affine, src/cpu_ref.h:25-45): W[N][K] quantized in
 * groups of `group` consecutive elements along K.
 *  - 4-bit: q uint32 [N][K/8], nibble k of a row at word k/8, bits 4*(k%8).
 *  - 8-bit: q uint32 [N][K/4], code k at word k/4, bits 8*(k%4).
 *  - scales, biases: bf16 [N][K/group]; w = float(code)*scale + bias.
 * Activations are bf16 [M][K] row-major; outputs are [M][N] row-major in
 * fp32 (out_dtype MIORI_F32, the reference's `device float* y`) or bf16
 * (MIORI_BF16, round-to-nearest-even as src/cpu_ref.h:16-23).
 */
#ifndef MIORI_HIP_H
#define MIORI_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIORI_HIP_ABI_VERSION 2

/* status codes */
#define MIORI_OK 0
#define MIORI_E_NULL (-1)      /* a required pointer is NULL */
#define MIORI_E_SHAPE (-2)     /* unsupported M/N/K/group combination */
#define MIORI_E_ALIGN (-3)     /* pointer misaligned for the kernel's loads */
#define MIORI_E_DTYPE (-4)     /* unknown out_dtype */
#define MIORI_E_HIP (-5)       /* a HIP runtime call failed */
#define MIORI_E_SCRATCH (-6)   /* split-K partials exceed a fixed scratch buffer */

/* output element types */
#define MIORI_F32 0
#define MIORI_BF16 1

typedef void* miori_stream; /* hipStream_t */

/* Library version (MIORI_HIP_ABI_VERSION). */
int miori_abi_version(void);
/* Human-readable text for a status code (static storage). */
const char* miori_status_string(int status);
/* Wait for all work enqueued on `stream`
 * (replaces Metal::submit(cb, wait=true), src/metal.cpp:56-59). */
int miori_sync(miori_stream stream);

/* ---- decode GEMVs -------------------------------------------------------
 * 4-bit GEMV, y[1][N] = x[1][K] . dequant4(W)^T, fp32 accumulation.
 * Replaces gemv4 / gemv4_raw / gemv4x4 / gemv4x2
 * (src/ops.h:8-10, 113-115, 105-107, 126-128; kernels shaders/ops.metal:6-42,
 * :563-602, :711-751).
 * Requires K % 32 == 0, group in {32, 64, 128}, K % group == 0,
 * K <= 32768, q and x 16-byte aligned. */
int miori_gemv_q4(const void* q, const void* scales, const void* biases,
                  const void* x, void* y, uint32_t N, uint32_t K, uint32_t group,
                  int out_dtype, miori_stream stream);

/* 8-bit GEMV (tied embedding / lm_head). Replaces gemv8 / gemv8_off
 * (src/ops.h:12-14, 135-138; kernel shaders/ops.metal:46-82).
 * Requires K % 16 == 0, group in {16, 32, 64, 128}, K % group == 0,
 * K <= 16384, q and x 16-byte aligned. */
int miori_gemv_q8(const void* q, const void* scales, const void* biases,
                  const void* x, void* y, uint32_t N, uint32_t K, uint32_t group,
                  int out_dtype, miori_stream stream);

/* Batched 4-bit GEMV over M activation rows, y[M][N] = x[M][K] . W^T, with
 * one pass over the weights for all rows. Replaces gemv4_b
 * (src/ops.h:164-166; kernel shaders/batch.metal:145-188), which is limited
 * to M <= 4; here 1 <= M <= 32 (larger M belongs to the GEMMs below).
 * Same K/group/alignment rules as miori_gemv_q4. */
int miori_gemv_q4_batched(const void* q, const void* scales, const void* biases,
                          const void* x, void* y, uint32_t M, uint32_t N,
                          uint32_t K, uint32_t group, int out_dtype,
                          miori_stream stream);

/* Batched 8-bit GEMV (batched lm_head). Replaces gemv8_b / gemv8_b_off
 * (src/ops.h:168-179; kernel shaders/batch.metal:192-236). 1 <= M <= 32.
 * Same K/group/alignment rules as miori_gemv_q8. */
int miori_gemv_q8_batched(const void* q, const void* scales, const void* biases,
                          const void* x, void* y, uint32_t M, uint32_t N,
                          uint32_t K, uint32_t group, int out_dtype,
                          miori_stream stream);

/* ---- fused decode ops ----------------------------------------------------
 * The decode layer steps around the GEMVs, fused into the 4-bit GEMV so the
 * bf16 activation never makes an HBM round trip (src/engine.cpp:388-400:
 * rmsnorm -> gemv4 w1/w3, silu_mul -> gemv4 w2). One activation row.
 *
 * miori_rmsnorm_gemv_q4: y = W . h with h = bf16(x * rsqrt(sum(x^2)/K + eps) * w),
 * x fp32 [K], w the bf16 norm weight [K] (rmsnorm, shaders/ops.metal:86-114).
 * miori_silu_mul_gemv_q4: y = W . a with a = bf16(g / (1 + exp(-g)) * u), g and
 * u fp32 [K] (silu_mul, shaders/ops.metal:129-139).
 * Same shape/group/alignment rules as miori_gemv_q4, plus K <= 8192 and the
 * fp32 / bf16 input vectors 16-byte aligned. */
int miori_rmsnorm_gemv_q4(const float* x, const void* norm_weight, float eps, const void* q,
                          const void* scales, const void* biases, void* y, uint32_t N,
                          uint32_t K, uint32_t group, int out_dtype, miori_stream stream);
int miori_silu_mul_gemv_q4(const float* gate, const float* up, const void* q,
                           const void* scales, const void* biases, void* y, uint32_t N,
                           uint32_t K, uint32_t group, int out_dtype, miori_stream stream);

/* ---- prefill GEMMs ------------------------------------------------------
 * C[M][N] = A[M][K] . B[N][K]^T, bf16 operands, fp32 accumulation on MFMA.
 * B is the bf16 weight cache in this library's layout, which is plain
 * row-major [N][K] (K contiguous, the operand order MFMA wants); it is what
 * miori_dequant_q4_tile writes. Replaces gemm_mpp / gemm_mpp_off / gemm_mpp32
 * (src/ops.h:94-103, 207-209; kernels shaders/gemm_mpp.metal:36-73), whose B
 * is the Apple-MPP tile-major [N/64][K][64] layout.
 * Requires K % 64 == 0, N % 16 == 0, A, B and C 16-byte aligned. */
int miori_gemm_bf16(const void* A, const void* B, void* C, uint32_t M,
                    uint32_t N, uint32_t K, int out_dtype, miori_stream stream);

/* Fused 4-bit GEMM: as miori_gemm_bf16 with B = bf16(dequant4(W)), the
 * dequantisation done inside the GEMM (M > 32: in registers, just before the
 * MFMAs that use it), so the bf16 cache is never materialised. Numerically identical in operands to
 * miori_dequant_q4_tile followed by miori_gemm_bf16 (the reference's two-step
 * dequant_tile + gemm_mpp, src/engine.cpp:144-146, 508-518).
 * Requires K % 64 == 0, N % 16 == 0, group in {32, 64, 128}. */
int miori_gemm_q4(const void* A, const void* q, const void* scales,
                  const void* biases, void* C, uint32_t M, uint32_t N, uint32_t K,
                  uint32_t group, int out_dtype, miori_stream stream);

/* Size of the fixed scratch array of miori_gemm_q4_static (bytes per GPU). */
#define MIORI_STATIC_SCRATCH_BYTES (32u << 20)

/* Allocation-free variant of miori_gemm_q4 (no counterpart in the
 * reference): for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, shape rules and results as miori_gemm_q4, but the split-K
 * partials go to a fixed per-GPU device array of MIORI_STATIC_SCRATCH_BYTES
 * instead of the library's growable workspace, so the call never allocates.
 * A shape whose partials (splits x M x N x 4 bytes) exceed the array returns
 * MIORI_E_SCRATCH before anything is enqueued. All calls on one GPU share
 * the array: calls that overlap on one GPU (other streams, other threads)
 * race, and calls on one stream are ordered. */
int miori_gemm_q4_static(const void* A, const void* q, const void* scales,
                         const void* biases, void* C, uint32_t M, uint32_t N, uint32_t K,
                         uint32_t group, int out_dtype, miori_stream stream);

/* Batch-engine projection policy: C[M][N] = A[M][K] . W^T for 4-bit MLX
 * weights W (q, scales, biases) with an optional bf16 cache of the same W
 * (row-major [N][K], as miori_dequant_q4_tile writes it; NULL if none).
 * Replaces BatchEngine::linear (src/batch.cpp:223-230), which runs the exact
 * 4-bit gemv4_b at <= 4 active slots and otherwise the bf16-cache GEMM
 * (gemm_mpp32 up to 32 rows, gemm_mpp beyond). Here:
 *  - M <= 32: the exact batched 4-bit GEMV (miori_gemv_q4_batched), the
 *    reference's gemv4_b semantics (no bf16 rounding of the weights). It
 *    reads a quarter of the bytes of the bf16 cache and is faster than the
 *    cache GEMM at every M = 1..32 on the decode projection shapes (1.3-2.7x),
 *    so the cache is never read for decode;
 *  - M > 32: miori_gemm_bf16 on the cache when one is given, else the fused
 *    4-bit GEMM (miori_gemm_q4).
 * Shape rules are those of the entry point taken. */
int miori_linear_q4(const void* A, const void* q, const void* scales, const void* biases,
                    const void* bf16_cache, void* C, uint32_t M, uint32_t N, uint32_t K,
                    uint32_t group, int out_dtype, miori_stream stream);

/* Strided GEMM for any shape: C[m*ldc + n] = sum_k A[m*lda + k] * B[n*ldb + k],
 * bf16 operands, fp32 output, each output one fp32 FMA chain over k = 0..K-1
 * (the reference kernel's accumulation). The fallback for shapes the MFMA
 * GEMM does not take. Replaces gemm_naive (src/ops.h:30-32, kernel
 * shaders/ops.metal:199-251); byte offsets are applied by the caller.
 * Requires lda >= K, ldb >= K, ldc >= N; A and B 2-byte, C 4-byte aligned. */
int miori_gemm_naive(const void* A, const void* B, float* C, uint32_t M, uint32_t N,
                     uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc,
                     miori_stream stream);

/* ---- weight-cache builders ----------------------------------------------
 * out = bf16(float(code)*scale + bias), RNE, bit-exact with the CPU dequant.
 * dequant_q4_tile writes the layout miori_gemm_bf16 reads (row-major [N][K]);
 * it replaces dequant_tile (src/ops.h:90-92, shaders/gemm_mpp.metal:9-34).
 * dequant_q4 replaces dequant4 (src/ops.h:26-28, shaders/ops.metal:142-166),
 * dequant_q8 replaces dequant8 (src/ops.h:203-205, shaders/ops.metal:754-779);
 * both write row-major [N][K]. */
int miori_dequant_q4_tile(const void* q, const void* scales, const void* biases,
                          void* out, uint32_t N, uint32_t K, uint32_t group,
                          miori_stream stream);
int miori_dequant_q4(const void* q, const void* scales, const void* biases,
                     void* out, uint32_t N, uint32_t K, uint32_t group,
                     miori_stream stream);
int miori_dequant_q8(const void* q, const void* scales, const void* biases,
                     void* out, uint32_t N, uint32_t K, uint32_t group,
                     miori_stream stream);

/* ---- diagnostics ---------------------------------------------------------
 * No counterpart in the reference. Launches one wave on `stream` that records
 * n pairs (shader-clock cycles from s_memtime, wall-clock ticks from
 * s_memrealtime) into samples[2n], one pair every gap_ticks wall-clock ticks,
 * and writes the wall-clock rate in kHz to *wall_khz (host pointer, set
 * before the launch returns). Run beside a kernel on another stream, the
 * clock it ran at over an interval is d(cycles) / d(ticks) x wall_khz. The
 * wave holds a few registers of one CU until it ends, so a concurrent kernel
 * that fills every CU runs slower meanwhile: use the samples for clocks, not
 * for timing. Bounds: n <= 2^20, n x gap_ticks <= 2 s of wall clock;
 * samples 8-byte aligned device memory. */
int miori_diag_clock_sample(uint64_t* samples, uint32_t n, uint32_t gap_ticks,
                            uint32_t* wall_khz, miori_stream stream);
/* No counterpart in the reference. miori_gemv_q4 (M = 1, K <= 2048 and a
 * multiple of 32) on the same kernel with one extra full load wait, also
 * writing four wall-clock stamps per wave (s_memrealtime ticks) into
 * stamps[4w .. 4w+3]: entry, all of the wave's loads landed, arithmetic and
 * reduction done, stores complete. *nwaves (host pointer) receives the wave
 * count, ceil(N / 16) * 4; cap is the capacity of stamps in values and must
 * be >= 4 * nwaves. y is the same as miori_gemv_q4's. For decomposing a
 * launch's time, not for production. */
int miori_diag_gemv_q4_timeline(const void* q, const void* scales, const void* biases,
                                const void* x, void* y, uint32_t N, uint32_t K, uint32_t group,
                                int out_dtype, uint64_t* stamps, uint32_t cap,
                                uint32_t* nwaves, miori_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* MIORI_HIP_H */
