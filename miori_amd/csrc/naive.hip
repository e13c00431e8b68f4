// Strided bf16 GEMM with fp32 output for any shape:
//   C[m][n] = sum_k float(A[m][k]) * float(B[n][k]),   A row stride lda,
//   B row stride ldb, C row stride ldc (elements).
// Replaces shaders/ops.metal:199-251 (gemm_naive) behind src/ops.h:30-32:
// the fallback for shapes the MFMA GEMM does not take (N % 16 != 0, K % 64
// != 0, strided operands: gate_proj N=16, the bf16 batch lm_head).
//
// Each output is one fp32 FMA chain over k = 0, 1, ..., K-1 starting from
// +0, the reference kernel's accumulation, so results are reproducible bit
// for bit by a sequential fmaf loop on the CPU.
//
// Structure: 256 threads own a TM x TN output tile, RM x RN outputs each
// (rows TM/RM apart, columns TN/RN apart).
// K advances in KT-deep slices; each slice of A and B is loaded coalesced
// (16-byte chunks along k when strides allow) into row-major LDS rows padded
// by 16 bytes, and the next slice's loads are in flight while the current one
// is computed. A is converted to fp32 as it is stored (each A element feeds
// TN/RN threads); B stays bf16 and is converted at use. A thread reads 8
// consecutive k of each of its B rows as one 16-byte LDS read (two for an A
// row) and runs the 8 FMAs of every chain in k order. The chains
// cannot be split over k, so the slice depth sets how many load round trips
// a chain waits for. A thread converts RN B values per k for RM x RN FMAs,
// so taller register tiles cost fewer conversions. Tile shapes (KT 64):
// 64 x 64 (4 x 4 per thread) for general M; 8 x 256 (2 x 4), 16 x 256
// (4 x 4) and 32 x 256 (8 x 4) for M <= 8 / 16 / 32 (the batch lm_head,
// where a taller tile would spend half or more of its FMAs on padding rows);
// 16 x 16 (1 x 1, KT 512) for N <= 32 (gate_proj N=16). Element loads (any
// stride) use a quarter of the slice depth.
#include "common.hpp"
#include "kernels.hpp"

namespace miori {

namespace {

// VEC: 16-byte global loads (lda, ldb multiples of 8, A and B 16-byte
// aligned, K a multiple of 8); otherwise element loads.
template <int TM, int TN, int RM, int RN, int KT, bool VEC>
__global__ __launch_bounds__(256) void naive_gemm_kernel(const uint16_t* __restrict__ A,
                                                         const uint16_t* __restrict__ B,
                                                         float* __restrict__ C, uint32_t M,
                                                         uint32_t N, uint32_t K, uint32_t lda,
                                                         uint32_t ldb, uint32_t ldc) {
    static_assert((TM / RM) * (TN / RN) == 256, "one register tile per thread");
    static_assert(KT % 8 == 0, "8-k chunks");
    constexpr int P = KT + 8;                     // B row stride in LDS (bf16), 16-byte pad
    constexpr int PA = KT + 4;                    // A row stride in LDS (fp32), 16-byte pad
    constexpr int CPR = KT / 8;                   // 16-byte chunks per row per slice
    // chunks (VEC) or elements per thread; an A slice smaller than 256
    // chunks leaves the threads past its end idle (tiles of 8 rows)
    constexpr int CA = (TM * CPR + 255) / 256, CB = TN * CPR / 256;
    constexpr int LA = (TM * KT + 255) / 256, LB = TN * KT / 256;
    static_assert(VEC ? TN * CPR % 256 == 0 : TN * KT % 256 == 0, "B slices in whole passes");
    static_assert(VEC ? (TM * CPR % 256 == 0 || TM * CPR < 256) : (TM * KT % 256 == 0 || TM * KT < 256),
                  "A slice: whole passes or one partial pass");
    // A is kept as fp32 (converted once when stored; each A element feeds
    // TN/RN threads), B as bf16 (converted at each use)
    __shared__ __attribute__((aligned(16))) float As[TM][PA];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[TN][P];

    // a thread's rows are XT (YT) apart, so the lanes of a wave read
    // consecutive LDS rows (a 16-byte-padded row stride spreads them over the
    // banks; rows RN apart would put lanes on the same banks)
    constexpr uint32_t XT = TN / RN, YT = TM / RM;
    const uint32_t t = threadIdx.x;
    const uint32_t tx = t % XT, ty = t / XT;
    const uint32_t m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;

    // one K slice in registers (the next is loaded while this one is used)
    u32x4_t va[VEC ? CA : 1], vb[VEC ? CB : 1];
    uint16_t sa[VEC ? 1 : LA], sb[VEC ? 1 : LB];
    auto load = [&](uint32_t k0) {
        if constexpr (VEC) {
#pragma unroll
            for (int e = 0; e < CA; ++e) {
                const uint32_t idx = e * 256u + t, r = idx / CPR, k = k0 + (idx % CPR) * 8, m = m0 + r;
                va[e] = (idx < (uint32_t)(TM * CPR) && m < M && k < K)
                            ? *reinterpret_cast<const u32x4_t*>(A + (size_t)m * lda + k)
                            : u32x4_t{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int e = 0; e < CB; ++e) {
                const uint32_t idx = e * 256u + t, r = idx / CPR, k = k0 + (idx % CPR) * 8, n = n0 + r;
                vb[e] = (n < N && k < K) ? *reinterpret_cast<const u32x4_t*>(B + (size_t)n * ldb + k)
                                         : u32x4_t{0u, 0u, 0u, 0u};
            }
        } else {
#pragma unroll
            for (int e = 0; e < LA; ++e) {
                const uint32_t idx = e * 256u + t, r = idx / KT, k = k0 + idx % KT, m = m0 + r;
                sa[e] = (idx < (uint32_t)(TM * KT) && m < M && k < K) ? A[(size_t)m * lda + k] : (uint16_t)0;
            }
#pragma unroll
            for (int e = 0; e < LB; ++e) {
                const uint32_t idx = e * 256u + t, r = idx / KT, k = k0 + idx % KT, n = n0 + r;
                sb[e] = (n < N && k < K) ? B[(size_t)n * ldb + k] : (uint16_t)0;
            }
        }
    };
    auto stash = [&]() {
        if constexpr (VEC) {
#pragma unroll
            for (int e = 0; e < CA; ++e) {
                const uint32_t idx = e * 256u + t;
                if (idx < (uint32_t)(TM * CPR)) {
                    const u32x4_t v = va[e];
                    float* dst = &As[idx / CPR][(idx % CPR) * 8];
                    *reinterpret_cast<f32x4_t*>(dst) =
                        f32x4_t{bf16_bits_to_f32(v[0] & 0xFFFFu), bf16_bits_to_f32(v[0] >> 16),
                                bf16_bits_to_f32(v[1] & 0xFFFFu), bf16_bits_to_f32(v[1] >> 16)};
                    *reinterpret_cast<f32x4_t*>(dst + 4) =
                        f32x4_t{bf16_bits_to_f32(v[2] & 0xFFFFu), bf16_bits_to_f32(v[2] >> 16),
                                bf16_bits_to_f32(v[3] & 0xFFFFu), bf16_bits_to_f32(v[3] >> 16)};
                }
            }
#pragma unroll
            for (int e = 0; e < CB; ++e) {
                const uint32_t idx = e * 256u + t;
                *reinterpret_cast<u32x4_t*>(&Bs[idx / CPR][(idx % CPR) * 8]) = vb[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < LA; ++e) {
                const uint32_t idx = e * 256u + t;
                if (idx < (uint32_t)(TM * KT)) As[idx / KT][idx % KT] = bf16_bits_to_f32(sa[e]);
            }
#pragma unroll
            for (int e = 0; e < LB; ++e) {
                const uint32_t idx = e * 256u + t;
                Bs[idx / KT][idx % KT] = sb[e];
            }
        }
    };

    float acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = 0.f;

    // 8 consecutive k of a B row as one 16-byte LDS read (two for A in fp32);
    // the 8 FMAs of a chain run in k order
    auto chunk = [&](uint32_t kk, int cnt) {
        f32x4_t a[RM][2];
        u32x4_t b[RN];
#pragma unroll
        for (int i = 0; i < RM; ++i) {
            a[i][0] = *reinterpret_cast<const f32x4_t*>(&As[ty + i * YT][kk]);
            a[i][1] = *reinterpret_cast<const f32x4_t*>(&As[ty + i * YT][kk + 4]);
        }
#pragma unroll
        for (int j = 0; j < RN; ++j) b[j] = *reinterpret_cast<const u32x4_t*>(&Bs[tx + j * XT][kk]);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if (q < cnt) {
#pragma unroll
                for (int i = 0; i < RM; ++i) {
                    const float av = a[i][q >> 2][q & 3];
#pragma unroll
                    for (int j = 0; j < RN; ++j) {
                        const float bv = bf16_bits_to_f32((b[j][q >> 1] >> (16 * (q & 1))) & 0xFFFFu);
                        acc[i][j] = __builtin_fmaf(av, bv, acc[i][j]);
                    }
                }
            }
        }
    };

    load(0);
    for (uint32_t k0 = 0; k0 < K; k0 += KT) {
        stash();
        __syncthreads();
        if (k0 + KT < K) load(k0 + KT);  // next slice in flight during the FMAs
        const uint32_t kn = min((uint32_t)KT, K - k0);  // padding k (zeros) are skipped
        const uint32_t full = kn / 8;
#pragma unroll 4
        for (uint32_t c = 0; c < full; ++c) chunk(c * 8, 8);
        if (kn % 8) chunk(full * 8, (int)(kn % 8));
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < RM; ++i) {
        const uint32_t m = m0 + ty + i * YT;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < RN; ++j) {
            const uint32_t n = n0 + tx + j * XT;
            if (n < N) C[(size_t)m * ldc + n] = acc[i][j];
        }
    }
}

template <int TM, int TN, int RM, int RN, int KT>
void launch_cfg(bool vec, const void* A, const void* B, float* C, uint32_t M, uint32_t N,
                uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc, hipStream_t st) {
    const dim3 grid((N + TN - 1) / TN, (M + TM - 1) / TM);
    if (vec)
        hipLaunchKernelGGL((naive_gemm_kernel<TM, TN, RM, RN, KT, true>), grid, dim3(256), 0, st,
                           (const uint16_t*)A, (const uint16_t*)B, C, M, N, K, lda, ldb, ldc);
    else
        hipLaunchKernelGGL((naive_gemm_kernel<TM, TN, RM, RN, KT / 4, false>), grid, dim3(256), 0,
                           st, (const uint16_t*)A, (const uint16_t*)B, C, M, N, K, lda, ldb, ldc);
}

}  // namespace

hipError_t launch_gemm_naive(const void* A, const void* B, float* C, uint32_t M, uint32_t N,
                             uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc,
                             hipStream_t st) {
    const bool vec = lda % 8 == 0 && ldb % 8 == 0 && K % 8 == 0 &&
                     ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0;
    // Deep K slices cut the number of load round trips a chain waits for.
    if (N <= 32)
        launch_cfg<16, 16, 1, 1, 512>(vec, A, B, C, M, N, K, lda, ldb, ldc, st);
    else if (M <= 8)
        launch_cfg<8, 256, 2, 4, 64>(vec, A, B, C, M, N, K, lda, ldb, ldc, st);
    else if (M <= 16)
        launch_cfg<16, 256, 4, 4, 64>(vec, A, B, C, M, N, K, lda, ldb, ldc, st);
    else if (M <= 32)
        launch_cfg<32, 256, 8, 4, 64>(vec, A, B, C, M, N, K, lda, ldb, ldc, st);
    else
        launch_cfg<64, 64, 4, 4, 64>(vec, A, B, C, M, N, K, lda, ldb, ldc, st);
    return hipGetLastError();
}

}  // namespace miori
