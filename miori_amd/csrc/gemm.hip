// Prefill GEMM on bf16 MFMA for gfx950: C[M][N] = A[M][K] . B[N][K]^T with
// fp32 accumulation, B either the bf16 weight cache (row-major [N][K]) or the
// 4-bit MLX-affine weights dequantised to bf16 while the tile is staged to LDS.
//
// Replaces shaders/gemm_mpp.metal:36-73 (gemm_mpp / gemm_mpp32, Apple MPP
// matmul2d on a tile-major bf16 cache) and, for the fused variant, the
// two-step dequant_tile + gemm_mpp of src/engine.cpp:144-146, 508-518.
//
// Structure: a 256x128 (M x N) macro tile per 256-thread workgroup, K in
// steps of 64. The four waves form a 2x2 grid of 128x64 wave tiles, each a
// 4x2 array of v_mfma_f32_32x32x16_bf16 accumulators. Operand tiles are
// double-buffered in LDS (A 32 KiB + B 16 KiB per stage); global loads of
// step k+1 are in flight while step k runs on the matrix cores. Rows in LDS
// are 128 bytes (64 bf16) and the eight 16-byte chunks of a row are XOR-
// swizzled by (row & 7), so the 32 rows an MFMA fragment read touches fall in
// distinct banks. Workgroups are renumbered so that each XCD (workgroup id
// mod 8 on MI355X) works on a contiguous block of output tiles and shares its
// operand slabs in its own L2.
#include "common.hpp"
#include "kernels.hpp"

namespace miori {

namespace {

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int ROWB = BK * 2;                 // bytes per LDS row
constexpr int A_BYTES = BM * ROWB;           // 32 KiB
constexpr int B_BYTES = BN * ROWB;           // 16 KiB
constexpr int STAGE = A_BYTES + B_BYTES;

__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t kb) {
    return row * ROWB + ((kb ^ (row & 7u)) << 4);
}

template <bool Q4>
__global__ __launch_bounds__(256) void gemm_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
    const uint4* __restrict__ q, const uint16_t* __restrict__ s,
    const uint16_t* __restrict__ bsc, void* __restrict__ C, uint32_t M, uint32_t N,
    uint32_t K, uint32_t G, int out_bf16, uint32_t tiles_m) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

    const uint32_t t = threadIdx.x;
    const uint32_t lane = t & 63u, wave = t >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;

    uint32_t pid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if ((nwg & 7u) == 0) pid = (pid & 7u) * (nwg >> 3) + (pid >> 3);
    const uint32_t tm = pid % tiles_m, tn = pid / tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t KT = K / BK;

    // ---- global -> register staging
    uint4 ra[8];
    uint4 rb[Q4 ? 1 : 4];
    uint32_t rs = 0, rbias = 0;

    auto load_tiles = [&](uint32_t kt) {
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const uint32_t row = min(m0 + p * 32 + (t >> 3), M - 1u);
            ra[p] = *reinterpret_cast<const uint4*>(A + (size_t)row * K + kt * BK + (t & 7u) * 8);
        }
        if constexpr (Q4) {
            const uint32_t row = min(n0 + (t >> 1), N - 1u);
            const uint32_t half = t & 1u;
            rb[0] = q[(size_t)row * (K / 32) + kt * 2 + half];
            const uint32_t g = (kt * BK + half * 32) / G;
            rs = s[(size_t)row * (K / G) + g];
            rbias = bsc[(size_t)row * (K / G) + g];
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t row = min(n0 + p * 32 + (t >> 3), N - 1u);
                rb[p] = *reinterpret_cast<const uint4*>(B + (size_t)row * K + kt * BK + (t & 7u) * 8);
            }
        }
    };

    auto store_tiles = [&](int buf) {
        uint8_t* base = lds + buf * STAGE;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const uint32_t r = p * 32 + (t >> 3);
            *reinterpret_cast<uint4*>(base + swz(r, t & 7u)) = ra[p];
        }
        uint8_t* bb = base + A_BYTES;
        if constexpr (Q4) {
            const uint32_t r = t >> 1, half = t & 1u;
            const float sc = bf16_bits_to_f32(rs), bi = bf16_bits_to_f32(rbias);
            const uint32_t wv[4] = {rb[0].x, rb[0].y, rb[0].z, rb[0].w};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t o[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float v0 = fmaf((float)((wv[w] >> (8 * j)) & 0xFu), sc, bi);
                    const float v1 = fmaf((float)((wv[w] >> (8 * j + 4)) & 0xFu), sc, bi);
                    o[j] = pack_bf16x2(v0, v1);
                }
                *reinterpret_cast<uint4*>(bb + swz(r, half * 4 + w)) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t r = p * 32 + (t >> 3);
                *reinterpret_cast<uint4*>(bb + swz(r, t & 7u)) = rb[p];
            }
        }
    };

    f32x16_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    load_tiles(0);
    store_tiles(0);
    __syncthreads();

    for (uint32_t kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) load_tiles(kt + 1);
        const uint8_t* base = lds + buf * STAGE;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const uint32_t kb = 2 * ks + (lane >> 5);
            bf16x8_t af[4], bf[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t r = wm * 128 + i * 32 + (lane & 31u);
                af[i] = *reinterpret_cast<const bf16x8_t*>(base + swz(r, kb));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t r = wn * 64 + j * 32 + (lane & 31u);
                bf[j] = *reinterpret_cast<const bf16x8_t*>(base + A_BYTES + swz(r, kb));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) store_tiles(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: lane l of a 32x32 accumulator holds column l%32 and rows
    // 8*(e/4) + 4*(l/32) + e%4 for its 16 elements e.
    const bool bf = out_bf16 != 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t col = n0 + wn * 64 + j * 32 + (lane & 31u);
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t row = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) store_out(C, (size_t)row * N + col, acc[i][j][e], bf);
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm(const void* A, const void* B, const void* q, const void* s,
                       const void* b, void* C, uint32_t M, uint32_t N, uint32_t K,
                       uint32_t G, int out_bf16, hipStream_t st) {
    const uint32_t tiles_m = (M + BM - 1) / BM;
    const uint32_t tiles_n = (N + BN - 1) / BN;
    const dim3 grid(tiles_m * tiles_n);
    if (q)
        hipLaunchKernelGGL(gemm_kernel<true>, grid, dim3(256), 0, st, (const uint16_t*)A,
                           (const uint16_t*)nullptr, (const uint4*)q, (const uint16_t*)s,
                           (const uint16_t*)b, C, M, N, K, G, out_bf16, tiles_m);
    else
        hipLaunchKernelGGL(gemm_kernel<false>, grid, dim3(256), 0, st, (const uint16_t*)A,
                           (const uint16_t*)B, (const uint4*)nullptr, (const uint16_t*)nullptr,
                           (const uint16_t*)nullptr, C, M, N, K, G, out_bf16, tiles_m);
    return hipGetLastError();
}

}  // namespace miori
