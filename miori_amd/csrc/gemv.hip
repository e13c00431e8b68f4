// Decode GEMVs on the VALU for gfx950: y[M][N] = x[M][K] . dequant(W)^T for
// small M (1..4 activation rows per launch), 4-bit and 8-bit MLX-affine W.
//
// Replaces shaders/ops.metal:6-42 (gemv4), :46-82 (gemv8) and
// shaders/batch.metal:145-236 (gemv4_b / gemv8_b). The reference kernels put
// one 32-lane simdgroup on a row, each lane dequantising a 32-element group
// into fp32 and multiplying by x re-read from memory. Here:
//
//  * A lane owns a 16-byte "chunk" of a weight row (32 nibbles or 16 codes)
//    and one wave instruction loads 64 consecutive chunks, a contiguous 1 KiB
//    of the row (global_load_dwordx4). A wave works on R rows at once and
//    issues all of their loads before any arithmetic, so a launch keeps most
//    of the matrix in flight.
//  * The activation chunk a lane needs is the same for every row, so it is
//    loaded once and kept in registers, pre-arranged for the unpacking order.
//  * The affine dequant is factored out of the inner loop:
//        sum_k (q_k*s + b) x_k = s * sum_k q_k x_k + b * sum_k x_k
//    per (row, group) piece, with sum_k x_k computed once per chunk. The
//    integer codes and bf16 x are exact operands, so only the fp32 sums round.
//  * 4-bit: nibble pairs become bf16 pairs with one AND-OR:
//        ((w >> 4j) & 0x000F000F) | 0x43004300 = bf16(128+q_j), bf16(128+q_{j+4})
//    and v_dot2c_f32_bf16 multiplies them with the matching x pair, so
//    D = sum (128+q) x and the bias becomes (b - 128 s).
//  * 8-bit: v_cvt_f32_ubyte{0..3} and an fp32 FMA per code.
//  * Lane partial sums are reduced with DPP inside the wave; when K is split
//    across the 4 waves of a workgroup (K > 2048 for 4-bit) the per-wave sums
//    are added through LDS in a fixed order.
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace miori {

namespace {

// Load the activation chunk c of one row and arrange it for the unpacking.
// 4-bit: chunk = 32 bf16 = 16 dwords. For word w of the weight chunk (nibbles
// k = 8w..8w+7), pair j (j = 0..3) multiplies nibbles j and j+4, so the x pair
// register holds (x[8w+j], x[8w+j+4]).
// 8-bit: chunk = 16 bf16 kept as 16 fp32.
template <int BITS>
__device__ __forceinline__ void load_x_chunk(const uint16_t* __restrict__ xrow, uint32_t c,
                                             bool valid, uint32_t xr[16], float& xs) {
    if constexpr (BITS == 4) {
        uint32_t d[16];
        if (valid) {
            const uint4* p = reinterpret_cast<const uint4*>(xrow) + (size_t)c * 4;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint4 v = p[t];
                d[4 * t + 0] = v.x; d[4 * t + 1] = v.y; d[4 * t + 2] = v.z; d[4 * t + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) d[t] = 0u;
        }
        float sum = 0.f;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            sum += bf16_bits_to_f32(d[t] & 0xFFFFu);
            sum += bf16_bits_to_f32(d[t] >> 16);
        }
        xs = sum;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t a = d[4 * w + (j >> 1)];
                const uint32_t b = d[4 * w + 2 + (j >> 1)];
                xr[4 * w + j] = (j & 1) ? ((a >> 16) | (b & 0xFFFF0000u))
                                        : ((a & 0xFFFFu) | (b << 16));
            }
        }
    } else {
        uint32_t d[8];
        if (valid) {
            const uint4* p = reinterpret_cast<const uint4*>(xrow) + (size_t)c * 2;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint4 v = p[t];
                d[4 * t + 0] = v.x; d[4 * t + 1] = v.y; d[4 * t + 2] = v.z; d[4 * t + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) d[t] = 0u;
        }
        float sum = 0.f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float lo = bf16_bits_to_f32(d[t] & 0xFFFFu);
            const float hi = bf16_bits_to_f32(d[t] >> 16);
            xr[2 * t] = __float_as_uint(lo);
            xr[2 * t + 1] = __float_as_uint(hi);
            sum += lo;
            sum += hi;
        }
        xs = sum;
    }
}

// sum over the chunk of code_k * x_k (4-bit: of (128 + code_k) * x_k).
template <int BITS>
__device__ __forceinline__ float chunk_dot(const uint4 qv, const uint32_t xr[16]) {
    const uint32_t wv[4] = {qv.x, qv.y, qv.z, qv.w};
    float d = 0.f;
    if constexpr (BITS == 4) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t p = ((wv[w] >> (4 * j)) & 0x000F000Fu) | 0x43004300u;
                d = dot2_bf16(p, xr[4 * w + j], d);
            }
        }
    } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float code = (float)((wv[w] >> (8 * j)) & 0xFFu);
                d = fmaf(code, __uint_as_float(xr[4 * w + j]), d);
            }
        }
    }
    return d;
}

template <int BITS, int MR, int R, int CPL>
__global__ __launch_bounds__(256) void gemv_valu_kernel(
    const uint4* __restrict__ q, const uint16_t* __restrict__ s,
    const uint16_t* __restrict__ bs, const uint16_t* __restrict__ x,
    void* __restrict__ y, uint32_t N, uint32_t K, uint32_t G, uint32_t S,
    int out_bf16) {
    constexpr uint32_t E = (BITS == 4) ? 32u : 16u;  // elements per 16-byte chunk
    __shared__ float red[4][R][MR];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t js = wave % S;   // K slice handled by this wave
    const uint32_t rb = wave / S;   // row block inside the workgroup
    const uint32_t rows_per_wg = R * (4u / S);
    const uint32_t row0 = blockIdx.x * rows_per_wg + rb * R;
    const uint32_t C = K / E;       // chunks per row
    const uint32_t ng = K / G;

    uint32_t cidx[CPL];
    bool cval[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const uint32_t c = (js * CPL + i) * 64u + lane;
        cval[i] = c < C;
        cidx[i] = cval[i] ? c : 0u;
    }

    // Weight loads for all R rows first: they are the HBM stream.
    uint4 qv[R][CPL];
    uint32_t sv[R][CPL], bv[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t rr = min(row0 + r, N - 1u);
        const uint4* qrow = q + (size_t)rr * C;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            qv[r][i] = cval[i] ? load_stream(qrow + cidx[i]) : make_uint4(0u, 0u, 0u, 0u);
            const uint32_t g = cidx[i] * E / G;
            sv[r][i] = s[(size_t)rr * ng + g];
            bv[r][i] = bs[(size_t)rr * ng + g];
        }
    }

    uint32_t xr[MR][CPL][16];
    float xs[MR][CPL];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int i = 0; i < CPL; ++i)
            load_x_chunk<BITS>(x + (size_t)m * K, cidx[i], cval[i], xr[m][i], xs[m][i]);

    float acc[R][MR];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = 0.f;

#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const float sc = bf16_bits_to_f32(sv[r][i]);
            const float bi = bf16_bits_to_f32(bv[r][i]);
            // 4-bit sums carry the +128 offset of the bf16 trick: fold it into the bias.
            const float bx = (BITS == 4) ? fmaf(-128.f, sc, bi) : bi;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float d = chunk_dot<BITS>(qv[r][i], xr[m][i]);
                acc[r][m] = fmaf(sc, d, fmaf(bx, xs[m][i], acc[r][m]));
            }
        }
    }

    float tot[R][MR];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) tot[r][m] = wave_sum(acc[r][m]);

    const bool bf = out_bf16 != 0;
    if (S == 1) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t row = row0 + r;
                if (row < N) {
#pragma unroll
                    for (int m = 0; m < MR; ++m) store_out(y, (size_t)m * N + row, tot[r][m], bf);
                }
            }
        }
        return;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) red[wave][r][m] = tot[r][m];
    }
    __syncthreads();
    if (js == 0 && lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = row0 + r;
            if (row >= N) continue;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float v = red[wave][r][m];
                for (uint32_t j = 1; j < S; ++j) v += red[wave + j][r][m];
                store_out(y, (size_t)m * N + row, v, bf);
            }
        }
    }
}

template <int BITS, int MR, int R, int CPL>
hipError_t launch_valu(const void* q, const void* s, const void* b, const void* x, void* y,
                       uint32_t N, uint32_t K, uint32_t G, uint32_t S, int out_bf16,
                       hipStream_t st) {
    const uint32_t rows_per_wg = R * (4u / S);
    const uint32_t grid = (N + rows_per_wg - 1) / rows_per_wg;
    hipLaunchKernelGGL((gemv_valu_kernel<BITS, MR, R, CPL>), dim3(grid), dim3(256), 0, st,
                       (const uint4*)q, (const uint16_t*)s, (const uint16_t*)b,
                       (const uint16_t*)x, y, N, K, G, S, out_bf16);
    return hipGetLastError();
}

template <int BITS, int MR, int R>
hipError_t dispatch_cpl(int cpl, const void* q, const void* s, const void* b, const void* x,
                        void* y, uint32_t N, uint32_t K, uint32_t G, uint32_t S, int out_bf16,
                        hipStream_t st) {
    switch (cpl) {
        case 1: return launch_valu<BITS, MR, R, 1>(q, s, b, x, y, N, K, G, S, out_bf16, st);
        case 2:
            if constexpr (MR <= 2) return launch_valu<BITS, MR, R, 2>(q, s, b, x, y, N, K, G, S, out_bf16, st);
            break;
        case 4:
            if constexpr (MR == 1) return launch_valu<BITS, MR, R, 4>(q, s, b, x, y, N, K, G, S, out_bf16, st);
            break;
    }
    return hipErrorInvalidValue;
}

template <int BITS>
hipError_t dispatch_mr(int mr, int rows, int cpl, const void* q, const void* s, const void* b,
                       const void* x, void* y, uint32_t N, uint32_t K, uint32_t G, uint32_t S,
                       int out_bf16, hipStream_t st) {
    if (mr == 1) {
        switch (rows) {
            case 1: return dispatch_cpl<BITS, 1, 1>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
            case 2: return dispatch_cpl<BITS, 1, 2>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
            case 8: return dispatch_cpl<BITS, 1, 8>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
            default: return dispatch_cpl<BITS, 1, 4>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
        }
    }
    switch (mr) {
        case 2: return dispatch_cpl<BITS, 2, 2>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
        case 3: return dispatch_cpl<BITS, 3, 2>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
        case 4: return dispatch_cpl<BITS, 4, 2>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
    }
    return hipErrorInvalidValue;
}

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

}  // namespace

// Split of the chunk range of a row: S K-slices over the 4 waves of a
// workgroup, each lane taking `cpl` chunks per slice.
void gemv_split(int bits, uint32_t K, uint32_t* S, int* cpl) {
    const uint32_t E = bits == 4 ? 32u : 16u;
    const uint32_t C = K / E;
    uint32_t s = C <= 64 ? 1u : (C <= 128 ? 2u : 4u);
    uint32_t c = (C + 64u * s - 1u) / (64u * s);
    *S = s;
    *cpl = c <= 1 ? 1 : (c <= 2 ? 2 : 4);
}

hipError_t launch_gemv_valu(int bits, const void* q, const void* s, const void* b,
                            const void* x, void* y, uint32_t M, uint32_t N, uint32_t K,
                            uint32_t G, int out_bf16, hipStream_t st) {
    uint32_t S;
    int cpl;
    gemv_split(bits, K, &S, &cpl);
    static const int rows_m1 = env_int("MIORI_GEMV_ROWS", 4);
    const int mr_max = cpl == 1 ? 4 : (cpl == 2 ? 2 : 1);
    const size_t ybytes = out_bf16 ? 2 : 4;
    for (uint32_t m0 = 0; m0 < M; m0 += mr_max) {
        const int mr = (int)std::min<uint32_t>(mr_max, M - m0);
        const void* xm = (const uint16_t*)x + (size_t)m0 * K;
        void* ym = (char*)y + (size_t)m0 * N * ybytes;
        hipError_t e = bits == 4
            ? dispatch_mr<4>(mr, rows_m1, cpl, q, s, b, xm, ym, N, K, G, S, out_bf16, st)
            : dispatch_mr<8>(mr, rows_m1, cpl, q, s, b, xm, ym, N, K, G, S, out_bf16, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace miori
