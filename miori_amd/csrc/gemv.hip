// Decode GEMVs on the VALU for gfx950: y[M][N] = x[M][K] . dequant(W)^T for
// small M (1..4 activation rows per launch), 4-bit and 8-bit MLX-affine W.
//
// Replaces shaders/ops.metal:6-42 (gemv4), :46-82 (gemv8) and
// shaders/batch.metal:145-236 (gemv4_b / gemv8_b, rows <= 4). The reference
// kernels put one 32-lane simdgroup on a row, each lane dequantising a
// 32-element group into fp32 and multiplying by x re-read from memory. Here:
//
//  * A lane owns a 16-byte "chunk" of a weight row (32 nibbles or 16 codes)
//    and one wave instruction loads 64 consecutive chunks, a contiguous 1 KiB
//    of the row (buffer_load_dwordx4). A wave works on R rows at once and
//    issues all of their loads before any arithmetic.
//  * The activation chunk a lane needs is the same for every row, so it is
//    loaded once and kept in registers, pre-arranged for the unpacking order.
//  * The affine dequant is factored out of the inner loop:
//        sum_k (q_k*s + b) x_k = s * sum_k q_k x_k + b * sum_k x_k
//    per (row, group) piece, with sum_k x_k computed once per chunk. The
//    integer codes and bf16 x are exact operands, so only the fp32 sums round.
//  * 4-bit: nibble pairs become bf16 pairs with one AND-OR:
//        ((w >> 4j) & 0x000F000F) | 0x43004300 = bf16(128+q_j), bf16(128+q_{j+4})
//    and v_dot2c_f32_bf16 multiplies them with the matching x pair, so
//    D = sum (128+q) x and the bias becomes (b - 128 s). 11 VALU ops per
//    8 weights.
//  * 8-bit: v_cvt_f32_ubyte{0..3} and an fp32 FMA per code.
//  * The R x M row sums are reduced across the wave with permlane swaps and
//    DPP (wave_reduce); when K is split across the 4 waves of a workgroup
//    (K > 2048 for 4-bit) the per-wave sums are added through LDS in a fixed
//    order. Every row's arithmetic is independent of R and M, so a batched
//    row is bit-identical to the single-row product.
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <stdlib.h>

namespace miori {

namespace {

constexpr uint32_t kNibMask = 0x000F000Fu;
constexpr uint32_t kBf128 = 0x43004300u;   // bf16 pair (128, 128)
constexpr uint32_t kBfOnes = 0x3F803F80u;  // bf16 pair (1, 1)

// Activation chunk c of one row, arranged for the unpacking order.
// 4-bit: chunk = 32 bf16 = 16 dwords. For word w of the weight chunk
// (nibbles k = 8w..8w+7) pair j (j = 0..3) multiplies nibbles j and j+4, so
// register 4w+j holds the bf16 pair (x[8w+j], x[8w+j+4]).
// 8-bit: chunk = 16 bf16 kept as 16 fp32.
template <int BITS>
__device__ __forceinline__ void prep_x(const u32x4_t (&d)[BITS == 4 ? 4 : 2], uint32_t (&xr)[16],
                                       float& xs) {
    float sum = 0.f;
    if constexpr (BITS == 4) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const u32x4_t v = d[w];
            xr[4 * w + 0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
            xr[4 * w + 1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
            xr[4 * w + 2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
            xr[4 * w + 3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
#pragma unroll
            for (int t = 0; t < 4; ++t) sum = dot2_bf16(v[t], kBfOnes, sum);
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t u = d[h][t];
                xr[8 * h + 2 * t] = u << 16;
                xr[8 * h + 2 * t + 1] = u & 0xFFFF0000u;
                sum = dot2_bf16(u, kBfOnes, sum);
            }
        }
    }
    xs = sum;
}

// Input transforms of the fused decode ops (one activation row, K <= 8192):
// the bf16 x vector is built in LDS by the whole workgroup from fp32 inputs
// that are L2-resident, so it never makes an HBM round trip.
//   XM_NORM: x = bf16(xf * rsqrt(sum(xf^2)/K + eps) * w)     (ops.metal:86-114)
//   XM_SILU: x = bf16(g / (1 + exp(-g)) * u)                 (ops.metal:129-139)
enum { XM_PLAIN = 0, XM_NORM = 1, XM_SILU = 2 };
constexpr uint32_t kXmMaxK = 8192;

// bf16(silu(a) * u), silu(a) = a / (1 + e^-a), rounded as the CPU's expf
// and IEEE divide would round it. The hardware exp2 of -a*log2(e) plus a
// reciprocal is a few fp32 ulp off; that only matters when the fp32 product
// lies near a bf16 rounding tie (low half 0x8000), where it can flip the
// rounding. Those lanes (about 0.1%) recompute with expf and a divide.
__device__ __forceinline__ uint32_t silu_mul_bf16(float a, float u) {
    const float e = __builtin_amdgcn_exp2f(-a * 1.44269504088896341f);
    float v = (a * __builtin_amdgcn_rcpf(1.0f + e)) * u;
    const uint32_t lo = __builtin_bit_cast(uint32_t, v) & 0xFFFFu;
    if (lo - (0x8000u - 32u) <= 64u) v = (a / (1.0f + expf(-a))) * u;
    return f32_to_bf16_bits(v);
}

// DIAG = 1 (a diagnostic build, miori_diag_gemv_q4_timeline): each wave
// also records four wall-clock stamps (s_memrealtime, 100 MHz) into
// stamps[4 * wave]: at entry, once all its loads have landed (an extra full
// vmcnt wait), after its arithmetic and reduction, and once its stores have
// completed. Only for S = 1 (every row in one wave).
template <int BITS, int MR, int R, int CPL, int XM = XM_PLAIN, int DIAG = 0>
__global__ __launch_bounds__(256) void gemv_valu_kernel(
    const void* __restrict__ q, const void* __restrict__ s, const void* __restrict__ bs,
    const void* __restrict__ x, void* __restrict__ y, uint32_t N, uint32_t K, uint32_t G,
    uint32_t S, int out_bf16, const void* __restrict__ x2 = nullptr, float eps = 0.f,
    uint64_t* __restrict__ stamps = nullptr) {
    uint64_t t_in = 0, t_land = 0, t_math = 0;
    if constexpr (DIAG) t_in = __builtin_amdgcn_s_memrealtime();
    static_assert(XM == XM_PLAIN || MR == 1, "fused input transforms take one row");
    constexpr uint32_t E = (BITS == 4) ? 32u : 16u;  // elements per 16-byte chunk
    constexpr int XL = (BITS == 4) ? 4 : 2;          // 16-byte x loads per chunk
    constexpr int RV0 = R * MR;
    constexpr int RV = RV0 <= 1 ? 1 : RV0 <= 2 ? 2 : RV0 <= 4 ? 4 : RV0 <= 8 ? 8 : 16;
    static_assert(RV0 <= 16, "at most 16 row sums per wave");
    __shared__ float red[4][RV];

    // Index arithmetic in scalar registers where it is wave-uniform, and by
    // shifts: S (1, 2 or 4) and G (16..128) are powers of two, checked by
    // the callers, so no integer division is emitted and the first weight
    // load issues after a few instructions.
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lgS = (uint32_t)__builtin_ctz(S), lgG = (uint32_t)__builtin_ctz(G);
    const uint32_t js = wave & (S - 1u);  // K slice handled by this wave
    const uint32_t rb = wave >> lgS;      // row block inside the workgroup
    const uint32_t rows_per_wg = R * (4u >> lgS);
    const uint32_t row0 = blockIdx.x * rows_per_wg + rb * R;
    const uint32_t C = K / E;       // chunks per row
    const uint32_t ng = K >> lgG;

    const rsrc_t rq = make_rsrc(q, N * C * 16u);
    const rsrc_t rs = make_rsrc(s, N * ng * 2u);
    const rsrc_t rb_ = make_rsrc(bs, N * ng * 2u);
    const rsrc_t rx = make_rsrc(x, MR * K * 2u);

    // Fused transforms: issue the fp32 input loads before the weight loads
    // (vmcnt completes in issue order, so waiting for them does not wait for
    // the weight stream). Thread t owns elements 8t + 2048 i.
    constexpr int XI = kXmMaxK / 2048;
    __shared__ __attribute__((aligned(16))) uint16_t xl[XM == XM_PLAIN ? 8 : kXmMaxK];
    f32x4_t xa[XM == XM_PLAIN ? 1 : XI][2], xb[XM == XM_PLAIN ? 1 : XI][2];
    if constexpr (XM != XM_PLAIN) {
        const rsrc_t r1 = make_rsrc(x, K * 4u);
        const rsrc_t r2 = make_rsrc(x2, K * (XM == XM_NORM ? 2u : 4u));
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const uint32_t e = i * 2048u + threadIdx.x * 8u;
            const bool in = e < K;
            xa[i][0] = __builtin_bit_cast(f32x4_t, buf_load16(r1, in ? e * 4u : kOOB));
            xa[i][1] = __builtin_bit_cast(f32x4_t, buf_load16(r1, in ? e * 4u + 16u : kOOB));
            if constexpr (XM == XM_NORM) {
                const u32x4_t wv = buf_load16(r2, in ? e * 2u : kOOB);  // 8 bf16 weights
                xb[i][0] = __builtin_bit_cast(f32x4_t, wv);
            } else {
                xb[i][0] = __builtin_bit_cast(f32x4_t, buf_load16(r2, in ? e * 4u : kOOB));
                xb[i][1] = __builtin_bit_cast(f32x4_t, buf_load16(r2, in ? e * 4u + 16u : kOOB));
            }
        }
    }

    uint32_t cidx[CPL];
    bool cval[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const uint32_t c = (js * CPL + i) * 64u + lane;
        cval[i] = c < C;
        cidx[i] = c;
    }

    // x chunks (plain GEMV) are loaded before the weights: they come from L2
    // and, since vmcnt completes in issue order, loading them after the
    // weights would hold the x preparation (and every row's arithmetic) until
    // the last weight byte has landed. Issued first, they are ready while the
    // weight stream is still in flight, and row r's arithmetic waits only for
    // the loads of rows 0..r.
    u32x4_t xd[XM == XM_PLAIN ? MR : 1][CPL][XL];
    if constexpr (XM == XM_PLAIN) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int i = 0; i < CPL; ++i)
#pragma unroll
                for (int t = 0; t < XL; ++t)
                    xd[m][i][t] = buf_load16(rx, cval[i] ? (m * K + cidx[i] * E) * 2u + t * 16u : kOOB);
    }

    // Weight loads for all R rows, row by row: they are the HBM stream. Rows
    // past N and chunks past the row read as zero (out-of-range offsets).
    // Weights are read once per launch, so their loads are non-temporal (nt);
    // so are the 4-bit scales/biases (measured faster), while the 8-bit
    // lm_head keeps its scales/biases cached (measured faster that way).
    constexpr int kQAux = 2, kSbAux = BITS == 4 ? 2 : 0;
    u32x4_t qv[R][CPL];
    uint32_t sv[R][CPL], bv[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = row0 + r;
        const bool rv = row < N;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const bool ok = rv && cval[i];
            qv[r][i] = buf_load16_aux<kQAux>(rq, ok ? (row * C + cidx[i]) * 16u : kOOB);
            const uint32_t g = (cidx[i] * E) >> lgG;
            const uint32_t so = ok ? (row * ng + g) * 2u : kOOB;
            sv[r][i] = buf_load_u16_aux<kSbAux>(rs, so);
            bv[r][i] = buf_load_u16_aux<kSbAux>(rb_, so);
        }
    }

    if constexpr (DIAG) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        t_land = __builtin_amdgcn_s_memrealtime();
        __builtin_amdgcn_sched_barrier(0);
    }

    if constexpr (XM != XM_PLAIN) {
        float inv = 0.f;
        if constexpr (XM == XM_NORM) {
            // sum of squares: per-thread, then the wave, then the 4 waves (fixed order)
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < XI; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int e = 0; e < 4; ++e) ss = fmaf(xa[i][h][e], xa[i][h][e], ss);
            ss = wave_sum(ss);
            if (lane == 0) red[wave][0] = ss;
            __syncthreads();
            const float tot = ((red[0][0] + red[1][0]) + red[2][0]) + red[3][0];
            inv = 1.0f / sqrtf(tot / (float)K + eps);
        }
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const uint32_t e = i * 2048u + threadIdx.x * 8u;
            if (e >= K) continue;
            uint32_t o[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t v[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = 2 * p + h;  // element 8t + j
                    const float a = xa[i][j >> 2][j & 3];
                    if constexpr (XM == XM_NORM) {
                        const uint32_t wb = __builtin_bit_cast(u32x4_t, xb[i][0])[j >> 1];
                        v[h] = f32_to_bf16_bits((a * inv) *
                                                bf16_bits_to_f32((wb >> (16 * (j & 1))) & 0xFFFFu));
                    } else {
                        v[h] = silu_mul_bf16(a, xb[i][j >> 2][j & 3]);
                    }
                }
                o[p] = v[0] | (v[1] << 16);
            }
            *reinterpret_cast<u32x4_t*>(&xl[e]) = u32x4_t{o[0], o[1], o[2], o[3]};
        }
        __syncthreads();
    }

    uint32_t xr[MR][CPL][16];
    float xs[MR][CPL];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            u32x4_t d[XL];
#pragma unroll
            for (int t = 0; t < XL; ++t) {
                if constexpr (XM == XM_PLAIN) {
                    d[t] = xd[m][i][t];
                } else {
                    d[t] = cval[i] ? *reinterpret_cast<const u32x4_t*>(&xl[cidx[i] * E + t * 8u])
                                   : u32x4_t{0u, 0u, 0u, 0u};
                }
            }
            prep_x<BITS>(d, xr[m][i], xs[m][i]);
        }
    }

    float acc[RV];
#pragma unroll
    for (int v = 0; v < RV; ++v) acc[v] = 0.f;

    const uint32_t c128 = kBf128;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const float sc = bf16_bits_to_f32(sv[r][i]);
            const float bi = bf16_bits_to_f32(bv[r][i]);
            float d[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) d[m] = 0.f;
            if constexpr (BITS == 4) {
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t v = qv[r][i][w];
                    const uint32_t p0 = and_or(v, kNibMask, c128);
                    const uint32_t p1 = and_or(v >> 4, kNibMask, c128);
                    const uint32_t p2 = and_or(v >> 8, kNibMask, c128);
                    const uint32_t p3 = and_or(v >> 12, kNibMask, c128);
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        d[m] = dot2_bf16(p0, xr[m][i][4 * w + 0], d[m]);
                        d[m] = dot2_bf16(p1, xr[m][i][4 * w + 1], d[m]);
                        d[m] = dot2_bf16(p2, xr[m][i][4 * w + 2], d[m]);
                        d[m] = dot2_bf16(p3, xr[m][i][4 * w + 3], d[m]);
                    }
                }
            } else {
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t v = qv[r][i][w];
                    const float c0 = (float)(v & 0xFFu);
                    const float c1 = (float)((v >> 8) & 0xFFu);
                    const float c2 = (float)((v >> 16) & 0xFFu);
                    const float c3 = (float)(v >> 24);
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        d[m] = fmaf(c0, __uint_as_float(xr[m][i][4 * w + 0]), d[m]);
                        d[m] = fmaf(c1, __uint_as_float(xr[m][i][4 * w + 1]), d[m]);
                        d[m] = fmaf(c2, __uint_as_float(xr[m][i][4 * w + 2]), d[m]);
                        d[m] = fmaf(c3, __uint_as_float(xr[m][i][4 * w + 3]), d[m]);
                    }
                }
            }
            // 4-bit sums carry the +128 offset of the bf16 trick: fold it into the bias.
            const float bx = (BITS == 4) ? fmaf(-128.f, sc, bi) : bi;
#pragma unroll
            for (int m = 0; m < MR; ++m)
                acc[r * MR + m] = fmaf(sc, d[m], fmaf(bx, xs[m][i], acc[r * MR + m]));
        }
    }

    float tot[(RV + 3) / 4];
    wave_reduce<RV>(acc, tot);
    if constexpr (DIAG) {
#pragma unroll
        for (int i = 0; i < (RV + 3) / 4; ++i) asm volatile("" ::"v"(tot[i]));
        __builtin_amdgcn_sched_barrier(0);
        t_math = __builtin_amdgcn_s_memrealtime();
        __builtin_amdgcn_sched_barrier(0);
    }

    // Lane 0 of each 16-lane row that holds a distinct value stores it.
    const uint32_t row16 = lane >> 4;
    const bool lead = (lane & 15u) == 0u &&
                      (RV >= 4 || (RV == 2 ? (row16 & 1u) == 0u : row16 == 0u));
    const bool bf = out_bf16 != 0;
    if (S == 1) {
        (void)x2;
        if (lead) {
#pragma unroll
            for (int i = 0; i < (RV + 3) / 4; ++i) {
                const int v = reduce_value(RV, i, (int)row16);
                if (v < RV0) {
                    const uint32_t row = row0 + v / MR;
                    const uint32_t m = v % MR;
                    if (row < N) store_out(y, (size_t)m * N + row, tot[i], bf);
                }
            }
        }
        if constexpr (DIAG) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            const uint64_t t_out = __builtin_amdgcn_s_memrealtime();
            if (lane == 0) {
                uint64_t* o = stamps + 4u * (blockIdx.x * 4u + (threadIdx.x >> 6));
                o[0] = t_in;
                o[1] = t_land;
                o[2] = t_math;
                o[3] = t_out;
            }
        }
        return;
    }
    if (lead) {
#pragma unroll
        for (int i = 0; i < (RV + 3) / 4; ++i) red[wave][reduce_value(RV, i, (int)row16)] = tot[i];
    }
    __syncthreads();
    if (js == 0 && lane < (uint32_t)RV0) {
        const uint32_t v = lane;
        float t = red[wave][v];
        for (uint32_t j = 1; j < S; ++j) t += red[wave + j][v];
        const uint32_t row = row0 + v / MR;
        if (row < N) store_out(y, (size_t)(v % MR) * N + row, t, bf);
    }
}

template <int BITS, int MR, int R, int CPL>
hipError_t launch_valu(const void* q, const void* s, const void* b, const void* x, void* y,
                       uint32_t N, uint32_t K, uint32_t G, uint32_t S, int out_bf16,
                       hipStream_t st) {
    const uint32_t rows_per_wg = R * (4u / S);
    const uint32_t grid = (N + rows_per_wg - 1) / rows_per_wg;
    hipLaunchKernelGGL((gemv_valu_kernel<BITS, MR, R, CPL>), dim3(grid), dim3(256), 0, st,
                       q, s, b, x, y, N, K, G, S, out_bf16, (const void*)nullptr, 0.f);
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
        // two rows of x: four weight rows per wave from N = 4096 (half the x
        // loads per weight byte; measured M=2 N=8192 4.74 -> 4.28 us, K=8192
        // 5.98 -> 4.86, 8-bit lm_head 65-70 -> 48-54), two below (a grid of
        // half the workgroups was 6-9% slower at N <= 2048)
        case 2:
            return N >= 4096 ? dispatch_cpl<BITS, 2, 4>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st)
                             : dispatch_cpl<BITS, 2, 2>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
        case 3:
            return N >= 4096 ? dispatch_cpl<BITS, 3, 4>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st)
                             : dispatch_cpl<BITS, 3, 2>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
        case 4:
            return N >= 4096 ? dispatch_cpl<BITS, 4, 4>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st)
                             : dispatch_cpl<BITS, 4, 2>(cpl, q, s, b, x, y, N, K, G, S, out_bf16, st);
    }
    return hipErrorInvalidValue;
}


}  // namespace

// Diagnostic GEMV (4-bit, M = 1, K <= 2048 so that S = 1, four rows per
// wave): the headline kernel with per-wave wall-clock stamps. Returns the
// number of waves through *nwaves; stamps must hold 4 * nwaves values.
hipError_t launch_gemv_q4_timeline(const void* q, const void* s, const void* b, const void* x,
                                   void* y, uint32_t N, uint32_t K, uint32_t G, int out_bf16,
                                   uint64_t* stamps, uint32_t cap, uint32_t* nwaves,
                                   hipStream_t st) {
    uint32_t S;
    int cpl;
    gemv_split(4, K, &S, &cpl);
    if (S != 1 || cpl != 1) return hipErrorInvalidValue;
    const uint32_t grid = (N + 15u) / 16u;  // 4 rows x 4 waves per workgroup
    *nwaves = grid * 4u;
    if ((uint64_t)grid * 16u > cap) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_valu_kernel<4, 1, 4, 1, XM_PLAIN, 1>), dim3(grid), dim3(256), 0, st,
                       q, s, b, x, y, N, K, G, S, out_bf16, (const void*)nullptr, 0.f, stamps);
    return hipGetLastError();
}

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
    // rows per wave for M = 1 (MIORI_GEMV_ROWS overrides it for tuning sweeps)
    static const int rows_m1 = tuning_env("MIORI_GEMV_ROWS", 4);
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

// Fused decode ops on the 4-bit GEMV, one activation row: y = W . t(x, x2)
// with t = rmsnorm (xm = 1: x fp32, x2 bf16 norm weight, eps) or silu-mul
// (xm = 2: x = gate fp32, x2 = up fp32). K <= 8192, a multiple of 32.
hipError_t launch_gemv_fused(int xm, const void* q, const void* s, const void* b, const void* x,
                             const void* x2, float eps, void* y, uint32_t N, uint32_t K,
                             uint32_t G, int out_bf16, hipStream_t st) {
    if (K > kXmMaxK || K % 32 != 0) return hipErrorInvalidValue;
    uint32_t S;
    int cpl;
    gemv_split(4, K, &S, &cpl);
    if (cpl != 1) return hipErrorInvalidValue;  // K <= 8192 takes one chunk per lane
    // Every workgroup rebuilds the whole transformed vector, so that work
    // grows with the grid: 8 rows per wave halve the grid once 4 rows would
    // give 512 or more workgroups (N=8192 at K=2048, N=2048 at K=7680);
    // smaller grids keep 4 rows so the weight stream has enough waves.
    // MIORI_FUSED_ROWS=4|8 overrides the choice for tuning sweeps.
    static const int r_env = tuning_env("MIORI_FUSED_ROWS", 0);
    const int R = r_env == 8 || r_env == 4 ? r_env
                  : (N + 4u * (4u / S) - 1) / (4u * (4u / S)) >= 512u ? 8 : 4;
    const uint32_t rows_per_wg = R * (4u / S);
    const dim3 grid((N + rows_per_wg - 1) / rows_per_wg);
    if (xm != XM_NORM && xm != XM_SILU) return hipErrorInvalidValue;
    if (R == 8) {
        if (xm == XM_NORM)
            hipLaunchKernelGGL((gemv_valu_kernel<4, 1, 8, 1, XM_NORM>), grid, dim3(256), 0, st, q,
                               s, b, x, y, N, K, G, S, out_bf16, x2, eps);
        else
            hipLaunchKernelGGL((gemv_valu_kernel<4, 1, 8, 1, XM_SILU>), grid, dim3(256), 0, st, q,
                               s, b, x, y, N, K, G, S, out_bf16, x2, eps);
    } else {
        if (xm == XM_NORM)
            hipLaunchKernelGGL((gemv_valu_kernel<4, 1, 4, 1, XM_NORM>), grid, dim3(256), 0, st, q,
                               s, b, x, y, N, K, G, S, out_bf16, x2, eps);
        else
            hipLaunchKernelGGL((gemv_valu_kernel<4, 1, 4, 1, XM_SILU>), grid, dim3(256), 0, st, q,
                               s, b, x, y, N, K, G, S, out_bf16, x2, eps);
    }
    return hipGetLastError();
}

}  // namespace miori
