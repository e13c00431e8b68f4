// Batched decode GEMV on MFMA for gfx950: y[M][N] = x[M][K] . dequant(W)^T
// for 5 <= M <= 32 activation rows (the fixed-slot batch decode), 4-bit or
// 8-bit MLX-affine W, with the exact affine semantics of the M=1 kernel.
//
// Replaces shaders/batch.metal:145-236 (gemv4_b / gemv8_b), whose per-lane
// fp32 FMAs make the batch "instruction bound" (the reference caps it at 4
// rows). At M >= 8 the VALU cost of M FMAs per weight exceeds the HBM time,
// so the products run on v_mfma_f32_16x16x32_bf16 instead:
//
//  * B operand = the weights. A lane (column j = output row, k-block c) turns
//    its packed codes into bf16 with one AND-OR per pair:
//      4-bit: ((w >> 4i) & 0x000F000F) | 0x43004300 = bf16 pair (128+q, 128+q')
//      8-bit: the same on the low and the high nibble of each byte; the high
//             nibbles go to a second accumulator that is scaled by 16.
//    These bf16 values are exact integers, and x is bf16, so the MFMA
//    products are exact and only fp32 sums round.
//  * A operand = x rows (M padded to 16 or 32), pair-permuted to match.
//  * Each quantisation group is accumulated separately (D_g), together with
//    X_g = sum of x over the group (an MFMA against a constant-one B), and
//    folded into the fp32 result as  acc += s*D_g + (b - 128*s)*X_g
//    (8-bit: s*(D_lo + 16*D_hi) + (b - 2176*s)*X_g). This is the same
//    factorisation as the VALU kernel, so the dequantised weights are never
//    rounded to bf16.
//  * A workgroup = 4 waves on the same NT x 16 output rows, splitting the
//    groups of K four ways; the per-wave accumulators are added through LDS
//    in a fixed order.
#include "common.hpp"
#include "kernels.hpp"

namespace miori {

namespace {

template <int WPL>
struct Words { uint32_t w[WPL]; };

template <int WPL>
__device__ __forceinline__ Words<WPL> load_words(const uint32_t* p) {
    Words<WPL> r;
    if constexpr (WPL == 1) {
        r.w[0] = *p;
    } else if constexpr (WPL == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        r.w[0] = v.x; r.w[1] = v.y;
    } else {
#pragma unroll
        for (int h = 0; h < WPL / 4; ++h) {
            const uint4 v = *reinterpret_cast<const uint4*>(p + 4 * h);
            r.w[4 * h] = v.x; r.w[4 * h + 1] = v.y; r.w[4 * h + 2] = v.z; r.w[4 * h + 3] = v.w;
        }
    }
    return r;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4_t v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8_t, v);
}

// 8 consecutive bf16 x values starting at k0 (16-byte aligned), as the A
// fragment for one 4-bit word: slots (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ bf16x8_t x_frag4(const uint4 d) {
    return as_bf16x8((d.x & 0xFFFFu) | (d.z << 16), (d.x >> 16) | (d.z & 0xFFFF0000u),
                     (d.y & 0xFFFFu) | (d.w << 16), (d.y >> 16) | (d.w & 0xFFFF0000u));
}

// ... and for two 8-bit words: slots (x0,x2) (x1,x3) (x4,x6) (x5,x7).
__device__ __forceinline__ bf16x8_t x_frag8(const uint4 d) {
    return as_bf16x8((d.x & 0xFFFFu) | (d.y << 16), (d.x >> 16) | (d.y & 0xFFFF0000u),
                     (d.z & 0xFFFFu) | (d.w << 16), (d.z >> 16) | (d.w & 0xFFFF0000u));
}

__device__ __forceinline__ uint32_t nib_pair(uint32_t v, int sh) {
    return ((v >> sh) & 0x000F000Fu) | 0x43004300u;
}

// B fragment of a 4-bit word: pairs (q_i, q_{i+4}), i = 0..3.
__device__ __forceinline__ bf16x8_t w_frag4(uint32_t v) {
    return as_bf16x8(nib_pair(v, 0), nib_pair(v, 4), nib_pair(v, 8), nib_pair(v, 12));
}

// B fragments of two 8-bit words (codes c0..c7): low nibbles and high
// nibbles, slots (c0,c2) (c1,c3) (c4,c6) (c5,c7).
__device__ __forceinline__ bf16x8_t w_frag8_lo(uint32_t v0, uint32_t v1) {
    return as_bf16x8(nib_pair(v0, 0), nib_pair(v0, 8), nib_pair(v1, 0), nib_pair(v1, 8));
}
__device__ __forceinline__ bf16x8_t w_frag8_hi(uint32_t v0, uint32_t v1) {
    return as_bf16x8(nib_pair(v0, 4), nib_pair(v0, 12), nib_pair(v1, 4), nib_pair(v1, 12));
}

__device__ __forceinline__ f32x4_t mfma(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// WPL = 32-bit words of one row-group held by one lane (4 lanes per row).
template <int BITS, int MT, int NT, int WPL>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(
    const uint32_t* __restrict__ q, const uint16_t* __restrict__ s,
    const uint16_t* __restrict__ bs, const uint16_t* __restrict__ x,
    void* __restrict__ y, uint32_t M, uint32_t N, uint32_t K, int out_bf16) {
    constexpr uint32_t G = (BITS == 4) ? WPL * 32u : WPL * 16u;
    constexpr int NA = (BITS == 4) ? WPL : WPL / 2;   // A fragments per group
    __shared__ float red[4][NT * MT * 4 * 64];

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t j = lane & 15u, c = lane >> 4;
    const uint32_t n_base = blockIdx.x * (16u * NT);
    const uint32_t ng = K / G;
    const uint32_t wpr = K * BITS / 32u;           // words per weight row
    const uint32_t g0 = ng * wave / 4u, g1 = ng * (wave + 1u) / 4u;

    uint32_t nrow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) nrow[t] = min(n_base + t * 16u + j, N - 1u);
    bool mval[MT];
    uint32_t mrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        mval[mt] = mt * 16u + j < M;
        mrow[mt] = mval[mt] ? mt * 16u + j : 0u;
    }

    f32x4_t acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const bf16x8_t ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);

    for (uint32_t g = g0; g < g1; ++g) {
        Words<WPL> wv[NT];
        uint32_t sv[NT], bv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            wv[t] = load_words<WPL>(q + (size_t)nrow[t] * wpr + g * (G * BITS / 32u) + c * WPL);
            sv[t] = s[(size_t)nrow[t] * ng + g];
            bv[t] = bs[(size_t)nrow[t] * ng + g];
        }
        bf16x8_t af[MT][NA];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                // 4-bit: fragment a covers word c*WPL + a (8 codes);
                // 8-bit: words c*WPL + 2a, +1 (8 codes).
                const uint32_t k0 = g * G + (BITS == 4 ? (c * WPL + a) * 8u : (c * WPL + 2 * a) * 4u);
                uint4 d = make_uint4(0u, 0u, 0u, 0u);
                if (mval[mt]) d = *reinterpret_cast<const uint4*>(x + (size_t)mrow[mt] * K + k0);
                af[mt][a] = (BITS == 4) ? x_frag4(d) : x_frag8(d);
            }
        }
        f32x4_t dx[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            dx[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int a = 0; a < NA; ++a) dx[mt] = mfma(af[mt][a], ones, dx[mt]);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float sc = bf16_bits_to_f32(sv[t]);
            const float bi = bf16_bits_to_f32(bv[t]);
            f32x4_t d[MT], dh[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                d[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                dh[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                if constexpr (BITS == 4) {
                    const bf16x8_t bf = w_frag4(wv[t].w[a]);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) d[mt] = mfma(af[mt][a], bf, d[mt]);
                } else {
                    const bf16x8_t blo = w_frag8_lo(wv[t].w[2 * a], wv[t].w[2 * a + 1]);
                    const bf16x8_t bhi = w_frag8_hi(wv[t].w[2 * a], wv[t].w[2 * a + 1]);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        d[mt] = mfma(af[mt][a], blo, d[mt]);
                        dh[mt] = mfma(af[mt][a], bhi, dh[mt]);
                    }
                }
            }
            const float bx = (BITS == 4) ? fmaf(-128.f, sc, bi) : fmaf(-2176.f, sc, bi);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float dd = (BITS == 4) ? d[mt][r] : fmaf(16.f, dh[mt][r], d[mt][r]);
                    acc[t][mt][r] = fmaf(sc, dd, fmaf(bx, dx[mt][r], acc[t][mt][r]));
                }
            }
        }
    }

    // Cross-wave reduction in a fixed order, then the store. Element
    // e = ((t*MT + mt)*4 + r)*64 + lane of the accumulators is output row
    // n_base + t*16 + lane%16, activation row mt*16 + 4*(lane/16) + r.
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][((t * MT + mt) * 4 + r) * 64 + lane] = acc[t][mt][r];
    __syncthreads();
    const bool bf = out_bf16 != 0;
    constexpr int TOT = NT * MT * 4 * 64;
    for (int e = threadIdx.x; e < TOT; e += 256) {
        const float v = ((red[0][e] + red[1][e]) + red[2][e]) + red[3][e];
        const uint32_t ln = e & 63u, r = (e >> 6) & 3u, tm = e >> 8;
        const uint32_t t = tm / MT, mt = tm % MT;
        const uint32_t n = n_base + t * 16u + (ln & 15u);
        const uint32_t m = mt * 16u + 4u * (ln >> 4) + r;
        if (n < N && m < M) store_out(y, (size_t)m * N + n, v, bf);
    }
}

template <int BITS, int MT, int NT, int WPL>
hipError_t launch_one(const void* q, const void* s, const void* b, const void* x, void* y,
                      uint32_t M, uint32_t N, uint32_t K, int out_bf16, hipStream_t st) {
    const uint32_t grid = (N + 16u * NT - 1) / (16u * NT);
    hipLaunchKernelGGL((gemv_mfma_kernel<BITS, MT, NT, WPL>), dim3(grid), dim3(256), 0, st,
                       (const uint32_t*)q, (const uint16_t*)s, (const uint16_t*)b,
                       (const uint16_t*)x, y, M, N, K, out_bf16);
    return hipGetLastError();
}

template <int BITS, int MT, int NT>
hipError_t by_group(uint32_t G, const void* q, const void* s, const void* b, const void* x,
                    void* y, uint32_t M, uint32_t N, uint32_t K, int out_bf16, hipStream_t st) {
    if constexpr (BITS == 4) {
        switch (G) {
            case 32: return launch_one<4, MT, NT, 1>(q, s, b, x, y, M, N, K, out_bf16, st);
            case 64: return launch_one<4, MT, NT, 2>(q, s, b, x, y, M, N, K, out_bf16, st);
            case 128: return launch_one<4, MT, NT, 4>(q, s, b, x, y, M, N, K, out_bf16, st);
        }
    } else {
        switch (G) {
            case 32: return launch_one<8, MT, NT, 2>(q, s, b, x, y, M, N, K, out_bf16, st);
            case 64: return launch_one<8, MT, NT, 4>(q, s, b, x, y, M, N, K, out_bf16, st);
            case 128: return launch_one<8, MT, NT, 8>(q, s, b, x, y, M, N, K, out_bf16, st);
        }
    }
    return hipErrorInvalidValue;
}

template <int BITS, int MT>
hipError_t by_nt(int nt, uint32_t G, const void* q, const void* s, const void* b,
                 const void* x, void* y, uint32_t M, uint32_t N, uint32_t K, int out_bf16,
                 hipStream_t st) {
    switch (nt) {
        case 1: return by_group<BITS, MT, 1>(G, q, s, b, x, y, M, N, K, out_bf16, st);
        case 2: return by_group<BITS, MT, 2>(G, q, s, b, x, y, M, N, K, out_bf16, st);
        default: return by_group<BITS, MT, 4>(G, q, s, b, x, y, M, N, K, out_bf16, st);
    }
}

}  // namespace

bool gemv_mfma_supported(int bits, uint32_t M, uint32_t K, uint32_t G) {
    if (M == 0 || M > 32) return false;
    if (!(G == 32 || G == 64 || G == 128) || K % G) return false;
    return K / G >= 4;  // every wave of the workgroup gets a group
}

hipError_t launch_gemv_mfma(int bits, const void* q, const void* s, const void* b,
                            const void* x, void* y, uint32_t M, uint32_t N, uint32_t K,
                            uint32_t G, int out_bf16, hipStream_t st) {
    // Output rows per workgroup: enough workgroups to cover the 256 CUs.
    int nt = 1;
    if ((N + 63) / 64 >= 256) nt = 4;
    else if ((N + 31) / 32 >= 256) nt = 2;
    if (const char* e = getenv("MIORI_MFMA_NT")) nt = atoi(e);
    if (bits == 4)
        return M <= 16 ? by_nt<4, 1>(nt, G, q, s, b, x, y, M, N, K, out_bf16, st)
                       : by_nt<4, 2>(nt, G, q, s, b, x, y, M, N, K, out_bf16, st);
    return M <= 16 ? by_nt<8, 1>(nt, G, q, s, b, x, y, M, N, K, out_bf16, st)
                   : by_nt<8, 2>(nt, G, q, s, b, x, y, M, N, K, out_bf16, st);
}

}  // namespace miori
