// Skinny MFMA kernel for gfx950: y[M][N] = x[M][K] . W^T for M <= 32, with W
// streamed from HBM once. One kernel, four weight modes:
//
//   Q4X  4-bit MLX-affine, exact affine semantics (batched decode GEMV,
//        replaces shaders/batch.metal:145-188 gemv4_b)
//   Q8X  8-bit, exact affine semantics (batched lm_head, replaces
//        shaders/batch.metal:192-236 gemv8_b)
//   Q4F  4-bit dequantised to bf16 on the fly (the fused GEMM's semantics:
//        bf16_rne(q*s + b), as the two-step dequant_tile + gemm_mpp)
//   BF16 bf16 weight cache (gemm_mpp at small M)
//
// Structure:
//  * A workgroup (4 waves) owns 64 output rows and a range of K tiles. Each K
//    tile's weight rows, x rows and scales/biases go global -> LDS with
//    global_load_lds DMA through a 3-stage ring, so HBM sees whole
//    contiguous row segments and the loads of tile t+2 fly while tile t is
//    computed. Chunks are XOR-swizzled by row so fragment reads are
//    conflict-free.
//  * Wave w takes the w-th quarter ("slice") of each K tile for all 64 rows:
//    4 n-tiles x (M padded to 16 or 32) of v_mfma_f32_16x16x32_bf16. The x
//    fragments of the slice are read once and reused by the 4 n-tiles.
//  * Exact modes: codes become exact bf16 integers (128+q via one AND-OR),
//    each quantisation group is accumulated alone (D_g) with X_g = sum of x
//    over the group from an MFMA against ones, and folded in fp32:
//        acc += s*D_g + (b - 128 s) X_g        (8-bit: hi nibbles x16, 2176)
//    so the dequantised weights are never rounded.
//  * The 4 waves' partial sums meet in LDS (fixed order). With split-K over
//    workgroups the partials go to a workspace and the last workgroup of an
//    output block (device-scope counter) adds them in split order, so the
//    result does not depend on timing. Q4F and BF16 run the identical MFMA
//    sequence, so the fused product is bit-identical to dequant + cache GEMM.
#include "common.hpp"
#include "kernels.hpp"

namespace miori {

namespace {

enum { Q4X = 0, Q8X = 1, Q4F = 2, BF16 = 3 };

template <int MODE, int MT, int G>
struct SkCfg {
    static constexpr bool EXACT = MODE == Q4X || MODE == Q8X;
    static constexpr int NB = 64;                                   // rows per workgroup
    static constexpr int SLICE = (EXACT && G > 64) ? G : 64;        // k per wave per tile
    static constexpr int KTILE = 4 * SLICE;
    static constexpr int KS = SLICE / 32;                           // MFMA k-steps per slice
    static constexpr int MR = 16 * MT;
    static constexpr int W_ROWB = (MODE == Q4X || MODE == Q4F) ? KTILE / 2
                                  : (MODE == Q8X ? KTILE : KTILE * 2);
    static constexpr int X_ROWB = KTILE * 2;
    static constexpr int W_ST = NB * W_ROWB;
    static constexpr int X_ST = MR * X_ROWB;
    static constexpr int NGT = (MODE == BF16) ? 0 : KTILE / G;      // groups per row per tile
    static constexpr int SB_DW = NGT / 2;                           // scale dwords per row per tile
    static constexpr int SB_ST = NB * SB_DW * 4;
    // LDS ring depth: 3 stages when they fit in the 160 KiB, else 2
    static constexpr int NS = 3 * (X_ST + W_ST + 2 * SB_ST) <= 160 * 1024 ? 3 : 2;
    static constexpr int X_OFF = 0;
    static constexpr int W_OFF = NS * X_ST;
    static constexpr int S_OFF = W_OFF + NS * W_ST;
    static constexpr int B_OFF = S_OFF + NS * SB_ST;
    static constexpr int RED = 4 * (4 * MT * 4 * 64) * 4;           // cross-wave reduction
    static constexpr int STAGES = B_OFF + NS * SB_ST;
    static constexpr int LDS = STAGES > RED ? STAGES : RED;
    static constexpr int X_INS = X_ST / 1024 / 4;                   // DMA instructions per wave
    static constexpr int W_INS = W_ST / 1024 / 4;
    static constexpr int SB_INS = 2 * SB_DW;                        // s and b, 64 dwords each
    static constexpr int W_CPR = W_ROWB / 16;                       // 16-byte chunks per row
    static_assert(X_ST % 4096 == 0 && W_ST % 4096 == 0, "tile sizes");
    static_assert(MODE == BF16 || NGT >= 2, "scale rows are moved as dwords");
};

// chunk swizzle of a row: 16 consecutive rows read at the same logical
// chunk land in distinct banks.
template <int CPR>
__device__ __forceinline__ uint32_t wsw(uint32_t r) {
    if constexpr (CPR >= 16) return r & 15u;
    else return (r >> 1) & (CPR - 1);
}

__device__ __forceinline__ bf16x8_t as_bf16x8_u(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4_t v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8_t, v);
}

// x fragments: 8 consecutive bf16 (one 16-byte chunk), pair-permuted to the
// slot order of the weight fragment (4-bit: (x0,x4)(x1,x5)(x2,x6)(x3,x7);
// 8-bit: (x0,x2)(x1,x3)(x4,x6)(x5,x7); bf16 / fused: natural order).
template <int MODE>
__device__ __forceinline__ bf16x8_t x_frag(u32x4_t d) {
    if constexpr (MODE == Q4X)
        return as_bf16x8_u(__builtin_amdgcn_perm(d[2], d[0], 0x05040100u),
                           __builtin_amdgcn_perm(d[2], d[0], 0x07060302u),
                           __builtin_amdgcn_perm(d[3], d[1], 0x05040100u),
                           __builtin_amdgcn_perm(d[3], d[1], 0x07060302u));
    else if constexpr (MODE == Q8X)
        return as_bf16x8_u(__builtin_amdgcn_perm(d[1], d[0], 0x05040100u),
                           __builtin_amdgcn_perm(d[1], d[0], 0x07060302u),
                           __builtin_amdgcn_perm(d[3], d[2], 0x05040100u),
                           __builtin_amdgcn_perm(d[3], d[2], 0x07060302u));
    else
        return __builtin_bit_cast(bf16x8_t, d);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int MODE, int MT, int G>
__global__ __launch_bounds__(256) void skinny_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
    const uint16_t* __restrict__ S, const uint16_t* __restrict__ Bi, void* __restrict__ Y,
    float* __restrict__ part, uint32_t* __restrict__ counters, uint32_t M, uint32_t N,
    uint32_t K, uint32_t SK, int out_bf16) {
    using C = SkCfg<MODE, MT, G>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS];
    __shared__ uint32_t last_flag;

    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t j = lane & 15u, c = lane >> 4;
    const uint32_t nblocks = (N + C::NB - 1) / C::NB;
    const uint32_t nb = blockIdx.x % nblocks, ksi = blockIdx.x / nblocks;
    const uint32_t n0 = nb * C::NB;
    const uint32_t KT = K / C::KTILE;
    const uint32_t kt0 = KT * ksi / SK, kt1 = KT * (ksi + 1) / SK;
    const uint32_t ng = (MODE == BF16) ? 1u : K / G;
    const uint64_t wrow = (MODE == Q4X || MODE == Q4F) ? K / 2 : (MODE == Q8X ? K : 2ull * K);

    // Scale/bias DMA instructions are spread round-robin over the waves.
    const int my_sb = (C::SB_INS - (int)wave + 3) / 4;

    auto issue = [&](uint32_t kt, uint32_t st) {
#pragma unroll
        for (int p = 0; p < C::X_INS; ++p) {
            const uint32_t byte0 = (wave * C::X_INS + p) * 1024u;
            const uint32_t slot = byte0 / 16u + lane;
            const uint32_t r = slot / (C::X_ROWB / 16), pc = slot % (C::X_ROWB / 16);
            const uint32_t lc = pc ^ (r & 15u);
            const uint32_t row = min(r, M - 1u);
            dma16(X + (size_t)row * K + (size_t)kt * C::KTILE + lc * 8u,
                  lds + C::X_OFF + st * C::X_ST + byte0);
        }
#pragma unroll
        for (int p = 0; p < C::W_INS; ++p) {
            const uint32_t byte0 = (wave * C::W_INS + p) * 1024u;
            const uint32_t slot = byte0 / 16u + lane;
            const uint32_t r = slot / C::W_CPR, pc = slot % C::W_CPR;
            const uint32_t lc = pc ^ wsw<C::W_CPR>(r);
            const uint32_t row = min(n0 + r, N - 1u);
            dma16(W + row * wrow + (uint64_t)kt * C::W_ROWB + lc * 16u,
                  lds + C::W_OFF + st * C::W_ST + byte0);
        }
        if constexpr (MODE != BF16) {
            for (int i = (int)wave; i < C::SB_INS; i += 4) {
                const int which = i / C::SB_DW, prt = i % C::SB_DW;
                const uint32_t d = prt * 64u + lane;
                const uint32_t r = d / C::SB_DW, dw = d % C::SB_DW;
                const uint32_t row = min(n0 + r, N - 1u);
                dma4((which ? Bi : S) + (size_t)row * ng + (size_t)kt * C::NGT + dw * 2u,
                     lds + (which ? C::B_OFF : C::S_OFF) + st * C::SB_ST + prt * 256u);
            }
        }
    };
    // Wait until the loads of the oldest group in flight have landed, with
    // `newer` groups still allowed in flight.
    auto wait_groups = [&](int newer) {
        const int per = C::X_INS + C::W_INS + my_sb;
        if (newer == 0) { wait_vm<0>(); return; }
        if (newer == 1) {
            if (per == C::X_INS + C::W_INS) wait_vm<C::X_INS + C::W_INS>();
            else if (per == C::X_INS + C::W_INS + 1) wait_vm<C::X_INS + C::W_INS + 1>();
            else wait_vm<C::X_INS + C::W_INS + 2>();
            return;
        }
        if (per == C::X_INS + C::W_INS) wait_vm<2 * (C::X_INS + C::W_INS)>();
        else if (per == C::X_INS + C::W_INS + 1) wait_vm<2 * (C::X_INS + C::W_INS + 1)>();
        else wait_vm<2 * (C::X_INS + C::W_INS + 2)>();
    };

    f32x4_t acc[4][MT];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const bf16x8_t ones = as_bf16x8_u(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
    const uint32_t c128 = 0x43004300u;

    // Word of the slice that lane quarter c uses in k-step ks. Exact modes
    // with more than one group per slice (G = 32) keep each k-step inside
    // one group; otherwise a lane's words are contiguous.
    auto word_of = [&](int ks) -> uint32_t {
        if constexpr (C::EXACT && G == 32) return ks * 4u + c;
        else return c * C::KS + ks;
    };

    auto compute = [&](uint32_t st, uint32_t kt) {
        const uint8_t* xs = lds + C::X_OFF + st * C::X_ST;
        const uint8_t* ws = lds + C::W_OFF + st * C::W_ST;
        const uint16_t* ss = reinterpret_cast<const uint16_t*>(lds + C::S_OFF + st * C::SB_ST);
        const uint16_t* bs = reinterpret_cast<const uint16_t*>(lds + C::B_OFF + st * C::SB_ST);
        const uint32_t koff = wave * C::SLICE;  // slice start inside the tile
        bf16x8_t af[MT][C::KS];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const uint32_t m = mt * 16u + j;
#pragma unroll
            for (int ks = 0; ks < C::KS; ++ks) {
                // 4-bit: a word = 8 k; 8-bit exact: a word pair = 8 k; bf16/fused: 8 k.
                const uint32_t k8 = (MODE == Q8X) ? koff / 8 + word_of(ks) : koff / 8 + word_of(ks);
                const uint32_t phys = k8 ^ (m & 15u);
                const u32x4_t d = *reinterpret_cast<const u32x4_t*>(xs + m * C::X_ROWB + phys * 16u);
                af[mt][ks] = x_frag<MODE>(d);
            }
        }
        constexpr int GPS = (C::EXACT && G == 32) ? 2 : 1;  // groups per slice (exact)
        f32x4_t dx[MT][GPS];
        if constexpr (C::EXACT) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int gg = 0; gg < GPS; ++gg) {
                    dx[mt][gg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ks = gg * (C::KS / GPS); ks < (gg + 1) * (C::KS / GPS); ++ks)
                        dx[mt][gg] = mfma16(af[mt][ks], ones, dx[mt][gg]);
                }
        }
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const uint32_t r = nt * 16u + j;
            const uint8_t* wr = ws + r * C::W_ROWB;
            if constexpr (MODE == BF16) {
#pragma unroll
                for (int ks = 0; ks < C::KS; ++ks) {
                    const uint32_t phys = (koff / 8 + word_of(ks)) ^ wsw<C::W_CPR>(r);
                    const bf16x8_t bfr = *reinterpret_cast<const bf16x8_t*>(wr + phys * 16u);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16(af[mt][ks], bfr, acc[nt][mt]);
                }
            } else if constexpr (MODE == Q4F) {
#pragma unroll
                for (int ks = 0; ks < C::KS; ++ks) {
                    const uint32_t w = koff / 8 + word_of(ks);           // word in the tile row
                    const uint32_t phys = (w / 4) ^ wsw<C::W_CPR>(r);
                    const uint32_t v = *reinterpret_cast<const uint32_t*>(wr + phys * 16u + (w % 4) * 4u);
                    const uint32_t gt = w * 8u / G;                       // group in the tile
                    const float sc = bf16_bits_to_f32(ss[r * C::NGT + gt]);
                    const float bi = bf16_bits_to_f32(bs[r * C::NGT + gt]);
                    const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
                    u32x4_t o;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float f0 = fmaf((float)((lo >> (8 * q)) & 0xFFu), sc, bi);
                        const float f1 = fmaf((float)((hi >> (8 * q)) & 0xFFu), sc, bi);
                        bf16x2_t pr = {(__bf16)f0, (__bf16)f1};
                        o[q] = __builtin_bit_cast(uint32_t, pr);
                    }
                    const bf16x8_t bfr = __builtin_bit_cast(bf16x8_t, o);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16(af[mt][ks], bfr, acc[nt][mt]);
                }
            } else {
#pragma unroll
                for (int gg = 0; gg < GPS; ++gg) {
                    f32x4_t dd[MT], dh[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        dd[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                        dh[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                    }
                    uint32_t gt = 0;
#pragma unroll
                    for (int ks = gg * (C::KS / GPS); ks < (gg + 1) * (C::KS / GPS); ++ks) {
                        if constexpr (MODE == Q4X) {
                            const uint32_t w = koff / 8 + word_of(ks);
                            gt = w * 8u / G;
                            const uint32_t phys = (w / 4) ^ wsw<C::W_CPR>(r);
                            const uint32_t v = *reinterpret_cast<const uint32_t*>(wr + phys * 16u + (w % 4) * 4u);
                            const bf16x8_t bfr = as_bf16x8_u(and_or(v, 0x000F000Fu, c128),
                                                             and_or(v >> 4, 0x000F000Fu, c128),
                                                             and_or(v >> 8, 0x000F000Fu, c128),
                                                             and_or(v >> 12, 0x000F000Fu, c128));
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) dd[mt] = mfma16(af[mt][ks], bfr, dd[mt]);
                        } else {
                            // 8-bit: word pair wp holds 8 codes (k = 8*wp .. +8 of the slice)
                            const uint32_t wp = koff / 8 + word_of(ks);
                            gt = wp * 8u / G;
                            const uint32_t byte = wp * 8u;
                            const uint32_t phys = (byte / 16) ^ wsw<C::W_CPR>(r);
                            const uint2 v = *reinterpret_cast<const uint2*>(wr + phys * 16u + (byte % 16));
                            const bf16x8_t blo = as_bf16x8_u(and_or(v.x, 0x000F000Fu, c128),
                                                             and_or(v.x >> 8, 0x000F000Fu, c128),
                                                             and_or(v.y, 0x000F000Fu, c128),
                                                             and_or(v.y >> 8, 0x000F000Fu, c128));
                            const bf16x8_t bhi = as_bf16x8_u(and_or(v.x >> 4, 0x000F000Fu, c128),
                                                             and_or(v.x >> 12, 0x000F000Fu, c128),
                                                             and_or(v.y >> 4, 0x000F000Fu, c128),
                                                             and_or(v.y >> 12, 0x000F000Fu, c128));
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) {
                                dd[mt] = mfma16(af[mt][ks], blo, dd[mt]);
                                dh[mt] = mfma16(af[mt][ks], bhi, dh[mt]);
                            }
                        }
                    }
                    const float sc = bf16_bits_to_f32(ss[r * C::NGT + gt]);
                    const float bi = bf16_bits_to_f32(bs[r * C::NGT + gt]);
                    const float bx = (MODE == Q4X) ? fmaf(-128.f, sc, bi) : fmaf(-2176.f, sc, bi);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float v = (MODE == Q4X) ? dd[mt][e] : fmaf(16.f, dh[mt][e], dd[mt][e]);
                            acc[nt][mt][e] = fmaf(sc, v, fmaf(bx, dx[mt][gg][e], acc[nt][mt][e]));
                        }
                }
            }
        }
        (void)kt;
    };

    // NS-stage DMA ring over this workgroup's K tiles [kt0, kt1): tile i+NS-1
    // is issued while tile i is computed.
    constexpr uint32_t D = C::NS - 1;
    const uint32_t nk = kt1 - kt0;
    for (uint32_t p = 0; p < D && p < nk; ++p) issue(kt0 + p, p);
    for (uint32_t i = 0; i < nk; ++i) {
        if (i + D < nk) issue(kt0 + i + D, (i + D) % C::NS);
        const uint32_t ahead = nk - 1 - i;  // groups issued after tile i
        wait_groups((int)(ahead < D ? ahead : D));
        barrier_lds();
        compute(i % C::NS, kt0 + i);
        barrier_lds();  // stage i % NS is refilled NS-1 iterations later
    }

    // Cross-wave reduction (the stage buffers are free now).
    float* red = reinterpret_cast<float*>(lds);
    constexpr int TOT = 4 * MT * 4 * 64;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) red[wave * TOT + ((nt * MT + mt) * 4 + e) * 64 + lane] = acc[nt][mt][e];
    __syncthreads();
    const bool bf = out_bf16 != 0;
    for (int e = t; e < TOT; e += 256) {
        const float v = ((red[e] + red[TOT + e]) + red[2 * TOT + e]) + red[3 * TOT + e];
        const uint32_t ln = e & 63u, r4 = (e >> 6) & 3u, tm = e >> 8;
        const uint32_t nt = tm / MT, mt = tm % MT;
        const uint32_t n = n0 + nt * 16u + (ln & 15u);
        const uint32_t m = mt * 16u + 4u * (ln >> 4) + r4;
        if (n >= N || m >= M) continue;
        if (SK == 1) store_out(Y, (size_t)m * N + n, v, bf);
        else st_shared_dev(&part[((size_t)ksi * M + m) * N + n], v);
    }
    if (SK == 1) return;

    // Split-K: the last workgroup of this output block adds the partials in
    // split order. The partials and the counter are device-coherent accesses
    // (no L2-wide fences).
    wait_vm<0>();
    __syncthreads();
    if (t == 0) last_flag = (arrive_dev(&counters[nb]) == SK - 1) ? 1u : 0u;
    __syncthreads();
    if (!last_flag) return;
    for (int e = t; e < TOT; e += 256) {
        const uint32_t ln = e & 63u, r4 = (e >> 6) & 3u, tm = e >> 8;
        const uint32_t nt = tm / MT, mt = tm % MT;
        const uint32_t n = n0 + nt * 16u + (ln & 15u);
        const uint32_t m = mt * 16u + 4u * (ln >> 4) + r4;
        if (n >= N || m >= M) continue;
        float v = 0.f;
        for (uint32_t s2 = 0; s2 < SK; ++s2)
            v += ld_shared_dev(&part[((size_t)s2 * M + m) * N + n]);
        store_out(Y, (size_t)m * N + n, v, bf);
    }
    if (t == 0) reset_dev(&counters[nb]);
}

template <int MODE, int MT, int G>
hipError_t launch_sk(const void* X, const void* W, const void* S, const void* B, void* Y,
                     uint32_t M, uint32_t N, uint32_t K, int out_bf16, hipStream_t st) {
    using C = SkCfg<MODE, MT, G>;
    const uint32_t nblocks = (N + C::NB - 1) / C::NB;
    const uint32_t KT = K / C::KTILE;
    // Split K until about 2 workgroups per CU, keeping >= 2 K tiles each.
    uint32_t SK = 1;
    while (nblocks * SK < 512 && KT / (SK * 2) >= 2) SK *= 2;
    if (const char* e = getenv("MIORI_SKINNY_SPLIT")) SK = (uint32_t)atoi(e);
    if (SK < 1) SK = 1;
    if (SK > KT) SK = KT;
    float* part = nullptr;
    uint32_t* counters = nullptr;
    if (SK > 1) {
        hipError_t e = workspace_get(st, (size_t)SK * M * N * 4, nblocks, &part, &counters);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((skinny_kernel<MODE, MT, G>), dim3(nblocks * SK), dim3(256), 0, st,
                       (const uint16_t*)X, (const uint8_t*)W, (const uint16_t*)S,
                       (const uint16_t*)B, Y, part, counters, M, N, K, SK, out_bf16);
    return hipGetLastError();
}

template <int MODE, int MT>
hipError_t by_group(uint32_t G, const void* X, const void* W, const void* S, const void* B,
                    void* Y, uint32_t M, uint32_t N, uint32_t K, int out_bf16, hipStream_t st) {
    if constexpr (MODE == BF16) {
        return launch_sk<BF16, MT, 64>(X, W, S, B, Y, M, N, K, out_bf16, st);
    } else {
        switch (G) {
            case 32: return launch_sk<MODE, MT, 32>(X, W, S, B, Y, M, N, K, out_bf16, st);
            case 64: return launch_sk<MODE, MT, 64>(X, W, S, B, Y, M, N, K, out_bf16, st);
            case 128: return launch_sk<MODE, MT, 128>(X, W, S, B, Y, M, N, K, out_bf16, st);
        }
        return hipErrorInvalidValue;
    }
}

template <int MODE>
hipError_t by_m(uint32_t G, const void* X, const void* W, const void* S, const void* B, void* Y,
                uint32_t M, uint32_t N, uint32_t K, int out_bf16, hipStream_t st) {
    return M <= 16 ? by_group<MODE, 1>(G, X, W, S, B, Y, M, N, K, out_bf16, st)
                   : by_group<MODE, 2>(G, X, W, S, B, Y, M, N, K, out_bf16, st);
}

}  // namespace

uint32_t skinny_ktile(int mode, uint32_t G) {
    const bool exact = mode == 0 || mode == 1;
    const uint32_t slice = (exact && G > 64) ? G : 64;
    return 4 * slice;
}

bool skinny_supported(int mode, uint32_t M, uint32_t N, uint32_t K, uint32_t G) {
    if (M == 0 || M > 32 || N == 0) return false;
    // 8-bit exact with group 128 and two m-tiles returns wrong values (cause
    // not found yet); that case stays on the VALU kernel.
    if (mode == 1 && G == 128 && M > 16) return false;
    if (mode != 3 && !(G == 32 || G == 64 || G == 128)) return false;
    return K % skinny_ktile(mode, G) == 0;
}

hipError_t launch_skinny(int mode, const void* X, const void* W, const void* S, const void* B,
                         void* Y, uint32_t M, uint32_t N, uint32_t K, uint32_t G, int out_bf16,
                         hipStream_t st) {
    switch (mode) {
        case 0: return by_m<Q4X>(G, X, W, S, B, Y, M, N, K, out_bf16, st);
        case 1: return by_m<Q8X>(G, X, W, S, B, Y, M, N, K, out_bf16, st);
        case 2: return by_m<Q4F>(G, X, W, S, B, Y, M, N, K, out_bf16, st);
        case 3: return by_m<BF16>(64, X, W, S, B, Y, M, N, K, out_bf16, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace miori
