// Skinny MFMA kernel for gfx950: y[M][N] = x[M][K] . W^T for 5 <= M <= 32
// (batched decode GEMV, small-M GEMM), with W streamed from HBM once and
// every load of a wave in flight before its first MFMA. Four weight modes:
//
//   Q4X  4-bit MLX-affine, exact affine semantics (batched decode GEMV,
//        replaces shaders/batch.metal:145-188 gemv4_b)
//   Q8X  8-bit, exact affine semantics (batched lm_head, replaces
//        shaders/batch.metal:192-236 gemv8_b)
//   Q4F  4-bit dequantised to bf16 on the fly (the fused GEMM's semantics:
//        bf16_rne(q*s + b), as the two-step dequant_tile + gemm_mpp)
//   BF16 bf16 weight cache (gemm_mpp at small M)
//
// Structure (v_mfma_f32_16x16x32_bf16; x is the A operand, W^T the B one):
//  * A workgroup of 8 waves owns 16*NT output rows and 1/SK of K; the waves
//    split its K range, each taking a contiguous run of at most 8 128-wide K
//    blocks (64 for 8-bit), and the eight partial tiles meet in LDS at the
//    end (fixed order). SK = 1: one pass, one store. SK > 1 (split over
//    gridDim.y, for products whose activation rows outweigh a workgroup's
//    weights): fp32 partials, added in split order by a second kernel.
//  * Weights go straight from memory to registers, 16 bytes per lane: lane
//    (row n = lane % 16, quarter c = lane / 16) loads 32 codes (4-bit) or 16
//    codes (8-bit) of row n. The MFMA sums over the 32 k of a step, so the k
//    a lane quarter supplies in step r can be any 8 as long as x matches;
//    exact modes keep every step inside one quantisation group by exchanging
//    words between lane quarters with v_permlane32/16_swap (group 32: a 4x4
//    word transpose; group 64 and 8-bit: one 32-lane swap; group >= 128:
//    none), and x fragments are loaded at the matching k (kmap below).
//  * Exact modes: codes become exact bf16 integers (4-bit: 128+q via one
//    AND-OR per code pair; 8-bit: q itself, byte convert + pack), each group
//    is accumulated alone (D_g) with X_g = sum of x over the group from an
//    MFMA against ones, and folded in fp32:
//        acc += s*D_g + (b - 128 s) X_g        (8-bit: acc += s*D_g + b X_g)
//    so the dequantised weights are never rounded.
//  * Q4F and BF16 run the identical MFMA sequence (same k order, same
//    accumulation order), so the fused product is bit-identical to
//    dequant + cache GEMM.
#include "common.hpp"
#include "kernels.hpp"

#include <stdlib.h>

#include <algorithm>
#include <type_traits>
#include <utility>

namespace miori {

namespace {

enum { Q4X = 0, Q8X = 1, Q4F = 2, BF16 = 3 };
constexpr int NW = 8;  // waves per workgroup (widest form; exact modes also use 4)

template <int N>
using ic = std::integral_constant<int, N>;
// f(ic<I>) for each I of the sequence, in order
template <int... I, class F>
__device__ __forceinline__ void each(std::integer_sequence<int, I...>, F&& f) {
    (f(ic<I>{}), ...);
}

template <int MODE, int MT, int NT, int G, int NBW, int NWV>
struct Sk {
    static constexpr bool EXACT = MODE == Q4X || MODE == Q8X;
    static constexpr int KB = MODE == Q8X ? 64 : 128;          // k per block
    static constexpr int STEPS = KB / 32;                      // MFMA k-steps per block
    static constexpr int WL = MODE == BF16 ? STEPS : 1;        // 16-byte weight loads per n-tile
    // k-steps folded together (one quantisation group inside the block)
    static constexpr int SPF = !EXACT ? STEPS : ((G < KB ? G : KB) / 32);
    static constexpr int NB = 16 * NT;
    // scale / bias tiles of the workgroup's rows in LDS (all K/G groups of up
    // to NBW * NWV blocks), rounded up to whole 1 KiB DMA chunks
    // (all K / G groups of a row: sized for the largest supported K, 8 blocks
    // per wave, so a workgroup of a K split indexes groups absolutely)
    static constexpr int NGMAX = EXACT || MODE == Q4F ? (8 * NWV * KB) / G : 0;
    // (+ room for the masked reads of padding blocks past a row's end)
    static constexpr int SB_BYTES = ((NB * NGMAX * 2 + NBW * KB / 16 + 1023) / 1024) * 1024;
    static constexpr int TOT = NT * MT * 4 * 64;                  // partial floats per wave
    static constexpr int RED_BYTES = NWV * TOT * 4;
    // x tile in LDS (XL): the workgroup's 16*MT rows of x over its whole K
    // range, rows padded to whole 128-element (256-byte) lengths, loaded once
    // by 1 KiB DMAs; the x fragments are then LDS reads and the vector memory
    // path carries only the weight stream. Taken wherever the tile (at the
    // largest K range of the form, KW) fits beside the scale / bias tiles;
    // the cross-wave reduction then reuses the tile's memory.
    static constexpr int KW = NBW * NWV * KB;
    static constexpr int XT_MAX = ((16 * MT * ((KW + 127) / 128 * 128) * 2 + 1023) / 1024) * 1024;
    // A 64-128 KiB tile leaves one workgroup per CU, which only pays where
    // the grid is one round: the eight-wave two-m-tile forms (M > 16, whose
    // n-tiles per workgroup keep config-sized grids at <= 256 workgroups),
    // and the 8-bit four-wave one-m-tile form (M <= 8, a 33 KiB tile).
    // Measured against x loads per block (us): M=32 N=8192 K=2048 10.20 ->
    // 9.67, fused GEMM M=24 N=2048 6.22 -> 5.67; one m-tile at M=16, N=16384
    // (512 workgroups) 11.1 -> 13.1, so those forms keep the loads.
    static constexpr bool XL =
        2 * SB_BYTES + (XT_MAX > RED_BYTES ? XT_MAX : RED_BYTES) <= 160 * 1024 &&
        ((NWV == 8 && MT == 2) || (MODE == Q8X && NWV == 4 && MT == 1 && NT == 2));
    // registers (dwords) per block slot, to size the pipeline depth
    static constexpr int REGS = NT * WL * 4 + (XL ? 0 : MT * STEPS * 4);
    static constexpr int PD0 = 136 / REGS;
    static constexpr int PD = PD0 < 2 ? 2 : (PD0 > 4 ? 4 : PD0);   // blocks in flight per wave
    static constexpr int L = NT * WL + (XL ? 0 : MT * STEPS);     // loads per block
    // static LDS: the scale / bias tiles, and without XL the reduction buffer
    static constexpr int LDS = (XL || 2 * SB_BYTES > RED_BYTES) ? 2 * SB_BYTES : RED_BYTES;
    static constexpr int DEPTH = PD < NBW ? PD : NBW;             // slots actually used
    static_assert((DEPTH - 1) * L < 64, "vmcnt range");
};

// k offset (within a block) of the 8 values lane quarter c supplies in step r.
template <int MODE, int G>
__device__ __forceinline__ uint32_t kmap(uint32_t c, int r) {
    if constexpr (MODE == Q4X && G == 32) return 32u * r + 8u * c;
    else if constexpr (MODE == Q4X && G == 64)
        return 32u * ((c & 1u) + 2u * (r >> 1)) + 8u * ((r & 1) + 2u * (c >> 1));
    else if constexpr (MODE == Q8X) return 32u * r + 8u * (((c & 1u) << 1) | (c >> 1));
    else return 32u * c + 8u * r;  // Q4X group >= 128, Q4F, BF16: no exchange
}

__device__ __forceinline__ void swap32u(uint32_t& a, uint32_t& b) {
    auto p = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = p[0];
    b = p[1];
}
__device__ __forceinline__ void swap16u(uint32_t& a, uint32_t& b) {
    auto p = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    a = p[0];
    b = p[1];
}

__device__ __forceinline__ bf16x8_t as_bf16x8_u(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4_t v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8_t, v);
}

// x fragment: 8 consecutive bf16, pair-permuted to the slot order of the
// weight fragment (4-bit exact: (x0,x4)(x1,x5)(x2,x6)(x3,x7); 8-bit exact,
// Q4F, BF16: natural order).
template <int MODE>
__device__ __forceinline__ bf16x8_t x_frag(u32x4_t d) {
    if constexpr (MODE == Q4X)
        return as_bf16x8_u(__builtin_amdgcn_perm(d[2], d[0], 0x05040100u),
                           __builtin_amdgcn_perm(d[2], d[0], 0x07060302u),
                           __builtin_amdgcn_perm(d[3], d[1], 0x05040100u),
                           __builtin_amdgcn_perm(d[3], d[1], 0x07060302u));
    else
        return __builtin_bit_cast(bf16x8_t, d);
}

// Loads as inline asm with hand-placed waits (vmcnt counts them in issue
// order), so PD blocks stay in flight. The kernel body is straight-line code
// (the per-wave block loop is unrolled for a compile-time block count, no
// branches), so a register a load is still filling is never copied; tie()
// makes each value depend on its wait so no use is scheduled above it.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void ld16(u32x4_t& d, const void* p) {
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(d) : "v"(p));
}
__device__ __forceinline__ void ld16nt(u32x4_t& d, const void* p) {
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(d) : "v"(p));
}
// Weight loads. A 4- or 8-bit block reads 64 bytes of each row, half a
// 128-byte line, and the next block of the same wave reads the other half.
// With a non-temporal hint L2 let such lines go in between and fetched them
// again: FETCH_SIZE of the 8-bit lm_head was 1.26x (M=8) and 1.62x (M=32)
// the weight bytes, 1.00x without the hint, and the launches 10-13% faster
// (bf16 weights: 12-20%). The fused 4-bit mode measured mixed (+-3%) and
// keeps the hint.
template <int MODE>
__device__ __forceinline__ void ldw(u32x4_t& d, const void* p) {
    if constexpr (MODE == Q4F)
        ld16nt(d, p);
    else
        ld16(d, p);
}
// (16 bytes at byte offset off + OFF of a buffer, OFF in the instruction's
// immediate field)
template <int OFF>
__device__ __forceinline__ void buf16_at(u32x4_t& d, rsrc_t r, uint32_t off) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:%3" : "=v"(d) : "v"(off), "s"(r), "i"(OFF));
}
// an offset past any buffer of the persistent kernel (N * K < 2^31) even
// with the largest immediate added
constexpr uint32_t kLmhOOB = 0x80000000u;
// an x-row offset past the skinny kernel's x buffer (M * K * 2 <= 512 KiB)
// however far into a row a load reaches (K * 2 <= 16 KiB)
constexpr uint32_t kXOOB = 0x80000000u;
__device__ __forceinline__ void ld8(u32x2_t& d, const void* p) {
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(d) : "v"(p));
}
__device__ __forceinline__ void ld4(uint32_t& d, const void* p) {
    asm volatile("global_load_dword %0, %1, off" : "=v"(d) : "v"(p));
}
__device__ __forceinline__ void ld2(uint32_t& d, const void* p) {
    asm volatile("global_load_ushort %0, %1, off" : "=v"(d) : "v"(p));
}
__device__ __forceinline__ void tie(u32x4_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void tie(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void tie(u32x2_t& v) { asm volatile("" : "+v"(v)); }

// 128 + two 4-bit codes as exact bf16 integers: (v & m) | c with m =
// 0x000F000F in an SGPR and c = 0x43004300 in a VGPR, so the compiler can
// select one v_and_or_b32 (this encoding takes no literal). The AND-OR itself
// stays compiler code (not inline asm): its results feed MFMA operands and the
// compiler must see the VALU write to insert the wait states an MFMA read of a
// just-written VGPR needs. The two constants come from asm moves so they are
// not folded back into literals.
struct NibConst {
    uint32_t m, c;
};
__device__ __forceinline__ NibConst nib_const() {
    NibConst k;
    asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(k.m));
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(k.c));
    return k;
}
__device__ __forceinline__ uint32_t nib2(uint32_t v, NibConst k) { return (v & k.m) | k.c; }

// Eight 8-bit codes (bytes of a then b, k order) as bf16: every integer
// 0..255 is exact in bf16, so convert + pack loses nothing. The bytes are
// made opaque first so each converts with one v_cvt_f32_ubyte<i>.
__device__ __forceinline__ bf16x8_t codes8_bf16(uint32_t a, uint32_t b) {
    asm volatile("" : "+v"(a), "+v"(b));
    u32x4_t o;
    const uint32_t w[2] = {a, b};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        bf16x2_t p0 = {(__bf16)(float)(w[h] & 0xFFu), (__bf16)(float)((w[h] >> 8) & 0xFFu)};
        bf16x2_t p1 = {(__bf16)(float)((w[h] >> 16) & 0xFFu), (__bf16)(float)(w[h] >> 24)};
        o[2 * h] = __builtin_bit_cast(uint32_t, p0);
        o[2 * h + 1] = __builtin_bit_cast(uint32_t, p1);
    }
    return __builtin_bit_cast(bf16x8_t, o);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int MODE, int MT, int NT, int G, int NBW, int NWV>
__global__ __launch_bounds__(NWV * 64) void skinny_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
    const uint16_t* __restrict__ S, const uint16_t* __restrict__ Bi, void* __restrict__ Y,
    uint32_t M, uint32_t N, uint32_t K, int out_bf16, float* __restrict__ part, uint32_t xrot) {
    using C = Sk<MODE, MT, NT, G, NBW, NWV>;
    // scale / bias tiles first, the cross-wave reduction buffer at the end
    __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS];
    // x tile (C::XL), sized by the launch; the reduction buffer reuses it
    extern __shared__ __attribute__((aligned(1024))) uint8_t xdyn[];
    float* red = reinterpret_cast<float*>(C::XL ? xdyn : lds);
    // LDS-typed pointers (ds_read, not flat loads that would wait on vmcnt)
    typedef __attribute__((address_space(3))) const uint16_t* lds_u16;
    const lds_u16 s_lds = (lds_u16)(lds);
    const lds_u16 b_lds = (lds_u16)(lds + C::SB_BYTES);

    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t j = lane & 15u, c = lane >> 4;
    const uint32_t n0 = blockIdx.x * 16u * NT;
    const uint32_t nblk = K / C::KB;
    // this workgroup's K blocks: [kb0, kb0 + nloc) (split gridDim.y ways)
    // (the unsplit launches skip the integer divisions: gridDim.y and
    // gridDim.z are uniform, so these are scalar branches)
    const uint32_t nloc = gridDim.y == 1 ? nblk : nblk / gridDim.y, kb0 = blockIdx.y * nloc;
    const uint32_t b0 = kb0 + wave * nloc / NWV, b1 = kb0 + (wave + 1) * nloc / NWV;
    const uint32_t nb = b1 - b0;
    const uint32_t ng = (MODE == BF16) ? 1u : K / G;

    // per-lane row pointers (rows clamped into the matrices; clamped rows are
    // never stored)
    const uint8_t* wrow[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t n = min(n0 + nt * 16u + j, N - 1u);
        const size_t rb = (MODE == Q4X || MODE == Q4F) ? K / 2 : (MODE == Q8X ? K : 2ull * K);
        wrow[nt] = W + (size_t)n * rb;
    }
    // x rows as byte offsets into a buffer over x (loads per block, forms
    // without the LDS x tile): rows outside the workgroup's range [m0, m1)
    // take an out-of-range offset and read as zeros without touching memory
    // (their outputs are never stored; each output row depends only on its
    // own x row)
    uint32_t xro[MT];
    // rows [m0, m0 + mstep) of y (M split over gridDim.z); lanes of x rows
    // past that range compute outputs that are never stored
    const uint32_t mstep = gridDim.z == 1 ? M : (M + gridDim.z - 1) / gridDim.z;
    const uint32_t m0 = blockIdx.z * mstep;
    const uint32_t m1 = min(M, m0 + mstep);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const uint32_t m = m0 + mt * 16u + j;
        xro[mt] = m < m1 ? m * K * 2u : kXOOB;
    }
    const rsrc_t rx = make_rsrc(X, M * K * 2u);

    // x tile in LDS (C::XL): rows m0 .. m0+xrows-1 over the workgroup's K
    // range [kbase, kbase + nloc*KB), row r at r * rsb bytes; 16-byte chunk
    // ch of a row is stored at chunk ch ^ (r & 15), so the 16 rows a
    // fragment read touches at one k fall on distinct banks. DMA u fills
    // tile bytes [1024u, 1024u + 1024), each lane the chunk its slot holds
    // (source row and chunk clamped into x; such slots are never read). The
    // wait for the first block covers the DMAs (issue order below).
    typedef __attribute__((address_space(3))) const u32x4_t* lds_v4;
    const uint32_t xrows = min(16u * MT, m1 - m0);
    const uint32_t kbase = kb0 * C::KB;
    const uint32_t rsb = ((nloc * C::KB + 127u) & ~127u) * 2u;
    uint32_t xrb[MT], xsw[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const uint32_t row = min(mt * 16u + j, xrows - 1u);
        xrb[mt] = __umul24(row, rsb);
        xsw[mt] = row & 15u;
    }
    // (issued after block 0's weight loads, below)
    auto issue_xtile = [&]() {
      if constexpr (C::XL) {
        const uint32_t nins = (xrows * rsb + 1023u) / 1024u;
        const uint32_t nch = nloc * C::KB / 8u;
        // xrot != 0: the workgroups of one XCD (blockIdx.x % 8 alike) start
        // at chunks spread over the tile, so they do not all fetch the same
        // lines at the same moment (the same DMAs, in a rotated order)
        const uint32_t per_xcd = max(1u, gridDim.x >> 3);
        const uint32_t r0 = xrot ? (blockIdx.x >> 3) % per_xcd * nins / per_xcd : 0u;
        // The row of a lane's 16-byte slot p is p / rsb. rsb is a multiple of
        // 256 bytes, so r = floor(a / d) with a = p / 256 and d = rsb / 256,
        // computed in fp32 as trunc((a + 1/2) / d): that quotient lies at
        // least 1/(2d) >= 2^-7 from an integer, and its rounding error is
        // below a * 2^-23 <= 2^-12 (a < 2^11, d <= 64). This replaces an
        // integer division (about 20 VALU instructions, five of them
        // quarter-rate) per DMA with four full-rate ones; the offsets fit
        // 24-bit multiplies (r < 2^11, rsb <= 2^14; x rows < 32, K <= 2^15).
        const float inv_d = 1.0f / (float)(rsb >> 8);
        const uint32_t xoff0 = __umul24(m0, K) + kbase;
        for (uint32_t v = wave; v < nins; v += NWV) {
            const uint32_t u = v + r0 < nins ? v + r0 : v + r0 - nins;
            const uint32_t p = u * 1024u + lane * 16u;
            const uint32_t a = u * 4u + (lane >> 4);
            const uint32_t r = (uint32_t)(((float)a + 0.5f) * inv_d);
            const uint32_t rr = min(r, xrows - 1u);
            const uint32_t ch = min(((p - __umul24(r, rsb)) >> 4) ^ (r & 15u), nch - 1u);
            dma16(X + (xoff0 + __umul24(rr, K) + ch * 8u), xdyn + u * 1024u);
        }
      }
    };

    // block slots
    u32x4_t wr[C::DEPTH][NT][C::WL];
    u32x4_t xr[C::XL ? 1 : C::DEPTH][MT][C::STEPS];

    auto issue = [&](uint32_t blk, auto slot_c) {
        constexpr int sl = decltype(slot_c)::value;
        const uint32_t k0 = blk * C::KB;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            if constexpr (MODE == BF16) {
#pragma unroll
                for (int r = 0; r < C::STEPS; ++r)
                    ldw<MODE>(wr[sl][nt][r], wrow[nt] + 2u * (k0 + kmap<MODE, G>(c, r)));
            } else {
                const uint32_t byte = (MODE == Q8X) ? k0 + 16u * c : k0 / 2 + 16u * c;
                ldw<MODE>(wr[sl][nt][0], wrow[nt] + byte);
            }
        }
        if constexpr (!C::XL) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < C::STEPS; ++r)
                    buf16_at<0>(xr[sl][mt][r], rx, xro[mt] + 2u * (k0 + kmap<MODE, G>(c, r)));
        }
    };

    f32x4_t acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const bf16x8_t ones = as_bf16x8_u(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
    const NibConst nk = nib_const();

    // scale / bias of this lane's row of n-tile nt, group (first group of the
    // wave) + d: one LDS read at a per-n-tile base with an immediate offset d.
    const uint32_t g_w0 = b0 * C::KB / G;
    lds_u16 srl[NT];
    lds_u16 brl[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        srl[nt] = s_lds + (nt * 16u + j) * ng + g_w0;
        brl[nt] = b_lds + (nt * 16u + j) * ng + g_w0;
    }
    auto s_of = [&](int nt, int d) { return bf16_bits_to_f32(srl[nt][d]); };
    auto b_of = [&](int nt, int d) { return bf16_bits_to_f32(brl[nt][d]); };

    // valid = false (a padding block of a wave with fewer than NBW blocks):
    // the block's loads were clamped to a real block and its contribution is
    // zeroed by selects (x fragments, or the fold coefficients).
    // block i (0-based in the wave) from slot i % DEPTH; group offsets inside
    // the wave's groups are compile-time: (i*KB + k) / G
    auto compute = [&](auto i_c, bool valid) {
        constexpr int i = decltype(i_c)::value;
        constexpr int sl = i % C::DEPTH;
        bf16x8_t xf[MT][C::STEPS];
        // (the block's k base inside the workgroup's range, for the LDS x tile)
        const uint32_t kx = (min(b0 + (uint32_t)i, kb0 + nloc - 1u) - kb0) * C::KB;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < C::STEPS; ++r) {
                u32x4_t d;
                if constexpr (C::XL) {
                    const uint32_t ch = (kx + kmap<MODE, G>(c, r)) / 8u;
                    d = *(lds_v4)(xdyn + xrb[mt] + ((ch ^ xsw[mt]) << 4));
                }
                else
                    d = xr[sl][mt][r];
                if constexpr (!C::EXACT) {
                    d[0] = valid ? d[0] : 0u;
                    d[1] = valid ? d[1] : 0u;
                    d[2] = valid ? d[2] : 0u;
                    d[3] = valid ? d[3] : 0u;
                }
                xf[mt][r] = x_frag<MODE>(d);
            }
        if constexpr (!C::EXACT) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int r = 0; r < C::STEPS; ++r) {
                    bf16x8_t bfr;
                    if constexpr (MODE == BF16) {
                        bfr = __builtin_bit_cast(bf16x8_t, wr[sl][nt][r]);
                    } else {
                        // this lane's group: codes i*KB + 32c .. +31 of the wave's range
                        const uint32_t d = (i * C::KB + 32u * c) / G;
                        const float sc = bf16_bits_to_f32(srl[nt][d]);
                        const float bi = bf16_bits_to_f32(brl[nt][d]);
                        const uint32_t v = wr[sl][nt][0][r];
                        const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
                        u32x4_t o;
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const float f0 = fmaf((float)((lo >> (8 * q)) & 0xFFu), sc, bi);
                            const float f1 = fmaf((float)((hi >> (8 * q)) & 0xFFu), sc, bi);
                            bf16x2_t pr = {(__bf16)f0, (__bf16)f1};
                            o[q] = __builtin_bit_cast(uint32_t, pr);
                        }
                        bfr = __builtin_bit_cast(bf16x8_t, o);
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16(xf[mt][r], bfr, acc[nt][mt]);
                }
        } else {
            // x sums of each fold (shared by the n-tiles)
            constexpr int NF = C::STEPS / C::SPF;
            f32x4_t dx[NF][MT];
#pragma unroll
            for (int f = 0; f < NF; ++f)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    dx[f][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int r = f * C::SPF; r < (f + 1) * C::SPF; ++r)
                        dx[f][mt] = mfma16(xf[mt][r], ones, dx[f][mt]);
                }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                uint32_t w0 = wr[sl][nt][0][0], w1 = wr[sl][nt][0][1];
                uint32_t w2 = wr[sl][nt][0][2], w3 = wr[sl][nt][0][3];
                if constexpr (MODE == Q8X || G == 64 || G == 32) {
                    swap32u(w0, w2);
                    swap32u(w1, w3);
                }
                if constexpr (MODE == Q4X && G == 32) {
                    swap16u(w0, w1);
                    swap16u(w2, w3);
                }
                const uint32_t wv[4] = {w0, w1, w2, w3};
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    f32x4_t dd[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) dd[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int r = f * C::SPF; r < (f + 1) * C::SPF; ++r) {
                        if constexpr (MODE == Q4X) {
                            const uint32_t v = wv[r];
                            const bf16x8_t bfr = as_bf16x8_u(nib2(v, nk),
                                                             nib2(v >> 4, nk),
                                                             nib2(v >> 8, nk),
                                                             nib2(v >> 12, nk));
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) dd[mt] = mfma16(xf[mt][r], bfr, dd[mt]);
                        } else {
                            // 8 codes in k order; a code (0..255) is an exact bf16
                            const bf16x8_t bq = codes8_bf16(wv[2 * r], wv[2 * r + 1]);
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) dd[mt] = mfma16(xf[mt][r], bq, dd[mt]);
                        }
                    }
                    const int d = (i * C::KB + f * C::SPF * 32) / G;
                    const float sv = s_of(nt, d), bv = b_of(nt, d);
                    const float sc = valid ? sv : 0.f;
                    const float bi = valid ? bv : 0.f;
                    // 4-bit codes carry the +128 of the bf16 trick
                    const float bx = (MODE == Q4X) ? fmaf(-128.f, sc, bi) : bi;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[nt][mt][e] = fmaf(sc, dd[mt][e], fmaf(bx, dx[f][mt][e], acc[nt][mt][e]));
                }
            }
        }
    };

    // DEPTH-deep pipeline over NBW block slots of this wave, fully unrolled:
    // block i is computed from slot i % DEPTH once the blocks issued after it
    // (at most DEPTH-1, L loads each) are the only ones in flight, then block
    // i + DEPTH is issued into the same slot.
    auto blk_of = [&](int i) { return min(b0 + (uint32_t)i, nblk - 1u); };
    auto step = [&](auto i_c) {
        constexpr int i = decltype(i_c)::value;
        constexpr int sl = i % C::DEPTH;
        constexpr int after = (NBW - 1 - i) < (C::DEPTH - 1) ? (NBW - 1 - i) : (C::DEPTH - 1);
        wait_vm<after * C::L>();
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
            for (int q = 0; q < C::WL; ++q) tie(wr[sl][nt][q]);
        }
        if constexpr (!C::XL) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < C::STEPS; ++r) tie(xr[sl][mt][r]);
        }
        // scale/bias tiles (and the x tile) landed for all waves
        if constexpr (i == 0 && (MODE != BF16 || C::XL)) barrier_lds();
        // keep each block's work (and its scale reads) inside its step
        __builtin_amdgcn_sched_barrier(0);
        compute(ic<i>{}, (uint32_t)i < nb);
        if constexpr (i + C::DEPTH < NBW) issue(blk_of(i + C::DEPTH), ic<sl>{});
        __builtin_amdgcn_sched_barrier(0);
    };
    // Issue order: block 0's loads, then the x tile's DMAs, then the scale /
    // bias tiles' DMAs, then blocks 1 .. DEPTH-1. The wait of block 0 keeps
    // only the DEPTH-1 youngest blocks in flight, so it covers both DMA sets;
    // block 0's weights (from HBM) go out first and their latency overlaps
    // the DMA issue (the x tile mostly comes from L2).
    issue(blk_of(0), ic<0>{});
    issue_xtile();
    // Scale / bias tiles of rows n0 .. n0+NB-1 (contiguous in S and B): 1 KiB
    // DMA chunks spread over the waves. Sources are clamped inside the arrays.
    if constexpr (MODE != BF16) {
        const uint32_t tb = C::NB * ng * 2u;                 // tile bytes
        const size_t total = (size_t)N * ng * 2u;            // array bytes
        const size_t base = (size_t)n0 * ng * 2u;
        for (uint32_t q = wave; q * 1024u < tb; q += NWV) {
            const size_t off = min(base + q * 1024u + lane * 16u, total - 16u);
            dma16(reinterpret_cast<const uint8_t*>(S) + off, lds + q * 1024u);
            dma16(reinterpret_cast<const uint8_t*>(Bi) + off, lds + C::SB_BYTES + q * 1024u);
        }
    }
    if constexpr (C::DEPTH > 1) issue(blk_of(1), ic<1 % C::DEPTH>{});
    if constexpr (C::DEPTH > 2) issue(blk_of(2), ic<2 % C::DEPTH>{});
    if constexpr (C::DEPTH > 3) issue(blk_of(3), ic<3 % C::DEPTH>{});
    step(ic<0>{});
    if constexpr (NBW > 1) step(ic<1>{});
    if constexpr (NBW > 2) { step(ic<2>{}); step(ic<3>{}); }
    if constexpr (NBW > 4) { step(ic<4>{}); step(ic<5>{}); step(ic<6>{}); step(ic<7>{}); }

    // Cross-wave reduction in fixed wave order (the LDS tiles are dead).
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) red[wave * C::TOT + ((nt * MT + mt) * 4 + e) * 64 + lane] = acc[nt][mt][e];
    __syncthreads();
    const bool bf = out_bf16 != 0;
    for (uint32_t e = t; e < (uint32_t)C::TOT; e += NWV * 64) {
        float v = red[e];
#pragma unroll
        for (int w = 1; w < NWV; ++w) v += red[w * C::TOT + e];
        const uint32_t ln = e & 63u, e4 = (e >> 6) & 3u, tm = e >> 8;
        const uint32_t nt = tm / MT, mt = tm % MT;
        const uint32_t n = n0 + nt * 16u + (ln & 15u);
        const uint32_t m = m0 + mt * 16u + 4u * (ln >> 4) + e4;
        if (n < N && m < m1) {
            if (gridDim.y == 1)
                store_out(Y, (size_t)m * N + n, v, bf);
            else
                part[((size_t)blockIdx.y * M + m) * N + n] = v;
        }
    }
}

// Persistent 8-bit exact kernel for vocabulary-sized N and 5 <= M <= 32 (the
// batched lm_head): one workgroup of eight waves per CU stages x (M x K bf16)
// in LDS once, and every wave then streams whole 16-row tiles of W over the
// full K, tile w, w + W, w + 2W, ... of the grid's W waves. A wave keeps
// DEPTH (16 or 32) 64-k blocks of its weight stream in flight, across tile
// boundaries, and needs no cross-wave reduction: each tile's 16 x M outputs
// are stored by the wave that computed them. The per-block arithmetic is the
// skinny kernel's Q8X mode (codes as exact bf16 integers, D_g and X_g by
// MFMA, acc += s*D_g + b*X_g), with the k order of its lane quarters.
//  * x is loaded once per CU instead of once per 64 rows, so the vector
//    memory path carries only the weight stream. Measured at N = 131072,
//    K = 2048 against the four-wave skinny form (us): M=32 81.7 -> 68.1,
//    M=24 78.3 -> 67.1, M=17 75.1 -> 65.1, M=16 67.8 -> 59.8, M=9 63.5 ->
//    58.5. Four waves per workgroup were slower than eight (M=32 82.6: one
//    wave per SIMD serialises its VALU and MFMA work), and so was the same
//    loop with per-block address arithmetic instead of per-chunk bases with
//    immediate offsets (73.2: 30% more VALU instructions).
//    Up to M = 8 it replaced the four-wave form with x in LDS: M=8 65.8 ->
//    60.5, M=6 62.4 -> 60.6, M=5 61.7 -> 60.1 (that form keeps the shapes
//    this kernel does not take).
//  * A tile's scales and biases (16 rows x K/G, contiguous) are DMA'd into a
//    per-wave LDS double buffer just before the tile's first weight load,
//    one 1 KiB chunk per instruction, so the wait for that block covers them;
//    the buffer's previous tile is finished by then because a tile has at
//    least DEPTH blocks. (Loading them per block with the weights, 2-byte
//    loads from 16 rows, took 93 us at M = 32.)
//  * Requires G in {64, 128}, K / 64 a power of two >= DEPTH, and the x tile
//    (16*MT rows of 2K bytes) plus the scale buffers within 160 KiB.
//
// XS = true (MIORI_LMH_XSUM=1, a tuning experiment): the x sums X_g of each
// 64-k block and m-tile, which do not depend on the weight rows, are made
// once per workgroup into LDS (the same two MFMAs against ones as the
// per-block code, so the products stay bit-identical) and each block reads
// them instead of recomputing them: half the MFMAs per block.
template <int MT, int G, int DEPTH, int NWV, bool XS = false>
__global__ __launch_bounds__(NWV * 64) void lmh_kernel(const uint16_t* __restrict__ X,
                                                  const uint8_t* __restrict__ W,
                                                  const uint16_t* __restrict__ S,
                                                  const uint16_t* __restrict__ Bi,
                                                  void* __restrict__ Y, uint32_t M, uint32_t N,
                                                  uint32_t K, int out_bf16, uint32_t xrot) {
    constexpr int KB = 64;
    static_assert(G == 64 || G == 128, "one scale / bias per 64-k block");
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
    const uint32_t t = threadIdx.x, lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t j = lane & 15u, c = lane >> 4;
    const uint32_t XR = K * 2u;  // LDS row stride (bytes)
    const uint32_t rows = min(M, 16u * MT);
    const uint32_t ng = K / G;
    const uint32_t sbc = (32u * ng + 1023u) / 1024u;  // 1 KiB chunks per scale tile
    // this wave's scale / bias buffers: [buffer][s, b][sbc KiB]
    uint8_t* sbw = xs + 16u * MT * XR + wave * (4u * sbc * 1024u);

    // x rows 0 .. rows-1 into LDS, one 1 KiB DMA per (row, 512-k chunk).
    // The 16-byte chunk q of row r sits at chunk q ^ (r & 15) of the row, so
    // the 16 rows of an MFMA fragment read fall on distinct banks; the DMA
    // writes lanes in order, so each lane fetches the chunk its slot holds.
    const uint32_t nch = K / 512u;
    // xrot != 0: each workgroup starts at a different DMA of the tile (the
    // same DMAs, rotated), so the CUs do not fetch the same lines together
    const uint32_t nx = rows * nch;
    const uint32_t r0 = xrot ? (blockIdx.x * 37u) % nx : 0u;
    for (uint32_t v = wave; v < nx; v += NWV) {
        const uint32_t u = v + r0 < nx ? v + r0 : v + r0 - nx;
        const uint32_t r = u / nch, ch = u % nch;
        dma16(X + (size_t)r * K + (ch * 64u + (lane ^ (r & 15u))) * 8u, xs + r * XR + ch * 1024u);
    }

    const uint32_t nbpt = K / KB;  // blocks per tile (a power of two, >= DEPTH)
    const uint32_t lg = 31u - __builtin_clz(nbpt);
    const uint32_t ntiles = (N + 15u) / 16u;
    const uint32_t nw = gridDim.x * NWV, w = blockIdx.x * NWV + wave;
    const uint32_t T = w < ntiles ? (ntiles - 1u - w) / nw + 1u : 0u;
    const uint32_t total = T << lg;  // blocks in this wave's stream
    // scale / bias tile of tile ti into buffer ti % 2 (sources clamped inside
    // the arrays; rows past N are never stored)
    const size_t sb_total = (size_t)N * ng * 2u;
    auto issue_sb = [&](uint32_t ti) {
        const size_t base = (size_t)min((w + ti * nw) * 16u, N - 1u) * ng * 2u;
        uint8_t* dst = sbw + (ti & 1u) * (2u * sbc * 1024u);
        for (uint32_t q = 0; q < sbc; ++q) {
            const size_t off = min(base + q * 1024u + lane * 16u, sb_total - 16u);
            dma16(reinterpret_cast<const uint8_t*>(S) + off, dst + q * 1024u);
            dma16(reinterpret_cast<const uint8_t*>(Bi) + off, dst + (sbc + q) * 1024u);
        }
    };
    if (T > 0) issue_sb(0);
    wait_vm<0>();
    barrier_lds();
    // (XS) x sums after the scale buffers: [block][m-tile][quarter c] x 4
    // floats, rows 4c + e of the m-tile; the MFMA against ones gives every
    // column the same sums, so lane 16c stores them.
    uint8_t* const xsum = xs + 16u * MT * XR + NWV * (4u * sbc * 1024u);
    if constexpr (XS) {
        typedef __attribute__((address_space(3))) const u32x4_t* lds_v4x;
        const bf16x8_t ones1 = as_bf16x8_u(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
        for (uint32_t kb = wave; kb < nbpt; kb += NWV) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const uint32_t r = min(mt * 16u + j, rows - 1u), sw = r & 15u;
                const uint32_t base = (kb & ~1u) * (KB * 2u) + r * XR;
                bf16x8_t f[2];
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    f[q] = __builtin_bit_cast(
                        bf16x8_t, *(lds_v4x)(xs + base + ((((kb & 1u) * 8u + kmap<Q8X, G>(c, q) / 8u) ^ sw) << 4)));
                f32x4_t dx = mfma16(f[0], ones1, f32x4_t{0.f, 0.f, 0.f, 0.f});
                dx = mfma16(f[1], ones1, dx);
                if ((lane & 15u) == 0)
                    *reinterpret_cast<f32x4_t*>(xsum + ((kb * MT + mt) * 4u + c) * 16u) = dx;
            }
        }
        barrier_lds();
    }
    if (T == 0) return;

    u32x4_t wr[DEPTH];
    // The stream moves in chunks of DEPTH blocks, each inside one tile
    // (DEPTH divides a tile's blocks). Per chunk the weight, x and scale
    // addresses are computed once; block i of the chunk adds a compile-time
    // offset (the load's and the LDS reads' immediate fields).
    // weight offset of the chunk starting at block bn
    // (a chunk past the stream's end loads through an out-of-range offset:
    // zeros, counted by vmcnt like any load, with no memory traffic)
    const rsrc_t rw = make_rsrc(W, N * K);
    auto wbase = [&](uint32_t bn) {
        const uint32_t ti = bn >> lg, kb = bn & (nbpt - 1u);
        const uint32_t n = min((w + ti * nw) * 16u + j, N - 1u);
        return bn < total ? n * K + kb * KB + 16u * c : kLmhOOB;
    };
    auto issue = [&](uint32_t base, auto i_c) {
        constexpr int i = decltype(i_c)::value;
        buf16_at<i * KB>(wr[i], rw, base);
    };
    typedef __attribute__((address_space(3))) const u32x4_t* lds_v4;
    typedef __attribute__((address_space(3))) const uint16_t* lds_u16;
    // x fragment (m-tile mt, step r) of block i of a chunk at k-block kb0 (a
    // multiple of 16): row chunk ((kb0 + i) * 8 + k8) ^ sw with sw < 16, which
    // is kb0 * 8 + (i / 2) * 16 + (((i % 2) * 8 + k8) ^ sw)
    uint32_t xa[MT][2][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const uint32_t r = min(mt * 16u + j, rows - 1u), sw = r & 15u;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int p = 0; p < 2; ++p)
                xa[mt][q][p] = r * XR + ((((uint32_t)p * 8u + kmap<Q8X, G>(c, q) / 8u) ^ sw) << 4);
    }
    const bf16x8_t ones = as_bf16x8_u(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // block i of the chunk: xc = x tile + kb0 * 128 bytes, sc_b / bi_b = this
    // lane's scale / bias row at the chunk's first group
    auto compute = [&](const uint8_t* xc, lds_u16 sc_b, lds_u16 bi_b, const uint8_t* xsc,
                       auto i_c) {
        constexpr int i = decltype(i_c)::value;
        bf16x8_t xf[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                xf[mt][q] = __builtin_bit_cast(bf16x8_t, *(lds_v4)(xc + (i / 2) * 256 + xa[mt][q][i % 2]));
        const float sc = bf16_bits_to_f32(sc_b[i * KB / G]);
        const float bi = bf16_bits_to_f32(bi_b[i * KB / G]);
        uint32_t w0 = wr[i][0], w1 = wr[i][1], w2 = wr[i][2], w3 = wr[i][3];
        swap32u(w0, w2);
        swap32u(w1, w3);
        const bf16x8_t q0 = codes8_bf16(w0, w1), q1 = codes8_bf16(w2, w3);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            f32x4_t dx;
            if constexpr (XS) {
                dx = *(const __attribute__((address_space(3))) f32x4_t*)(xsc + ((i * MT + mt) * 4 + c) * 16u);
            } else {
                dx = mfma16(xf[mt][0], ones, f32x4_t{0.f, 0.f, 0.f, 0.f});
                dx = mfma16(xf[mt][1], ones, dx);
            }
            f32x4_t dd = mfma16(xf[mt][0], q0, f32x4_t{0.f, 0.f, 0.f, 0.f});
            dd = mfma16(xf[mt][1], q1, dd);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt][e] = fmaf(sc, dd[e], fmaf(bi, dx[e], acc[mt][e]));
        }
    };
    const bool bf = out_bf16 != 0;
    {
        const uint32_t base = wbase(0);
        each(std::make_integer_sequence<int, DEPTH>{}, [&](auto i) { issue(base, i); });
    }
    for (uint32_t b0 = 0; b0 < total; b0 += DEPTH) {
        const uint32_t kb0 = b0 & (nbpt - 1u), bn = b0 + DEPTH;
        const uint8_t* xc = xs + kb0 * (KB * 2u);
        const uint8_t* xsc = xsum + kb0 * (MT * 64u);
        const uint8_t* sbb = sbw + ((b0 >> lg) & 1u) * (2u * sbc * 1024u);
        const lds_u16 sc_b = (lds_u16)sbb + j * ng + kb0 * KB / G;
        const lds_u16 bi_b = (lds_u16)(sbb + sbc * 1024u) + j * ng + kb0 * KB / G;
        const uint32_t nb = wbase(bn);
        // one block: wait until only the blocks issued after it are in flight
        // (DEPTH-1 weight loads, plus at most the next tile's scale DMAs,
        // which are younger), compute it, refill its slot with the block
        // DEPTH later; at the chunk's first block, when that later chunk
        // starts a tile, its scales go first, into the other buffer (whose
        // tile is done)
        each(std::make_integer_sequence<int, DEPTH>{}, [&](auto i_c) {
            constexpr int i = decltype(i_c)::value;
            wait_vm<DEPTH - 1>();
            tie(wr[i]);
            __builtin_amdgcn_sched_barrier(0);
            compute(xc, sc_b, bi_b, xsc, i_c);
            if constexpr (i == 0)
                if ((bn & (nbpt - 1u)) == 0 && (bn >> lg) < T) issue_sb(bn >> lg);
            issue(nb, i_c);
            __builtin_amdgcn_sched_barrier(0);
        });
        if ((bn & (nbpt - 1u)) == 0) {
            // tile done: rows 4c + e of each m-tile, column j
            const uint32_t n = (w + (b0 >> lg) * nw) * 16u + j;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t m = mt * 16u + 4u * c + e;
                    if (m < M && n < N) store_out(Y, (size_t)m * N + n, acc[mt][e], bf);
                }
                acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
    // the last DEPTH issues fill slots that are never read
    wait_vm<0>();
    each(std::make_integer_sequence<int, DEPTH>{}, [&](auto i) { tie(wr[decltype(i)::value]); });
}

// x tile plus the waves' double-buffered scale / bias tiles
inline size_t lmh_lds_bytes(int mt, uint32_t K, uint32_t G, int nwv, bool xsum = false) {
    const size_t sbc = (32u * (K / G) + 1023u) / 1024u;
    return (size_t)16 * mt * 2u * K + (size_t)nwv * 4 * sbc * 1024 +
           (xsum ? (size_t)(K / 64) * mt * 64 : 0);
}

template <int MT, int G, int DEPTH, int NWV, bool XS = false>
hipError_t launch_lmh(const void* X, const void* W, const void* S, const void* B, void* Y,
                      uint32_t M, uint32_t N, uint32_t K, int out_bf16, hipStream_t st) {
    // CU count of each device, and (dynamic LDS above 64 KiB is opted into
    // once per device, up to the whole 160 KiB) the kernel's LDS attribute
    static std::atomic<int> cus[64];
    static PerDeviceOnce setup;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = setup.run(dev, [&] {
        int n = 0;
        hipError_t r = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (r != hipSuccess) return r;
        if (n <= 0) return hipErrorInvalidDevice;
        r = hipFuncSetAttribute((const void*)lmh_kernel<MT, G, DEPTH, NWV, XS>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (r == hipSuccess) cus[dev].store(n, std::memory_order_relaxed);
        return r;
    });
    if (e != hipSuccess) return e;
    const size_t lds = lmh_lds_bytes(MT, K, G, NWV, XS);
    static const uint32_t xrot = (uint32_t)tuning_env("MIORI_SKINNY_XROT", 0);
    const uint32_t ntiles = (N + 15u) / 16u;
    const uint32_t grid = std::min<uint32_t>((uint32_t)cus[dev].load(std::memory_order_relaxed),
                                             (ntiles + NWV - 1u) / NWV);
    hipLaunchKernelGGL((lmh_kernel<MT, G, DEPTH, NWV, XS>), dim3(grid), dim3(NWV * 64), lds, st,
                       (const uint16_t*)X, (const uint8_t*)W, (const uint16_t*)S,
                       (const uint16_t*)B, Y, M, N, K, out_bf16, xrot);
    return hipGetLastError();
}

template <int MODE, int MT, int NT, int G, int NBW, int NWV>
hipError_t launch_sk(const void* X, const void* W, const void* S, const void* B, void* Y,
                     uint32_t M, uint32_t N, uint32_t K, int out_bf16, uint32_t SK,
                     hipStream_t st, uint32_t MZ = 1) {
    // (the kernel's scale / bias LDS tiles hold 8 blocks per wave)
    if (K / SK / (MODE == Q8X ? 64u : 128u) > 8u * NWV) return hipErrorInvalidValue;
    const uint32_t nwg = (N + 16 * NT - 1) / (16 * NT);
    using C = Sk<MODE, MT, NT, G, NBW, NWV>;
    // the shape checks come before the split-K workspace is taken, so a
    // rejected shape allocates nothing
    size_t xbytes = 0;
    if constexpr (C::XL) {
        // 16-byte aligned rows (K % 8 == 0 and an aligned X, which the C ABI
        // checks); the tile of the workgroup's rows, or the reduction buffer
        if (((uintptr_t)X & 15) != 0 || K % 8 != 0) return hipErrorInvalidValue;
        const size_t rows = std::min<uint32_t>(16u * MT, (M + MZ - 1) / MZ);
        const size_t tile = (rows * (((K / SK) + 127u) / 128u * 128u) * 2 + 1023) / 1024 * 1024;
        xbytes = std::max<size_t>(tile, C::RED_BYTES);
        if (tile > (size_t)C::XT_MAX) return hipErrorInvalidValue;
        if (xbytes > 64 * 1024) {
            // (dynamic LDS above 64 KiB is opted into once per device)
            static PerDeviceOnce attr;
            int dev = 0;
            hipError_t e = hipGetDevice(&dev);
            if (e != hipSuccess) return e;
            e = attr.run(dev, [] {
                return hipFuncSetAttribute((const void*)skinny_kernel<MODE, MT, NT, G, NBW, NWV>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           160 * 1024 - C::LDS);
            });
            if (e != hipSuccess) return e;
        }
    }
    float* part = nullptr;
    if (SK > 1) {
        const hipError_t e = scratch_get(st, (size_t)SK * M * N * 4, &part);
        if (e != hipSuccess) return e;
    }
    // (MIORI_SKINNY_XROT=1: rotated x-tile DMA order per workgroup, a tuning
    // experiment, off by default)
    static const uint32_t xrot = (uint32_t)tuning_env("MIORI_SKINNY_XROT", 0);
    hipLaunchKernelGGL((skinny_kernel<MODE, MT, NT, G, NBW, NWV>), dim3(nwg, SK, MZ), dim3(NWV * 64),
                       xbytes, st, (const uint16_t*)X, (const uint8_t*)W, (const uint16_t*)S,
                       (const uint16_t*)B, Y, M, N, K, out_bf16, part, xrot);
    if (SK > 1) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_splitk_reduce(part, Y, (size_t)M * N, SK, out_bf16, st);
    }
    return hipGetLastError();
}

// blocks per wave, rounded up to 1, 2, 4 or 8
inline int nbw_of(uint32_t K, uint32_t kb, int nw = NW) {
    const uint32_t per = (K / kb + nw - 1) / nw;
    return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

template <int MODE, int MT, int NT, int G, int NWV>
hipError_t by_nbw(const void* X, const void* W, const void* S, const void* B, void* Y,
                  uint32_t M, uint32_t N, uint32_t K, int out_bf16, uint32_t SK, hipStream_t st,
                  uint32_t MZ = 1) {
    switch (nbw_of(K / SK, MODE == Q8X ? 64u : 128u, NWV)) {
        case 1: return launch_sk<MODE, MT, NT, G, 1, NWV>(X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
        case 2: return launch_sk<MODE, MT, NT, G, 2, NWV>(X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
        case 4: return launch_sk<MODE, MT, NT, G, 4, NWV>(X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
    }
    return launch_sk<MODE, MT, NT, G, 8, NWV>(X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
}

template <int MODE, int MT, int NT, int NWV = NW>
hipError_t by_group(uint32_t G, const void* X, const void* W, const void* S, const void* B,
                    void* Y, uint32_t M, uint32_t N, uint32_t K, int out_bf16, uint32_t SK,
                    hipStream_t st, uint32_t MZ = 1) {
    if constexpr (MODE == BF16) {
        return by_nbw<BF16, MT, NT, 64, NWV>(X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
    } else {
        switch (G) {
            case 32: return by_nbw<MODE, MT, NT, 32, NWV>(X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
            case 64: return by_nbw<MODE, MT, NT, 64, NWV>(X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
            case 128: return by_nbw<MODE, MT, NT, 128, NWV>(X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
        }
        return hipErrorInvalidValue;
    }
}

// (an element's k order and wave reduction do not depend on NT)
template <int MODE, int MT>
hipError_t by_nt(int nt, uint32_t G, const void* X, const void* W, const void* S, const void* B,
                 void* Y, uint32_t M, uint32_t N, uint32_t K, int out_bf16, uint32_t SK,
                 hipStream_t st, uint32_t MZ = 1) {
    // (bf16 weights need 4x the load registers of a 4-bit n-tile: at most 2)
    if constexpr (MODE != BF16)
        if (nt >= 4) return by_group<MODE, MT, 4>(G, X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
    if (nt >= 2) return by_group<MODE, MT, 2>(G, X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
    return by_group<MODE, MT, 1>(G, X, W, S, B, Y, M, N, K, out_bf16, SK, st, MZ);
}

template <int MODE>
hipError_t by_shape(uint32_t G, const void* X, const void* W, const void* S, const void* B,
                    void* Y, uint32_t M, uint32_t N, uint32_t K, int out_bf16, hipStream_t st) {
    // n-tiles per workgroup: x is loaded once per workgroup and reused by
    // each n-tile; two while that still gives >= 256 workgroups (more rows
    // per workgroup measured slower: fewer workgroups in flight)
    // four for the 32-row products of N > 8192, where x (M x K bf16, loaded
    // once per workgroup) outweighs a 2-tile workgroup's weights and the
    // x tile in LDS leaves one workgroup per CU (grids of <= 256 up to
    // N = 16384; N=12288 M=32 14.8 -> 13.6 us, N=10240 M=24 13.3 -> 12.5)
    int nt = (N >= 8192) ? 2 : 1;
    if (M > 16 && N > 8192) nt = 4;
    // K split over workgroups for K >= 8192 at M > 8: a workgroup then loads
    // a quarter of x (M x 8192 bf16 is 512 KB at M = 32, against 64 KB of
    // its weights), and the fp32 partials are added by a second kernel.
    // Measured (N = 2048, K = 8192): M=32 19.3 -> 12.2 us, M=16 12.0 -> 10.4;
    // at M = 8 and at K = 2048 the split was slower.
    uint32_t sk = 1;
    if (M > 8 && K >= 8192) {
        sk = 4;
        nt = 2;
    }
    // tuning overrides (MIORI_SKINNY_*), read once per process
    static const int e_nt = tuning_env("MIORI_SKINNY_NT", -1);
    static const int e_split = tuning_env("MIORI_SKINNY_SPLIT", -1);
    static const int e_nw = tuning_env("MIORI_SKINNY_NW", -1);
    static const int e_mz = tuning_env("MIORI_SKINNY_MZ", -1);
    if (e_nt >= 0) nt = e_nt;
    // N a multiple of 16 so the partials' reduction covers whole 8-element
    // groups; the split must divide the K blocks
    if (e_split >= 0) sk = (uint32_t)e_split;
    const uint32_t kb = MODE == Q8X ? 64u : 128u;
    if (sk < 1 || N % 16 != 0) sk = 1;
    // (a function of N and K only, so the fused 4-bit and the bf16 products
    // of one shape split alike and stay bit-identical)
    while (sk > 1 && (K / kb) % sk != 0) --sk;
    // Vocabulary-sized N, exact modes: workgroups of four waves, with four
    // n-tiles above M = 8 and two up to it. Each wave streams twice the K
    // blocks of the eight-wave form, and x is loaded once per 64 rows.
    // Measured (N = 131072, K = 2048, against the best eight-wave form):
    // 8-bit M=32 140 -> 117 us, M=16 90 -> 85, M=8 80.5 -> 78.7; 4-bit at
    // N = 65536 M=32 45.5 -> 38.5 us, M=8 25.0 -> 24.5 (four n-tiles: 26.4).
    // Needs the whole K in 8 blocks per wave and no K split.
    const bool nw4_ok = sk == 1 && K / kb <= 32;
    // 8-bit at vocabulary-sized N: the persistent form with x in LDS
    static const int e_lmh = tuning_env("MIORI_SKINNY_LMH", 1);
    if constexpr (MODE == Q8X) {
        const uint32_t nbpt = K / 64u;
        const bool lmh_ok = e_lmh && N >= 32768 && (G == 64 || G == 128) &&
                            (uint64_t)N * K < 0x7FFF0000u &&
                            nbpt >= 16 && (nbpt & (nbpt - 1u)) == 0 &&
                            lmh_lds_bytes(M > 16 ? 2 : 1, K, G, 8) <= 160u * 1024u &&
                            ((uintptr_t)X & 15) == 0 && e_nt < 0 && e_nw < 0;
        if (lmh_ok) {
            // (MIORI_LMH_NWV=12 or 16, M <= 16: twelve or sixteen waves of
            // 16 blocks in flight per workgroup instead of eight of 32, three
            // or four waves per SIMD to hide each other's unpack and fold
            // (116 VGPRs); a tuning experiment, off by default)
            static const int e_lmh_nwv = tuning_env("MIORI_LMH_NWV", 8);
            if ((e_lmh_nwv == 12 || e_lmh_nwv == 16) && M <= 16 &&
                lmh_lds_bytes(1, K, G, e_lmh_nwv) <= 160u * 1024u) {
                if (e_lmh_nwv == 12)
                    return G == 64 ? launch_lmh<1, 64, 16, 12>(X, W, S, B, Y, M, N, K, out_bf16, st)
                                   : launch_lmh<1, 128, 16, 12>(X, W, S, B, Y, M, N, K, out_bf16, st);
                return G == 64 ? launch_lmh<1, 64, 16, 16>(X, W, S, B, Y, M, N, K, out_bf16, st)
                               : launch_lmh<1, 128, 16, 16>(X, W, S, B, Y, M, N, K, out_bf16, st);
            }
            // 32 blocks in flight per wave from K = 2048, else 16
            const int sel = (M > 16 ? 4 : 0) + (G == 64 ? 0 : 2) + (nbpt >= 32 ? 1 : 0);
            // (MIORI_LMH_XSUM=1: x sums made once per workgroup, an experiment)
            static const int e_xs = tuning_env("MIORI_LMH_XSUM", 0);
            if (e_xs && lmh_lds_bytes(M > 16 ? 2 : 1, K, G, 8, true) <= 160u * 1024u) {
                switch (sel) {
                    case 0: return launch_lmh<1, 64, 16, 8, true>(X, W, S, B, Y, M, N, K, out_bf16, st);
                    case 1: return launch_lmh<1, 64, 32, 8, true>(X, W, S, B, Y, M, N, K, out_bf16, st);
                    case 2: return launch_lmh<1, 128, 16, 8, true>(X, W, S, B, Y, M, N, K, out_bf16, st);
                    case 3: return launch_lmh<1, 128, 32, 8, true>(X, W, S, B, Y, M, N, K, out_bf16, st);
                    case 4: return launch_lmh<2, 64, 16, 8, true>(X, W, S, B, Y, M, N, K, out_bf16, st);
                    case 5: return launch_lmh<2, 64, 32, 8, true>(X, W, S, B, Y, M, N, K, out_bf16, st);
                    case 6: return launch_lmh<2, 128, 16, 8, true>(X, W, S, B, Y, M, N, K, out_bf16, st);
                    default: return launch_lmh<2, 128, 32, 8, true>(X, W, S, B, Y, M, N, K, out_bf16, st);
                }
            }
            switch (sel) {
                case 0: return launch_lmh<1, 64, 16, 8>(X, W, S, B, Y, M, N, K, out_bf16, st);
                case 1: return launch_lmh<1, 64, 32, 8>(X, W, S, B, Y, M, N, K, out_bf16, st);
                case 2: return launch_lmh<1, 128, 16, 8>(X, W, S, B, Y, M, N, K, out_bf16, st);
                case 3: return launch_lmh<1, 128, 32, 8>(X, W, S, B, Y, M, N, K, out_bf16, st);
                case 4: return launch_lmh<2, 64, 16, 8>(X, W, S, B, Y, M, N, K, out_bf16, st);
                case 5: return launch_lmh<2, 64, 32, 8>(X, W, S, B, Y, M, N, K, out_bf16, st);
                case 6: return launch_lmh<2, 128, 16, 8>(X, W, S, B, Y, M, N, K, out_bf16, st);
                default: return launch_lmh<2, 128, 32, 8>(X, W, S, B, Y, M, N, K, out_bf16, st);
            }
        }
    }
    int nw = 8;
    if ((MODE == Q4X || MODE == Q8X) && N >= 32768 && nw4_ok && e_nt < 0)
        nw = 4;
    if (e_nw >= 0) nw = (e_nw == 4 && nw4_ok) ? 4 : 8;
    if constexpr (MODE == Q4X || MODE == Q8X) {
        if (nw == 4) {
            if (M <= 8) return by_group<MODE, 1, 2, 4>(G, X, W, S, B, Y, M, N, K, out_bf16, sk, st);
            if (M <= 16) return by_group<MODE, 1, 4, 4>(G, X, W, S, B, Y, M, N, K, out_bf16, sk, st);
            return by_group<MODE, 2, 4, 4>(G, X, W, S, B, Y, M, N, K, out_bf16, sk, st);
        }
    }
    // M split above M = 8 when the doubled grid still fits one round of
    // 256 workgroups: the rows go to two workgroups (gridDim.z) of one
    // 16-row m-tile each, half of it idle up to M = 16, and the second reads
    // the weights from L2. Every output element is computed as without the
    // split. Measured at M = 32, K = 2048: N = 2048 7.09 -> 5.23 us (fused
    // 7.36 -> 5.73, bf16 9.85 -> 8.04), N = 512 6.79 -> 5.12; at N = 3072
    // (192 -> 384 workgroups) it was slower, bf16 10.3 -> 14.2 us.
    uint32_t mz = 1;
    const uint32_t wgs = (N + 16u * nt - 1) / (16u * nt) * sk;
    if (M > 8 && wgs <= 128) mz = 2;
    if (e_mz >= 0) mz = (e_mz == 2 && M > 8) ? 2 : 1;
    if (M <= 16 || mz == 2)
        return by_nt<MODE, 1>(nt, G, X, W, S, B, Y, M, N, K, out_bf16, sk, st, mz);
    return by_nt<MODE, 2>(nt, G, X, W, S, B, Y, M, N, K, out_bf16, sk, st);
}

}  // namespace

bool skinny_supported(int mode, uint32_t M, uint32_t N, uint32_t K, uint32_t G) {
    if (M == 0 || M > 32 || N == 0) return false;
    if (mode != 3 && !(G == 32 || G == 64 || G == 128)) return false;
    const uint32_t kb = mode == 1 ? 64u : 128u;
    // whole blocks, at most 8 per wave; scale rows in whole 16-byte chunks
    if (mode != 3 && (K / G) % 8 != 0) return false;
    return K % kb == 0 && K <= kb * NW * 8;
}

hipError_t launch_skinny(int mode, const void* X, const void* W, const void* S, const void* B,
                         void* Y, uint32_t M, uint32_t N, uint32_t K, uint32_t G, int out_bf16,
                         hipStream_t st) {
    switch (mode) {
        case 0: return by_shape<Q4X>(G, X, W, S, B, Y, M, N, K, out_bf16, st);
        case 1: return by_shape<Q8X>(G, X, W, S, B, Y, M, N, K, out_bf16, st);
        case 2: return by_shape<Q4F>(G, X, W, S, B, Y, M, N, K, out_bf16, st);
        case 3: return by_shape<BF16>(64, X, W, S, B, Y, M, N, K, out_bf16, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace miori
