// Prefill GEMM on bf16 MFMA for gfx950: C[M][N] = A[M][K] . B[N][K]^T with
// fp32 accumulation, B either the bf16 weight cache (row-major [N][K]) or the
// 4-bit MLX-affine weights dequantised to bf16 on the fly.
//
// Replaces shaders/gemm_mpp.metal:36-73 (gemm_mpp / gemm_mpp32, Apple MPP
// matmul2d on a tile-major bf16 cache) and, for the fused variant, the
// two-step dequant_tile + gemm_mpp of src/engine.cpp:144-146, 508-518.
//
// Four kernels share the LDS layout and the epilogue. gemm_kernel and
// gemm_pcq_kernel run one MFMA sequence (32x32x16), so their results for one
// K split are bit-identical; gemm_pc_kernel and gemm_w8_kernel run 16x16x32
// MFMAs (one order, bit-identical with each other), whose results differ
// from those by fp32 rounding of the k sums:
//  * gemm_kernel: four waves, each loading (DMA) and multiplying; the 64x64
//    bf16 small-grid tiles, and (tuning overrides only) the 256x256 and
//    192x256 bf16 tiles and the fused form with B dequantised into LDS.
//  * gemm_pc_kernel: bf16, eight waves, four consumers that only read LDS and
//    run MFMAs, four producers that DMA the operands (256x128, 128x128).
//  * gemm_pcq_kernel: fused 4-bit, eight waves, producers DMA A, each
//    consumer loads and dequantises its own strip of B in registers
//    (256x128, 128x128).
//  * gemm_w8_kernel: bf16, eight waves that each DMA and multiply, 16x16x32
//    MFMAs with gemm_pc_kernel's order (bit-identical with it): the 256x256
//    and 192x256 tiles.
// Common structure (K in steps of 64):
//  * Operand tiles move HBM/L2 -> LDS with global_load_lds_dwordx4 (gfx950
//    direct-to-LDS DMA): no staging registers, several K tiles in flight
//    (LDS ring, one workgroup barrier per step, vmcnt waits placed by hand).
//  * Rows in LDS are 128 bytes (64 bf16); the 16-byte chunk kb of row r sits
//    at slot kb ^ (r & 7) ^ ((r >> 3) & 1), so the 32 rows of an MFMA
//    fragment read hit distinct banks. The DMA writes lanes in order, so the
//    swizzle is applied by choosing which global chunk each lane fetches.
//  * gemm_kernel / gemm_pcq_kernel: v_mfma_f32_32x32x16_bf16; in k-step s of
//    a 64-wide K tile, lane half h = lane/32 of a fragment holds chunk 4h + s
//    (any k order is valid as long as A and B use the same one).
//    gemm_pc_kernel: v_mfma_f32_16x16x32_bf16, lane quarter q holds chunk
//    2q + s in k-step s. Per flop the 16x16 MFMA reads and writes half the
//    accumulator registers: 42.5 -> 37.3-39.9 us at M=1024, N=8192, K=2048,
//    with a shader clock ~3% higher over the replay and fewer cycles.
//  * Fused 4-bit B is dequantised to bf16_rne(q*s + b), the exact bf16 value
//    the dequant kernels write, so the MFMA operands equal the two-step
//    path's, and so do the results wherever the two-step product runs on
//    gemm_kernel (its small-grid tiles).
//  * Workgroups are renumbered so each XCD (workgroup id mod 8) works on a
//    contiguous block of output tiles and keeps its operand slabs in its own
//    L2. The epilogue stages the fp32 tile through LDS so every lane stores
//    8 consecutive outputs (one 16-byte bf16 store).
#include "common.hpp"
#include "kernels.hpp"

#include <stdlib.h>

#include <type_traits>

namespace miori {

namespace {

constexpr int BK = 64;
constexpr int ROWB = BK * 2;  // bytes per LDS row of a bf16 tile

__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t kb) {
    return r * ROWB + ((kb ^ (r & 7u) ^ ((r >> 3) & 1u)) << 4);
}

// Buffer loads as inline asm (the compiler inserts no waits for them; the
// caller places s_waitcnt vmcnt by hand and ties the result below it).
__device__ __forceinline__ void asm_load16(u32x4_t& d, rsrc_t r, uint32_t off) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(d) : "v"(off), "s"(r));
}
__device__ __forceinline__ void asm_load_u16(uint32_t& d, rsrc_t r, uint32_t off) {
    asm volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(d) : "v"(off), "s"(r));
}
__device__ __forceinline__ void tie(u32x4_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void tie(uint32_t& v) { asm volatile("" : "+v"(v)); }
// After the wait that covers a slot's LDS fragment reads, the slot's
// registers are tied before its MFMAs: each read's output then stays live
// until that point, so the compiler cannot give its register to other code
// while the read is still in flight (it would if the output were dead, as in
// a build with the MFMAs compiled out, which faulted the GPU).
__device__ __forceinline__ void tie(bf16x8_t& v) { asm volatile("" : "+v"(v)); }

template <int BM, int BN, bool Q4, int G>
struct Cfg {
    static constexpr int WM = BM / 2, WN = BN / 2;   // wave tile
    static constexpr int TM = WM / 32, TN = WN / 32; // 32x32 MFMA tiles per wave
    static constexpr int A_ST = BM * ROWB;
    static constexpr int B_ST = BN * ROWB;
    static constexpr int RAW_ST = BN * 32;          // 4-bit codes: 32 B per row per K tile
    // scale/bias bytes per row per K tile in LDS: the DMA writes one dword per
    // lane whatever the load size, so each row gets a 4-byte slot (G = 32: the
    // two groups of the K tile; otherwise one bf16 in the low half)
    static constexpr int SB_W = 4;
    static constexpr int SB_ST = BN * SB_W;
    // LDS ring depth: 3 stages, or 2 when three 256x256 stages would not fit
    static constexpr int NST = (!Q4 && BM * BN > 256 * 128) ? 2 : 3;
    static constexpr int A_OFF = 0;
    static constexpr int B_OFF = NST * A_ST;        // bf16 B ring
    static constexpr int RAW_OFF = B_OFF + NST * B_ST;
    static constexpr int S_OFF = RAW_OFF + 3 * RAW_ST;
    static constexpr int BI_OFF = S_OFF + 3 * SB_ST;
    static constexpr int LDS = Q4 ? BI_OFF + 3 * SB_ST : RAW_OFF;
    // DMA instructions per wave per K tile (each moves 64 lanes x size bytes)
    static constexpr int A_INS = BM / 32;
    static constexpr int B_INS = Q4 ? 0 : BN / 32;
    static constexpr int RAW_INS = Q4 ? BN * 32 / 1024 / 4 : 0;             // per wave
    static constexpr int SB_INS = Q4 ? BN / 64 / 2 : 0;   // per wave (s or b), 64 rows each
    static constexpr int L = A_INS + B_INS + RAW_INS + SB_INS;
    static_assert(!Q4 || BN == 128, "fused dequant maps one thread per 32-code chunk");
    // epilogue: each wave stages EPR rows of its fp32 tile at a time
    static constexpr int EPR = (4 * WM * (WN + 8) * 4 <= LDS) ? WM : 32;
    static_assert(4 * EPR * (WN + 8) * 4 <= LDS, "epilogue staging fits in the stage buffers");
    static_assert(!Q4 || NST == 3, "the fused pipeline is written for three stages");
};

// Epilogue of one wave's WM x WN accumulator tile, through LDS (the stage
// buffers are free once every wave is past the main loop; the caller
// synchronises the workgroup first). Accumulator element e of lane l is row
// 8*(e/4) + 4*(l/32) + e%4, column l%32 of its 32x32 tile. Each wave writes
// EPR rows of its fp32 tile at a time to its own LDS region (row stride
// WN + 8 floats: the two half-waves of a write land on disjoint banks), then
// reads them back 8 columns per lane and stores 16 bytes (bf16) or 2 x 16
// bytes (fp32) per lane, or, split-K, the fp32 partial tile to part[ksp].
// Only this wave touches its region, and a wave's LDS accesses complete in
// order, so passes need no barrier.
// (stage(ep, ps) writes the pass-ps rows of the wave's accumulators to ep,
// row stride CF::WN + 8 floats)
template <class CF, class Stage>
__device__ __forceinline__ void store_wave_rows(Stage&& stage, uint8_t* lds, uint32_t wave,
                                                uint32_t lane, uint32_t wm, uint32_t wn,
                                                uint32_t m0, uint32_t n0, uint32_t M, uint32_t N,
                                                void* __restrict__ C, int out_bf16,
                                                float* __restrict__ part, uint32_t ksp,
                                                uint32_t SK) {
    constexpr uint32_t RS = CF::WN + 8;  // floats per LDS row
    constexpr int EPR = CF::EPR;         // rows per pass
    float* ep = reinterpret_cast<float*>(lds) + wave * (EPR * RS);
    constexpr uint32_t CPR = CF::WN / 8;          // 8-column chunks per row
    constexpr uint32_t RPI = 64 / CPR;            // rows per read-back iteration
    const uint32_t cc = lane % CPR, rr = lane / CPR;
    const uint32_t col = n0 + wn * CF::WN + cc * 8u;
    auto store8 = [&](uint32_t row, f32x4_t v0, f32x4_t v1) {
        if (out_bf16) {
            u32x4_t o;
            bf16x2_t p0 = {(__bf16)v0[0], (__bf16)v0[1]}, p1 = {(__bf16)v0[2], (__bf16)v0[3]};
            bf16x2_t p2 = {(__bf16)v1[0], (__bf16)v1[1]}, p3 = {(__bf16)v1[2], (__bf16)v1[3]};
            o[0] = __builtin_bit_cast(uint32_t, p0);
            o[1] = __builtin_bit_cast(uint32_t, p1);
            o[2] = __builtin_bit_cast(uint32_t, p2);
            o[3] = __builtin_bit_cast(uint32_t, p3);
            *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(C) + (size_t)row * N + col) = o;
        } else {
            float* dst = reinterpret_cast<float*>(C) + (size_t)row * N + col;
            *reinterpret_cast<f32x4_t*>(dst) = v0;
            *reinterpret_cast<f32x4_t*>(dst + 4) = v1;
        }
    };
    static_assert(CF::WM % EPR == 0 && EPR % 32 == 0, "passes cover whole 32-row MFMA tiles");
#pragma unroll
    for (int ps = 0; ps < CF::WM / EPR; ++ps) {
        stage(ep, ps);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const uint32_t rbase = m0 + wm * CF::WM + ps * EPR;  // first output row of this pass
        if (SK == 1) {
#pragma unroll 4
            for (uint32_t r = rr; r < (uint32_t)EPR; r += RPI) {
                const uint32_t row = rbase + r;
                const f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(ep + r * RS + cc * 8u);
                const f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(ep + r * RS + cc * 8u + 4u);
                if (row < M && col < N) store8(row, v0, v1);
            }
        } else {
            // Split-K: the fp32 partial tile goes to part[ksp]; a second kernel
            // adds the SK partials in split order (deterministic, and spread
            // over every CU rather than funnelled through one workgroup per tile).
            for (uint32_t r = rr; r < (uint32_t)EPR; r += RPI) {
                const uint32_t row = rbase + r;
                if (row >= M || col >= N) continue;
                float* dst = part + ((size_t)ksp * M + row) * N + col;
                *reinterpret_cast<f32x4_t*>(dst) = *reinterpret_cast<const f32x4_t*>(ep + r * RS + cc * 8u);
                *reinterpret_cast<f32x4_t*>(dst + 4) = *reinterpret_cast<const f32x4_t*>(ep + r * RS + cc * 8u + 4u);
            }
        }
        // the next pass rewrites this region: its reads must have returned
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
}

// 32x32 MFMA tiles: element e of lane l is row 8*(e/4) + 4*(l/32) + e%4,
// column l%32 of its tile.
template <class CF>
__device__ __forceinline__ void store_wave_tile(f32x16_t (&acc)[CF::TM][CF::TN], uint8_t* lds,
                                                uint32_t wave, uint32_t lane, uint32_t wm,
                                                uint32_t wn, uint32_t m0, uint32_t n0, uint32_t M,
                                                uint32_t N, void* __restrict__ C, int out_bf16,
                                                float* __restrict__ part, uint32_t ksp,
                                                uint32_t SK) {
    constexpr uint32_t RS = CF::WN + 8;
    constexpr int EPR = CF::EPR;
    auto stage = [&](float* ep, int ps) {
#pragma unroll
        for (int i = 0; i < CF::TM; ++i) {
            if (i < ps * (EPR / 32) || i >= (ps + 1) * (EPR / 32)) continue;
#pragma unroll
            for (int j = 0; j < CF::TN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint32_t r = (i - ps * (EPR / 32)) * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                    ep[r * RS + j * 32 + (lane & 31u)] = acc[i][j][e];
                }
        }
    };
    store_wave_rows<CF>(stage, lds, wave, lane, wm, wn, m0, n0, M, N, C, out_bf16, part, ksp, SK);
}

// 16x16 MFMA tiles (WM / 16 x WN / 16 of them): element e of lane l is row
// 4*(l/16) + e, column l%16 of its tile.
template <class CF>
__device__ __forceinline__ void store_wave_tile16(f32x4_t (&acc)[CF::WM / 16][CF::WN / 16],
                                                  uint8_t* lds, uint32_t wave, uint32_t lane,
                                                  uint32_t wm, uint32_t wn, uint32_t m0,
                                                  uint32_t n0, uint32_t M, uint32_t N,
                                                  void* __restrict__ C, int out_bf16,
                                                  float* __restrict__ part, uint32_t ksp,
                                                  uint32_t SK) {
    constexpr uint32_t RS = CF::WN + 8;
    constexpr int EPR = CF::EPR;
    auto stage = [&](float* ep, int ps) {
#pragma unroll
        for (int i = 0; i < CF::WM / 16; ++i) {
            if (i < ps * (EPR / 16) || i >= (ps + 1) * (EPR / 16)) continue;
#pragma unroll
            for (int j = 0; j < CF::WN / 16; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t r = (i - ps * (EPR / 16)) * 16 + 4 * (lane >> 4) + e;
                    ep[r * RS + j * 16 + (lane & 15u)] = acc[i][j][e];
                }
        }
    };
    store_wave_rows<CF>(stage, lds, wave, lane, wm, wn, m0, n0, M, N, C, out_bf16, part, ksp, SK);
}

template <int BM, int BN, bool Q4, int G>
__global__ __launch_bounds__(256) void gemm_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
    const uint32_t* __restrict__ q, const uint16_t* __restrict__ s,
    const uint16_t* __restrict__ bsc, void* __restrict__ C, uint32_t M, uint32_t N,
    uint32_t K, int out_bf16, uint32_t tiles_m, int remap, float* __restrict__ part,
    uint32_t SK, uint32_t ntiles) {
    using CF = Cfg<BM, BN, Q4, G>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[CF::LDS];

    const uint32_t t = threadIdx.x;
    const uint32_t lane = t & 63u, wave = t >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1u;

    uint32_t pid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if (remap && (nwg & 7u) == 0) pid = (pid & 7u) * (nwg >> 3) + (pid >> 3);
    // Split-K: workgroup pid computes K tiles [kt0, kt0 + KT) of output tile
    // pid % ntiles; KT below counts this workgroup's tiles only.
    const uint32_t tile = pid % ntiles, ksp = pid / ntiles;
    const uint32_t tm = tile % tiles_m, tn = tile / tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t KT_ALL = K / BK;
    const uint32_t kt0 = KT_ALL * ksp / SK;
    const uint32_t KT = KT_ALL * (ksp + 1) / SK - kt0;
    const uint32_t ng = Q4 ? K / G : 1;

    // Per-lane DMA source rows (clamped: rows past M / N load valid memory and
    // their results are never stored).
    // One DMA group: A(kt) into A stage `stage_a`; bf16 B(kt) into B stage
    // `stage_b`, or, fused, the raw codes + scale/bias of K tile `kr` into raw
    // slot `stage_b`. with_a = false issues only the B part.
    auto issue = [&](uint32_t kt, uint32_t stage_a, uint32_t kr, uint32_t stage_b, bool with_a) {
        if (with_a) {
            // A: instruction p of this wave covers 8 rows; lane -> (row, physical chunk)
#pragma unroll
            for (int p = 0; p < CF::A_INS; ++p) {
                const uint32_t r0 = (wave * CF::A_INS + p) * 8u;
                const uint32_t r = r0 + (lane >> 3);
                const uint32_t kb = (lane & 7u) ^ (r & 7u) ^ ((r >> 3) & 1u);
                const uint32_t row = min(m0 + r, M - 1u);
                dma16(A + (size_t)row * K + (kt0 + kt) * BK + kb * 8u,
                      lds + CF::A_OFF + stage_a * CF::A_ST + r0 * ROWB);
            }
        }
        if constexpr (!Q4) {
#pragma unroll
            for (int p = 0; p < CF::B_INS; ++p) {
                const uint32_t r0 = (wave * CF::B_INS + p) * 8u;
                const uint32_t r = r0 + (lane >> 3);
                const uint32_t kb = (lane & 7u) ^ (r & 7u) ^ ((r >> 3) & 1u);
                const uint32_t row = min(n0 + r, N - 1u);
                dma16(B + (size_t)row * K + (kt0 + kt) * BK + kb * 8u, lds + CF::B_OFF + stage_b * CF::B_ST + r0 * ROWB);
            }
        } else {
            // raw codes of K tile kt (clamped to a valid tile): row r, chunk c at slot 2r + c
            const uint32_t ktc = kt0 + min(kr, KT - 1u);
            {
                const uint32_t slot = wave * 64u + lane;
                const uint32_t r = slot >> 1, c = slot & 1u;
                const uint32_t row = min(n0 + r, N - 1u);
                dma16(q + (size_t)row * (K / 8) + ktc * 8u + c * 4u,
                      lds + CF::RAW_OFF + stage_b * CF::RAW_ST + wave * 1024u);
            }
            // scales (waves 0,1) or biases (waves 2,3): 64 rows per instruction
            {
                const uint32_t r = (wave & 1u) * 64u + lane;
                const uint32_t row = min(n0 + r, N - 1u);
                const uint16_t* src = (wave < 2) ? s : bsc;
                uint8_t* dst = lds + ((wave < 2) ? CF::S_OFF : CF::BI_OFF) + stage_b * CF::SB_ST +
                               (wave & 1u) * 64u * CF::SB_W;
                if constexpr (G == 32)
                    dma4(src + (size_t)row * ng + ktc * 2u, dst);
                else
                    dma2(src + (size_t)row * ng + ktc * BK / G, dst);
            }
        }
    };

    // bf16 path: DMA instruction p (0 <= p < L) of group kt into stage st, so
    // a group can be spread over the MFMA stream. Issued between MFMAs, so it
    // must cost no vector instructions: the per-lane byte offsets (row and
    // swizzled chunk) are computed once, the K-slice base is a wave-uniform
    // pointer (global_load_lds with an SGPR base and a VGPR offset), and the
    // LDS destination comes from the wave index held in an SGPR, so M0 is set
    // by scalar instructions.
    const uint32_t wave_s = __builtin_amdgcn_readfirstlane(wave);
    uint32_t ab_off[Q4 ? 1 : CF::L];
    if constexpr (!Q4) {
#pragma unroll
        for (int p = 0; p < CF::L; ++p) {
            const bool is_a = p < CF::A_INS;
            const int pp = is_a ? p : p - CF::A_INS;
            const uint32_t r = (wave * (is_a ? CF::A_INS : CF::B_INS) + pp) * 8u + (lane >> 3);
            const uint32_t kb = (lane & 7u) ^ (r & 7u) ^ ((r >> 3) & 1u);
            const uint32_t row = is_a ? min(m0 + r, M - 1u) : min(n0 + r, N - 1u);
            ab_off[p] = row * K * 2u + kb * 16u;
        }
    }
    auto issue_one = [&](uint32_t kt, uint32_t st, int p) {
        const bool is_a = p < CF::A_INS;
        const int pp = is_a ? p : p - CF::A_INS;
        const uint32_t r0 = (wave_s * (is_a ? CF::A_INS : CF::B_INS) + pp) * 8u;
        const uint8_t* base = reinterpret_cast<const uint8_t*>(is_a ? A : B) + (size_t)(kt0 + kt) * BK * 2u;
        dma16(base + ab_off[p], lds + (is_a ? CF::A_OFF + st * CF::A_ST : CF::B_OFF + st * CF::B_ST) + r0 * ROWB);
    };

    // Fused 4-bit: dequantise raw slot `stage` into bf16 buffer bb.
    auto dequant_tile = [&](uint32_t stage, uint32_t bb) {
        const uint32_t r = t >> 1, c = t & 1u;
        const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(lds + CF::RAW_OFF + stage * CF::RAW_ST + t * 16u);
        const uint8_t* sp = lds + CF::S_OFF + stage * CF::SB_ST + r * CF::SB_W;
        const uint8_t* bp = lds + CF::BI_OFF + stage * CF::SB_ST + r * CF::SB_W;
        const uint32_t sub = (G == 32) ? c * 2u : 0u;  // G = 32: the chunk's own group
        const float sc = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(sp + sub));
        const float bi = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(bp + sub));
        uint8_t* dst = lds + CF::B_OFF + bb * CF::B_ST;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t v = raw[w];
            const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
            float f[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f[2 * j] = fmaf((float)((lo >> (8 * j)) & 0xFFu), sc, bi);
                f[2 * j + 1] = fmaf((float)((hi >> (8 * j)) & 0xFFu), sc, bi);
            }
            u32x4_t o;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                bf16x2_t p = {(__bf16)f[2 * j], (__bf16)f[2 * j + 1]};
                o[j] = __builtin_bit_cast(uint32_t, p);
            }
            *reinterpret_cast<u32x4_t*>(dst + swz(r, c * 4u + w)) = o;
        }
    };

    f32x16_t acc[CF::TM][CF::TN];
#pragma unroll
    for (int i = 0; i < CF::TM; ++i)
#pragma unroll
        for (int j = 0; j < CF::TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    // MFMA fragments, double-buffered: k-step ks+1 is read while ks runs.
    // The reads are issued as inline asm with hand-placed lgkmcnt waits (the
    // compiler's own waits drain every LDS read before each MFMA group). A
    // fragment row r = (multiple of 16) + lane%32, so its swizzle term is
    // f = (lane & 7) ^ ((lane >> 3) & 1) for every fragment, and k-step ks of
    // lane half h reads chunk (4h ^ f) ^ ks.
    bf16x8_t af[2][CF::TM], bf[2][CF::TN];
    const uint32_t fsw = (lane & 7u) ^ ((lane >> 3) & 1u);
    const uint32_t c0 = (4u * (lane >> 5)) ^ fsw;
    const uint32_t lrow = (lane & 31u) * ROWB;
    auto read_frags = [&](uint32_t kt, int ks, int slot) {
        const uint32_t chunk = ((c0 ^ (uint32_t)ks) << 4) + lrow;
        const uint32_t a_addr = CF::A_OFF + (kt % CF::NST) * CF::A_ST + wm * CF::WM * ROWB + chunk;
        const uint32_t b_addr = CF::B_OFF + (kt % CF::NST) * CF::B_ST + wn * CF::WN * ROWB + chunk;
#pragma unroll
        for (int i = 0; i < CF::TM; ++i)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[slot][i]) : "v"(a_addr), "i"(i * 32 * ROWB));
#pragma unroll
        for (int j = 0; j < CF::TN; ++j)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(bf[slot][j]) : "v"(b_addr), "i"(j * 32 * ROWB));
    };
    constexpr int NFR = CF::TM + CF::TN;  // LDS reads per k-step
    // With 8 reads per k-step a full double buffer would put 16 reads in
    // flight, more than the 4-bit lgkm counter holds (15). This variant
    // issues the A fragments of the next k-step, waits until only they are
    // outstanding (the previous slot has landed), then issues the B ones.
    auto read_frags_capped = [&](uint32_t kt, int ks, int slot) {
        const uint32_t chunk = ((c0 ^ (uint32_t)ks) << 4) + lrow;
        const uint32_t a_addr = CF::A_OFF + (kt % CF::NST) * CF::A_ST + wm * CF::WM * ROWB + chunk;
        const uint32_t b_addr = CF::B_OFF + (kt % CF::NST) * CF::B_ST + wn * CF::WN * ROWB + chunk;
#pragma unroll
        for (int i = 0; i < CF::TM; ++i)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[slot][i]) : "v"(a_addr), "i"(i * 32 * ROWB));
        asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(CF::TM) : "memory");
#pragma unroll
        for (int j = 0; j < CF::TN; ++j)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(bf[slot][j]) : "v"(b_addr), "i"(j * 32 * ROWB));
    };
    auto mfmas = [&](int slot) {
#pragma unroll
        for (int i = 0; i < CF::TM; ++i) tie(af[slot][i]);
#pragma unroll
        for (int j = 0; j < CF::TN; ++j) tie(bf[slot][j]);
#pragma unroll
        for (int i = 0; i < CF::TM; ++i)
#pragma unroll
            for (int j = 0; j < CF::TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bf[slot][j],
                                                                    acc[i][j], 0, 0, 0);
    };
    // The MFMAs of one k-step with DMA instructions [P0, P1) of group dkt
    // (stage dst) spread evenly between them: the wave issues each DMA while
    // the matrix core is busy instead of stalling on a burst of them.
    constexpr int NM = CF::TM * CF::TN;
    constexpr int PER = (CF::L + 2) / 3;  // DMA instructions per k-step (k-steps 0..2)
    // (small tiles have fewer MFMAs than DMA instructions per k-step: then
    // several DMAs follow one MFMA)
    auto mfmas_dma = [&](int slot, bool dma, uint32_t dkt, uint32_t dst, auto p0c, auto p1c) {
        constexpr int P0 = decltype(p0c)::value, P1 = decltype(p1c)::value;
        constexpr int CNT = P1 - P0;
#pragma unroll
        for (int i = 0; i < CF::TM; ++i) tie(af[slot][i]);
#pragma unroll
        for (int j = 0; j < CF::TN; ++j) tie(bf[slot][j]);
#pragma unroll
        for (int q = 0; q < NM; ++q) {
            const int i = q / CF::TN, j = q % CF::TN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bf[slot][j],
                                                                acc[i][j], 0, 0, 0);
            if constexpr (CNT > 0) {
                // DMAs [P0 + q*CNT/NM, P0 + (q+1)*CNT/NM) after MFMA q
#pragma unroll
                for (int p = (q * CNT) / NM; p < ((q + 1) * CNT) / NM; ++p)
                    if (dma) issue_one(dkt, dst, P0 + p);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Pipeline. Group p = {A(p), B(p)} (bf16) or {A(p), raw(p+1)} (fused; the
    // codes travel one group early and are dequantised two tiles ahead into a
    // 3-deep bf16 ring). In step kt the barrier sits before the last k-step,
    // where tile kt's LDS reads are done: it publishes group kt+1, frees stage
    // kt % 3, and the first fragments of tile kt+1 are read while the last
    // MFMAs of kt run. Fused: groups 0..2 are issued up front and group kt+3
    // right after the barrier of step kt. bf16: groups 0 and 1 up front, and
    // group kt+2 interleaved with the MFMAs of tile kt.
    if constexpr (Q4) {
        issue(0, 0, 0, 0, false);  // raw(0)
        issue(0, 0, 1, 1, true);
        if (KT > 1) issue(1, 1, 2, 2, true);
        if (KT > 1) wait_vm<CF::L>(); else wait_vm<0>();
        barrier_lds();
        dequant_tile(0, 0);
        if (KT > 1) dequant_tile(1, 1);
        barrier_lds();             // raw slot 0 is free again
        if (KT > 2) issue(2, 2, 3, 0, true);
    } else {
        issue(0, 0, 0, 0, true);
        if (KT > 1) issue(1, 1, 1, 1, true);
        if (KT > 1) wait_vm<CF::L>(); else wait_vm<0>();
        barrier_lds();
    }
    read_frags(0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (Q4) {
        for (uint32_t kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int ks = 0; ks < BK / 16 - 1; ++ks) {
                read_frags(kt, ks + 1, (ks + 1) & 1);
                asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(NFR) : "memory");  // k-step ks has landed
                __builtin_amdgcn_sched_barrier(0);
                mfmas(ks & 1);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (kt + 1 < KT) {
                if (kt + 2 < KT) wait_vm<CF::L>(); else wait_vm<0>();
                barrier_lds();  // also completes the reads of the last k-step
                if (kt + 2 < KT) dequant_tile((kt + 2) % 3, (kt + 2) % 3);
                if (kt + 3 < KT) issue(kt + 3, kt % 3, kt + 4, (kt + 4) % 3, true);
                read_frags(kt + 1, 0, 0);
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            __builtin_amdgcn_sched_barrier(0);
            mfmas((BK / 16 - 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else if constexpr (CF::NST == 2) {
        // bf16, two stages: group kt+1 is the only one in flight during tile
        // kt. The barrier of step kt (before its last k-step, whose fragments
        // are already in registers) publishes group kt+1 and frees stage
        // kt % 2, so group kt+2 is issued into it during that last k-step.
        for (uint32_t kt = 0; kt < KT; ++kt) {
            const bool dma = kt + 2 < KT;
            read_frags_capped(kt, 1, 1);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(0);
            __builtin_amdgcn_sched_barrier(0);
            read_frags_capped(kt, 2, 0);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(1);
            __builtin_amdgcn_sched_barrier(0);
            read_frags_capped(kt, 3, 1);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(0);
            __builtin_amdgcn_sched_barrier(0);
            if (kt + 1 < KT) {
                wait_vm<0>();
                barrier_lds();  // also completes the reads of the last k-step
                read_frags(kt + 1, 0, 0);
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            __builtin_amdgcn_sched_barrier(0);
            using I0 = std::integral_constant<int, 0>;
            mfmas_dma(1, dma, kt + 2, kt % 2, I0{}, std::integral_constant<int, CF::L>{});
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        // bf16: group kt+2 goes into stage (kt+2) % 3, freed by the barrier of
        // step kt-1, spread over k-steps 0..2 of tile kt. The barrier of step
        // kt then needs group kt+1, which is everything but the last L
        // instructions.
        for (uint32_t kt = 0; kt < KT; ++kt) {
            const bool dma = kt + 2 < KT;
            const uint32_t dkt = kt + 2, dst = (kt + 2) % 3;
            using I0 = std::integral_constant<int, 0>;
            read_frags(kt, 1, 1);
            asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(NFR) : "memory");
            __builtin_amdgcn_sched_barrier(0);
            mfmas_dma(0, dma, dkt, dst, I0{}, std::integral_constant<int, (PER < CF::L ? PER : CF::L)>{});
            read_frags(kt, 2, 0);
            asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(NFR) : "memory");
            __builtin_amdgcn_sched_barrier(0);
            mfmas_dma(1, dma, dkt, dst, std::integral_constant<int, (PER < CF::L ? PER : CF::L)>{},
                      std::integral_constant<int, (2 * PER < CF::L ? 2 * PER : CF::L)>{});
            read_frags(kt, 3, 1);
            asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(NFR) : "memory");
            __builtin_amdgcn_sched_barrier(0);
            mfmas_dma(0, dma, dkt, dst, std::integral_constant<int, (2 * PER < CF::L ? 2 * PER : CF::L)>{},
                      std::integral_constant<int, CF::L>{});
            if (kt + 1 < KT) {
                if (dma) wait_vm<CF::L>(); else wait_vm<0>();
                barrier_lds();  // also completes the reads of the last k-step
                read_frags(kt + 1, 0, 0);
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            __builtin_amdgcn_sched_barrier(0);
            mfmas(1);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Every fragment read has landed before any epilogue code runs: the last
    // k-step already waited for them, but the epilogue's address arithmetic
    // must not be scheduled above a point where that holds on every path.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    __syncthreads();
    store_wave_tile<CF>(acc, lds, wave, lane, wm, wn, m0, n0, M, N, C, out_bf16, part, ksp, SK);
}

// Producer / consumer form of the bf16 GEMM: eight waves, two per SIMD.
// Waves 0-3 (consumers, 2x2 grid of (BM/2) x (BN/2) tiles) only read MFMA
// fragments from LDS and run the MFMAs; waves 4-7 (producers) fill the
// 3-stage LDS ring with A and B by global -> LDS DMA, two tiles in flight
// behind the one being multiplied. A consumer never waits on vector memory,
// so while one wave of a SIMD waits for its operands the other keeps the
// matrix core busy. At the barrier of tile kt the consumers have read all of
// tile kt (stage kt % 3 is free) and tiles kt+1 and kt+2 are complete in LDS;
// the producers then fill the freed stage with tile kt+3. The consumers run
// 16x16x32 MFMAs (two k-steps per K tile); results differ from gemm_kernel's
// 32x32x16 ones by fp32 rounding of the k sums.
template <int BM, int BN>
__global__ __launch_bounds__(512) void gemm_pc_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C,
    uint32_t M, uint32_t N, uint32_t K, int out_bf16, uint32_t tiles_m, int remap,
    float* __restrict__ part, uint32_t SK, uint32_t ntiles) {
    using CF = Cfg<BM, BN, false, 64>;
    static_assert(CF::NST == 3, "the producer / consumer ring has three stages");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[CF::LDS];

    const uint32_t t = threadIdx.x;
    const uint32_t lane = t & 63u, wave = t >> 6;
    const bool producer = wave >= 4;
    const uint32_t w4 = wave & 3u;
    const uint32_t wm = w4 >> 1, wn = w4 & 1u;

    uint32_t pid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if (remap && (nwg & 7u) == 0) pid = (pid & 7u) * (nwg >> 3) + (pid >> 3);
    const uint32_t tile = pid % ntiles, ksp = pid / ntiles;
    const uint32_t tm = tile % tiles_m, tn = tile / tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t KT_ALL = K / BK;
    const uint32_t kt0 = KT_ALL * ksp / SK;
    const uint32_t KT = KT_ALL * (ksp + 1) / SK - kt0;

    constexpr int TM = CF::WM / 16, TN = CF::WN / 16;  // 16x16 MFMA tiles per wave
    f32x4_t acc[TM][TN];

    if (producer) {
        // DMA: producer wave w4 moves 8-row groups [w4*PA, (w4+1)*PA) of the A
        // tile and [w4*PB, (w4+1)*PB) of the B tile; one instruction = 8 rows
        // x 128 bytes, lane -> (row, swizzled chunk).
        constexpr int PA = BM / 32, PB = BN / 32, PL = PA + PB;
        const uint32_t w4s = __builtin_amdgcn_readfirstlane(w4);
        uint32_t off[PL];
#pragma unroll
        for (int p = 0; p < PL; ++p) {
            const bool is_a = p < PA;
            const uint32_t r = (w4 * (is_a ? PA : PB) + (is_a ? p : p - PA)) * 8u + (lane >> 3);
            const uint32_t kb = (lane & 7u) ^ (r & 7u) ^ ((r >> 3) & 1u);
            const uint32_t row = is_a ? min(m0 + r, M - 1u) : min(n0 + r, N - 1u);
            off[p] = row * K * 2u + kb * 16u;
        }
        auto issue = [&](uint32_t kt, uint32_t st) {
#pragma unroll
            for (int p = 0; p < PL; ++p) {
                const bool is_a = p < PA;
                const uint32_t r0 = (w4s * (is_a ? PA : PB) + (is_a ? p : p - PA)) * 8u;
                const uint8_t* base =
                    reinterpret_cast<const uint8_t*>(is_a ? A : B) + (size_t)(kt0 + kt) * BK * 2u;
                dma16(base + off[p], lds + (is_a ? CF::A_OFF + st * CF::A_ST
                                                 : CF::B_OFF + st * CF::B_ST) + r0 * ROWB);
            }
        };
        issue(0, 0);
        if (KT > 1) issue(1, 1);
        if (KT > 2) issue(2, 2);
        if (KT > 2) wait_vm<2 * PL>(); else if (KT > 1) wait_vm<PL>(); else wait_vm<0>();
        barrier_lds();  // tile 0 has landed
        for (uint32_t kt = 0; kt + 1 < KT; ++kt) {
            if (kt + 2 < KT) wait_vm<PL>(); else wait_vm<0>();
            barrier_lds();  // tile kt+1 has landed; stage kt % 3 is free
            if (kt + 3 < KT) issue(kt + 3, kt % 3);
        }
    } else {
        __builtin_amdgcn_s_setprio(2);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        // 16x16x32 MFMAs, two 32-deep k-steps per K tile. A fragment is 16
        // rows (lane % 16) x 8 k; lane group q = lane / 16 supplies 16-byte
        // chunk 2q + ks of the row in k-step ks, so over a K tile each lane
        // reads the 32 contiguous bytes of k 16q .. 16q+15 (the B operand
        // uses the same map, which is all an MFMA's k sum needs). A fragment
        // row r = (multiple of 16) + lane % 16, so its swizzle term is
        // f = (lane & 7) ^ ((lane >> 3) & 1) for every fragment.
        bf16x8_t af[2][TM], bf[2][TN];
        const uint32_t fsw = (lane & 7u) ^ ((lane >> 3) & 1u);
        const uint32_t c0 = (2u * (lane >> 4)) ^ fsw;
        const uint32_t lrow = (lane & 15u) * ROWB;
        auto frag_base = [&](uint32_t kt, int ks, bool b) {
            const uint32_t chunk = ((c0 ^ (uint32_t)ks) << 4) + lrow;
            return b ? CF::B_OFF + (kt % 3u) * CF::B_ST + wn * CF::WN * ROWB + chunk
                     : CF::A_OFF + (kt % 3u) * CF::A_ST + wm * CF::WM * ROWB + chunk;
        };
        auto read_b = [&](uint32_t kt, int ks, int slot) {
            const uint32_t b_addr = frag_base(kt, ks, true);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(bf[slot][j]) : "v"(b_addr), "i"(j * 16 * ROWB));
        };
        auto read_a = [&](uint32_t kt, int ks, int slot) {
            const uint32_t a_addr = frag_base(kt, ks, false);
#pragma unroll
            for (int i = 0; i < TM; ++i)
                asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[slot][i]) : "v"(a_addr), "i"(i * 16 * ROWB));
        };
        auto read_first = [&](uint32_t kt, int ks, int slot) {
            read_b(kt, ks, slot);
            read_a(kt, ks, slot);
        };
        auto read_next = [&](uint32_t kt, int ks, int slot) {
            if constexpr (TM + TN + TN > 15) asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(15 - TN) : "memory");
            read_b(kt, ks, slot);
            asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(TN) : "memory");
            read_a(kt, ks, slot);
        };
        auto mfmas = [&](int slot) {
#pragma unroll
            for (int i = 0; i < TM; ++i) tie(af[slot][i]);
#pragma unroll
            for (int j = 0; j < TN; ++j) tie(bf[slot][j]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[slot][i], bf[slot][j],
                                                                        acc[i][j], 0, 0, 0);
        };
        barrier_lds();  // tile 0 has landed
        read_first(0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        for (uint32_t kt = 0; kt < KT; ++kt) {
            read_next(kt, 1, 1);  // k-step 0 has landed
            __builtin_amdgcn_sched_barrier(0);
            mfmas(0);
            __builtin_amdgcn_sched_barrier(0);
            if (kt + 1 < KT) {
                barrier_lds();  // completes k-step 1's reads; tile kt+1 has landed
                read_first(kt + 1, 0, 0);
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            __builtin_amdgcn_sched_barrier(0);
            mfmas(1);
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_setprio(0);
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    if (!producer)
        store_wave_tile16<CF>(acc, lds, w4, lane, wm, wn, m0, n0, M, N, C, out_bf16, part, ksp, SK);
}

// Fused 4-bit GEMM with the weight operand straight to registers. Eight
// waves as in gemm_pc_kernel: waves 4-7 only DMA the A tiles into the 3-stage
// LDS ring; consumer wave w (0-3) owns the 32 columns n0 + 32w .. +31 of the
// BM x 128 tile over all BM rows (BM/32 MFMA tiles of 32x32). It loads its
// own 4-bit codes, scales and biases with buffer loads two K tiles ahead,
// dequantises them in registers to the MFMA B fragment (bf16_rne(q*s + b),
// the dequant kernels' value) between its MFMAs, and reads only A from LDS.
//  * B never passes through LDS, and each code is dequantised once: one
//    32-code word per lane per k-step feeds BM/32 MFMAs.
//  * Fragment layout: in k-step ks lane half h = lane/32 holds k chunk
//    4h + ks (the A fragments use the same order), so a lane's four k-steps
//    are 32 consecutive codes of its row: one 16-byte load per K tile.
//  * Rows past N load zeros (buffer loads out of range) and are never stored.
// The MFMA operands and their order per output are those of gemm_kernel, so
// results are bit-identical with the two-step dequant + bf16 GEMM wherever
// that runs on gemm_kernel (its small-grid tiles).
template <int BM>
struct CfgQ {  // wave tile of the fused register-B form, for the epilogue
    static constexpr int WM = BM, WN = 32, TM = BM / 32, TN = 1;
    // rows per epilogue pass: 4 waves x 128 (or 64) rows x 40 floats fit the
    // kernel's LDS (checked in the kernel)
    static constexpr int EPR = BM % 128 == 0 ? 128 : 64;
};

template <int BM, int BN, int G>
__global__ __launch_bounds__(512) void gemm_pcq_kernel(
    const uint16_t* __restrict__ A, const uint32_t* __restrict__ q,
    const uint16_t* __restrict__ s, const uint16_t* __restrict__ bsc, void* __restrict__ C,
    uint32_t M, uint32_t N, uint32_t K, int out_bf16, uint32_t tiles_m, int remap,
    float* __restrict__ part, uint32_t SK, uint32_t ntiles) {
    using CF = Cfg<BM, BN, false, 64>;  // A ring layout of the bf16 form
    using WQ = CfgQ<BM>;
    static_assert(CF::NST == 3 && BN == 128, "three A stages, 128 columns = 4 waves x 32");
    static_assert(4 * WQ::EPR * (WQ::WN + 8) * 4 <= CF::LDS && BM % WQ::EPR == 0, "epilogue fits");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[CF::LDS];

    const uint32_t t = threadIdx.x;
    const uint32_t lane = t & 63u, wave = t >> 6;
    const bool producer = wave >= 4;
    const uint32_t w4 = wave & 3u;

    uint32_t pid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if (remap && (nwg & 7u) == 0) pid = (pid & 7u) * (nwg >> 3) + (pid >> 3);
    const uint32_t tile = pid % ntiles, ksp = pid / ntiles;
    const uint32_t tm = tile % tiles_m, tn = tile / tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t KT_ALL = K / BK;
    const uint32_t kt0 = KT_ALL * ksp / SK;
    const uint32_t KT = KT_ALL * (ksp + 1) / SK - kt0;

    f32x16_t acc[WQ::TM][1];

    if (producer) {
        // producer wave w4 moves 8-row groups [w4*PA, (w4+1)*PA) of the A tile
        constexpr int PA = BM / 32;
        const uint32_t w4s = __builtin_amdgcn_readfirstlane(w4);
        uint32_t off[PA];
#pragma unroll
        for (int p = 0; p < PA; ++p) {
            const uint32_t r = (w4 * PA + p) * 8u + (lane >> 3);
            const uint32_t kb = (lane & 7u) ^ (r & 7u) ^ ((r >> 3) & 1u);
            off[p] = min(m0 + r, M - 1u) * K * 2u + kb * 16u;
        }
        auto issue = [&](uint32_t kt, uint32_t st) {
            const uint8_t* base = reinterpret_cast<const uint8_t*>(A) + (size_t)(kt0 + kt) * BK * 2u;
#pragma unroll
            for (int p = 0; p < PA; ++p)
                dma16(base + off[p], lds + CF::A_OFF + st * CF::A_ST + (w4s * PA + p) * 8u * ROWB);
        };
        issue(0, 0);
        if (KT > 1) issue(1, 1);
        if (KT > 2) issue(2, 2);
        if (KT > 2) wait_vm<2 * PA>(); else if (KT > 1) wait_vm<PA>(); else wait_vm<0>();
        barrier_lds();  // tile 0 has landed
        for (uint32_t kt = 0; kt + 1 < KT; ++kt) {
            if (kt + 2 < KT) wait_vm<PA>(); else wait_vm<0>();
            barrier_lds();  // tile kt+1 has landed; stage kt % 3 is free
            if (kt + 3 < KT) issue(kt + 3, kt % 3);
        }
    } else {
        __builtin_amdgcn_s_setprio(2);
#pragma unroll
        for (int i = 0; i < WQ::TM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][0][e] = 0.f;

        // this lane's weight row and k half
        const uint32_t h = lane >> 5;
        const uint32_t ng = K / G;
        const rsrc_t rq = make_rsrc(q, N * (K / 2u));
        const rsrc_t rs = make_rsrc(s, N * ng * 2u);
        const rsrc_t rb = make_rsrc(bsc, N * ng * 2u);
        const uint32_t n = n0 + w4 * 32u + (lane & 31u);
        const uint32_t qoff = n < N ? n * (K / 2u) + h * 16u : kOOB;
        const uint32_t soff = n < N ? n * ng * 2u : kOOB;
        struct Codes {
            u32x4_t raw;
            uint32_t sc, bi;
        };
        constexpr int PQ = 3;  // vector loads per fetch
        auto fetch = [&](uint32_t kt, Codes& x) {
            const uint32_t kg = (kt0 + kt) * BK + h * 32u;  // first code of the lane's half
            asm_load16(x.raw, rq, qoff == kOOB ? kOOB : qoff + (kt0 + kt) * (BK / 2u));
            const uint32_t so = soff == kOOB ? kOOB : soff + (kg / G) * 2u;
            asm_load_u16(x.sc, rs, so);
            asm_load_u16(x.bi, rb, so);
        };
        auto settle = [](Codes& x) {
            tie(x.raw);
            tie(x.sc);
            tie(x.bi);
        };
        // B fragment of k-step ks from word ks of the codes: elements 2i, 2i+1
        // are nibbles 2i, 2i+1 of the word
        auto deq = [](uint32_t v, float sc, float bi) {
            uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
            tie(lo);
            tie(hi);
            u32x4_t o;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float f0 = fmaf((float)((lo >> (8 * i)) & 0xFFu), sc, bi);
                const float f1 = fmaf((float)((hi >> (8 * i)) & 0xFFu), sc, bi);
                bf16x2_t pr = {(__bf16)f0, (__bf16)f1};
                o[i] = __builtin_bit_cast(uint32_t, pr);
            }
            return __builtin_bit_cast(bf16x8_t, o);
        };

        bf16x8_t af[2][WQ::TM], bq[2];
        float fsc = 0.f, fbi = 0.f;
        const uint32_t fsw = (lane & 7u) ^ ((lane >> 3) & 1u);
        const uint32_t c0 = (4u * h) ^ fsw;
        const uint32_t lrow = (lane & 31u) * ROWB;
        auto read_a = [&](uint32_t kt, int ks, int slot) {
            const uint32_t chunk = ((c0 ^ (uint32_t)ks) << 4) + lrow;
            const uint32_t a_addr = CF::A_OFF + (kt % 3u) * CF::A_ST + chunk;
#pragma unroll
            for (int i = 0; i < WQ::TM; ++i)
                asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[slot][i]) : "v"(a_addr), "i"(i * 32 * ROWB));
        };
        auto scales = [&](const Codes& x) {
            fsc = bf16_bits_to_f32(x.sc);
            fbi = bf16_bits_to_f32(x.bi);
        };
        auto make_b = [&](const Codes& x, int ks, int slot) { bq[slot] = deq(x.raw[ks], fsc, fbi); };
        // (no ties here: they reorder this kernel's MFMA / dequant interleave;
        // every fragment feeds an MFMA of its own k-step, checked by the
        // hazard test on the compiled kernel)
        auto mfmas = [&](int slot) {
#pragma unroll
            for (int i = 0; i < WQ::TM; ++i)
                acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bq[slot], acc[i][0], 0, 0, 0);
        };
        // one MFMA, then up to three VALU instructions (the next k-step's B
        // fragment), so the dequant issues while the matrix core is busy
        auto interleave = [] {
#pragma unroll
            for (int m = 0; m < WQ::TM; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            }
        };
        auto cl = [&](uint32_t kt) { return kt < KT ? kt : KT - 1u; };  // clamped tile
        // Tile kt with cur = codes(kt) (settled; its k-step 0 fragment and
        // scales already made), nxt = codes(kt+1) in flight, fx free: fetch
        // codes(kt+2) into fx, run k-steps 0..2 while making the next
        // k-step's B fragment, then (past the barrier that publishes A(kt+1))
        // wait for codes(kt+1) and make tile kt+1's k-step 0 fragment while
        // k-step 3 runs. (last: no tile follows, so no A fragments are read
        // for one)
        auto step = [&](uint32_t kt, Codes& cur, Codes& nxt, Codes& fx, auto last) {
            fetch(cl(kt + 2), fx);
#pragma unroll
            for (int ks = 0; ks < BK / 16 - 1; ++ks) {
                // at most 15 fragment reads in flight (lgkmcnt's field): with
                // TM = 8 one of k-step ks's reads lands before the next batch
                if constexpr (2 * WQ::TM > 15)
                    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(15 - WQ::TM) : "memory");
                read_a(kt, ks + 1, (ks + 1) & 1);
                asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(WQ::TM) : "memory");  // k-step ks has landed
                __builtin_amdgcn_sched_barrier(0);
                make_b(cur, ks + 1, (ks + 1) & 1);
                mfmas(ks & 1);
                interleave();
                __builtin_amdgcn_sched_barrier(0);
            }
            if (!decltype(last)::value && kt + 1 < KT) {
                barrier_lds();  // completes the last k-step's reads; A(kt+1) has landed
                read_a(kt + 1, 0, 0);
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            wait_vm<PQ>();  // codes(kt+1) have landed; codes(kt+2) may be in flight
            settle(nxt);
            __builtin_amdgcn_sched_barrier(0);
            scales(nxt);
            make_b(nxt, 0, 0);
            mfmas((BK / 16 - 1) & 1);
            interleave();
            __builtin_amdgcn_sched_barrier(0);
        };
        Codes x0, x1, x2;
        fetch(0, x0);
        fetch(cl(1), x1);
        wait_vm<PQ>();
        settle(x0);
        scales(x0);
        make_b(x0, 0, 0);
        barrier_lds();  // A(0) has landed
        read_a(0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t kt = 0;
        using More = std::false_type;
        for (; kt + 3 <= KT; kt += 3) {
            step(kt, x0, x1, x2, More{});
            step(kt + 1, x1, x2, x0, More{});
            step(kt + 2, x2, x0, x1, More{});
        }
        if (kt < KT) {
            step(kt, x0, x1, x2, More{});
            if (kt + 1 < KT) step(kt + 1, x1, x2, x0, std::true_type{});
        }
        // every code set stays live until its last load has landed (the last
        // fetches fill sets that are never read)
        wait_vm<0>();
        settle(x0);
        settle(x1);
        settle(x2);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_setprio(0);
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    if (!producer)
        store_wave_tile<WQ>(acc, lds, w4, lane, 0u, w4, m0, n0, M, N, C, out_bf16, part, ksp, SK);
}

// Eight-wave bf16 GEMM for the tall 192x256 and 256x256 tiles: every wave
// both moves operands and multiplies. The waves form a 2 x 4 grid of
// (BM/2) x 64 tiles on 16x16x32 MFMAs, the fragment map and MFMA order of
// gemm_pc_kernel (so results are bit-identical with it), with accumulators
// small enough for two waves per SIMD: one wave of a SIMD multiplies while
// the other waits for LDS or issues DMA. Operands go global -> LDS by DMA
// through a 2-stage ring (A then B per stage, 112 or 128 KiB); each wave
// issues its share of K tile kt+2 between the MFMAs of tile kt's last k-step,
// right after the barrier that frees that stage. At most 15 fragment reads
// are in flight: a k-step's B reads go first, then a wait for the previous
// k-step's reads, then its A reads.
template <int BM, int BN>
struct CfgW8 {
    static constexpr int WM = BM / 2, WN = BN / 4;  // wave tile
    static constexpr int EPR = 32;                  // epilogue rows per pass
    static constexpr int A_ST = BM * ROWB, B_ST = BN * ROWB, ST = A_ST + B_ST;
    static constexpr int LDS = 2 * ST;
    static constexpr int INS = (BM + BN) / 8;       // DMA instructions per K tile
    static constexpr int PW = INS / 8;              // per wave
};

template <int BM, int BN>
__global__ __launch_bounds__(512) void gemm_w8_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C,
    uint32_t M, uint32_t N, uint32_t K, int out_bf16, uint32_t tiles_m, int remap,
    float* __restrict__ part, uint32_t SK, uint32_t ntiles) {
    using CF = CfgW8<BM, BN>;
    constexpr int TM = CF::WM / 16, TN = CF::WN / 16, NFR = TM + TN, PW = CF::PW;
    static_assert(CF::INS % 8 == 0 && NFR <= 15 && TN <= 15, "DMA split and lgkm range");
    static_assert(8 * CF::EPR * (CF::WN + 8) * 4 <= CF::LDS, "epilogue fits");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[CF::LDS];

    const uint32_t t = threadIdx.x;
    const uint32_t lane = t & 63u, wave = t >> 6;
    const uint32_t wm = wave >> 2, wn = wave & 3u;

    uint32_t pid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if (remap && (nwg & 7u) == 0) pid = (pid & 7u) * (nwg >> 3) + (pid >> 3);
    const uint32_t tile = pid % ntiles, ksp = pid / ntiles;
    const uint32_t tm = tile % tiles_m, tn = tile / tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t KT_ALL = K / BK;
    const uint32_t kt0 = KT_ALL * ksp / SK;
    const uint32_t KT = KT_ALL * (ksp + 1) / SK - kt0;

    // DMA instruction g = wave * PW + p moves 8 rows (lane -> row, swizzled
    // chunk) of A (g < BM/8) or of B; per-lane offsets computed once
    const uint32_t wave_s = __builtin_amdgcn_readfirstlane(wave);
    uint32_t off[PW];
#pragma unroll
    for (int p = 0; p < PW; ++p) {
        const uint32_t g = wave * PW + p;
        const bool is_a = g < (uint32_t)(BM / 8);
        const uint32_t r = (is_a ? g : g - BM / 8) * 8u + (lane >> 3);
        const uint32_t kb = (lane & 7u) ^ (r & 7u) ^ ((r >> 3) & 1u);
        const uint32_t row = is_a ? min(m0 + r, M - 1u) : min(n0 + r, N - 1u);
        off[p] = row * K * 2u + kb * 16u;
    }
    auto issue_one = [&](uint32_t kt, uint32_t st, int p) {
        const uint32_t g = wave_s * PW + p;
        const bool is_a = g < (uint32_t)(BM / 8);
        const uint8_t* base =
            reinterpret_cast<const uint8_t*>(is_a ? A : B) + (size_t)(kt0 + kt) * BK * 2u;
        const uint32_t dst = st * CF::ST + (is_a ? g * 8u * ROWB : CF::A_ST + (g - BM / 8) * 8u * ROWB);
        dma16(base + off[p], lds + dst);
    };
    auto issue = [&](uint32_t kt, uint32_t st) {
#pragma unroll
        for (int p = 0; p < PW; ++p) issue_one(kt, st, p);
    };

    f32x4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    bf16x8_t af[2][TM], bf[2][TN];
    const uint32_t fsw = (lane & 7u) ^ ((lane >> 3) & 1u);
    const uint32_t c0 = (2u * (lane >> 4)) ^ fsw;
    const uint32_t lrow = (lane & 15u) * ROWB;
    // fragments of k-step ks of tile kt into slot: B reads, then (read_next)
    // a wait until the other slot's NFR reads have landed, then A reads
    auto frag_addr = [&](uint32_t kt, int ks, bool b) {
        const uint32_t chunk = ((c0 ^ (uint32_t)ks) << 4) + lrow;
        return (kt & 1u) * CF::ST + (b ? CF::A_ST + wn * CF::WN * ROWB : wm * CF::WM * ROWB) + chunk;
    };
    auto read_b = [&](uint32_t kt, int ks, int slot) {
        const uint32_t b_addr = frag_addr(kt, ks, true);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(bf[slot][j]) : "v"(b_addr), "i"(j * 16 * ROWB));
    };
    auto read_a = [&](uint32_t kt, int ks, int slot) {
        const uint32_t a_addr = frag_addr(kt, ks, false);
#pragma unroll
        for (int i = 0; i < TM; ++i)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[slot][i]) : "v"(a_addr), "i"(i * 16 * ROWB));
    };
    auto read_first = [&](uint32_t kt, int ks, int slot) {  // nothing else in flight
        read_b(kt, ks, slot);
        read_a(kt, ks, slot);
    };
    auto read_next = [&](uint32_t kt, int ks, int slot) {
        if constexpr (NFR + TN > 15) asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(15 - TN) : "memory");
        read_b(kt, ks, slot);
        asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(TN) : "memory");
        read_a(kt, ks, slot);
    };
    // (no ties here: they change this kernel's register allocation and LDS
    // read order; every fragment feeds an MFMA of its own k-step, checked by
    // the hazard test on the compiled kernel)
    auto mfmas_dma = [&](int slot, bool dma, uint32_t dkt, uint32_t dst) {
        constexpr int NM = TM * TN;
#pragma unroll
        for (int q = 0; q < NM; ++q) {
            const int i = q / TN, j = q % TN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[slot][i], bf[slot][j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int p = (q * PW) / NM; p < ((q + 1) * PW) / NM; ++p)
                if (dma) issue_one(dkt, dst, p);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    issue(0, 0);
    if (KT > 1) issue(1, 1);
    if (KT > 1) wait_vm<PW>(); else wait_vm<0>();
    barrier_lds();  // tile 0 has landed
    read_first(0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    for (uint32_t kt = 0; kt < KT; ++kt) {
        read_next(kt, 1, 1);  // k-step 0's reads have landed
        __builtin_amdgcn_sched_barrier(0);
        mfmas_dma(0, false, 0u, 0u);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + 1 < KT) {
            wait_vm<0>();   // this wave's share of tile kt+1 has landed
            barrier_lds();  // k-step 1's reads done everywhere; tile kt+1 visible; stage kt&1 free
            read_first(kt + 1, 0, 0);
        } else {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        __builtin_amdgcn_sched_barrier(0);
        mfmas_dma(1, kt + 2 < KT, kt + 2, kt & 1u);
        __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    store_wave_tile16<CF>(acc, lds, wave, lane, wm, wn, m0, n0, M, N, C, out_bf16, part, ksp, SK);
}

// out[i] = sum over k = 0..SK-1 of part[k][i], in that order; 8 outputs per
// thread (M*N is a multiple of 16).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part,
                                                            void* __restrict__ C, size_t MN,
                                                            uint32_t SK, int out_bf16) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i >= MN) return;
    constexpr uint32_t MAXSK = 16;
    f32x4_t a[MAXSK][2];
#pragma unroll
    for (uint32_t k = 0; k < MAXSK; ++k)
        if (k < SK) {
            a[k][0] = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(part + k * MN + i));
            a[k][1] = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(part + k * MN + i + 4));
        }
    f32x4_t v0 = {0.f, 0.f, 0.f, 0.f}, v1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t k = 0; k < MAXSK; ++k)
        if (k < SK) {
            v0 += a[k][0];
            v1 += a[k][1];
        }
    if (out_bf16) {
        u32x4_t o;
        bf16x2_t p0 = {(__bf16)v0[0], (__bf16)v0[1]}, p1 = {(__bf16)v0[2], (__bf16)v0[3]};
        bf16x2_t p2 = {(__bf16)v1[0], (__bf16)v1[1]}, p3 = {(__bf16)v1[2], (__bf16)v1[3]};
        o[0] = __builtin_bit_cast(uint32_t, p0);
        o[1] = __builtin_bit_cast(uint32_t, p1);
        o[2] = __builtin_bit_cast(uint32_t, p2);
        o[3] = __builtin_bit_cast(uint32_t, p3);
        *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(C) + i) = o;
    } else {
        *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(C) + i) = v0;
        *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(C) + i + 4) = v1;
    }
}

}  // namespace

hipError_t launch_splitk_reduce(const float* part, void* C, size_t MN, uint32_t SK, int out_bf16,
                                hipStream_t st) {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((MN / 8 + 255) / 256)), dim3(256), 0,
                       st, part, C, MN, SK, out_bf16);
    return hipGetLastError();
}

namespace {

template <int BM, int BN, bool Q4, int G>
hipError_t launch_cfg(const void* A, const void* B, const void* q, const void* s, const void* b,
                      void* C, uint32_t M, uint32_t N, uint32_t K, int out_bf16, uint32_t SK,
                      hipStream_t st) {
    const uint32_t tiles_m = (M + BM - 1) / BM;
    const uint32_t tiles_n = (N + BN - 1) / BN;
    const uint32_t ntiles = tiles_m * tiles_n;
    static const int remap = tuning_env("MIORI_GEMM_REMAP", 1);
    float* part = nullptr;
    if (SK > 1) {
        const hipError_t e = scratch_get(st, (size_t)SK * M * N * 4, &part);
        if (e != hipSuccess) return e;
    }
    // the eight-wave forms for 256x128 and 128x128 tiles (MIORI_GEMM_PC=0:
    // the four-wave gemm_kernel, for comparisons)
    static const int pc = tuning_env("MIORI_GEMM_PC", 1);
    if constexpr (Cfg<BM, BN, false, 64>::NST == 3 && BM * BN >= 128 * 128 && BN == 128) {
        if (pc && Q4)
            hipLaunchKernelGGL((gemm_pcq_kernel<BM, BN, G>), dim3(ntiles * SK), dim3(512), 0, st,
                               (const uint16_t*)A, (const uint32_t*)q, (const uint16_t*)s,
                               (const uint16_t*)b, C, M, N, K, out_bf16, tiles_m, remap, part, SK,
                               ntiles);
        else if (pc)
            hipLaunchKernelGGL((gemm_pc_kernel<BM, BN>), dim3(ntiles * SK), dim3(512), 0, st,
                               (const uint16_t*)A, (const uint16_t*)B, C, M, N, K, out_bf16,
                               tiles_m, remap, part, SK, ntiles);
        else
            hipLaunchKernelGGL((gemm_kernel<BM, BN, Q4, G>), dim3(ntiles * SK), dim3(256), 0, st,
                               (const uint16_t*)A, (const uint16_t*)B, (const uint32_t*)q,
                               (const uint16_t*)s, (const uint16_t*)b, C, M, N, K, out_bf16,
                               tiles_m, remap, part, SK, ntiles);
    } else {
        hipLaunchKernelGGL((gemm_kernel<BM, BN, Q4, G>), dim3(ntiles * SK), dim3(256), 0, st,
                           (const uint16_t*)A, (const uint16_t*)B, (const uint32_t*)q,
                           (const uint16_t*)s, (const uint16_t*)b, C, M, N, K, out_bf16, tiles_m,
                           remap, part, SK, ntiles);
    }
    if (SK > 1) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_splitk_reduce(part, C, (size_t)M * N, SK, out_bf16, st);
    }
    return hipGetLastError();
}

template <int BM, int BN>
hipError_t launch_w8(const void* A, const void* B, void* C, uint32_t M, uint32_t N, uint32_t K,
                     int out_bf16, hipStream_t st) {
    const uint32_t tiles_m = (M + BM - 1) / BM;
    const uint32_t ntiles = tiles_m * ((N + BN - 1) / BN);
    static const int remap = tuning_env("MIORI_GEMM_REMAP", 1);
    hipLaunchKernelGGL((gemm_w8_kernel<BM, BN>), dim3(ntiles), dim3(512), 0, st,
                       (const uint16_t*)A, (const uint16_t*)B, C, M, N, K, out_bf16, tiles_m,
                       remap, nullptr, 1u, ntiles);
    return hipGetLastError();
}

template <int BM, int BN>
hipError_t launch_tile(const void* A, const void* B, const void* q, const void* s, const void* b,
                       void* C, uint32_t M, uint32_t N, uint32_t K, uint32_t G, int out_bf16,
                       uint32_t SK, hipStream_t st) {
    if (!q) return launch_cfg<BM, BN, false, 64>(A, B, q, s, b, C, M, N, K, out_bf16, SK, st);
    switch (G) {
        case 32: return launch_cfg<BM, BN, true, 32>(A, B, q, s, b, C, M, N, K, out_bf16, SK, st);
        case 64: return launch_cfg<BM, BN, true, 64>(A, B, q, s, b, C, M, N, K, out_bf16, SK, st);
        case 128: return launch_cfg<BM, BN, true, 128>(A, B, q, s, b, C, M, N, K, out_bf16, SK, st);
    }
    return hipErrorInvalidValue;
}

// K splits for `tiles` BM x BN output tiles of KT K tiles each, one
// workgroup per CU at a time. Cost in half-K-tile units (a 64-deep K tile of
// a 128x128 workgroup takes ~0.6 us): rounds of 256 workgroups x K tiles per
// workgroup, plus for a split ~3 us of fixed cost and the partials' traffic
// (SK*MN*4 bytes written and read back at ~5 TB/s, MN the padded output
// size). A function of the tile grid and K only, so the fused and the
// two-step products of one shape take the same path.
uint32_t pick_split(uint32_t tiles, uint32_t KT, uint64_t MN, uint64_t* cost_out = nullptr) {
    uint32_t best = 1;
    uint64_t best_cost = 2ull * ((tiles + 255) / 256) * KT;
    for (uint32_t sk = 2; sk <= 16 && KT / sk >= 4; ++sk) {
        const uint64_t rounds = (tiles * (uint64_t)sk + 255) / 256;
        const uint64_t traffic = sk * MN * 8 / 1500000;  // bytes / (5 TB/s * 0.3 us)
        const uint64_t cost = 2 * rounds * ((KT + sk - 1) / sk) + 10 + traffic;
        if (cost < best_cost) { best = sk; best_cost = cost; }
    }
    if (cost_out) *cost_out = best_cost;
    return best;
}

// 256x128 or 128x128 tiles: the cheaper by the split-K cost model (each on
// its padded grid, with its best split), a 256x128 round weighted 1.35x a
// 128x128 one (fused 4-bit: 56 us per 256x128 round at M=1024, N=8192, K=2048;
// 37 us per 128x128 round at M=1472). A function of the tile grids and K
// only, so the fused and the bf16 products of one shape pick alike.
// 192x128 tiles (tile 7) compete at 24/20, between the two: M=1472, K=8192,
// N=2048 then runs 8 x 16 = 128 tiles split in two, one full round of 256
// workgroups, instead of 96 256x128 tiles split in two on 192 CUs.
int pick_tile_256x128(uint32_t M, uint32_t N, uint32_t K) {
    const uint32_t t0 = ((M + 255) / 256) * ((N + 127) / 128);
    const uint32_t t1 = ((M + 127) / 128) * ((N + 127) / 128);
    const uint32_t t7 = ((M + 191) / 192) * ((N + 127) / 128);
    uint64_t c0 = 0, c1 = 0, c7 = 0;
    pick_split(t0, K / 64, (uint64_t)t0 * 256 * 128, &c0);
    pick_split(t1, K / 64, (uint64_t)t1 * 128 * 128, &c1);
    pick_split(t7, K / 64, (uint64_t)t7 * 192 * 128, &c7);
    static const int e_192 = tuning_env("MIORI_GEMM_192", 1);
    if (e_192 && c7 * 24 < c0 * 27 && c7 * 24 < c1 * 20) return 7;
    return c0 * 27 <= c1 * 20 ? 0 : 1;
}

}  // namespace

hipError_t launch_gemm(const void* A, const void* B, const void* q, const void* s,
                       const void* b, void* C, uint32_t M, uint32_t N, uint32_t K,
                       uint32_t G, int out_bf16, hipStream_t st) {
    // Tile choice (MIORI_GEMM_TILE overrides: 0 = 256x128, 1 = 128x128,
    // 2 = 256x256, 3 = 64x128, 4 = 64x64, 5 = 192x256, 6 = 128x128 split as
    // the 64x128 grid, 7 = 192x128 fused):
    //  * bf16 weight cache: 256x256 tiles (128 flop per operand byte, against
    //    85 for 256x128) once they fill at least 3/4 of the 256 CUs in a
    //    round; the split-K cost model is not applied to them (SK = 1).
    //    192x256 replaces them when its grid needs fewer rounds at 3/4 the
    //    cost per round: M=1472, N=8192, K=2048 62.7 -> 56.5 us, K=8192
    //    220 -> 194 us.
    //  * small grids (K <= 4096, at most 512 64x64 tiles): bf16 64x64 tiles,
    //    2-3 workgroups per CU; fused 4-bit 128x128 (gemm_pcq_kernel). Both
    //    paths take the K split the cost model picks for the 64x128 grid
    //    (usually none), so fused and bf16 products stay bit-identical.
    //    Measured against 128x128 tiles with their own split partials: bf16
    //    M=1024 N=2048 19.7 -> 15.0 us, M=256 N=8192 19.9 -> 15.3 us. The
    //    fused path's 128x128 register-B tiles against the four-wave 64x128
    //    form: M=256 N=8192 30.1 -> 24.8 us, M=1024 N=2048 29.9 -> 24.3,
    //    M=512 N=3072 28.7 -> 23.6, M=1024 N=512 17.6 -> 16.8.
    //  * otherwise 256x128 or 128x128 tiles, whichever the split-K cost
    //    model rates cheaper (pick_tile_256x128). Against the earlier rule
    //    (256x128 only in whole waves of 256): fused M=1472 N=8192 K=2048
    //    110 -> 101 us, M=1024 K=8192 N=2048 78.8 -> 67.3 us; bf16 M=1472
    //    K=8192 N=2048 92 -> 85 us.
    const uint64_t huge = (uint64_t)((M + 255) / 256) * ((N + 255) / 256);
    const uint64_t t64 = (uint64_t)((M + 63) / 64) * ((N + 63) / 64);
    int tile = pick_tile_256x128(M, N, K);
    if (!q && huge >= 192) {
        // M=1472, N=8192: 8 x 32 = 256 192x256 tiles in one round, against
        // 6 x 32 = 192 256x256 tiles that leave a quarter of the CUs idle
        const uint64_t t192 = (uint64_t)((M + 191) / 192) * ((N + 255) / 256);
        tile = (t192 + 255) / 256 * 3 < (huge + 255) / 256 * 4 ? 5 : 2;
    } else if (K <= 4096 && t64 <= 512) tile = q ? 6 : 4;
    static const int e_tile = tuning_env("MIORI_GEMM_TILE", -1);
    if (e_tile >= 0) tile = e_tile;
    // (MIORI_GEMM_W8=0: the four-wave gemm_kernel for these tiles, for comparisons)
    static const int e_w8 = tuning_env("MIORI_GEMM_W8", 1);
    if (tile == 2 && !q && e_w8) return launch_w8<256, 256>(A, B, C, M, N, K, out_bf16, st);
    if (tile == 5 && !q && e_w8) return launch_w8<192, 256>(A, B, C, M, N, K, out_bf16, st);
    if (tile == 2 && !q) return launch_cfg<256, 256, false, 64>(A, B, q, s, b, C, M, N, K, out_bf16, 1, st);
    if (tile == 5 && !q) return launch_cfg<192, 256, false, 64>(A, B, q, s, b, C, M, N, K, out_bf16, 1, st);
    const bool t5 = tile == 5;  // the bf16 path's 192x256 choice (fused: 192x128, unsplit)
    if (tile == 5 && q && e_tile < 0) {
        // Fused 4-bit where the bf16 path takes 192x256 tiles (M=1472,
        // N=8192): 192x128 tiles when their grid's rounds cost less than
        // 256x128 ones, a round of 192-row tiles taking about 3/4 of a
        // 256-row one. M=1472, N=8192: 8 x 64 = 512 tiles in two full rounds
        // (2 x 3/4) against 6 x 64 = 384 256x128 tiles in two rounds, the
        // second half empty (2 x 1). Unsplit, like the bf16 tall tiles.
        const uint64_t t192 = (uint64_t)((M + 191) / 192) * ((N + 127) / 128);
        const uint64_t t256 = (uint64_t)((M + 255) / 256) * ((N + 127) / 128);
        if ((t192 + 255) / 256 * 3 < (t256 + 255) / 256 * 4) tile = 7;
    }
    if (tile == 7 && q && t5) return launch_tile<192, 128>(A, B, q, s, b, C, M, N, K, G, out_bf16, 1, st);
    if (tile == 2 || tile == 5) tile = pick_tile_256x128(M, N, K);  // fused: no 256x256 variant
    // (64x64, and the fused path's 128x128 tiles on these small grids, split
    // as the 64x128 grid)
    const uint32_t tbm = tile == 0 ? 256 : tile == 7 ? 192 : (tile == 3 || tile == 4 || tile == 6) ? 64 : 128;
    const uint32_t tbn = 128;
    const uint32_t ntiles = ((M + tbm - 1) / tbm) * ((N + tbn - 1) / tbn);
    // partial traffic from the padded tile grid, so every M in one row-tile
    // count splits alike (rows of a small product equal those of a larger one)
    const uint64_t tile_elems = (uint64_t)tbm * tbn;
    uint32_t SK = pick_split(ntiles, K / 64, ntiles * tile_elems);
    static const int e_split = tuning_env("MIORI_GEMM_SPLIT", -1);
    if (e_split >= 0) SK = (uint32_t)e_split;
    if (SK < 1) SK = 1;
    if (SK > 16) SK = 16;
    if (SK > K / 64) SK = K / 64;
    if (tile == 0) return launch_tile<256, 128>(A, B, q, s, b, C, M, N, K, G, out_bf16, SK, st);
    if (tile == 7) return launch_tile<192, 128>(A, B, q, s, b, C, M, N, K, G, out_bf16, SK, st);
    if (tile == 3) return launch_tile<64, 128>(A, B, q, s, b, C, M, N, K, G, out_bf16, SK, st);
    if (tile == 4 && !q) return launch_cfg<64, 64, false, 64>(A, B, q, s, b, C, M, N, K, out_bf16, SK, st);
    return launch_tile<128, 128>(A, B, q, s, b, C, M, N, K, G, out_bf16, SK, st);
}

}  // namespace miori
