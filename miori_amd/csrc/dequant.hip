// Weight-cache builders: MLX-affine 4-bit / 8-bit -> bf16 row-major [N][K].
//
// Replaces shaders/ops.metal:142-166 (dequant4), :754-779 (dequant8) and
// shaders/gemm_mpp.metal:9-34 (dequant_tile). Each element is
// bf16_rne(float(code) * scale + bias). float(code)*scale is exact in fp32
// (a <= 8-bit integer times an 8-bit-mantissa bf16), so the value has a single
// rounding whether or not the compiler fuses the multiply-add, and the bf16
// result is bit-identical to the CPU reference.
//
// One thread per 16-byte weight chunk (32 nibbles or 16 codes): a coalesced
// dwordx4 load, then 64 or 32 bytes of bf16 written as dwordx4 stores.
#include "common.hpp"
#include "kernels.hpp"

namespace miori {

namespace {

template <int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(
    const uint4* __restrict__ q, const uint16_t* __restrict__ s,
    const uint16_t* __restrict__ bs, uint4* __restrict__ out, uint32_t N, uint32_t K,
    uint32_t G) {
    constexpr uint32_t E = (BITS == 4) ? 32u : 16u;
    const uint32_t C = K / E;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)N * C) return;
    const uint32_t row = (uint32_t)(idx / C);
    const uint32_t c = (uint32_t)(idx % C);
    const uint4 qv = q[idx];
    const uint32_t g = c * E / G;
    const size_t sidx = (size_t)row * (K / G) + g;
    const float sc = bf16_bits_to_f32(s[sidx]);
    const float bi = bf16_bits_to_f32(bs[sidx]);
    const uint32_t wv[4] = {qv.x, qv.y, qv.z, qv.w};
    uint32_t o[E / 2];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        if constexpr (BITS == 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v0 = fmaf((float)((wv[w] >> (8 * j)) & 0xFu), sc, bi);
                const float v1 = fmaf((float)((wv[w] >> (8 * j + 4)) & 0xFu), sc, bi);
                o[4 * w + j] = pack_bf16x2(v0, v1);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float v0 = fmaf((float)((wv[w] >> (16 * j)) & 0xFFu), sc, bi);
                const float v1 = fmaf((float)((wv[w] >> (16 * j + 8)) & 0xFFu), sc, bi);
                o[2 * w + j] = pack_bf16x2(v0, v1);
            }
        }
    }
    uint4* dst = out + idx * (E / 8);
#pragma unroll
    for (uint32_t t = 0; t < E / 8; ++t)
        dst[t] = make_uint4(o[4 * t], o[4 * t + 1], o[4 * t + 2], o[4 * t + 3]);
}

}  // namespace

hipError_t launch_dequant(int bits, const void* q, const void* s, const void* b, void* out,
                          uint32_t N, uint32_t K, uint32_t G, hipStream_t st) {
    const uint32_t E = bits == 4 ? 32u : 16u;
    const size_t total = (size_t)N * (K / E);
    const size_t grid = (total + 255) / 256;
    if (bits == 4)
        hipLaunchKernelGGL(dequant_kernel<4>, dim3((uint32_t)grid), dim3(256), 0, st,
                           (const uint4*)q, (const uint16_t*)s, (const uint16_t*)b,
                           (uint4*)out, N, K, G);
    else
        hipLaunchKernelGGL(dequant_kernel<8>, dim3((uint32_t)grid), dim3(256), 0, st,
                           (const uint4*)q, (const uint16_t*)s, (const uint16_t*)b,
                           (uint4*)out, N, K, G);
    return hipGetLastError();
}

}  // namespace miori
