// Shared device helpers for the gfx950 kernels of libmiori_hip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

namespace miori {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// bf16 bits -> fp32 (the bf16 is the upper half of the fp32).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t v) {
    return __uint_as_float(v << 16);
}

// fp32 -> bf16 bits, round to nearest even by the add-and-truncate rule
// (no NaN special case), the same bit rule as the CPU reference conversion.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// Two fp32 -> packed bf16 pair (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// D = a.lo*b.lo + a.hi*b.hi + c on packed bf16 pairs (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wave. DPP inside each row of 16 lanes
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror),
// then the four row sums are read out and added in a fixed order, so the
// result is uniform across the wave and deterministic.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
}

// 16-byte streaming load (weights are read once per launch).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Buffer resource over [base, base + bytes) (bytes < 4 GiB). Loads whose
// offset is outside the range return zero, which the kernels use for ragged
// edges instead of clamping addresses.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
constexpr uint32_t kOOB = 0xFFFFFFF0u;  // an offset that is always out of range

__device__ __forceinline__ u32x4_t buf_load16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
// AUX: cache-policy bits of the load (2 = nt, streaming data read once)
template <int AUX>
__device__ __forceinline__ u32x4_t buf_load16_aux(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX);
}
template <int AUX>
__device__ __forceinline__ uint32_t buf_load_u16_aux(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, AUX);
}
__device__ __forceinline__ uint32_t buf_load_u16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

// (a & m) | c in one v_and_or_b32 (m in an SGPR, c in a VGPR: the VOP3
// encoding takes no literal and one scalar operand on this target).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(c));
    return r;
}

// Reduce RV (1, 2, 4 or 8) per-lane values over the 64 lanes of a wave.
// Halves are folded with v_permlane32_swap / v_permlane16_swap (each swap
// moves one value's partial sums next to another's, so RV values cost about
// as much as one), then DPP finishes each 16-lane row. On return, value t
// is complete in every lane of one 16-lane row of one out[] register, as
// reduce_value() maps it; for RV = 2 value t is in rows 2t and 2t+1; for
// RV = 1 in all lanes.
__device__ __forceinline__ void swap32(float& a, float& b) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(p[0]);
    b = __uint_as_float(p[1]);
}
__device__ __forceinline__ void swap16(float& a, float& b) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(p[0]);
    b = __uint_as_float(p[1]);
}
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    return v;
}
template <int RV>
__device__ __forceinline__ void wave_reduce(float (&v)[RV], float (&out)[(RV + 3) / 4]) {
    if constexpr (RV == 1) {
        float a = v[0], b = v[0];
        swap32(a, b);
        float c = a + b, d = c;
        swap16(c, d);
        out[0] = row_sum16(c + d);
    } else if constexpr (RV == 2) {
        float a = v[0], b = v[1];
        swap32(a, b);           // lanes 0-31: value 0, lanes 32-63: value 1
        float c = a + b, d = c;
        swap16(c, d);
        out[0] = row_sum16(c + d);
    } else {
        constexpr int H = RV / 2;
        float h[H];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            // pair value i (kept in lanes 0-31) with value i + H (lanes 32-63)
            float a = v[i], b = v[i + H];
            swap32(a, b);
            h[i] = a + b;
        }
        // h[i]: lanes 0-31 value i, lanes 32-63 value i + H
#pragma unroll
        for (int i = 0; i < H / 2; ++i) {
            float a = h[2 * i], b = h[2 * i + 1];
            swap16(a, b);
            // rows: 0 -> value 2i, 1 -> value 2i+1, 2 -> value 2i+H, 3 -> value 2i+1+H
            out[i] = row_sum16(a + b);
        }
    }
}
// Which value register out[i], 16-lane row `row`, holds after wave_reduce:
// for RV >= 4, rows 0..3 of out[i] hold values 2i, 2i+1, 2i+H, 2i+1+H
// (H = RV / 2).
__device__ __forceinline__ int reduce_value(int RV, int i, int row) {
    if (RV == 1) return 0;
    if (RV == 2) return row >> 1;
    const int H = RV / 2;
    return 2 * i + (row & 1) + ((row >> 1) ? H : 0);
}

// Tuning override MIORI_*: its integer value, or dflt when unset. Call sites
// keep the result in a function-local static, so each variable is read once
// per process (later changes to the environment are not seen).
inline int tuning_env(const char* name, int dflt) {
    const char* v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

// Per-device set-up run once (a kernel attribute, a device property), safe
// against host threads making their first call on a device together: the
// first caller runs f under a lock and later callers see the flag. A failed
// f is retried by the next call.
struct PerDeviceOnce {
    std::atomic<bool> done[64] = {};
    std::mutex mu;
    template <class F>
    hipError_t run(int dev, F&& f) {
        if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
        if (done[dev].load(std::memory_order_acquire)) return hipSuccess;
        std::lock_guard<std::mutex> g(mu);
        if (done[dev].load(std::memory_order_relaxed)) return hipSuccess;
        const hipError_t e = f();
        if (e == hipSuccess) done[dev].store(true, std::memory_order_release);
        return e;
    }
};

// ---- direct-to-LDS DMA and barriers (gfx950)
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gptr_t;

__device__ __forceinline__ void dma16(const void* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds((gptr_t)g, (lds_ptr_t)l, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds((gptr_t)g, (lds_ptr_t)l, 4, 0, 0);
}
__device__ __forceinline__ void dma2(const void* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds((gptr_t)g, (lds_ptr_t)l, 2, 0, 0);
}

// Workgroup barrier that neither waits for outstanding DMA (the fence of
// __syncthreads would) nor lets the compiler move memory accesses across it.
__device__ __forceinline__ void barrier_lds() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}



// Store one output element as fp32 or bf16.
__device__ __forceinline__ void store_out(void* y, size_t idx, float v, bool bf16) {
    if (bf16)
        reinterpret_cast<uint16_t*>(y)[idx] = (uint16_t)f32_to_bf16_bits(v);
    else
        reinterpret_cast<float*>(y)[idx] = v;
}

}  // namespace miori
