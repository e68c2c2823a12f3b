// Shared device helpers for the gfx950 LNCC kernels: buffer resources, bf16 conversion, tile
// geometry. Included by the kernel translation units only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "lncc_geometry.h"

namespace fl {

// gfx9 buffer resource word 3 (raw buffer, 32-bit data format); out-of-range loads return 0 and
// out-of-range stores are dropped, which gives the zero padding of the box window for free.
constexpr int kRsrcWord3 = 0x00020000;
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

// Resource for plane z (clamped into [0, D)) of a volume; `valid == false` gives a zero-sized
// buffer, so loads through it return 0 and stores through it are dropped. z and valid must be
// workgroup-uniform; the explicit readfirstlane keeps the address arithmetic on the scalar unit
// (a clamp that the compiler selects as a VALU op would otherwise force a per-lane loop around
// every access through the resource).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(const void* vol, int z, int D, int64_t plane_bytes,
                                                               bool valid) {
    const int zc = __builtin_amdgcn_readfirstlane(z < 0 ? 0 : (z >= D ? D - 1 : z));
    const int nb = __builtin_amdgcn_readfirstlane(valid ? (int)plane_bytes : 0);
    return make_rsrc((const char*)vol + (int64_t)zc * plane_bytes, (uint32_t)nb);
}

// Resource for `bytes` bytes at a workgroup-uniform address; `valid == false` gives a zero-sized
// buffer (the address is then never dereferenced).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_at(uint64_t addr, uint32_t bytes, bool valid) {
    return make_rsrc((const void*)(uintptr_t)addr, valid ? bytes : 0u);
}

// Cache-policy operand of the buffer instructions: 0 = default, kNT = non-temporal (the line is
// streamed: a store does not displace data that will be read again from the L2, a load marks the
// line as the first to evict).
constexpr int kNT = 2;

template <bool BF16, int AUX = 0>
__device__ __forceinline__ float load_elem(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    if constexpr (BF16) {
        uint32_t u = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, 0, AUX);
        return __uint_as_float(u << 16);
    } else {
        // the builtin returns the raw 32 bits; reinterpret, do not convert
        return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, AUX));
    }
}

template <bool BF16>
__device__ __forceinline__ float load_elem_ptr(const void* base, int64_t idx) {
    if constexpr (BF16) {
        return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(base)[idx] << 16);
    } else {
        return reinterpret_cast<const float*>(base)[idx];
    }
}

// float32 -> bfloat16 bits, round to nearest even; NaN stays a NaN. gfx950 converts in one
// instruction (v_cvt_pk_bf16_f32), which the compiler selects for the __bf16 conversion.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
}

template <bool BF16, int AUX = 0>
__device__ __forceinline__ void store_elem_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, float v) {
    if constexpr (BF16) {
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)f32_to_bf16_bits(v), r, (int)voff, 0, AUX);
    } else {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)voff, 0, AUX);
    }
}

template <bool BF16>
__device__ __forceinline__ void store_elem(void* base, int64_t idx, float v) {
    if constexpr (BF16) {
        reinterpret_cast<uint16_t*>(base)[idx] = f32_to_bf16_bits(v);
    } else {
        reinterpret_cast<float*>(base)[idx] = v;
    }
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E), so that register arrays
// indexed by I stay in registers.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

}  // namespace fl
