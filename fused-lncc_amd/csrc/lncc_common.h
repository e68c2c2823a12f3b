// Shared device helpers for the gfx950 LNCC kernels: buffer resources, bf16 conversion, tile
// geometry. Included by the kernel translation units only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fl {

// Workgroup: 512 lanes (8 wave64s). Output tile: TX x TY columns of one volume, marched along D.
constexpr int NT = 512;
constexpr int TX = 64;
constexpr int TY = 16;

// gfx9 buffer resource word 3 (raw buffer, 32-bit data format); out-of-range loads return 0 and
// out-of-range stores are dropped, which gives the zero padding of the box window for free.
constexpr int kRsrcWord3 = 0x00020000;
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

template <bool BF16>
__device__ __forceinline__ float load_elem(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    if constexpr (BF16) {
        uint32_t u = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, 0, 0);
        return __uint_as_float(u << 16);
    } else {
        // the builtin returns the raw 32 bits; reinterpret, do not convert
        return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, 0));
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

// float32 -> bfloat16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
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

constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
constexpr int odd(int a) { return a | 1; }

// Tile geometry for halo H (k = 2H+1). Coordinates inside a workgroup:
//   input region   ix in [0,IX), iy in [0,IY)  <-> global (x0-2H+ix, y0-2H+iy)
//   adjoint region ax in [0,AX), ay in [0,AY)  <-> global (x0-H+ax,  y0-H+ay)
//   output tile    ox in [0,TX), oy in [0,TY)  <-> global (x0+ox,    y0+oy)
template <int H>
struct Geo {
    static constexpr int K = 2 * H + 1;
    static constexpr int IX = TX + 4 * H, IY = TY + 4 * H;
    static constexpr int AX = TX + 2 * H, AY = TY + 2 * H;
    static constexpr int NIN = IX * IY;
    static constexpr int J = cdiv(NIN, NT);               // input columns per lane
    // forward x-pass: rows iy in [0,IY), SX outputs per item
    static constexpr int SX = 4;
    static constexpr int XSEG = cdiv(AX, SX);
    static constexpr int XITEMS = IY * XSEG;
    static constexpr int ZSTRIDE = odd(cmax(XSEG * SX + 2 * H, IX));
    // forward y-pass: columns ax in [0,AX), SY outputs per item
    static constexpr int SY = 4;
    static constexpr int YSEG = cdiv(AY, SY);
    static constexpr int YITEMS = AX * YSEG;
    static constexpr int XROWS = cmax(IY, YSEG * SY + 2 * H);
    static constexpr int XSTRIDE = odd(XSEG * SX);
    // adjoint x-pass: rows ay in [0,AY), SX2 outputs per item
    static constexpr int SX2 = 4;
    static constexpr int X2SEG = TX / SX2;
    static constexpr int X2ITEMS = AY * X2SEG;
    static constexpr int GSTRIDE = odd(AX);
    static constexpr int GXSTRIDE = odd(TX);
    // adjoint y-pass + combine: one lane per (ox, pair of oy)
    static_assert(TX * TY / 2 == NT, "combine stage maps one lane to two output columns");
    // LDS plan (floats)
    static constexpr int Z_FLOATS = 5 * IY * ZSTRIDE;
    static constexpr int X_FLOATS = 5 * XROWS * XSTRIDE;
    static constexpr int G_FLOATS = 3 * AY * GSTRIDE;
    static constexpr int GX_FLOATS = 3 * AY * GXSTRIDE;
    static constexpr int PT_FLOATS = 2 * 2 * TY * TX;
};

}  // namespace fl
