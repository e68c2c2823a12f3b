// Shared device helpers for the gfx950 LNCC kernels: buffer resources, bf16 conversion, tile
// geometry. Included by the kernel translation units only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fl {

// Workgroup: 1024 lanes (16 wave64s, one workgroup per CU). Output tile: TX x TY columns of one
// volume, marched along D.
constexpr int NT = 1024;
constexpr int WG_PER_CU = 1;
constexpr int TX = 32;
constexpr int TY = 32;

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

constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
constexpr int odd(int a) { return a | 1; }

// Row stride (floats) for LDS rows read as float4 by lanes that step from row to row: = 4 mod 8,
// so that the 8 lanes served per cycle by a 128-bit read land on distinct groups of 4 banks.
constexpr int stride4(int n) { return n + ((12 - n % 8) % 8); }
constexpr int rup4(int n) { return (n + 3) / 4 * 4; }
constexpr int rup64(int n) { return (n + 63) / 64 * 64; }

// Tile geometry for halo H (k = 2H+1). Coordinates inside a workgroup:
//   input region   ix in [0,IX), iy in [0,IY)  <-> global (x0-2H+ix, y0-2H+iy)
//   adjoint region ax in [0,AX), ay in [0,AY)  <-> global (x0-H+ax,  y0-H+ay)
//   output tile    ox in [0,TX), oy in [0,TY)  <-> global (x0+ox,    y0+oy)
// Running-sum passes work on segments of S consecutive outputs. The X and Y passes round their
// output range up to whole segments: the extra outputs read row padding and land in padding rows
// of the destination that no later pass reads (and that the loss never counts), so no lane needs
// a per-output store mask.
// NA = number of adjoint fields carried from Y to AZ: 3 (alpha, beta, gamma of the pred gradient)
// or 5 (with alpha', beta' of the target gradient; gamma is shared)
template <int H, int NA = 3>
struct Geo {
    static constexpr int K = 2 * H + 1;
    static constexpr int TY = fl::TY;
    static constexpr int IX = TX + 4 * H, IY = TY + 4 * H;
    static constexpr int AX = TX + 2 * H, AY = TY + 2 * H;
    static constexpr int NIN = IX * IY;
    static constexpr int J = cdiv(NIN, NT);               // input columns per lane
    static constexpr int NOUT = TX * TY;                  // output columns (one lane each)
    // X: x-sums of the five z-sums; items (iy, seg) over rows iy < IY, outputs ax < XR (>= AX)
    static constexpr int SX = rup4(cdiv(AX, 2)), XSEG = 2, XR = XSEG * SX, XITEMS = IY * XSEG;
    // Y: y-sums -> box sums, ncc, adjoints; items (ax, seg), outputs ay < YR (>= AY)
    static constexpr int SY = 4, YSEG = cdiv(AY, SY), YR = YSEG * SY, YITEMS = AX * YSEG;
    // AX: x-sums of alpha, beta, gamma; items (ay, seg), outputs ox < TX
    static constexpr int SA = 16, ASEG = TX / SA, AITEMS = AY * ASEG;
    // AYs: y-sums of the three; items (ox, seg), outputs oy < TY
    static constexpr int SB = TY / 2, BSEG = TY / SB, BITEMS = TX * BSEG;
    // Work units of the running-sum passes are single quantities of one segment. Waves are
    // spread over the 4 SIMDs of the CU round-robin (wave w on SIMD w % 4), so the heavy items
    // are placed to even out each SIMD's share of a phase: in phase P1 the X units (5 per item)
    // fill the first waves and the AX units (3 per item) start on the next wave boundary; in
    // phase P0 the Y items fill the first waves (SIMDs 0 and 1 get the extra ones) and the AYs
    // units (3 per item) go to waves 10, 11, 14, 15 (SIMDs 2 and 3), B_PER_WAVE each.
    // With five adjoint fields the AYs units (two rows of 32 per field) take five whole waves.
    static constexpr int UX = 5 * XITEMS, UA = NA * AITEMS, AX_LANE0 = rup64(UX), U1 = 1;
    static constexpr int UB = NA * BITEMS, B_PER_WAVE = NA == 3 ? UB / 4 : 64;
    static_assert(YITEMS <= 10 * 64 && AX_LANE0 + UA <= NT && BSEG == 2 && TX == 32 &&
                      (NA == 3 ? (UB == 192 && B_PER_WAVE == 48) : (NA == 5 && UB == 320)),
                  "lanes");
    // every segment starts on a 16-byte boundary (rows are read as float4)
    static_assert(XR >= AX && TX % SA == 0 && TY % SB == 0 && SX % 4 == 0 && SY % 4 == 0 &&
                      SA % 4 == 0 && SB % 4 == 0, "segments");
    // LDS layout (floats): Zs[5][IY][ZS], XsT[5][XR][XS] (transposed), Gs[NA][YR][GS],
    // GXsT[NA][TX][GXS] (transposed), GY[NA][TY][GYS]; each buffer but GY ends in PAD spare floats
    static constexpr int ZS = stride4(IX), XS = stride4(cmax(IY, AY)), GS = stride4(AX), GXS = XS;
    static constexpr int GYS = TX + 1, PAD = 16;
    static constexpr int ZP = IY * ZS, XP = XR * XS, GP = YR * GS, GXP = TX * GXS, GYP = TY * GYS;
    // A segment reads rup4(S + 2H) floats from its start; reads past a row's end stay inside the
    // buffer (the next row or the spare floats) and only feed outputs that are never used.
    static_assert(SX + rup4(SX + 2 * H) <= ZS + PAD && YR - SY + rup4(SY + 2 * H) <= XS + PAD &&
                      TX - SA + rup4(SA + 2 * H) <= GS + PAD && TY - SB + rup4(SB + 2 * H) <= GXS + PAD,
                  "row reads");
    static constexpr int LDS_FLOATS = 5 * (ZP + XP) + NA * (GP + GXP + GYP) + 4 * PAD;
    static_assert(LDS_FLOATS * 4 <= 160 * 1024, "LDS");
};

}  // namespace fl
