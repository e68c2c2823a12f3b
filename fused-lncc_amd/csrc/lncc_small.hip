// The fused LNCC kernel for small volumes (each of D, H, W at most 16), gfx950.
//
// The plane-marching kernel (lncc_fused_kernel.h) works on 32 x 32 tiles and a D-pipeline of
// 4h+3 steps: on many small volumes, as in a network's feature maps (the reference benchmarks
// (1,256,16^3)), three quarters of its lanes idle and the pipeline steps outnumber the planes.
// Here one 1024-lane workgroup holds one whole volume, zero-padded to 16^3, in LDS, and forms the
// same sums and the same per-voxel arithmetic in four phases separated by workgroup barriers:
//
//   A  lane (q, y, x): the five fields p, t, p^2, t^2, p t on planes 4q-h .. 4q+3+h of its (y, x)
//      column (read from HBM, zero outside the volume), their z window sums for planes 4q..4q+3,
//      then the x window sums across the 16 lanes of its DPP row (the lanes of one x line): F.
//   B  lane (q, z, x): the y window sums of F for rows 4q..4q+3 of its (z, x) line -> the five
//      box sums of four voxels; ncc (clamped), the loss partials, the adjoint coefficients
//      alpha, beta, gamma (zero outside the volume), their y window sums along the same line: G.
//   C  the x window sums of G across the DPP row: G2.
//   D  lane (q, y, x): the z window sums of G2 for planes 4q..4q+3 of its column: box(alpha),
//      box(beta), box(gamma), and the gradient of those four voxels.
//
// Every window sum is a sum of its own values (z and y: lncc_window.h's block sums; x: a direct
// sum of the 2h+1 lanes of the window), so windows of zeros sum to exactly 0 and windows of one
// constant as the reference's direct sums do. The formula, its clamp, its NaN policy and the
// range scale are those of the plane-marching kernel (lncc_fused_kernel.h). One workgroup writes
// one float64 ncc partial sum per volume, summed over its lanes and waves in a fixed order.
//
// The four lane quarters q are whole waves (256 lanes = 4 waves each), so the ranges of a
// quarter's line reads are wave-uniform: the first and the last quarter, whose windows reach past
// the volume's 16 positions, run code in which those reads are compile-time zeros.
#include "lncc_common.h"
#include "lncc_launch.h"
#include "lncc_window.h"

namespace fl {

constexpr int SNT = kSmallLanes;   // 1024
constexpr int SQ = 4;              // outputs per lane along its line
constexpr int SF = kSmallEdge * kSmallEdge * kSmallEdge;   // floats per field (16^3)
static_assert(SNT == 4 * kSmallEdge * kSmallEdge && kSmallEdge == 4 * SQ, "lane quarters");

// LDS offset of (z, y, x) in one field (rows rotated by z: conflict-free for every phase's waves)
__device__ __forceinline__ int sidx(int z, int y, int x) { return small_lds(z, y, x); }

template <int D>
__device__ __forceinline__ float dpp_from_below(float v) {   // lane x gets x - D of its row, 0 past the edge
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + D, 0xF, 0xF, true));
}
template <int D>
__device__ __forceinline__ float dpp_from_above(float v) {   // lane x gets x + D of its row, 0 past the edge
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + D, 0xF, 0xF, true));
}
// x window sum over the 16 lanes of a DPP row (one x line, zero padded): v[x] + v[x-1] + v[x+1] +
// ... + v[x-h] + v[x+h], one v_add_f32_dpp per term
template <int HH, int D = 1>
__device__ __forceinline__ float xsum16(float v, float s) {
    if constexpr (D > HH) {
        return s;
    } else {
        return xsum16<HH, D + 1>(v, (s + dpp_from_below<D>(v)) + dpp_from_above<D>(v));
    }
}

// The window sums of four consecutive outputs 4q..4q+3 along a line of 16 LDS values (positions
// p = 4q - h + i, i < 4 + 2h), read by `at(p)`; positions outside [0, 16) are zero. QC = the
// lane quarter's class: 0 (q = 0, windows start below 0), 3 (q = 3, they end past 15), 1 (q = 1
// or 2, every position inside).
template <int HH, int QC, class At>
__device__ __forceinline__ void line4(int q, At at, float (&out)[SQ]) {
    float v[SQ + 2 * HH];
#pragma unroll
    for (int i = 0; i < SQ + 2 * HH; ++i) v[i] = small_skip(QC, HH, i) ? 0.f : at(4 * q - HH + i);
    box_sums<HH, SQ>(v, out);
}

template <int HH, bool BF16, int MODE>
__global__ __launch_bounds__(SNT, 1) void lncc_small_kernel(FusedArgs a) {
    constexpr bool ADJ = (MODE == MODE_GRAD);
    constexpr int ELEM = BF16 ? 2 : 4;
    constexpr float VS = range_scale(2 * HH + 1);
    __shared__ __align__(16) float F[5 * SF];    // phase A -> B; G (B -> C) reuses its first 3 fields
    __shared__ __align__(16) float G2[ADJ ? 3 * SF : 1];
    __shared__ double red[SNT / 64];
    float* const G = F;

    const int tid = threadIdx.x;
    const int q = __builtin_amdgcn_readfirstlane(tid >> 8);   // the lane quarter, wave-uniform
    const int r = (tid >> 4) & 15, x = tid & 15;            // A, D: r = y; B, C: r = z
    const int D = a.dimD, Hd = a.dimH, Wd = a.dimW;
    const int64_t b = blockIdx.x;
    const int64_t vox = (int64_t)D * Hd * Wd;
    const uint32_t vol_bytes = (uint32_t)(vox * ELEM);
    const char* pvol = (const char*)a.pred + b * vox * ELEM;
    const char* tvol = (const char*)a.target + b * vox * ELEM;
    const float nf = a.nf, ndr = a.ndr, inv_n = a.inv_n;

    // ---- A: lane (q, y = r, x)
    float pk[SQ], tk[SQ];   // p, t of the lane's four output voxels (phase D's gradient)
    {
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(pvol, vol_bytes), rt = make_rsrc(tvol, vol_bytes);
        const bool col = r < Hd && x < Wd;
        float p[SQ + 2 * HH], t[SQ + 2 * HH];
#pragma unroll
        for (int i = 0; i < SQ + 2 * HH; ++i) {
            const int z = 4 * q - HH + i;
            const uint32_t off = col && z >= 0 && z < D ? (uint32_t)(((z * Hd + r) * Wd + x) * ELEM) : kOOB;
            p[i] = load_elem<BF16>(rp, off);
            t[i] = load_elem<BF16>(rt, off);
        }
#pragma unroll
        for (int j = 0; j < SQ; ++j) {
            pk[j] = p[HH + j];
            tk[j] = t[HH + j];
        }
#pragma unroll
        for (int f = 0; f < 5; ++f) {
            float v[SQ + 2 * HH], zs[SQ];
#pragma unroll
            for (int i = 0; i < SQ + 2 * HH; ++i)
                v[i] = f == 0 ? p[i] : f == 1 ? t[i] : f == 2 ? p[i] * p[i] : f == 3 ? t[i] * t[i] : p[i] * t[i];
            box_sums<HH, SQ>(v, zs);
#pragma unroll
            for (int j = 0; j < SQ; ++j) F[f * SF + sidx(4 * q + j, r, x)] = xsum16<HH>(zs[j], zs[j]);
        }
    }
    __syncthreads();

    // Line reads of the four output positions 4q..4q+3 (plus the window halo) of NF fields, `at(f, p)`
    // giving field f at line position p; the quarter's class picks the code (a uniform branch).
    auto read_lines = [&](auto nf_c, auto at, float (&out)[decltype(nf_c)::value][SQ]) __attribute__((always_inline)) {
        constexpr int NF = decltype(nf_c)::value;
        auto run = [&](auto qc) __attribute__((always_inline)) {
            constexpr int QC = decltype(qc)::value;
#pragma unroll
            for (int f = 0; f < NF; ++f) line4<HH, QC>(q, [&](int pos) { return at(f, pos); }, out[f]);
        };
        const int qc = small_class(q);
        if (qc == 0)
            run(std::integral_constant<int, 0>{});
        else if (qc == 3)
            run(std::integral_constant<int, 3>{});
        else
            run(std::integral_constant<int, 1>{});
    };

    // ---- B: lane (q, z = r, x): box sums, ncc, adjoint coefficients and their y window sums
    double lsum_d = 0.0;
    {
        float S[5][SQ];
        read_lines(std::integral_constant<int, 5>{}, [&](int f, int y) { return F[f * SF + sidx(r, y, x)]; }, S);
        if constexpr (ADJ) __syncthreads();   // G overwrites F
        float adj[3][SQ];
        float lsum = -0.f;
        const bool zin = r < D && x < Wd;
#pragma unroll
        for (int j = 0; j < SQ; ++j) {
            const int y = 4 * q + j;
            const bool in = zin && y < Hd;
            const float Sp = S[0][j], St = S[1][j], Spp = S[2][j], Stt = S[3][j], Spt = S[4][j];
            const float X = fmaf(-Sp, St, nf * Spt);
            const float VP = fmaxf(fmaf(-Sp, Sp, nf * Spp), 0.f) + ndr;
            const float VT = (fmaxf(fmaf(-St, St, nf * Stt), 0.f) + ndr) * VS;   // VT s
            const float rr = __builtin_amdgcn_rcpf(VP * VT);
            const float cr = X * rr;            // c / s
            const float ncc = (X * VS) * cr;    // ncc
            const bool live = in && (ncc < 1.0f);
            const float nccc = (ncc >= 1.0f) ? 1.0f : ncc;
            if (in) lsum += nccc;
            const float crm = live ? cr : 0.f;
            const float uu = crm * VT;
            const float w = fmaf(-Sp, uu, St);
            adj[0][j] = crm * w;
            adj[1][j] = crm * uu;
            adj[2][j] = crm;
            if constexpr (MODE == MODE_MAPS) {
                if (in) {
                    const int64_t o = ((b * D + r) * Hd + y) * (int64_t)Wd + x;
                    a.ncc_map[o] = nccc;
                    if (a.a_map) {
                        const float c0 = cr * VT, w0 = fmaf(-Sp, c0, St);
                        a.a_map[o] = live ? (-2.f * VS) * (cr * w0) : 0.f;
                        a.b_map[o] = live ? (-nf * VS) * (cr * c0) : 0.f;
                        a.c_map[o] = live ? (2.f * nf * VS) * cr : 0.f;
                    }
                }
            }
        }
        lsum_d = (double)lsum;
        if constexpr (ADJ) {
#pragma unroll
            for (int c = 0; c < 3; ++c)
#pragma unroll
                for (int j = 0; j < SQ; ++j) G[c * SF + sidx(r, 4 * q + j, x)] = adj[c][j];
        }
    }

    if constexpr (ADJ) {
        __syncthreads();
        // ---- C: lane (q, z = r, x): y window sums of G along the line, x window sums across the row
        {
            float ys[3][SQ];
            read_lines(std::integral_constant<int, 3>{}, [&](int c, int y) { return G[c * SF + sidx(r, y, x)]; }, ys);
#pragma unroll
            for (int c = 0; c < 3; ++c)
#pragma unroll
                for (int j = 0; j < SQ; ++j) G2[c * SF + sidx(r, 4 * q + j, x)] = xsum16<HH>(ys[c][j], ys[c][j]);
        }
        __syncthreads();
        // ---- D: lane (q, y = r, x): z window sums of G2 and the gradient of planes 4q..4q+3
        {
            float gw[3][SQ];
            read_lines(std::integral_constant<int, 3>{}, [&](int c, int z) { return G2[c * SF + sidx(z, r, x)]; }, gw);
            const bool col = r < Hd && x < Wd;
            char* const gvol = (char*)a.grad + b * vox * ELEM;
            const __amdgpu_buffer_rsrc_t rg = make_rsrc(gvol, vol_bytes);
#pragma unroll
            for (int j = 0; j < SQ; ++j) {
                const int z = 4 * q + j;
                const uint32_t off = col && z < D ? (uint32_t)(((z * Hd + r) * Wd + x) * ELEM) : kOOB;
                const float g = a.gscale * fmaf(inv_n, gw[0][j], fmaf(pk[j], gw[1][j], -tk[j] * gw[2][j]));
                store_elem_buf<BF16>(rg, off, g);
            }
        }
    }

    // ---- the volume's ncc partial sum: wave64 reduction, then the waves in a fixed order
    if constexpr (MODE == MODE_MAPS) return;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) lsum_d += __shfl_xor(lsum_d, off, 64);
    if ((tid & 63) == 0) red[tid >> 6] = lsum_d;
    __syncthreads();
    if (tid == 0) {
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < SNT / 64; ++w) s += red[w];
        a.partials[b] = s;
    }
}

template <int HH>
static hipError_t launch_small_h(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st) {
    const dim3 grid(nblocks), block(SNT);
#define FL_LAUNCH(BF, MD) hipLaunchKernelGGL((lncc_small_kernel<HH, BF, MD>), grid, block, 0, st, a)
    if (mode == MODE_LOSS) {
        if (bf16) FL_LAUNCH(true, MODE_LOSS); else FL_LAUNCH(false, MODE_LOSS);
    } else if (mode == MODE_GRAD) {
        if (bf16) FL_LAUNCH(true, MODE_GRAD); else FL_LAUNCH(false, MODE_GRAD);
    } else if (mode == MODE_MAPS) {
        if (bf16) FL_LAUNCH(true, MODE_MAPS); else FL_LAUNCH(false, MODE_MAPS);
    } else {
        return hipErrorInvalidValue;
    }
#undef FL_LAUNCH
    return hipGetLastError();
}

hipError_t launch_small(int halo, int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st) {
    switch (halo) {
        case 1: return launch_small_h<1>(mode, bf16, a, nblocks, st);
        case 2: return launch_small_h<2>(mode, bf16, a, nblocks, st);
        case 3: return launch_small_h<3>(mode, bf16, a, nblocks, st);
        case 4: return launch_small_h<4>(mode, bf16, a, nblocks, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace fl
