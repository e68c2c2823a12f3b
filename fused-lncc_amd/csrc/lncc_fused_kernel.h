// Fused 3D LNCC kernels for gfx950 (MI355X).
//
// One workgroup owns a TX x TY tile of output columns of one (D,H,W) volume and marches along D
// over a chunk [z0,z1) of planes. For each input plane zi it runs a software pipeline whose stages
// are lagged along D, so that every quantity is produced from data already on chip:
//
//   F  (registers) each lane owns input columns of the (TX+4h) x (TY+4h) region; it loads p,t of
//      plane zi (prefetched one plane ahead), keeps a k-deep ring of raw p,t and running z-sums of
//      p, t, p^2, t^2, p*t, and writes the five z-sums of the plane to LDS.
//   X  (LDS) running x-sums of the five z-sums over the (TX+2h)-wide adjoint range.
//   Y  (LDS) running y-sums -> the five k^3 box-sums at plane zc = zi-h on the (TX+2h) x (TY+2h)
//      adjoint region; per voxel squared NCC (clamped to 1) and the three adjoint coefficients
//      alpha, beta, gamma (zero where ncc >= 1 or outside the volume); loss partial sums.
//   AX (LDS) running x-sums of alpha, beta, gamma over the TX output columns.
//   AY (registers) running y-sums for two output rows per lane, a k-deep ring of the xy-sums and
//      running z-sums -> box(alpha), box(beta), box(gamma) at plane zo = zi-2h, combined with p,t
//      of plane zo into the gradient, which is the only per-voxel write to HBM.
//
// Reference semantics (fused_lncc/csrc/lncc3d.cu:93-107, baselines/torch_lncc.py:25-32):
//   cross = Spt - Sp St/n ; vp = max(Spp - Sp^2/n, 0) + dr ; vt likewise ; ncc = cross^2/(vp vt);
//   ncc >= 1 -> ncc = 1 and zero adjoints; NaN keeps NaN ncc and zero adjoints;
//   A = dncc/dSp, Bc = dncc/dvp, Cc = dncc/dcross; grad = -(1/M)(box A + 2p box Bc + t box Cc).
// With r = 1/(vp vt), cr = cross r, u = cr vt, w = St - Sp u the kernel carries
//   alpha = cr w, beta = cr u, gamma = cr   (A = -2 alpha/n, Bc = -beta, Cc = 2 gamma)
// so that grad = (2/M) (box(alpha)/n + p box(beta) - t box(gamma)).
#pragma once
#include "lncc_common.h"
#include "lncc_launch.h"

namespace fl {

template <int HH, bool BF16, int MODE>
__global__ __launch_bounds__(NT, 1) void lncc_fused_kernel(FusedArgs a) {
    using G = Geo<HH>;
    constexpr int K = G::K;
    constexpr bool ADJ = (MODE == MODE_GRAD);
    constexpr int ELEM = BF16 ? 2 : 4;
    constexpr int J = G::J;
    constexpr int ZP = G::IY * G::ZSTRIDE;
    constexpr int XP = G::XROWS * G::XSTRIDE;
    constexpr int GP = G::AY * G::GSTRIDE;
    constexpr int GXP = G::AY * G::GXSTRIDE;
    constexpr int PTP = TY * TX;

    __shared__ float zs[G::Z_FLOATS];
    __shared__ float xs[G::X_FLOATS];
    __shared__ float gs[ADJ ? G::G_FLOATS : 1];
    __shared__ float gxs[ADJ ? G::GX_FLOATS : 1];
    __shared__ float pts[ADJ ? G::PT_FLOATS : 1];
    __shared__ double red[NT / 64];

    const int tid = threadIdx.x;
    const int D = a.dimD, Hd = a.dimH, Wd = a.dimW;

    // workgroup -> tile; consecutive logical tiles (x-neighbours sharing halos) go to one XCD
    const uint32_t nb = gridDim.x, bid = blockIdx.x;
    uint32_t L = (nb % 8u == 0u) ? (bid % 8u) * (nb / 8u) + bid / 8u : bid;
    const int tx = (int)(L % (uint32_t)a.ntx); L /= (uint32_t)a.ntx;
    const int ty = (int)(L % (uint32_t)a.nty); L /= (uint32_t)a.nty;
    const int tz = (int)(L % (uint32_t)a.nzc); L /= (uint32_t)a.nzc;
    const int64_t b = (int64_t)L;
    const int x0 = tx * TX, y0 = ty * TY;
    const int z0 = tz * a.dchunk, z1 = min(z0 + a.dchunk, D);
    const int64_t HW = (int64_t)Hd * Wd;
    const uint32_t plane_bytes = (uint32_t)(HW * ELEM);
    const char* pvol = (const char*)a.pred + b * D * HW * ELEM;
    const char* tvol = (const char*)a.target + b * D * HW * ELEM;

    for (int i = tid; i < G::Z_FLOATS; i += NT) zs[i] = 0.f;
    for (int i = tid; i < G::X_FLOATS; i += NT) xs[i] = 0.f;
    if constexpr (ADJ) {
        for (int i = tid; i < G::G_FLOATS; i += NT) gs[i] = 0.f;
        for (int i = tid; i < G::GX_FLOATS; i += NT) gxs[i] = 0.f;
    }

    // ---- per-lane input columns
    uint32_t voff[J];
    int zoff[J], ptoff[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = tid + j * NT;
        voff[j] = kOOB;
        zoff[j] = -1;
        ptoff[j] = -1;
        if (c < G::NIN) {
            const int iy = c / G::IX, ix = c - iy * G::IX;
            const int gx = x0 - 2 * HH + ix, gy = y0 - 2 * HH + iy;
            if (gx >= 0 && gx < Wd && gy >= 0 && gy < Hd) voff[j] = (uint32_t)((gy * Wd + gx) * ELEM);
            zoff[j] = iy * G::ZSTRIDE + ix;
            const int cx = ix - 2 * HH, cy = iy - 2 * HH;
            if (cx >= 0 && cx < TX && cy >= 0 && cy < TY) ptoff[j] = cy * TX + cx;
        }
    }

    constexpr int LEAD = ADJ ? 2 * HH : HH;
    const int zlo = max(z0 - LEAD, 0);
    const int zhi = z1 + LEAD;
    const int zc_lo = ADJ ? max(z0 - HH, 0) : z0;
    const int zc_hi = ADJ ? min(z1 + HH, D) : z1;

    float pring[J][K], tring[J][K], zsum[J][5], pnext[J], tnext[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int r = 0; r < K; ++r) { pring[j][r] = 0.f; tring[j][r] = 0.f; }
#pragma unroll
        for (int q = 0; q < 5; ++q) zsum[j][q] = 0.f;
    }
    {
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(pvol + (int64_t)zlo * HW * ELEM, plane_bytes);
        const __amdgpu_buffer_rsrc_t rt = make_rsrc(tvol + (int64_t)zlo * HW * ELEM, plane_bytes);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            pnext[j] = load_elem<BF16>(rp, voff[j]);
            tnext[j] = load_elem<BF16>(rt, voff[j]);
        }
    }

    // adjoint-side state: lane owns output columns (ox, oy) and (ox, oy+1)
    const int ox = tid % TX;
    const int oy = 2 * (tid / TX);
    float gring[2][3][K], gz[2][3];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            gz[m][c] = 0.f;
#pragma unroll
            for (int r = 0; r < K; ++r) gring[m][c][r] = 0.f;
        }

    double loss_acc = 0.0;
    const float inv_n = a.inv_n, dr = a.dr;
    __syncthreads();

    for (int base = zlo; base < zhi; base += K) {
        static_for<0, K>([&](auto rc) __attribute__((always_inline)) {
            constexpr int r = decltype(rc)::value;
            const int zi = base + r;
            if (zi >= zhi) return;
            const int s = zi - zlo;

            // ---------------- F: z-sums of the input region ----------------
            float pc[J], tc[J];
#pragma unroll
            for (int j = 0; j < J; ++j) { pc[j] = pnext[j]; tc[j] = tnext[j]; }
            if (zi + 1 < zhi && zi + 1 < D) {
                const __amdgpu_buffer_rsrc_t rp = make_rsrc(pvol + (int64_t)(zi + 1) * HW * ELEM, plane_bytes);
                const __amdgpu_buffer_rsrc_t rt = make_rsrc(tvol + (int64_t)(zi + 1) * HW * ELEM, plane_bytes);
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    pnext[j] = load_elem<BF16>(rp, voff[j]);
                    tnext[j] = load_elem<BF16>(rt, voff[j]);
                }
            } else {
#pragma unroll
                for (int j = 0; j < J; ++j) { pnext[j] = 0.f; tnext[j] = 0.f; }
            }
            constexpr int ro = (r + 1) % K;  // oldest ring slot after this step: plane zi-2h
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const float p = pc[j], t = tc[j];
                const float po = pring[j][r], to = tring[j][r];
                zsum[j][0] += p - po;
                zsum[j][1] += t - to;
                zsum[j][2] = fmaf(p, p, fmaf(-po, po, zsum[j][2]));
                zsum[j][3] = fmaf(t, t, fmaf(-to, to, zsum[j][3]));
                zsum[j][4] = fmaf(p, t, fmaf(-po, to, zsum[j][4]));
                pring[j][r] = p;
                tring[j][r] = t;
                if (zoff[j] >= 0) {
#pragma unroll
                    for (int q = 0; q < 5; ++q) zs[q * ZP + zoff[j]] = zsum[j][q];
                }
                if constexpr (ADJ) {
                    if (ptoff[j] >= 0) {
                        pts[(s & 1) * 2 * PTP + ptoff[j]] = pring[j][ro];
                        pts[(s & 1) * 2 * PTP + PTP + ptoff[j]] = tring[j][ro];
                    }
                }
            }
            __syncthreads();

            const int zc = zi - HH;
            const bool fwd = (zc >= zc_lo) && (zc < zc_hi);
            if (fwd) {
                // ---------------- X: running x-sums of the five z-sums ----------------
#pragma unroll
                for (int u = 0; u < cdiv(G::XITEMS, NT); ++u) {
                    const int it = tid + u * NT;
                    if (it < G::XITEMS) {
                        const int iy = it % G::IY, seg = it / G::IY;
                        const float* src = zs + iy * G::ZSTRIDE + seg * G::SX;
                        float* dst = xs + iy * G::XSTRIDE + seg * G::SX;
#pragma unroll
                        for (int q = 0; q < 5; ++q) {
                            float v[G::SX + 2 * HH];
#pragma unroll
                            for (int i = 0; i < G::SX + 2 * HH; ++i) v[i] = src[q * ZP + i];
                            float acc = v[0];
#pragma unroll
                            for (int i = 1; i <= 2 * HH; ++i) acc += v[i];
                            dst[q * XP] = acc;
#pragma unroll
                            for (int i = 1; i < G::SX; ++i) {
                                acc += v[i + 2 * HH] - v[i - 1];
                                dst[q * XP + i] = acc;
                            }
                        }
                    }
                }
                __syncthreads();

                // ---------------- Y: box-sums, ncc, adjoint coefficients ----------------
                const bool count = (zc >= z0) && (zc < z1);
                float lsum = 0.f;
#pragma unroll
                for (int u = 0; u < cdiv(G::YITEMS, NT); ++u) {
                    const int it = tid + u * NT;
                    if (it < G::YITEMS) {
                        const int ax = it % G::AX, seg = it / G::AX;
                        const float* src = xs + seg * G::SY * G::XSTRIDE + ax;
                        float S[5][G::SY];
#pragma unroll
                        for (int q = 0; q < 5; ++q) {
                            float v[G::SY + 2 * HH];
#pragma unroll
                            for (int i = 0; i < G::SY + 2 * HH; ++i) v[i] = src[q * XP + i * G::XSTRIDE];
                            float acc = v[0];
#pragma unroll
                            for (int i = 1; i <= 2 * HH; ++i) acc += v[i];
                            S[q][0] = acc;
#pragma unroll
                            for (int i = 1; i < G::SY; ++i) {
                                acc += v[i + 2 * HH] - v[i - 1];
                                S[q][i] = acc;
                            }
                        }
                        const int gx = x0 - HH + ax;
                        const bool inx = gx >= 0 && gx < Wd;
                        const bool corex = ax >= HH && ax < HH + TX;
#pragma unroll
                        for (int i = 0; i < G::SY; ++i) {
                            const int ay = seg * G::SY + i;
                            const float Sp = S[0][i], St = S[1][i], Spp = S[2][i], Stt = S[3][i], Spt = S[4][i];
                            const float mp = Sp * inv_n, mt = St * inv_n;
                            const float cross = fmaf(-mp, St, Spt);
                            const float vp = fmaxf(fmaf(-mp, Sp, Spp), 0.f) + dr;
                            const float vt = fmaxf(fmaf(-mt, St, Stt), 0.f) + dr;
                            const float rr = __builtin_amdgcn_rcpf(vp * vt);
                            const float cr = cross * rr;
                            const float ncc = cross * cr;
                            const int gy = y0 - HH + ay;
                            const bool inv = inx && gy >= 0 && gy < Hd && ay < G::AY;
                            const bool live = inv && (ncc < 1.0f);
                            const float nccc = (ncc >= 1.0f) ? 1.0f : ncc;
                            const bool core = corex && ay >= HH && ay < HH + TY;
                            if (count && inv && core) lsum += nccc;
                            if constexpr (ADJ) {
                                const float uu = cr * vt;
                                const float w = fmaf(-Sp, uu, St);
                                if (ay < G::AY) {
                                    gs[0 * GP + ay * G::GSTRIDE + ax] = live ? cr * w : 0.f;
                                    gs[1 * GP + ay * G::GSTRIDE + ax] = live ? cr * uu : 0.f;
                                    gs[2 * GP + ay * G::GSTRIDE + ax] = live ? cr : 0.f;
                                }
                            }
                            if constexpr (MODE == MODE_MAPS) {
                                if (count && inv && core) {
                                    const float uu = cr * vt;
                                    const float w = fmaf(-Sp, uu, St);
                                    const int64_t o = ((b * D + zc) * Hd + gy) * (int64_t)Wd + gx;
                                    a.ncc_map[o] = nccc;
                                    a.a_map[o] = live ? -2.f * inv_n * (cr * w) : 0.f;
                                    a.b_map[o] = live ? -(cr * uu) : 0.f;
                                    a.c_map[o] = live ? 2.f * cr : 0.f;
                                }
                            }
                        }
                    }
                }
                loss_acc += (double)lsum;
            }

            if constexpr (ADJ) {
                if (fwd) {
                    __syncthreads();
                    // ---------------- AX: running x-sums of alpha, beta, gamma ----------------
#pragma unroll
                    for (int u = 0; u < cdiv(G::X2ITEMS, NT); ++u) {
                        const int it = tid + u * NT;
                        if (it < G::X2ITEMS) {
                            const int ay = it % G::AY, seg = it / G::AY;
                            const float* src = gs + ay * G::GSTRIDE + seg * G::SX2;
                            float* dst = gxs + ay * G::GXSTRIDE + seg * G::SX2;
#pragma unroll
                            for (int c = 0; c < 3; ++c) {
                                float v[G::SX2 + 2 * HH];
#pragma unroll
                                for (int i = 0; i < G::SX2 + 2 * HH; ++i) v[i] = src[c * GP + i];
                                float acc = v[0];
#pragma unroll
                                for (int i = 1; i <= 2 * HH; ++i) acc += v[i];
                                dst[c * GXP] = acc;
#pragma unroll
                                for (int i = 1; i < G::SX2; ++i) {
                                    acc += v[i + 2 * HH] - v[i - 1];
                                    dst[c * GXP + i] = acc;
                                }
                            }
                        }
                    }
                    __syncthreads();
                }
                // ---------------- AY: y-sums, z ring, combine ----------------
                float ys[2][3];
                if (fwd) {
                    const float* src = gxs + oy * G::GXSTRIDE + ox;
#pragma unroll
                    for (int c = 0; c < 3; ++c) {
                        float v[2 + 2 * HH];
#pragma unroll
                        for (int i = 0; i < 2 + 2 * HH; ++i) v[i] = src[c * GXP + i * G::GXSTRIDE];
                        float acc = v[0];
#pragma unroll
                        for (int i = 1; i <= 2 * HH; ++i) acc += v[i];
                        ys[0][c] = acc;
                        ys[1][c] = acc + v[2 * HH + 1] - v[0];
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < 2; ++m)
#pragma unroll
                        for (int c = 0; c < 3; ++c) ys[m][c] = 0.f;
                }
#pragma unroll
                for (int m = 0; m < 2; ++m)
#pragma unroll
                    for (int c = 0; c < 3; ++c) {
                        gz[m][c] += ys[m][c] - gring[m][c][r];
                        gring[m][c][r] = ys[m][c];
                    }
                const int zo = zi - 2 * HH;
                if (zo >= z0 && zo < z1) {
                    const int gx = x0 + ox;
#pragma unroll
                    for (int m = 0; m < 2; ++m) {
                        const int gy = y0 + oy + m;
                        const float p = pts[(s & 1) * 2 * PTP + (oy + m) * TX + ox];
                        const float t = pts[(s & 1) * 2 * PTP + PTP + (oy + m) * TX + ox];
                        const float g = a.gscale * fmaf(inv_n, gz[m][0], fmaf(p, gz[m][1], -t * gz[m][2]));
                        if (gx < Wd && gy < Hd) store_elem<BF16>(a.grad, ((b * D + zo) * Hd + gy) * (int64_t)Wd + gx, g);
                    }
                }
            }
        });
    }

    // ---- workgroup partial of the ncc sum: wave64 reduction, then the 8 waves in fixed order
    if constexpr (MODE == MODE_MAPS) return;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) loss_acc += __shfl_xor(loss_acc, off, 64);
    if ((tid & 63) == 0) red[tid >> 6] = loss_acc;
    __syncthreads();
    if (tid == 0) {
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) sum += red[w];
        a.partials[bid] = sum;
    }
}

template <int HH>
hipError_t launch_fused(int mode, bool bf16, const FusedArgs& a, uint32_t nblocks, hipStream_t st) {
    const dim3 grid(nblocks), block(NT);
#define FL_LAUNCH(BF, MD) hipLaunchKernelGGL((lncc_fused_kernel<HH, BF, MD>), grid, block, 0, st, a)
    if (mode == MODE_LOSS) {
        if (bf16) FL_LAUNCH(true, MODE_LOSS); else FL_LAUNCH(false, MODE_LOSS);
    } else if (mode == MODE_GRAD) {
        if (bf16) FL_LAUNCH(true, MODE_GRAD); else FL_LAUNCH(false, MODE_GRAD);
    } else {
        if (bf16) FL_LAUNCH(true, MODE_MAPS); else FL_LAUNCH(false, MODE_MAPS);
    }
#undef FL_LAUNCH
    return hipGetLastError();
}

}  // namespace fl
