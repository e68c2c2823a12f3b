// Fused 3D LNCC kernels for gfx950 (MI355X).
//
// One workgroup (1024 lanes) owns a TX x TY tile of output columns of one (D,H,W) volume and
// marches along D over a chunk [z0,z1) of planes. Per input plane zi it runs six stages, lagged
// along D so that every quantity is produced from data already on chip:
//
//   F   (registers) lanes own the input columns of the (TX+4h) x (TY+4h) region and keep the
//       last k planes of p, t in a register ring; the z-sums of p, t, p^2, t^2, p*t over planes
//       [zi-k+1, zi] are formed from the ring (below) and written to LDS.
//   X   x-sums of the five z-sums over the (TX+2h)-wide adjoint range.
//   Y   y-sums -> the five k^3 box-sums on the (TX+2h) x (TY+2h) adjoint region; per voxel
//       squared NCC (clamped to 1), loss partial sums, and the adjoint coefficients alpha, beta,
//       gamma (zero where ncc >= 1 or outside the volume).
//   AX  x-sums of alpha, beta, gamma over the TX output columns.
//   AYs y-sums of the three over the TY output rows.
//   AZ  (registers) one lane per output column: a k-deep ring of the xy-sums -> z-sums
//       box(alpha), box(beta), box(gamma), combined with p,t of the output plane (re-read from
//       the L2 as their last use, non-temporal) into the gradient, the only per-voxel write to HBM.
//
// Every box-sum is a sum of its window's own values (lncc_window.h): in x and y blocks of k
// values give each window as a block suffix plus the next block's prefix; along D the march is
// unrolled by k, the ring slot r of plane zi is its position in its block of k planes, and the
// z-sum at zi is the prefix of the current block (planes of slots 0..r, carried in registers)
// plus the suffix of the previous block still in the ring (slots r+1..k-1). So windows of zeros
// sum to exactly zero and windows of one constant to exactly k^3 c, as the reference's direct
// sums do; running sums (add the entering value, subtract the leaving one) would carry the
// rounding of every earlier plane into them.
//
// Software pipeline: the chain F -> X -> Y -> AX -> AYs -> AZ alternates between two phases per
// plane, P0 = {F(zi), Y(zi-1), AYs(zi-2)} and P1 = {X(zi), AX(zi-1), AZ(zi-2)}, so each plane costs
// two workgroup barriers. F and AZ run on every lane; the Y items and the AYs units, and the X and
// the AX units, sit on disjoint waves.
//
// Reference semantics (fused_lncc/csrc/lncc3d.cu:93-107, baselines/torch_lncc.py:25-32):
//   cross = Spt - Sp St/n ; vp = max(Spp - Sp^2/n, 0) + dr ; vt likewise ; ncc = cross^2/(vp vt);
//   ncc >= 1 -> ncc = 1 and zero adjoints; NaN keeps NaN ncc and zero adjoints;
//   A = dncc/dSp, Bc = dncc/dvp, Cc = dncc/dcross; grad = -(1/M)(box A + 2p box Bc + t box Cc).
// The kernel forms the n-fold quantities X = n Spt - Sp St, VP = max(n Spp - Sp^2, 0) + n dr and
// VT likewise (ncc = X^2/(VP VT)): an integer n times a sum and one fused multiply-add, so a
// window of one constant c gives exactly X = 0 and VP - n dr = 0 whenever n^2 c^2 is a float, as
// the reference's Sp St / n division does (a reciprocal 1/n would leave a residue there that the
// division by dr^2 blows up). With r = 1/(VP VT), c = X r, u = c VT, w = St - Sp u it carries
//   alpha = c w, beta = c u, gamma = c   (A = -2 alpha, Bc = -n beta, Cc = 2 n gamma)
// so that grad = (2n/M) (box(alpha)/n + p box(beta) - t box(gamma)).
#pragma once
#include "lncc_common.h"
#include "lncc_launch.h"
#include "lncc_window.h"

namespace fl {

// Loads NV consecutive floats from a 16-byte aligned LDS address: float4s, then a tail of 2 or 1
// floats as a float2 or a float (a tail of 3 as one more float4, which reads one float past the
// row; it is not used), row_read(NV) floats in all. Each vector passes through an empty asm
// operand that needs all of its lanes, so that the loads stay whole: otherwise the optimizer
// re-partitions them along the box-sums' blocks (a row of 10 floats became b128 + b96 + read2_b32
// + b32 instead of b128 + b128 + b64), which costs LDS instructions and bank cycles. The 2-float
// tail (rather than a third float4) also keeps two registers per row free.
typedef float lds_f4 __attribute__((ext_vector_type(4)));
typedef float lds_f2 __attribute__((ext_vector_type(2)));
template <int NV>
__device__ __forceinline__ void lds_row(const float* __restrict__ src, float (&v)[NV]) {
    static_assert(row_read(NV) >= NV, "row read");
#pragma unroll
    for (int m = 0; m < NV / 4; ++m) {
        lds_f4 f = reinterpret_cast<const lds_f4*>(src)[m];
        asm("" : "+v"(f));
        v[4 * m] = f.x;
        v[4 * m + 1] = f.y;
        v[4 * m + 2] = f.z;
        v[4 * m + 3] = f.w;
    }
    constexpr int t = NV / 4 * 4;
    if constexpr (NV % 4 == 3) {
        lds_f4 f = reinterpret_cast<const lds_f4*>(src)[NV / 4];
        asm("" : "+v"(f));
        v[t] = f.x;
        v[t + 1] = f.y;
        v[t + 2] = f.z;
    } else if constexpr (NV % 4 == 2) {
        lds_f2 f = *reinterpret_cast<const lds_f2*>(src + t);
        asm("" : "+v"(f));
        v[t] = f.x;
        v[t + 1] = f.y;
    } else if constexpr (NV % 4 == 1) {
        float f = src[t];
        asm("" : "+v"(f));
        v[t] = f;
    }
}

template <int HH, bool BF16, int MODE>
__global__ __launch_bounds__(NT, WG_PER_CU) void lncc_fused_kernel(FusedArgs a) {
    constexpr bool ADJ = (MODE == MODE_GRAD);
    using G = Geo<HH>;
    constexpr int K = G::K;
    constexpr int ELEM = BF16 ? 2 : 4;
    constexpr int J = G::J;
    constexpr int TY = G::TY;

    // one __shared__ array per buffer, so the compiler knows that the reads of one stage do not
    // alias the writes of another and can overlap them
    __shared__ __align__(16) float Zs[5 * G::ZP + G::PAD];
    __shared__ __align__(16) float Xs[5 * G::XP + G::PAD];
    __shared__ __align__(16) float Gs[ADJ ? 3 * G::GP + G::PAD : 4];
    __shared__ __align__(16) float GXs[ADJ ? 3 * G::GXP + G::PAD : 4];
    __shared__ __align__(16) float GY[ADJ ? 3 * G::GYP : 2];
    __shared__ double red[NT / 64];

    const int tid = threadIdx.x;
    // the wave's index in the workgroup, wave-uniform (a scalar register): at k >= 7 the reduction
    // after the march uses it with the lane index (recomputed there), so that no vector register
    // carries the thread index across the march (at the register limit of those kernels it was
    // spilled to scratch: 6 MB of extra HBM traffic per launch at (2,16,128^3)); at k <= 5, where
    // nothing spills, keeping the thread index measured 1% faster
    const int wave_id = __builtin_amdgcn_readfirstlane(tid) >> 6;
    const int D = a.dimD, Hd = a.dimH, Wd = a.dimW;

    // workgroup -> tile. Workgroups go to the 8 XCDs round-robin (workgroup i on XCD i % 8); XCD j
    // takes the j-th contiguous range of logical tiles (q + (j < r) of them, q = nb / 8, r = nb % 8),
    // so that neighbouring tiles, which share halo columns, share one L2
    const uint32_t nb = gridDim.x, bid = blockIdx.x;
    const uint32_t xcd = bid % 8u, q8 = nb / 8u, r8 = nb % 8u;
    uint32_t L = xcd * q8 + min(xcd, r8) + bid / 8u;
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
    char* const gvol = ADJ ? (char*)a.grad + b * D * HW * ELEM : nullptr;

    // ---- F: per-lane input columns
    uint32_t voff[J];
    int zaddr[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        int ix, iy;
        voff[j] = kOOB;
        zaddr[j] = -1;
        if (f_column<G>(tid + j * NT, ix, iy, zaddr[j])) {
            const int gx = x0 - 2 * HH + ix, gy = y0 - 2 * HH + iy;
            if (gx >= 0 && gx < Wd && gy >= 0 && gy < Hd) voff[j] = (uint32_t)((gy * Wd + gx) * ELEM);
        }
    }
    if constexpr (G::FPAIR) zaddr[1] = zaddr[0] + NT;  // a lane without a second column writes padding
    // P1 units: X (z-sums -> x-sums) then AX (adjoints -> x-sums); offsets into the source and
    // destination buffers and the unit kind (0 none, 1 X, 2 AX)
    int u_src[G::U1], u_dst[G::U1], u_kind[G::U1];
#pragma unroll
    for (int k = 0; k < G::U1; ++k) u_kind[k] = p1_unit<G, ADJ>(tid + k * NT, u_src[k], u_dst[k]);
    // P0: Y items on lanes [0, YITEMS), AYs units on waves 10, 11, 14, 15
    const bool has_y = tid < G::YITEMS;
    int y_seg = 0, y_ax = 0;  // rows seg of AX positions
    if (has_y) y_item<G>(tid, y_seg, y_ax);
    const int y_start = y_seg * G::SY;
    // per output of the Y segment: inside the volume (ncc and adjoints live) / counted in the loss
    // (inside the volume and in the output tile); the same on every plane
    bool y_inv[G::SY], y_core[G::SY];
    {
        const int gx = x0 - HH + y_ax;
        const bool inx = has_y && gx >= 0 && gx < Wd;
        const bool corex = y_ax >= HH && y_ax < HH + TX;
#pragma unroll
        for (int i = 0; i < G::SY; ++i) {
            const int ay = y_start + i, gy = y0 - HH + ay;
            y_inv[i] = inx && gy >= 0 && gy < Hd;
            y_core[i] = y_inv[i] && corex && ay >= HH && ay < HH + TY;
        }
    }
    int b_src, b_dst;
    const bool has_b = ays_unit<G>(tid, b_src, b_dst) && ADJ;
    const bool has_z = ADJ && tid < G::NOUT;
    int z_ox, z_oy;
    az_lane<G>(tid, z_ox, z_oy);
    const bool z_in = has_z && x0 + z_ox < Wd && y0 + z_oy < Hd;
    const uint32_t z_voff = z_in ? (uint32_t)(((y0 + z_oy) * Wd + x0 + z_ox) * ELEM) : kOOB;

    constexpr int LEAD = ADJ ? 2 * HH : HH;
    const int zlo = max(z0 - LEAD, 0);
    const int zhi = ADJ ? z1 + 2 + 2 * HH : z1 + 1 + HH;
    const int zc_lo = ADJ ? max(z0 - HH, 0) : z0;
    const int zc_hi = ADJ ? min(z1 + HH, D) : z1;

    // F state: the ring of the last k planes' p,t (slot r = position of the plane in its block of
    // k), the prefix sums of the five fields over the current block, and p,t of the next plane
    // (prefetched one step ahead). The ring starts at zero: nothing before the first plane of the
    // march enters a window that is used.
    float pring[J][K], tring[J][K], fpre[J][5], zsum[J][5], pnext[J], tnext[J];
    float pz = 0.f, tzz = 0.f;  // AZ: p,t at this step's output plane (prefetched one step ahead)
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            fpre[j][q] = 0.f;
            zsum[j][q] = 0.f;
        }
#pragma unroll
        for (int r = 0; r < K; ++r) {
            pring[j][r] = 0.f;
            tring[j][r] = 0.f;
        }
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
    // AZ state: the ring of the last k planes' xy-sums of alpha, beta, gamma and their prefix sums
    // over the current block
    float gring[3][K], gpre[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        gpre[c] = 0.f;
#pragma unroll
        for (int r = 0; r < K; ++r) gring[c][r] = 0.f;
    }

    double loss_acc = 0.0;
    const float inv_n = a.inv_n, nf = a.nf, ndr = a.ndr;

    // Plane addresses advance by one plane per step: zoff = zi * plane size, and every plane the
    // loop touches sits at a fixed plane distance from zi. A plane outside its valid range gets a
    // zero-sized resource (its address is never dereferenced).
    const uint64_t PB = (uint64_t)HW * ELEM;
    const uint64_t pva = (uint64_t)(uintptr_t)pvol, tva = (uint64_t)(uintptr_t)tvol;
    const uint64_t gva = (uint64_t)(uintptr_t)gvol;
    uint64_t zoff = (uint64_t)zlo * PB;
    const int zn_hi = min(zhi, D);                 // F: new plane zi+1 valid while zi+1 < zn_hi
    constexpr int ZO = 2 + 2 * HH;                 // AZ: output plane zi-ZO

    // Stage bodies; the march below orders them per phase.
    //
    // Y(zi-1): box sums S (y-sums of the rows of the five x-sums), then ncc and the adjoint
    // coefficients at plane zcY (y_math).
    auto y_math = [&](const float (&S)[5][G::SY], int zcY) __attribute__((always_inline)) {
        const bool count = zcY >= z0 && zcY < z1;
        float lsum = -0.f;  // -0 + x == x for every x, so the first add folds away
        float adj[3][G::SY];  // alpha, beta, gamma of the segment's outputs
#pragma unroll
        for (int i = 0; i < G::SY; ++i) {
            const int ay = y_start + i;
            const float Sp = S[0][i], St = S[1][i], Spp = S[2][i], Stt = S[3][i], Spt = S[4][i];
            const float X = fmaf(-Sp, St, nf * Spt);
            // n dr is added after the cancellation: folded into the fma that rounds n Spp, it
            // would break that rounding's ties (frequent when n Spp has few significant bits)
            // always upwards, a bias of ~2e-5 in ncc on offset intensities at k = 3
            const float VP = fmaxf(fmaf(-Sp, Sp, nf * Spp), 0.f) + ndr;
            const float VT = fmaxf(fmaf(-St, St, nf * Stt), 0.f) + ndr;
            const float rr = __builtin_amdgcn_rcpf(VP * VT);
            const float cr = X * rr;
            const float ncc = X * cr;
            const bool live = y_inv[i] && (ncc < 1.0f);
            const float nccc = (ncc >= 1.0f) ? 1.0f : ncc;
            if (count && y_core[i]) lsum += nccc;
            if constexpr (ADJ) {
                // masking cr masks all three coefficients (alpha, beta, gamma are multiples of it)
                const float crm = live ? cr : 0.f;
                const float uu = crm * VT;
                const float w = fmaf(-Sp, uu, St);
                if constexpr (G::ASWAP) {
                    adj[0][i] = crm * w;
                    adj[1][i] = crm * uu;
                    adj[2][i] = crm;
                } else {
                    Gs[y_gs<G>(0, y_ax, ay)] = crm * w;
                    Gs[y_gs<G>(1, y_ax, ay)] = crm * uu;
                    Gs[y_gs<G>(2, y_ax, ay)] = crm;
                }
            }
            if constexpr (MODE == MODE_MAPS) {
                if (count && y_core[i]) {
                    const float uu = cr * VT;
                    const float w = fmaf(-Sp, uu, St);
                    const int gx = x0 - HH + y_ax, gy = y0 - HH + ay;
                    const int64_t o = ((b * D + zcY) * Hd + gy) * (int64_t)Wd + gx;
                    a.ncc_map[o] = nccc;
                    if (a.a_map) {  // null: the ncc map alone
                        a.a_map[o] = live ? -2.f * (cr * w) : 0.f;
                        a.b_map[o] = live ? -nf * (cr * uu) : 0.f;
                        a.c_map[o] = live ? (2.f * nf) * cr : 0.f;
                    }
                }
            }
        }
        if constexpr (ADJ && G::ASWAP) {  // Gs rows along y: one float4 per field
            static_assert(G::SY == 4, "float4 rows");
#pragma unroll
            for (int c = 0; c < 3; ++c)
                *reinterpret_cast<lds_f4*>(Gs + y_gs<G>(c, y_ax, y_start)) = lds_f4{adj[c][0], adj[c][1], adj[c][2], adj[c][3]};
        }
        loss_acc += (double)lsum;
    };
    // F(zi): z-sums of the input region over planes [zi-k+1, zi] (zstep5: the plane prefetched one
    // step ago joins the block prefix and the ring, the previous block's suffix comes from the
    // ring), then the prefetch of the next plane. Every global access of the loop is issued unconditionally
    // (inactive ones through a zero-sized buffer), so the number of outstanding memory operations
    // is the same on every path and the waits before use stay exact. With STORE the z-sums go to
    // the LDS column by column as they are formed; without, f_store writes them later.
    auto f_sums = [&](auto rc, auto store, int zi, uint64_t zoff) __attribute__((always_inline)) {
        constexpr int r = decltype(rc)::value;
        constexpr bool STORE = decltype(store)::value;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            zstep5<K, r>(pnext[j], tnext[j], fpre[j], pring[j], tring[j], zsum[j]);
            if constexpr (STORE) {
                if (G::FPAIR || zaddr[j] >= 0) {
#pragma unroll
                    for (int q = 0; q < 5; ++q) Zs[q * G::ZP + zaddr[j]] = zsum[j][q];
                }
            }
        }
        // prefetch plane zi+1
        const bool okn = zi + 1 < zn_hi;
        const __amdgpu_buffer_rsrc_t rpn = rsrc_at(pva + zoff + PB, plane_bytes, okn);
        const __amdgpu_buffer_rsrc_t rtn = rsrc_at(tva + zoff + PB, plane_bytes, okn);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            pnext[j] = load_elem<BF16>(rpn, voff[j]);
            tnext[j] = load_elem<BF16>(rtn, voff[j]);
        }
    };
    auto f_store = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            if (zaddr[j] >= 0) {
#pragma unroll
                for (int q = 0; q < 5; ++q) Zs[q * G::ZP + zaddr[j]] = zsum[j][q];
            }
        }
    };
    // X(zi) or AX(zi-1), the lane's unit: x-sums of one z-sum (feeds Y at the next plane) or of
    // one of alpha, beta, gamma at plane zcY, over one segment. The row is read early and the sums
    // formed by u_math later; the early read takes SX + 2h floats for both kinds (SX >= SA), and an
    // AX row's extra floats stay inside Gs, unused.
    static_assert(G::U1 == 1 && G::SX >= G::SA, "one unit per lane");
    auto u_math = [&](const float (&uv)[G::SX + 2 * HH], bool runX, bool runA) __attribute__((always_inline)) {
        if (runX) {
            float o[G::SX];
            box_sums<HH, G::SX>(uv, o);
#pragma unroll
            for (int i = 0; i < G::SX; ++i) Xs[u_dst[0] + i * G::XS] = o[i];
        } else if (runA) {
            float v[G::SA + 2 * HH], o[G::SA];
#pragma unroll
            for (int i = 0; i < G::SA + 2 * HH; ++i) v[i] = uv[i];
            box_sums<HH, G::SA>(v, o);
#pragma unroll
            for (int i = 0; i < G::SA; ++i) GXs[u_dst[0] + i * G::GXS] = o[i];
        }
    };

    // Stage order inside a phase. Each wave runs its stages in program order, so a stage placed
    // between the issue of another stage's LDS reads and their use hides part of their latency:
    //  * P0, k <= 5: Y's five rows are read, F's arithmetic and prefetch run while they arrive,
    //    then Y's math, AYs, and F's stores last.
    //  * P0, k = 7: three of Y's rows, then F whole (its z-sums stored as they are formed), then
    //    Y's other two rows: five rows held across F, or F's z-sums held until after Y, exceed the
    //    128-register budget of a 1024-lane workgroup (spills in the loop).
    //  * P0, k = 9: Y, AYs, then F (its two rings leave no room for rows read early).
    //  * P1: AZ's xy-sums are read before everything else, and the unit's row is read before AZ
    //    and its sums formed after AZ.
    constexpr int Y_EARLY = HH <= 2 ? 5 : HH == 3 ? 3 : 0;   // Y rows read before F
    constexpr bool F_STORE_AT_ONCE = Y_EARLY < 5;

    for (int base = zlo; base < zhi; base += K) {
        static_for<0, K>([&](auto rc) __attribute__((always_inline)) {
            const int zi = base + decltype(rc)::value;
            if (zi >= zhi) return;
            const int zcY = zi - 1 - HH;   // Y(zi-1) and AX(zi-1)
            const bool actY = zcY >= zc_lo && zcY < zc_hi;
            const int zcB = zi - 2 - HH;   // AYs(zi-2) and the xy-sums AZ(zi-2) reads
            const bool actB = ADJ && zcB >= zc_lo && zcB < zc_hi;

            // ============================ phase P0 ============================
            // Y(zi-1), AYs(zi-2), F(zi)
            if constexpr (Y_EARLY > 0) {
                float yv[5][G::SY + 2 * HH];
                if (actY && has_y) {
#pragma unroll
                    for (int q = 0; q < Y_EARLY; ++q) lds_row(Xs + q * G::XP + y_ax * G::XS + y_start, yv[q]);
                }
                f_sums(rc, std::integral_constant<bool, F_STORE_AT_ONCE>{}, zi, zoff);
                if (actY && has_y) {
#pragma unroll
                    for (int q = Y_EARLY; q < 5; ++q) lds_row(Xs + q * G::XP + y_ax * G::XS + y_start, yv[q]);
                    float S[5][G::SY];
#pragma unroll
                    for (int q = 0; q < 5; ++q) box_sums<HH, G::SY>(yv[q], S[q]);
                    y_math(S, zcY);
                }
            } else if (actY && has_y) {
                // one row at a time: all five held at once exceed the register budget here
                float S[5][G::SY];
#pragma unroll
                for (int q = 0; q < 5; ++q) {
                    float yv[G::SY + 2 * HH];
                    lds_row(Xs + q * G::XP + y_ax * G::XS + y_start, yv);
                    box_sums<HH, G::SY>(yv, S[q]);
                }
                y_math(S, zcY);
            }
            if constexpr (ADJ) {
                // AYs(zi-2): y-sums (x-sums with ASWAP) of alpha, beta, gamma at plane zcB (one
                // quantity per unit)
                if (actB && has_b) {
                    float v[G::SB + 2 * HH], o[G::SB];
                    lds_row(GXs + b_src, v);
                    box_sums<HH, G::SB>(v, o);
#pragma unroll
                    for (int i = 0; i < G::SB; ++i) {
                        if constexpr (G::ASWAP) {  // GY rows along x: float4s
                            if (i % 4 == 0)
                                *reinterpret_cast<lds_f4*>(GY + b_dst + i) = lds_f4{o[i], o[i + 1], o[i + 2], o[i + 3]};
                        } else {
                            GY[b_dst + i * G::BW] = o[i];
                        }
                    }
                }
            }
            if constexpr (Y_EARLY == 0) {
                f_sums(rc, std::true_type{}, zi, zoff);
            } else if constexpr (!F_STORE_AT_ONCE) {
                f_store();
            }
            __syncthreads();

            // ============================ phase P1 ============================
            // X(zi) and AX(zi-1) on the unit lanes, AZ(zi-2) on the output lanes
            float ys[3];
            if constexpr (ADJ) {
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    // read whatever actB says (the value is dropped when it is false), so that the
                    // three reads pair up
                    const float gy = GY[c * G::GYP + z_oy * G::GYS + z_ox];
                    ys[c] = actB ? gy : 0.f;
                }
            }
            const int zcX = zi - HH;
            const bool actX = zcX >= zc_lo && zcX < zc_hi;
            const bool runX = u_kind[0] == 1 && actX, runA = ADJ && u_kind[0] == 2 && actY;
            float uv[G::SX + 2 * HH];
            if (runX || runA) lds_row((runA ? Gs : Zs) + u_src[0], uv);
            if constexpr (ADJ) {
                // AZ(zi-2): z-sums of the xy-sums over the k planes of the output plane zo = the
                // prefix of the current block plus the previous block's suffix still in the ring
                // (lanes without an output column run on a clamped one and store out of range,
                // i.e. nothing)
                constexpr int r = decltype(rc)::value;
                float gw[3];
#pragma unroll
                for (int c = 0; c < 3; ++c) gw[c] = zstep1<K, r>(ys[c], gpre[c], gring[c]);
                const int zo = zi - ZO;
                const float g = a.gscale * fmaf(inv_n, gw[0], fmaf(pz, gw[1], -tzz * gw[2]));
                // Non-temporal: the gradient is never read back, and this re-read of p,t is the
                // last use of those lines. With the default policy both would be promoted in the
                // L2 and push out the planes that F loaded and this stage re-reads 2h+2 steps
                // later, so that every input byte would be fetched about twice; marked
                // evict-first, every input byte is fetched from HBM once. bf16 gradient rows of a
                // tile are half a 128-byte line (the x-neighbour tile writes the other half):
                // those stores keep the default policy, so that the L2 merges the two halves into
                // one write.
                store_elem_buf<BF16, BF16 ? 0 : kNT>(rsrc_at(gva + zoff - ZO * PB, plane_bytes, zo >= z0 && zo < z1), z_voff, g);
                // prefetch p,t at the next step's output plane; issued after this step's use, so
                // one register each suffices and no copy has to wait for the load
                const bool oko = zo + 1 >= z0 && zo + 1 < z1;
                pz = load_elem<BF16, kNT>(rsrc_at(pva + zoff - (ZO - 1) * PB, plane_bytes, oko), z_voff);
                tzz = load_elem<BF16, kNT>(rsrc_at(tva + zoff - (ZO - 1) * PB, plane_bytes, oko), z_voff);
            }
            u_math(uv, runX, runA);
            zoff += PB;
            __syncthreads();
        });
    }

    // ---- workgroup partial of the ncc sum: wave64 reduction, then the waves in fixed order
    if constexpr (MODE == MODE_MAPS) return;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) loss_acc += __shfl_xor(loss_acc, off, 64);
    const int lane = HH >= 3 ? (int)__lane_id() : (tid & 63);
    const int wave = HH >= 3 ? wave_id : (tid >> 6);
    if (lane == 0) red[wave] = loss_acc;
    __syncthreads();
    if (wave == 0 && lane == 0) {
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
    } else if (mode == MODE_MAPS) {
        if (bf16) FL_LAUNCH(true, MODE_MAPS); else FL_LAUNCH(false, MODE_MAPS);
    } else {
        return hipErrorInvalidValue;
    }
#undef FL_LAUNCH
    return hipGetLastError();
}

}  // namespace fl
