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
// plane, so each plane costs two workgroup barriers and every LDS buffer is written in one phase
// and read in the other:
//   P0 = {F(zi), Y(zi-1) y-sums, AX(zi-2), AZ(zi-3)}   P1 = {X(zi), Y(zi-1) ncc, AYs(zi-2)}
// Y is split over the phases: its y-sums (LDS reads of Xs) in P0, its ncc and adjoint arithmetic
// (the largest block of VALU work, registers only) in P1, where it runs while the X and AYs units
// wait for their LDS rows. F and AZ run on every lane; the Y items, the X units, the AX units and
// the AYs units sit on waves chosen per phase so that no lane holds two kinds of row at once.
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
// Both gradients (MODE_DUAL): the loss is symmetric in p and t, and with u' = c VP, w' = Sp - St u'
// the target's coefficients are alpha' = c w', beta' = c u' and gamma' = c = gamma, so that
// grad_t = (2n/M) (box(alpha')/n + t box(beta') - p box(gamma)): five adjoint fields through the
// adjoint passes instead of three, each formed by the same operations on the same values as in a
// pred-gradient pass over the swapped inputs, so both gradients equal those of two such passes bit
// for bit.
// Range: VP VT = n^2 vp vt would overflow n^2 times earlier than the reference's vp vt (at a
// local standard deviation ~20x smaller at k = 7). The kernel therefore forms VT s instead of VT,
// with s = 2^-E the power of two just below 1/n^2, so that r and c carry a factor 1/s; ncc is
// formed as (X s) (c/s), and alpha, beta, gamma carry 1/s, which the gradient's final scale (2n/M)
// s takes back. Each is one multiply by a literal per voxel (on gfx9 a select or an fma with a
// non-inline constant would need a vector register, and at k >= 5 the kernels are at the
// register limit). Scaling by a power of two is exact, so every result is bit for bit what the
// unscaled arithmetic gives wherever that does not overflow, and VP VT s overflows only where the
// reference's vp vt does (n^2 s lies in (1/2, 1]).
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

// Stores four floats to a 16-byte aligned LDS address as one 128-bit write. The vector passes
// through an empty asm operand that needs all of its lanes, for the reason given at lds_row: left
// alone, the compiler split the AYs stores into pairs of adjacent 32-bit writes (ds_write2_b32),
// and at the row stride of GY (36 floats) each such write served 64 lanes from 16 banks, 4-way
// conflicts: a quarter of the kernel's LDS bank-conflict cycles came from them.
__device__ __forceinline__ void lds_store4(float* __restrict__ dst, float x, float y, float z, float w) {
    lds_f4 f = {x, y, z, w};
    asm("" : "+v"(f));
    *reinterpret_cast<lds_f4*>(dst) = f;
}

template <int HH, bool BF16, int MODE>
__global__ __launch_bounds__(NT, WG_PER_CU) void lncc_fused_kernel(FusedArgs a) {
    constexpr bool DUAL = (MODE == MODE_DUAL);
    constexpr bool ADJ = (MODE == MODE_GRAD) || DUAL;
    constexpr int NADJ = DUAL ? 5 : 3;   // adjoint fields
    using G = Geo<HH, NADJ>;
    constexpr int K = G::K;
    constexpr int ELEM = BF16 ? 2 : 4;
    constexpr int J = G::J;
    constexpr int TY = G::TY;

    // one __shared__ array per buffer, so the compiler knows that the reads of one stage do not
    // alias the writes of another and can overlap them
    __shared__ __align__(16) float Zs[5 * G::ZP + G::PAD];
    __shared__ __align__(16) float Xs[5 * G::XP + G::PAD];
    __shared__ __align__(16) float Gs[ADJ ? NADJ * G::GP + G::PAD : 4];
    __shared__ __align__(16) float GXs[ADJ ? NADJ * G::GXP + G::PAD : 4];
    __shared__ __align__(16) float GY[ADJ ? NADJ * G::GYP : 2];
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
    char* const gtvol = DUAL ? (char*)a.grad_t + b * D * HW * ELEM : nullptr;

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
    // Y items on lanes [0, YITEMS) (y-sums in P0, ncc arithmetic in P1), X and AYs units in P1,
    // AX units in P0 (lncc_geometry.h); offsets into the source and destination buffers
    // (a lane has at most one unit of X and AYs, so the two share one pair of offsets; with five
    // adjoint fields the AYs units sit on Y lanes)
    int u_src, u_dst, a_src, a_dst, b_src, b_dst;
    const bool has_x = x_unit<G>(tid, u_src, u_dst);
    const bool has_a = ax_unit<G>(tid, a_src, a_dst) && ADJ;
    const bool has_b = ays_unit<G>(tid, b_src, b_dst) && ADJ;
    if (has_b) {
        u_src = b_src;
        u_dst = b_dst;
    }
    const bool has_y = tid < G::YITEMS;
    int y_seg = 0, y_ax = 0;  // rows seg of AX positions
    // the Y item's offsets into Xs and Gs. At k = 7 they take the registers of the X / AYs unit
    // offsets (a Y lane has no such unit), which with three of Y's rows in flight across F is
    // what keeps the kernel within 128 registers; at the other k separate registers measured
    // faster (k = 9: 1%). With both gradients the Y lanes carry AYs units, whose offsets those are.
    constexpr bool Y_SHARE = HH == 3 && !DUAL;
    int y_xs = 0, y_gs0 = 0;
    if (has_y) {
        y_item<G>(tid, y_seg, y_ax);
        if constexpr (Y_SHARE)
            y_offsets<G>(tid, u_src, u_dst);
        else
            y_offsets<G>(tid, y_xs, y_gs0);
    }
    const int y_xo = Y_SHARE ? u_src : y_xs, y_go = Y_SHARE ? u_dst : y_gs0;
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
    const bool has_z = ADJ && tid < G::NOUT;
    int z_ox, z_oy;
    az_lane<G>(tid, z_ox, z_oy);
    const bool z_in = has_z && x0 + z_ox < Wd && y0 + z_oy < Hd;
    const uint32_t z_voff = z_in ? (uint32_t)(((y0 + z_oy) * Wd + x0 + z_ox) * ELEM) : kOOB;

    constexpr int LEAD = ADJ ? 2 * HH : HH;
    const int zlo = max(z0 - LEAD, 0);
    const int zhi = ADJ ? z1 + 3 + 2 * HH : z1 + 1 + HH;
    const int zc_lo = ADJ ? max(z0 - HH, 0) : z0;
    const int zc_hi = ADJ ? min(z1 + HH, D) : z1;

    // F state: the ring of the last k planes' p,t (slot r = position of the plane in its block of
    // k), the prefix sums of the five fields over the current block, and p,t of the next plane
    // (prefetched one step ahead). The ring starts at zero: nothing before the first plane of the
    // march enters a window that is used.
    float pring[J][K], tring[J][K], fpre[J][5], fch[J][5], zsum[J][5], pnext[J], tnext[J];
    float pz = 0.f, tzz = 0.f;  // AZ: p,t at this step's output plane (prefetched one step ahead)
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            fpre[j][q] = 0.f;
            fch[j][q] = 0.f;
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
    // AZ state: the ring of the last k planes' xy-sums of the adjoint fields and their prefix sums
    // over the current block
    float gring[NADJ][K], gpre[NADJ];
#pragma unroll
    for (int c = 0; c < NADJ; ++c) {
        gpre[c] = 0.f;
#pragma unroll
        for (int r = 0; r < K; ++r) gring[c][r] = 0.f;
    }

    double loss_acc = 0.0;
    const float inv_n = a.inv_n, nf = a.nf, ndr = a.ndr;
    constexpr float VS = range_scale(K);   // the range scale s = 2^-E (header)

    // Plane addresses advance by one plane per step: zoff = zi * plane size, and every plane the
    // loop touches sits at a fixed plane distance from zi. A plane outside its valid range gets a
    // zero-sized resource (its address is never dereferenced).
    const uint64_t PB = (uint64_t)HW * ELEM;
    const uint64_t pva = (uint64_t)(uintptr_t)pvol, tva = (uint64_t)(uintptr_t)tvol;
    const uint64_t gva = (uint64_t)(uintptr_t)gvol, gtva = (uint64_t)(uintptr_t)gtvol;
    uint64_t zoff = (uint64_t)zlo * PB;
    const int zn_hi = min(zhi, D);                 // F: new plane zi+1 valid while zi+1 < zn_hi
    constexpr int ZO = 3 + 2 * HH;                 // AZ: output plane zi-ZO
    // z-window chains (zstep5 / zstep1): the previous block's sums over ring slots F_CHAIN..K-1
    // (F) and A_CHAIN..K-1 (AZ) kept as partial sums; 0 = none. F's chain (slots 4..6 at k = 7)
    // saves adds but holds five more registers per column; at k = 7 those registers measured
    // better spent on Y's rows in flight across F (three rows and no chain: 2.7% faster than one
    // row and the chain), and at k = 9 they are not there.
    constexpr int F_CHAIN = 0;
    constexpr int A_CHAIN = HH >= 2 && (HH <= 3 || !BF16) ? HH + 1 : 0;

    // Stage bodies; the march below orders them per phase.
    //
    // Y(zi-1): box sums S (y-sums of the rows of the five x-sums), then ncc and the adjoint
    // coefficients at plane zcY (y_math).
    auto y_math = [&](const float (&S)[5][G::SY], int zcY) __attribute__((always_inline)) {
        const bool count = zcY >= z0 && zcY < z1;
        float lsum = -0.f;  // -0 + x == x for every x, so the first add folds away
        float adj[NADJ][G::SY];  // alpha, beta, gamma (and alpha', beta') of the segment's outputs
#pragma unroll
        for (int i = 0; i < G::SY; ++i) {
            const int ay = y_start + i;
            const float Sp = S[0][i], St = S[1][i], Spp = S[2][i], Stt = S[3][i], Spt = S[4][i];
            const float X = fmaf(-Sp, St, nf * Spt);
            // n dr is added after the cancellation: folded into the fma that rounds n Spp, it
            // would break that rounding's ties (frequent when n Spp has few significant bits)
            // always upwards, a bias of ~2e-5 in ncc on offset intensities at k = 3
            const float VP = fmaxf(fmaf(-Sp, Sp, nf * Spp), 0.f) + ndr;
            const float VT = (fmaxf(fmaf(-St, St, nf * Stt), 0.f) + ndr) * VS;   // VT s
            const float rr = __builtin_amdgcn_rcpf(VP * VT);
            const float cr = X * rr;             // c / s
            const float ncc = (X * VS) * cr;     // ncc
            const bool live = y_inv[i] && (ncc < 1.0f);
            const float nccc = (ncc >= 1.0f) ? 1.0f : ncc;
            if (count && y_core[i]) lsum += nccc;
            if constexpr (ADJ) {
                // masking cr masks all three coefficients (alpha, beta, gamma are multiples of it)
                const float crm = live ? cr : 0.f;
                const float uu = crm * VT;
                const float w = fmaf(-Sp, uu, St);
                adj[0][i] = crm * w;
                adj[1][i] = crm * uu;
                adj[2][i] = crm;
                if constexpr (DUAL) {
                    // the target's: u' = (c/s)(VP s), w' = Sp - St u' (the swapped pass's uu, w)
                    const float uu2 = crm * (VP * VS);
                    adj[3][i] = crm * fmaf(-St, uu2, Sp);
                    adj[4][i] = crm * uu2;
                }
                if constexpr (!G::ASWAP) {
#pragma unroll
                    for (int c = 0; c < NADJ; ++c) Gs[y_go + c * G::GP + i * G::GST] = adj[c][i];
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
                        a.a_map[o] = live ? (-2.f * VS) * (cr * w) : 0.f;
                        a.b_map[o] = live ? (-nf * VS) * (cr * uu) : 0.f;
                        a.c_map[o] = live ? (2.f * nf * VS) * cr : 0.f;
                    }
                }
            }
        }
        if constexpr (ADJ && G::ASWAP) {  // Gs rows along y: one float4 per field
            static_assert(G::SY == 4, "float4 rows");
#pragma unroll
            for (int c = 0; c < NADJ; ++c)
                lds_store4(Gs + y_go + c * G::GP, adj[c][0], adj[c][1], adj[c][2], adj[c][3]);
        }
        loss_acc += (double)lsum;
    };
    // F(zi): z-sums of the input region over planes [zi-k+1, zi] (zstep5: the plane prefetched one
    // step ago joins the block prefix and the ring, the previous block's suffix comes from the
    // ring), then the prefetch of the next plane. Every global access of the loop is issued unconditionally
    // (inactive ones through a zero-sized buffer), so the number of outstanding memory operations
    // is the same on every path and the waits before use stay exact. With STORE the z-sums go to
    // the LDS column by column as they are formed; without, f_store writes them later.
    // F's columns [JB, JE) of this lane (f_sums runs them all, then the prefetch)
    auto f_cols = [&](auto rc, auto store, auto jb, auto je) __attribute__((always_inline)) {
        constexpr int r = decltype(rc)::value;
        constexpr bool STORE = decltype(store)::value;
#pragma unroll
        for (int j = decltype(jb)::value; j < decltype(je)::value; ++j) {
            zstep5<K, r, F_CHAIN>(pnext[j], tnext[j], fpre[j], pring[j], tring[j], fch[j], zsum[j]);
            if constexpr (STORE) {
                if (G::FPAIR || zaddr[j] >= 0) {
#pragma unroll
                    for (int q = 0; q < 5; ++q) Zs[q * G::ZP + zaddr[j]] = zsum[j][q];
                }
            }
        }
    };
    auto f_pref = [&](int zi, uint64_t zoff) __attribute__((always_inline)) {
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
    auto f_sums = [&](auto rc, auto store, int zi, uint64_t zoff) __attribute__((always_inline)) {
        f_cols(rc, store, std::integral_constant<int, 0>{}, std::integral_constant<int, J>{});
        f_pref(zi, zoff);
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
    // Stage order inside a phase. Each wave runs its stages in program order, so a stage placed
    // between the issue of another stage's LDS reads and their use hides part of their latency.
    //  * P0: AZ's xy-sums are read first. The Y lanes read Y_EARLY of their five rows (all five
    //    at k <= 5, three at k = 7, two for bf16 at k = 7: more rows held across F exceed the
    //    128-register budget of a 1024-lane workgroup) and at k <= 5 the AX lanes their row; F
    //    runs while they arrive, then the Y lanes read their other rows and form the five box
    //    sums, which stay in registers until P1, and the AX lanes their sums; AZ's z-sums and the
    //    gradient come last. At k = 9 (two rings of 9 planes) nothing is read before F, one row
    //    between F's two columns, and the others one at a time after F. (At k = 7 the AX row read
    //    before F measured 1% slower than after it.)
    //  * P1: the Y lanes turn their box sums into ncc and the adjoint coefficients (arithmetic
    //    only, no LDS reads: it keeps the SIMDs busy while the rows of the X and AYs units, on the
    //    other waves, arrive), then the X and AYs units (with both gradients, at k >= 5, also on
    //    the first Y lanes: units that do not fit after the X units, 2-7% faster than all AYs
    //    units on Y lanes).
    //  * Both gradients (five adjoint fields, fourteen more ring registers per lane at k = 7):
    //    fewer early rows, all five at k = 3, two (bf16) or none (fp32) at k = 5, one at k = 7
    //    (more early rows spill; the counts are the fastest measured: k = 5 fp32 with none 1.2% faster than with
    //    two, bf16 with two 0.4% faster than with none), and no AX row before F. At k = 9 the two
    //    9-plane rings and the five adjoint rings exceed the 128 registers even so: 36-46 spill to
    //    scratch, and the launch still runs 22-26% faster than two pred-gradient passes.
    constexpr int Y_EARLY = DUAL ? (HH <= 1 ? 5 : HH == 2 ? (BF16 ? 2 : 0) : HH == 3 ? 1 : 0)
                                 : HH <= 2 ? 5 : HH == 3 ? (BF16 ? 2 : 3) : 0;   // Y rows read before F
    constexpr bool F_STORE_AT_ONCE = Y_EARLY < 5;
    // Y_MID of Y's rows are read between F's two columns, after the box sums of the early rows
    // (whose registers they take); the rest after F. k = 9: one row (0.6-1% faster than none).
    // k = 7: one row measured 0.7% faster at (2,16,128^3) but 1.3% slower at (2,16,256^3), whose
    // re-reads of the output planes then missed the L2 more often (HBM reads 1.05x -> up to 1.46x
    // the inputs, growing from launch to launch); none.
    constexpr int Y_MID = HH == 4 && J == 2 && !DUAL ? 1 : 0;
    static_assert(Y_EARLY + Y_MID <= 5, "Y rows");
    constexpr bool AX_EARLY = HH <= 2 && !DUAL;               // the AX row read before F
    constexpr int NY = G::SY + 2 * HH, NA = G::SA + 2 * HH, NX = G::SX + 2 * HH, NB = G::SB + 2 * HH;
    // P0's early reads (Y's first rows or the AX row) share one register array: the two kinds of
    // lane sit on different waves
    constexpr int NE0 = cmax(cmax(Y_EARLY * NY, AX_EARLY ? NA : 0), NY);

    for (int base = zlo; base < zhi; base += K) {
        static_for<0, K>([&](auto rc) __attribute__((always_inline)) {
            const int zi = base + decltype(rc)::value;
            if (zi >= zhi) return;
            const int zcX = zi - HH;       // X(zi): the z-sums of F(zi) are centred on plane zi-h
            const bool actX = zcX >= zc_lo && zcX < zc_hi;
            const int zcY = zi - 1 - HH;   // Y(zi-1)
            const bool actY = zcY >= zc_lo && zcY < zc_hi;
            const int zcB = zi - 2 - HH;   // AX(zi-2) and AYs(zi-2)
            const bool actB = ADJ && zcB >= zc_lo && zcB < zc_hi;
            const int zcA = zi - 3 - HH;   // the xy-sums AZ(zi-3) reads
            const bool actA = ADJ && zcA >= zc_lo && zcA < zc_hi;

            // ============================ phase P0 ============================
            // AZ(zi-3) reads, Y(zi-1) y-sums, AX(zi-2), F(zi), AZ(zi-3)
            // AZ's xy-sums: read first, except at k = 9, where they would be held across F
            float ys[NADJ];
            auto az_read = [&]() __attribute__((always_inline)) {
#pragma unroll
                for (int c = 0; c < NADJ; ++c) {
                    // read whatever actA says (the value is dropped when it is false), so that the
                    // three reads pair up
                    const float gy = GY[c * G::GYP + z_oy * G::GYS + z_ox];
                    ys[c] = actA ? gy : 0.f;
                }
            };
            if constexpr (ADJ && HH <= 3) az_read();
            float er[NE0];
            if (has_y && actY) {
#pragma unroll
                for (int q = 0; q < Y_EARLY; ++q) {
                    float v[NY];
                    lds_row(Xs + q * G::XP + y_xo, v);
#pragma unroll
                    for (int i = 0; i < NY; ++i) er[q * NY + i] = v[i];
                }
            } else if (AX_EARLY && has_a && actB) {
                float v[NA];
                lds_row(Gs + a_src, v);
#pragma unroll
                for (int i = 0; i < NA; ++i) er[i] = v[i];
            }
            float S[5][G::SY];  // Y's box sums, carried into P1
            float em[Y_MID > 0 ? Y_MID * NY : 1];
            if constexpr (Y_MID > 0) {
                // F's first column; then the box sums of the early rows and the reads of the mid
                // rows; then F's second column and the prefetch
                f_cols(rc, std::true_type{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
                if (has_y && actY) {
#pragma unroll
                    for (int q = 0; q < Y_EARLY; ++q) {
                        float v[NY];
#pragma unroll
                        for (int i = 0; i < NY; ++i) v[i] = er[q * NY + i];
                        box_sums<HH, G::SY>(v, S[q]);
                    }
#pragma unroll
                    for (int q = 0; q < Y_MID; ++q) {
                        float v[NY];
                        lds_row(Xs + (Y_EARLY + q) * G::XP + y_xo, v);
#pragma unroll
                        for (int i = 0; i < NY; ++i) em[q * NY + i] = v[i];
                    }
                }
                f_cols(rc, std::true_type{}, std::integral_constant<int, 1>{}, std::integral_constant<int, J>{});
                f_pref(zi, zoff);
            } else {
                f_sums(rc, std::integral_constant<bool, F_STORE_AT_ONCE>{}, zi, zoff);
            }
            if (has_y && actY) {
                // the rows not yet summed: early rows (held in er), mid rows (em), the rest read now
#pragma unroll
                for (int q = Y_MID > 0 ? Y_EARLY : 0; q < 5; ++q) {
                    float v[NY];
                    if (q < Y_EARLY) {
#pragma unroll
                        for (int i = 0; i < NY; ++i) v[i] = er[(q < Y_EARLY ? q : 0) * NY + i];
                    } else if (q < Y_EARLY + Y_MID) {
#pragma unroll
                        for (int i = 0; i < NY; ++i) v[i] = em[(q < Y_EARLY + Y_MID ? q - Y_EARLY : 0) * NY + i];
                    } else {
                        lds_row(Xs + q * G::XP + y_xo, v);
                    }
                    box_sums<HH, G::SY>(v, S[q]);
                }
            } else if (has_a && actB) {
                // AX(zi-2): x-sums (y-sums with ASWAP) of one of alpha, beta, gamma over one segment
                float v[NA], o[G::SA];
                if constexpr (AX_EARLY) {
#pragma unroll
                    for (int i = 0; i < NA; ++i) v[i] = er[i];
                } else {
                    lds_row(Gs + a_src, v);
                }
                box_sums<HH, G::SA>(v, o);
#pragma unroll
                for (int i = 0; i < G::SA; ++i) GXs[a_dst + i * G::GXS] = o[i];
            }
            if constexpr (!F_STORE_AT_ONCE) f_store();
            if constexpr (ADJ && HH > 3) az_read();
            if constexpr (ADJ) {
                // AZ(zi-3): z-sums of the xy-sums over the k planes of the output plane zo = the
                // prefix of the current block plus the previous block's suffix (ring and chain)
                // (lanes without an output column run on a clamped one and store out of range,
                // i.e. nothing)
                constexpr int r = decltype(rc)::value;
                float gw[NADJ];
#pragma unroll
                for (int c = 0; c < NADJ; ++c) gw[c] = zstep1<K, r, A_CHAIN>(ys[c], gpre[c], gring[c]);
                const int zo = zi - ZO;
                const float g = a.gscale * fmaf(inv_n, gw[0], fmaf(pz, gw[1], -tzz * gw[2]));   // gscale holds s
                // Non-temporal: the gradient is never read back, and this re-read of p,t is the
                // last use of those lines. With the default policy both would be promoted in the
                // L2 and push out the planes that F loaded and this stage re-reads 2h+3 steps
                // later, so that every input byte would be fetched about twice; marked
                // evict-first, every input byte is fetched from HBM once. bf16 gradient rows of a
                // tile are half a 128-byte line (the x-neighbour tile writes the other half):
                // those stores keep the default policy, so that the L2 merges the two halves into
                // one write.
                store_elem_buf<BF16, BF16 ? 0 : kNT>(rsrc_at(gva + zoff - ZO * PB, plane_bytes, zo >= z0 && zo < z1), z_voff, g);
                if constexpr (DUAL) {
                    const float gt = a.gscale * fmaf(inv_n, gw[3], fmaf(tzz, gw[4], -pz * gw[2]));
                    store_elem_buf<BF16, BF16 ? 0 : kNT>(rsrc_at(gtva + zoff - ZO * PB, plane_bytes, zo >= z0 && zo < z1), z_voff, gt);
                }
                // prefetch p,t at the next step's output plane; issued after this step's use, so
                // one register each suffices and no copy has to wait for the load
                const bool oko = zo + 1 >= z0 && zo + 1 < z1;
                pz = load_elem<BF16, kNT>(rsrc_at(pva + zoff - (ZO - 1) * PB, plane_bytes, oko), z_voff);
                tzz = load_elem<BF16, kNT>(rsrc_at(tva + zoff - (ZO - 1) * PB, plane_bytes, oko), z_voff);
            }
            __syncthreads();

            // ============================ phase P1 ============================
            // Y(zi-1) ncc arithmetic, X(zi), AYs(zi-2)
            if (has_y && actY) y_math(S, zcY);
            if (has_x && actX) {
                // X(zi): x-sums of one of the five z-sums over one segment (feeds Y at the next plane)
                float v[NX], o[G::SX];
                lds_row(Zs + u_src, v);
                box_sums<HH, G::SX>(v, o);
#pragma unroll
                for (int i = 0; i < G::SX; ++i) Xs[u_dst + i * G::XS] = o[i];
            } else if (has_b && actB) {
                // AYs(zi-2): y-sums (x-sums with ASWAP) of one of alpha, beta, gamma at plane zcB
                float v[NB], o[G::SB];
                lds_row(GXs + u_src, v);
                box_sums<HH, G::SB>(v, o);
#pragma unroll
                for (int i = 0; i < G::SB; ++i) {
                    if constexpr (G::ASWAP) {  // GY rows along x: float4s
                        if (i % 4 == 0)
                            lds_store4(GY + u_dst + i, o[i], o[i + 1], o[i + 2], o[i + 3]);
                    } else {
                        GY[u_dst + i * G::BW] = o[i];
                    }
                }
            }
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
    } else if (mode == MODE_DUAL) {
        if (bf16) FL_LAUNCH(true, MODE_DUAL); else FL_LAUNCH(false, MODE_DUAL);
    } else {
        return hipErrorInvalidValue;
    }
#undef FL_LAUNCH
    return hipGetLastError();
}

}  // namespace fl
