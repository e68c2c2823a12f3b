// Tile geometry and per-lane work maps of the fused LNCC kernel. Plain C++ (no HIP builtins):
// the kernel takes every LDS offset it uses from these functions, and the host-side model of the
// kernel's LDS accesses (tests/lds_model.cpp) enumerates the same functions for every lane.
#pragma once

#if defined(__HIPCC__)
#define FL_HD __host__ __device__
#else
#define FL_HD
#endif

namespace fl {

// Workgroup: 1024 lanes (16 wave64s, one workgroup per CU). Output tile: TX x tile_rows(H)
// columns of one volume, marched along D. The tile is 32 x 32 for k <= 7 and 32 x 24 for k = 9,
// whose input region (48 x 40 columns) then still takes two columns per lane, so that the
// register ring of the last k planes fits (32 x 32 at k = 9 would need three).
constexpr int NT = 1024;
constexpr int WG_PER_CU = 1;
constexpr int TX = 32;
constexpr int TY_MAX = 32;
FL_HD constexpr int tile_rows(int halo) { return halo >= 4 ? 24 : 32; }

constexpr int cmax(int a, int b) { return a > b ? a : b; }

// The power of two 2^-E with 2^E the smallest power of two >= n^2, n = k^3: the factor by which the
// fused kernel scales VT so that VP VT stays within the float range wherever the reference's
// vp vt does (VP VT = n^2 vp vt; n^2 2^-E lies in (1/2, 1]).
FL_HD constexpr float range_scale(int k) {
    const long long n2 = (long long)k * k * k * k * k * k;
    float s = 1.0f;
    for (long long p = 1; p < n2; p *= 2) s *= 0.5f;
    return s;
}
constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
constexpr int odd(int a) { return a | 1; }

// Row stride (floats) for LDS rows read as float4 by lanes that step from row to row: = 4 mod 8,
// so that the 8 lanes served per cycle by a 128-bit read land on distinct groups of 4 banks.
constexpr int stride4(int n) { return n + ((12 - n % 8) % 8); }
constexpr int rup4(int n) { return (n + 3) / 4 * 4; }
constexpr int rup64(int n) { return (n + 63) / 64 * 64; }
// Floats fetched by the LDS read of a row of n values: float4 pieces, and a tail of 2 or 1 values
// as a float2 or a float (a tail of 3 as one more float4).
FL_HD constexpr int row_read(int n) { return n % 4 == 3 ? rup4(n) : n; }

// Tile geometry for halo H (k = 2H+1). Coordinates inside a workgroup:
//   input region   ix in [0,IX), iy in [0,IY)  <-> global (x0-2H+ix, y0-2H+iy)
//   adjoint region ax in [0,AX), ay in [0,AY)  <-> global (x0-H+ax,  y0-H+ay)
//   output tile    ox in [0,TX), oy in [0,TY)  <-> global (x0+ox,    y0+oy)
// The box-sum passes work on segments of S consecutive outputs. The X and Y passes round their
// output range up to whole segments: the extra outputs read row padding and land in padding rows
// of the destination that no later pass reads (and that the loss never counts), so no lane needs
// a per-output store mask. NA adjoint fields go from Y to AZ: three (alpha, beta, gamma) for the
// pred gradient, five for both gradients (the target's alpha' and beta' besides; its gamma' is
// gamma).
template <int H, int NA = 3>
struct Geo {
    static_assert(NA == 3 || NA == 5, "adjoint fields");
    static constexpr int HALO = H, NADJ = NA;
    static constexpr int K = 2 * H + 1;
    static constexpr int TY = tile_rows(H);
    static constexpr int IX = TX + 4 * H, IY = TY + 4 * H;
    static constexpr int AX = TX + 2 * H, AY = TY + 2 * H;
    static constexpr int NIN = IX * IY;
    static constexpr int J = cdiv(NIN, NT);               // input columns per lane
    static constexpr int NOUT = TX * TY;                  // output columns (one lane each)
    // X: x-sums of the five z-sums; items (iy, seg) over rows iy < IY, outputs ax < XR (>= AX)
    static constexpr int SX = rup4(cdiv(AX, 2)), XSEG = 2, XR = XSEG * SX, XITEMS = IY * XSEG;
    // Y: y-sums -> box sums, ncc, adjoints; items (ax, seg), outputs ay < YR (>= AY)
    static constexpr int SY = 4, YSEG = cdiv(AY, SY), YR = YSEG * SY, YITEMS = AX * YSEG;
    // Adjoint passes: AX (phase P0) box-sums alpha, beta, gamma along x, AYs (phase P1) along y.
    // At k = 7 (ASWAP) the order is swapped, y first and x second: the rows of Gs then run along
    // y, so Y stores the four outputs of a field as one float4, and the rows of GY along x, so AYs
    // stores its 16 outputs as four float4s (34 LDS store instructions fewer per plane than the
    // scattered 32-bit stores; measured 1.2% faster at k = 7, 0.4-0.7% slower at k = 3, 5, 5%
    // slower at k = 9).
    static constexpr bool ASWAP = (H == 3);
    // AX: items (pos, seg), pos over the AY rows (x-sums, outputs ox < TX) or, with ASWAP, over
    // the AX columns (y-sums, outputs oy < TY)
    static constexpr int SA = ASWAP ? TY / 2 : 16, ASEG = (ASWAP ? TY : TX) / SA, APOS = ASWAP ? AX : AY,
                         AITEMS = APOS * ASEG;
    // AYs: items (pos, seg), pos over the TX columns (y-sums, outputs oy < TY) or, with ASWAP,
    // over the TY rows (x-sums, outputs ox < TX); BW = the stride of its outputs in GY
    static constexpr int SB = (ASWAP ? TX : TY) / 2, BSEG = 2, BPOS = ASWAP ? TY : TX, BITEMS = BPOS * BSEG;
    // Work units of the box-sum passes are single quantities of one segment. Lanes by phase:
    //   P0  Y's y-sums on lanes [0, YITEMS); AX units on the NAW waves ax_wave(0..NAW-1), 64 each
    //   P1  Y's ncc arithmetic on the same lanes; X units on [XL0, XL0 + UX); AYs units on
    //       [BL0, BL0 + UB)
    // (F and AZ run on every lane in P0.) Waves sit on the CU's 4 SIMDs round-robin (wave w on
    // SIMD w % 4): with three adjoint fields the AX waves go to the SIMDs with fewer Y waves, which
    // evens out P0. With five the AX units run on the waves after Y's, and the AYs units that do
    // not fit on the lanes after the X units (BOWN of them do) run on the first Y lanes, after Y's
    // ncc arithmetic (which reads no LDS row).
    static constexpr int UX = 5 * XITEMS, UA = NA * AITEMS, UB = NA * BITEMS;
    static constexpr int NYW = cdiv(YITEMS, 64), XL0 = 64 * NYW, BL0 = rup64(XL0 + UX), NAW = cdiv(UA, 64);
    static constexpr int BOWN = UB < NT - BL0 ? UB : NT - BL0;
    static constexpr bool B_ON_Y = UB > BOWN;
    // Y items and X units on disjoint lanes, AYs units on lanes of their own or on Y lanes (the
    // kernel keeps a Y item's offsets in the registers of the X / AYs unit offsets at k = 7 with
    // three adjoint fields)
    static_assert(XL0 >= YITEMS && BL0 >= XL0 + UX && UB - BOWN <= YITEMS && (NA > 3 || !B_ON_Y), "lane kinds");
    static_assert(BL0 <= NT && (NA > 3 ? NYW + NAW <= NT / 64 : NAW <= 4) && (NYW == 5 || NYW == 6) &&
                      BPOS == 32 && TX == 32 && NIN <= 2 * NT && TY <= TY_MAX,
                  "lanes");
    // every segment starts on a 16-byte boundary (rows are read as float4)
    static_assert(XR >= AX && ASEG * SA == (ASWAP ? TY : TX) && BSEG * SB == (ASWAP ? TX : TY) && SX % 4 == 0 && SY % 4 == 0 &&
                      SA % 4 == 0 && SB % 4 == 0, "segments");
    // LDS layout (floats): Zs[5][IY][ZS], XsT[5][XR][XS] (transposed), Gs[3][YR][GS],
    // GXsT[3][TX][GXS] (transposed), GY[3][TY][GYS]; each buffer but GY ends in PAD spare floats
    static constexpr int ZS = stride4(IX), XS = stride4(cmax(IY, AY));
    // Gs rows along x (along y with ASWAP), GXs rows along y (x), GY rows along x
    static constexpr int GS = ASWAP ? stride4(YR) : stride4(AX), GXS = ASWAP ? stride4(AX) : XS;
    static constexpr int GYS = ASWAP ? stride4(TX) : TX + 1, BW = ASWAP ? 1 : GYS, PAD = 16;
    static constexpr int GST = ASWAP ? 1 : GS;  // stride of a Y item's consecutive outputs in Gs
    // The planes F writes (one column, five fields) and AZ reads (one column, three fields) are a
    // multiple of 64 floats apart for k >= 5, so that those accesses pair into write2st64 /
    // read2st64 (6 LDS instructions per lane and step instead of 10 for F, 5 with FPAIR; 2 instead
    // of 3 for AZ; 2-4% faster at k = 5..9, k = 3 measured 0.6% slower with it)
    // k = 7: a lane's two F columns are NT floats apart in every Zs plane (ZS == IX), planes of
    // 2 NT floats: a lane without a second column writes its (zero) z-sums into the padding, so
    // that every lane's ten z-sum stores pair into five write2st64
    static constexpr bool FPAIR = (H == 3 && ZS == IX && J == 2);
    static constexpr int ZP = FPAIR ? 2 * NT : H >= 2 ? rup64(IY * ZS) : IY * ZS, XP = XR * XS, GP = (ASWAP ? AX : YR) * GS, GXP = (ASWAP ? TY : TX) * GXS,
                         GYP = H >= 2 ? rup64(TY * GYS) : TY * GYS;
    // A segment reads row_read(S + 2H) floats from its start; reads past a row's end stay inside
    // the buffer (the next row or the spare floats) and only feed outputs that are never used.
    static_assert(SX + row_read(SX + 2 * H) <= ZS + PAD && YR - SY + row_read(SY + 2 * H) <= XS + PAD &&
                      (ASEG - 1) * SA + row_read(SA + 2 * H) <= GS + PAD && (BSEG - 1) * SB + row_read(SB + 2 * H) <= GXS + PAD,
                  "row reads");
    static constexpr int LDS_FLOATS = 5 * (ZP + XP) + NA * (GP + GXP + GYP) + 4 * PAD;
    static_assert(LDS_FLOATS * 4 <= 160 * 1024, "LDS");
};

// ---- the small-volume kernel (lncc_small.hip): one workgroup of kSmallLanes lanes per volume
// whose D, H, W are all at most kSmallEdge, the volume zero-padded to kSmallEdge^3 in LDS. Lanes
// form four quarters q (whole waves) of 16 x 16; a quarter owns positions 4q..4q+3 of a line and
// reads positions 4q-h+i, i < 4+2h, of it (zero outside [0, 16)).
constexpr int kSmallEdge = 16;
constexpr int kSmallLanes = 1024;
// LDS offset of (z, y, x) in one 16^3 field: each z plane's 16-float rows rotated by z, so that the
// 64 lanes of a wave, four consecutive y (or z) of one 16-wide x row each, hit 64 distinct banks.
FL_HD constexpr int small_lds(int z, int y, int x) { return (z << 8) | (((y + z) & 15) << 4) | x; }
// The code class of lane quarter q: 0 (q = 0: reads below position 0 are zeros), 3 (q = 3: reads
// past position 15 are zeros), 1 (q = 1, 2: every read is inside the line, for h <= 4).
FL_HD constexpr int small_class(int q) { return q == 0 ? 0 : q == 3 ? 3 : 1; }
// Whether read i (position 4q-h+i) of a quarter of class qc is a compile-time zero.
FL_HD constexpr bool small_skip(int qc, int h, int i) { return (qc == 0 && i < h) || (qc == 3 && i >= 4 + h); }

// Lane order for work over n_rows rows of LEN (>= 32) positions: indices [0, 32 n_rows) take
// positions 0..31 of one row per 32 consecutive lanes, so that each half-wave stores into a
// single destination row (consecutive LDS banks, no conflicts); the remaining indices take
// positions 32..LEN-1 row after row.
template <int LEN>
FL_HD inline void split32(int idx, int n_rows, int& row, int& pos) {
    static_assert(LEN >= 32, "rows of at least 32 positions");
    if constexpr (LEN == 32) {
        row = idx >> 5;
        pos = idx & 31;
    } else {
        if (idx < 32 * n_rows) {
            row = idx >> 5;
            pos = idx & 31;
        } else {
            const int e = idx - 32 * n_rows;
            row = e / (LEN - 32);
            pos = 32 + e % (LEN - 32);
        }
    }
}

// F: input column c (lane + j * NT) of the input region, if c < NIN: its position (ix, iy) and
// the offset of its z-sum in each of the five Zs planes.
template <class G>
FL_HD inline bool f_column(int c, int& ix, int& iy, int& zaddr) {
    if (c >= G::NIN) return false;
    iy = c / G::IX;
    ix = c - iy * G::IX;
    zaddr = iy * G::ZS + ix;
    return true;
}

// X unit of lane tid (phase P1): x-sums of one z-sum over one segment of row iy; reads Zs from
// src, writes Xs at dst + i * XS. Returns false for lanes without a unit.
template <class G>
FL_HD inline bool x_unit(int tid, int& src, int& dst) {
    src = 0;
    dst = 0;
    const int u = tid - G::XL0;
    if (u < 0 || u >= G::UX) return false;
    int row, iy;  // rows (q, seg) of IY positions
    split32<G::IY>(u, 5 * G::XSEG, row, iy);
    const int q = row / G::XSEG, start = (row % G::XSEG) * G::SX;
    src = q * G::ZP + iy * G::ZS + start;
    dst = q * G::XP + start * G::XS + iy;
    return true;
}

// The waves of the AX units. Three adjoint fields: those of the SIMDs with fewer Y waves first
// (6 Y waves: SIMDs 0 and 1 carry two each; 5: SIMD 0 does). Five: the waves after Y's.
template <class G>
FL_HD constexpr int ax_wave(int slot) {
    return G::NADJ > 3 ? G::NYW + slot
                       : G::NYW == 6 ? (slot == 0 ? 6 : slot == 1 ? 7 : slot == 2 ? 10 : 11)
                                     : (slot == 0 ? 5 : slot == 1 ? 6 : slot == 2 ? 7 : 9);
}

// AX unit of lane tid (phase P0): sums of one adjoint field over one segment of position pos
// (x-sums of adjoint row pos, or y-sums of adjoint column pos with ASWAP); reads Gs from src,
// writes GXs at dst + i * GXS. Returns false for lanes without a unit.
template <class G>
FL_HD inline bool ax_unit(int tid, int& src, int& dst) {
    src = 0;
    dst = 0;
    const int wave = tid >> 6;
    int slot = -1;
    for (int s = 0; s < G::NAW; ++s)
        if (ax_wave<G>(s) == wave) slot = s;
    const int u = slot * 64 + (tid & 63);
    if (slot < 0 || u >= G::UA) return false;
    int row, pos;  // rows (c, seg) of APOS positions
    split32<G::APOS>(u, G::NADJ * G::ASEG, row, pos);
    const int c = row / G::ASEG, start = (row % G::ASEG) * G::SA;
    src = c * G::GP + pos * G::GS + start;
    dst = c * G::GXP + start * G::GXS + pos;
    return true;
}

// Y item of lane tid < YITEMS: adjoint column ax and segment seg (rows y_start = seg * SY ...).
// It reads Xs at q * XP + ax * XS + y_start and writes adjoint c of row ay to Gs at y_gs(c, ax, ay).
template <class G>
FL_HD inline void y_item(int tid, int& seg, int& ax) {
    split32<G::AX>(tid, G::YSEG, seg, ax);
}
template <class G>
FL_HD inline int y_gs(int c, int ax, int ay) {
    return c * G::GP + (G::ASWAP ? ax * G::GS + ay : ay * G::GS + ax);
}
// The same as two offsets per lane: the item's rows start at xs in every Xs plane (q * XP + xs),
// and output i of adjoint field c goes to Gs at gs + c * GP + i * GST (= y_gs(c, ax, seg*SY + i)).
template <class G>
FL_HD inline void y_offsets(int tid, int& xs, int& gs) {
    int seg, ax;
    y_item<G>(tid, seg, ax);
    xs = ax * G::XS + seg * G::SY;
    gs = y_gs<G>(0, ax, seg * G::SY);
}

// AYs unit of lane tid (phase P1): sums of one adjoint field over one segment of position pos
// (y-sums of output column pos, or x-sums of output row pos with ASWAP); reads GXs from src,
// writes GY at dst + i * BW. Returns false for lanes without a unit.
template <class G>
FL_HD inline bool ays_unit(int tid, int& src, int& dst) {
    src = 0;
    dst = 0;
    // units [0, BOWN) on lanes BL0.., the rest on lanes 0..
    const int u = tid >= G::BL0 ? tid - G::BL0 : G::BOWN + tid;
    if (u >= G::UB) return false;
    const int row = u >> 5, pos = u & 31;  // rows (c, seg) of BPOS = 32 positions
    const int c = row / G::BSEG, start = (row % G::BSEG) * G::SB;
    src = c * G::GXP + pos * G::GXS + start;
    dst = c * G::GYP + (G::ASWAP ? pos * G::GYS + start : start * G::GYS + pos);
    return true;
}

// AZ: output column (ox, oy) of lane tid (lanes beyond the tile run on a clamped row); it reads
// GY at c * GYP + oy * GYS + ox.
template <class G>
FL_HD inline void az_lane(int tid, int& ox, int& oy) {
    ox = tid % TX;
    oy = tid / TX < G::TY - 1 ? tid / TX : G::TY - 1;
}

}  // namespace fl
