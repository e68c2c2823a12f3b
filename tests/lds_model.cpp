// Host-side model of the LDS accesses of the fused LNCC kernel (lncc_fused_kernel.h): for every
// halo h = 1..4 (tile 32 x 32, and 32 x 24 at h = 4), with three adjoint fields (pred gradient)
// and with five (both gradients), it enumerates the LDS reads and writes of every lane in every
// stage from the same lane maps the kernel uses (lncc_geometry.h) and checks
//   bounds    every access lies inside its __shared__ array (spare floats included);
//   races     within a phase no address is written twice, and no array written in a phase is read
//             in it (the two phases are separated by the workgroup barriers);
//   coverage  every read that feeds a used output (one inside the adjoint region or the output
//             tile) reads an address the producing stage writes, and each used output's window is
//             inside what its lane reads.
// ROCm has no LDS race checker and GPU address sanitizers do not cover LDS, so this stands in
// for the compute-sanitizer workloads of the reference (tests/_sanitize*.py).
//
// Usage: lds_model [plant]. plant = 0 checks the kernel's maps; 1..4 plant one mistake in the
// model's view of them (F writes one column too far, Y rows one float short, AYs stores with a
// row stride one too small, X rows read past their buffer), which must be reported. Prints one
// line per configuration and exits 0 when every check passes.
#include <cstdio>
#include <cstdlib>
#include <set>
#include <string>
#include <vector>

#include "lncc_geometry.h"

namespace {

enum Arr { ZS, XS, GS, GXS, GY, NARR };
const char* kName[NARR] = {"Zs", "Xs", "Gs", "GXs", "GY"};

struct Model {
    int plant = 0;
    long failures = 0;
    std::string cfg;
    std::vector<long> size;
    // per phase: addresses written per array (with multiplicity), arrays read
    std::vector<std::vector<int>> writes[2];
    std::set<int> read_arrays[2];
    std::set<int> written_arrays[2];

    void fail(const std::string& what) {
        if (failures < 8) std::printf("  FAIL %s: %s\n", cfg.c_str(), what.c_str());
        ++failures;
    }
    void write(int phase, int arr, long addr) {
        if (addr < 0 || addr >= size[arr]) {
            fail(std::string("write out of ") + kName[arr] + " at " + std::to_string(addr));
            return;
        }
        writes[phase][arr][addr] += 1;
        written_arrays[phase].insert(arr);
    }
    void read(int phase, int arr, long addr, int len) {
        if (addr < 0 || addr + len > size[arr])
            fail(std::string("read out of ") + kName[arr] + " at [" + std::to_string(addr) + ", " +
                 std::to_string(addr + len) + ")");
        read_arrays[phase].insert(arr);
    }
    // a used read: the addresses [addr, addr+len) must all have been written by the producer
    // (which runs in the other phase)
    void used(int phase, int arr, long addr, int len) {
        for (long a = addr; a < addr + len; ++a)
            if (a < 0 || a >= size[arr] || writes[1 - phase][arr][a] == 0) {
                fail(std::string("used read of unwritten ") + kName[arr] + "[" + std::to_string(a) + "]");
                return;
            }
    }
};

template <int H, int NADJ = 3>
long check(int plant) {
    using G = fl::Geo<H, NADJ>;
    constexpr int NA = G::NADJ;
    Model m;
    m.plant = plant;
    m.cfg = "h=" + std::to_string(H) + " tile 32x" + std::to_string(G::TY) + " " + std::to_string(NA) + " adjoint fields";
    m.size = {5L * G::ZP + G::PAD, 5L * G::XP + G::PAD, (long)NA * G::GP + G::PAD,
              (long)NA * G::GXP + G::PAD, (long)NA * G::GYP};
    for (int p = 0; p < 2; ++p) {
        m.writes[p].resize(NARR);
        for (int a = 0; a < NARR; ++a) m.writes[p][a].assign(m.size[a], 0);
    }
    const int rows_x = fl::row_read(G::SX + 2 * H);                       // X row read (floats)
    const int rows_a = fl::row_read(G::SA + 2 * H);                       // AX row read
    const int rows_y = fl::row_read(G::SY + 2 * H) - (plant == 2 ? 1 : 0);
    const int rows_b = fl::row_read(G::SB + 2 * H);

    // ---- writes of both phases first (each phase's reads use the other phase's writes)
    for (int tid = 0; tid < fl::NT; ++tid) {
        // P0 / F: the five z-sums of each input column
        for (int j = 0; j < G::J; ++j) {
            int ix, iy, zaddr;
            if (!fl::f_column<G>(tid + j * fl::NT, ix, iy, zaddr)) {
                if (!G::FPAIR) continue;
                // paired stores: a lane without this column writes zeros into the plane padding
                int ix0, iy0;
                fl::f_column<G>(tid, ix0, iy0, zaddr);
                zaddr += j * fl::NT;
                if (zaddr < G::IY * G::ZS) m.fail("F padding write inside the plane");
            }
            if (plant == 1) zaddr += 1;
            for (int q = 0; q < 5; ++q) m.write(0, ZS, (long)q * G::ZP + zaddr);
        }
        // P1 / Y: the NA adjoint fields of SY outputs of column ax
        if (tid < G::YITEMS) {
            int seg, ax, xs, gs;
            fl::y_item<G>(tid, seg, ax);
            fl::y_offsets<G>(tid, xs, gs);  // the kernel's per-lane form of the same addresses
            for (int c = 0; c < NA; ++c)
                for (int i = 0; i < G::SY; ++i) {
                    const int a = gs + c * G::GP + i * G::GST;
                    if (a != fl::y_gs<G>(c, ax, seg * G::SY + i)) m.fail("Y offsets disagree with y_gs");
                    m.write(1, GS, a);
                }
        }
        // P1 / AYs
        int bsrc, bdst;
        if (fl::ays_unit<G>(tid, bsrc, bdst))
            for (int i = 0; i < G::SB; ++i) m.write(1, GY, bdst + (long)i * (G::BW - (plant == 3 ? 1 : 0)));
        // P1 / X, P0 / AX
        int src, dst;
        if (fl::x_unit<G>(tid, src, dst))
            for (int i = 0; i < G::SX; ++i) m.write(1, XS, dst + (long)i * G::XS);
        if (fl::ax_unit<G>(tid, src, dst))
            for (int i = 0; i < G::SA; ++i) m.write(0, GXS, dst + (long)i * G::GXS);
        // lane kinds: a lane has at most one of Y, X, AYs (P1; with five adjoint fields the AYs
        // units run on Y lanes after Y's arithmetic, which reads no LDS row) and at most one of
        // Y, AX (P0)
        int s2, d2;
        const bool y = tid < G::YITEMS, x = fl::x_unit<G>(tid, s2, d2), b = fl::ays_unit<G>(tid, s2, d2);
        const bool two_p1 = (x && (y || b)) || (y && b && !G::B_ON_Y);
        const int p0 = y + fl::ax_unit<G>(tid, s2, d2);
        if (two_p1 || p0 > 1) m.fail("lane " + std::to_string(tid) + " has two units in one phase");
    }
    // ---- races: one write per address per phase
    for (int p = 0; p < 2; ++p)
        for (int a = 0; a < NARR; ++a)
            for (long x = 0; x < m.size[a]; ++x)
                if (m.writes[p][a][x] > 1) {
                    m.fail(std::string("address written twice in one phase: ") + kName[a] + "[" + std::to_string(x) + "]");
                    break;
                }

    // ---- reads, and the reads that feed used outputs
    long used_outputs = 0;
    for (int tid = 0; tid < fl::NT; ++tid) {
        // P0 / Y reads rows of Xs; outputs ay < AY are used, each reading its 2h+1 window
        if (tid < G::YITEMS) {
            int seg, ax, xs, gs;
            fl::y_item<G>(tid, seg, ax);
            fl::y_offsets<G>(tid, xs, gs);
            const int y0 = seg * G::SY;
            if (xs != ax * G::XS + y0) m.fail("Y row offset disagrees with the item");
            for (int q = 0; q < 5; ++q) {
                const long row = (long)q * G::XP + xs;
                m.read(0, XS, row, rows_y);
                for (int i = 0; i < G::SY; ++i) {
                    if (y0 + i >= G::AY || ax >= G::AX) continue;
                    if (i + 2 * H + 1 > rows_y) m.fail("Y window past the row read");
                    m.used(0, XS, row + i, 2 * H + 1);
                    ++used_outputs;
                }
            }
        }
        // P1 / AYs reads rows of GXs; every output oy < TY is used
        int bsrc, bdst;
        if (fl::ays_unit<G>(tid, bsrc, bdst)) {
            m.read(1, GXS, bsrc, rows_b);
            for (int i = 0; i < G::SB; ++i) {
                m.used(1, GXS, bsrc + i, 2 * H + 1);
                ++used_outputs;
            }
        }
        // P1 / X reads rows of Zs (outputs ax < AX used), P0 / AX reads rows of Gs (all used)
        int src, dst;
        if (fl::x_unit<G>(tid, src, dst)) {
            const long s = src + (plant == 4 ? 5L * G::ZP : 0);
            m.read(1, ZS, s, rows_x);
            const int start = (dst % G::XP) / G::XS;  // first output position of the segment
            for (int i = 0; i < G::SX; ++i) {
                if (start + i >= G::AX) continue;
                m.used(1, ZS, s + i, 2 * H + 1);
                ++used_outputs;
            }
        }
        if (fl::ax_unit<G>(tid, src, dst)) {
            m.read(0, GS, src, rows_a);
            for (int i = 0; i < G::SA; ++i) {
                if (i + 2 * H + 1 > rows_a) m.fail("AX window past the row read");
                m.used(0, GS, src + i, 2 * H + 1);
                ++used_outputs;
            }
        }
        // P0 / AZ reads one xy-sum per field of its output column
        if (tid < G::NOUT) {
            int ox, oy;
            fl::az_lane<G>(tid, ox, oy);
            for (int c = 0; c < NA; ++c) {
                const long a = (long)c * G::GYP + oy * G::GYS + ox;
                m.read(0, GY, a, 1);
                m.used(0, GY, a, 1);
                ++used_outputs;
            }
        }
    }
    // ---- phase separation: nothing read in a phase is written in it
    for (int p = 0; p < 2; ++p)
        for (int a : m.read_arrays[p])
            if (m.written_arrays[p].count(a)) m.fail(std::string(kName[a]) + " read and written in one phase");
    std::printf("%s: %ld used outputs checked, %s\n", m.cfg.c_str(), used_outputs,
                m.failures ? "FAILED" : "ok");
    return m.failures;
}

}  // namespace

int main(int argc, char** argv) {
    const int plant = argc > 1 ? std::atoi(argv[1]) : 0;
    long f = 0;
    f += check<1>(plant);
    f += check<2>(plant);
    f += check<3>(plant);
    f += check<4>(plant);
    f += check<1, 5>(plant);
    f += check<2, 5>(plant);
    f += check<3, 5>(plant);
    f += check<4, 5>(plant);
    std::printf("%s\n", f ? "FAILED" : "all ok");
    return f ? 1 : 0;
}
