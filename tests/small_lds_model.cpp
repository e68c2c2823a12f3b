// Host-side model of the LDS accesses of the small-volume kernel (lncc_small.hip), from the same
// index functions the kernel uses (lncc_geometry.h: small_lds, small_class, small_skip), for every
// halo h = 1..4. It checks
//   layout    small_lds maps the 16^3 positions of a field one to one onto [0, 4096);
//   banks     every LDS access instruction (one field, one of a lane's positions, the 64 lanes of
//             a wave) touches 64 distinct 4-byte banks;
//   reads     every line read that is not a compile-time zero lies inside [0, 16), and every
//             skipped one outside it, for each lane quarter's code class;
//   races     between two workgroup barriers no LDS float is both read and written;
//   coverage  every read finds what the previous interval wrote there.
// The barrier intervals: A writes F; B reads F; (barrier) B writes G over F's first three fields;
// (barrier) C reads G and writes G2; (barrier) D reads G2.
// Usage: small_lds_model [plant]: 1 leaves the rows unrotated (bank conflicts in B and C), 2 gives
// quarter 0 the interior class (reads below position 0), 3 puts G2 over F as G is (a race in C);
// each must be reported.
#include <cstdio>
#include <cstdlib>
#include <map>
#include <set>
#include <string>

#include "lncc_geometry.h"

namespace {

constexpr int E = fl::kSmallEdge, NT = fl::kSmallLanes, FIELD = E * E * E;
int g_plant = 0;
long g_fail = 0;

void fail(const std::string& what) {
    if (g_fail < 8) std::printf("  FAIL %s\n", what.c_str());
    ++g_fail;
}

int lds(int z, int y, int x) {
    if (g_plant == 1) return (z << 8) | (y << 4) | x;   // rows not rotated
    return fl::small_lds(z, y, x);
}
int qclass(int q) { return g_plant == 2 && q == 0 ? 1 : fl::small_class(q); }

// LDS float offsets: F at [0, 5 FIELD) (G over its first three fields), G2 after it
int f_at(int f, int a) { return f * FIELD + a; }
int g2_at(int c, int a) { return (g_plant == 3 ? 0 : 5 * FIELD) + c * FIELD + a; }

struct Interval {
    std::set<int> reads, writes;
};

void bank_check(const std::string& what, const int (&addr)[64], const bool (&on)[64]) {
    std::map<int, int> banks;
    for (int l = 0; l < 64; ++l)
        if (on[l]) banks[addr[l] % 64] += 1;
    for (auto& kv : banks)
        if (kv.second > 1) {
            fail(what + ": " + std::to_string(kv.second) + " lanes on bank " + std::to_string(kv.first));
            return;
        }
}

template <int H>
void check() {
    const long before = g_fail;
    const std::string tag = "h=" + std::to_string(H);
    {
        std::set<int> seen;
        for (int z = 0; z < E; ++z)
            for (int y = 0; y < E; ++y)
                for (int x = 0; x < E; ++x) {
                    const int a = lds(z, y, x);
                    if (a < 0 || a >= FIELD || !seen.insert(a).second) {
                        fail(tag + " layout not one to one");
                        z = y = x = E;
                    }
                }
    }
    // Lane tid: q = tid >> 8 (four whole waves), r = (tid >> 4) & 15, x = tid & 15. Phases A, D:
    // r = y, the lane's column (y, x) along z; phases B, C: r = z, the lane's line (z, x) along y.
    Interval iv[5];   // A, B reads, B writes, C, D
    auto access = [&](int interval, bool write, int nfields, auto addr_of, const std::string& what) {
        for (int w = 0; w < NT / 64; ++w) {
            const int q = (64 * w) >> 8;
            for (int k = 0; k < (write ? 4 : 4 + 2 * H); ++k)
                for (int f = 0; f < nfields; ++f) {
                    int addr[64];
                    bool on[64];
                    for (int l = 0; l < 64; ++l) {
                        const int tid = 64 * w + l, r = (tid >> 4) & 15, x = tid & 15;
                        on[l] = true;
                        int pos = 4 * q + k;
                        if (!write) {
                            pos = 4 * q - H + k;
                            const bool skip = fl::small_skip(qclass(q), H, k), inside = pos >= 0 && pos < E;
                            if (!skip && !inside) fail(tag + " " + what + ": quarter " + std::to_string(q) + " reads position " + std::to_string(pos));
                            if (skip && inside) fail(tag + " " + what + ": quarter " + std::to_string(q) + " skips position " + std::to_string(pos));
                            on[l] = !skip && inside;
                        }
                        addr[l] = on[l] ? addr_of(f, r, pos, x) : 0;
                        if (on[l]) (write ? iv[interval].writes : iv[interval].reads).insert(addr[l]);
                    }
                    bank_check(tag + " " + what, addr, on);
                }
        }
    };
    access(0, true, 5, [](int f, int y, int z, int x) { return f_at(f, lds(z, y, x)); }, "A writes F");
    access(1, false, 5, [](int f, int z, int y, int x) { return f_at(f, lds(z, y, x)); }, "B reads F");
    access(2, true, 3, [](int c, int z, int y, int x) { return f_at(c, lds(z, y, x)); }, "B writes G");
    access(3, false, 3, [](int c, int z, int y, int x) { return f_at(c, lds(z, y, x)); }, "C reads G");
    access(3, true, 3, [](int c, int z, int y, int x) { return g2_at(c, lds(z, y, x)); }, "C writes G2");
    access(4, false, 3, [](int c, int y, int z, int x) { return g2_at(c, lds(z, y, x)); }, "D reads G2");
    // races and coverage
    std::set<int> latest;   // the floats written by earlier intervals
    for (int i = 0; i < 5; ++i) {
        for (int a : iv[i].reads) {
            if (iv[i].writes.count(a)) {
                fail(tag + " interval " + std::to_string(i) + " reads and writes LDS float " + std::to_string(a));
                break;
            }
        }
        for (int a : iv[i].reads)
            if (!latest.count(a)) {
                fail(tag + " interval " + std::to_string(i) + " reads LDS float " + std::to_string(a) + " that no earlier interval wrote");
                break;
            }
        for (int a : iv[i].writes) latest.insert(a);
    }
    std::printf("small-volume kernel h=%d: %s\n", H, g_fail == before ? "ok" : "FAILED");
}

}  // namespace

int main(int argc, char** argv) {
    g_plant = argc > 1 ? std::atoi(argv[1]) : 0;
    check<1>();
    check<2>();
    check<3>();
    check<4>();
    std::printf("%s\n", g_fail ? "FAILED" : "all ok");
    return g_fail ? 1 : 0;
}
