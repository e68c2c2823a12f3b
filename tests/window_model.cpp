// Host-side check of the window sums the fused kernel uses (fused-lncc_amd/csrc/lncc_window.h):
// box_sums (x and y passes) and zstep5 / zstep1 (the march along D), run here exactly as the
// kernel runs them, against direct sums in float64.
//
//   exact    on integer data every partial sum is exact, so each window must equal its direct
//            sum bit for bit (catches a wrong index, a missing or doubled term, a wrong block);
//   zeros    a window of zeros inside random float data sums to exactly 0;
//   const    a window of one constant c (0.5, 7, 128) inside random data sums to exactly K*c, as
//            a direct sum does (constants whose partial sums are floats; for others, such as
//            0.1f, every order of summation rounds differently and only the bound applies);
//   bound    on random data every window is within (K-1) * 2^-24 * sum|v| of the float64 sum,
//            the error bound of a direct sum of K terms.
// The march is run over 300 planes with zero and constant slabs after signal, for K = 3..9 and
// every split M of the previous block's suffix (the chain of zstep5 / zstep1; M = 0: none).
//
// Usage: window_model [plant]. plant = 1 replaces zstep5's window by a running sum (add the
// entering plane, subtract the leaving one), plant = 2 drops the last term of box_sums' block
// suffix, plant = 3 halves zstep5's chain of the previous block's suffix (for every split M > 0);
// each must be reported. Prints one line per check group and exits 0 when all pass.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "lncc_window.h"

namespace {

int g_plant = 0;
long g_fail = 0;

void fail(const std::string& what) {
    if (g_fail < 10) std::printf("  FAIL %s\n", what.c_str());
    ++g_fail;
}

float direct32(const float* v, int K) {
    float s = 0.f;
    for (int i = 0; i < K; ++i) s += v[i];
    return s;
}

template <int H, int S>
void box_sums_under_test(const float (&v)[S + 2 * H], float (&out)[S]) {
    fl::box_sums<H, S>(v, out);
    if (g_plant == 2) {
        constexpr int K = 2 * H + 1;
        // model of a bug: the first window loses its last term
        out[0] -= v[K - 1];
    }
}

// x/y passes: random rows with integer, zero and constant windows planted
template <int H, int S>
void check_box(std::mt19937& rng, const char* name) {
    constexpr int K = 2 * H + 1, N = S + 2 * H;
    std::uniform_real_distribution<float> u(-3.f, 3.f);
    std::uniform_int_distribution<int> ui(-500, 500);
    const long before = g_fail;
    for (int trial = 0; trial < 2000; ++trial) {
        float v[N], out[S];
        const int mode = trial % 4;
        for (int i = 0; i < N; ++i) v[i] = mode == 0 ? (float)ui(rng) : u(rng) * std::pow(10.f, (float)(ui(rng) % 4));
        const float consts[4] = {0.f, 0.5f, 7.f, 128.f};
        int z0 = -1;
        if (mode >= 1) {  // plant a window of zeros or one constant
            z0 = rng() % S;
            const float c = consts[(trial / 4) % 4];
            for (int i = z0; i < z0 + K; ++i) v[i] = c;
        }
        box_sums_under_test<H, S>(v, out);
        for (int i = 0; i < S; ++i) {
            double ref = 0.0, mag = 0.0;
            for (int j = i; j < i + K; ++j) {
                ref += v[j];
                mag += std::fabs(v[j]);
            }
            if (mode == 0 && out[i] != (float)ref)
                fail(std::string(name) + ": integer window " + std::to_string(i) + " not exact");
            if (i == z0 && out[i] != direct32(v + i, K))
                fail(std::string(name) + ": zero/constant window " + std::to_string(i) + " = " + std::to_string(out[i]));
            if (std::fabs(out[i] - ref) > (K - 1) * std::ldexp(1.0, -24) * mag + 1e-30)
                fail(std::string(name) + ": window " + std::to_string(i) + " beyond the direct-sum bound");
        }
    }
    std::printf("box_sums h=%d S=%d (%s): %s\n", H, S, name, g_fail == before ? "ok" : "FAILED");
}

template <int K, int R, int M>
void step5(float p, float t, float (&pre)[5], float (&pr)[K], float (&tr)[K], float (&ch)[5], float (&out)[5]) {
    if (g_plant == 1) {
        // model of the bug this replaces: running sums over the whole march
        static float acc[5];
        const float po = pr[R], to = tr[R];
        acc[0] += p - po;
        acc[1] += t - to;
        acc[2] = std::fma(p, p, std::fma(-po, po, acc[2]));
        acc[3] = std::fma(t, t, std::fma(-to, to, acc[3]));
        acc[4] = std::fma(p, t, std::fma(-po, to, acc[4]));
        for (int q = 0; q < 5; ++q) out[q] = acc[q];
        pr[R] = p;
        tr[R] = t;
        (void)pre;
        (void)ch;
        return;
    }
    fl::zstep5<K, R, M>(p, t, pre, pr, tr, ch, out);
    if (g_plant == 3 && R == K - 1) ch[0] *= 0.5f;  // a chain that loses half of its p terms
}

template <int K, int M, int R = 0>
void march_step(int r, float p, float t, float (&pre)[5], float (&pr)[K], float (&tr)[K], float (&ch)[5],
                float (&out)[5], float y, float& gpre, float (&gr)[K], float& gout) {
    if constexpr (R < K) {
        if (r == R) {
            step5<K, R, M>(p, t, pre, pr, tr, ch, out);
            gout = fl::zstep1<K, R, M>(y, gpre, gr);
        } else {
            march_step<K, M, R + 1>(r, p, t, pre, pr, tr, ch, out, y, gpre, gr, gout);
        }
    }
}

// the D-march: one column over 300 planes, signal then zero then constant slabs; M = the split
// of the previous block's suffix (0 = none)
template <int K, int M>
void check_march(std::mt19937& rng) {
    const int Z = 300;
    const long before = g_fail;
    std::uniform_real_distribution<float> u(0.f, 255.f);
    for (int kind = 0; kind < 3; ++kind) {
        std::vector<float> p(Z), t(Z), y(Z);
        for (int z = 0; z < Z; ++z) {
            p[z] = kind == 0 ? std::floor(u(rng)) : u(rng);
            t[z] = kind == 0 ? std::floor(u(rng)) : 0.7f * p[z] + 0.3f * u(rng);
            y[z] = u(rng) - 100.f;
            if (kind >= 1 && z >= 100 && z < 180) p[z] = t[z] = y[z] = 0.f;         // zero slab
            if (kind >= 1 && z >= 220 && z < 280) p[z] = t[z] = y[z] = (kind == 1 ? 128.f : 0.5f);  // constant slab
        }
        float pre[5] = {0}, pr[K] = {0}, tr[K] = {0}, ch[5] = {0}, out[5], gpre = 0.f, gr[K] = {0}, gout;
        for (int z = 0; z < Z; ++z) {
            march_step<K, M>(z % K, p[z], t[z], pre, pr, tr, ch, out, y[z], gpre, gr, gout);
            // direct sums of the window [z-K+1, z] (planes before 0 are zero)
            double ref[5] = {0}, mag[5] = {0}, gref = 0.0, gmag = 0.0;
            float r32[5] = {0}, g32 = 0.f;
            for (int s = z - K + 1; s <= z; ++s) {
                if (s < 0) continue;
                const double a = p[s], b = t[s];
                const double f[5] = {a, b, a * a, b * b, a * b};
                for (int q = 0; q < 5; ++q) {
                    ref[q] += f[q];
                    mag[q] += std::fabs(f[q]);
                }
                r32[0] += p[s];
                r32[1] += t[s];
                r32[2] = std::fma(p[s], p[s], r32[2]);
                r32[3] = std::fma(t[s], t[s], r32[3]);
                r32[4] = std::fma(p[s], t[s], r32[4]);
                gref += y[s];
                gmag += std::fabs(y[s]);
                g32 += y[s];
            }
            const bool flat = z >= K - 1 && [&] {
                for (int s = z - K + 1; s <= z; ++s)
                    if (p[s] != p[z] || t[s] != t[z]) return false;
                return true;
            }();
            for (int q = 0; q < 5; ++q) {
                if (kind == 0 && out[q] != (float)ref[q])
                    fail("march K=" + std::to_string(K) + ": integer window at z=" + std::to_string(z) + " not exact");
                if (flat && out[q] != r32[q])
                    fail("march K=" + std::to_string(K) + ": flat window at z=" + std::to_string(z) + " field " +
                         std::to_string(q) + " = " + std::to_string(out[q]) + ", direct " + std::to_string(r32[q]));
                if (std::fabs(out[q] - ref[q]) > 2 * (K - 1) * std::ldexp(1.0, -24) * mag[q] + 1e-30)
                    fail("march K=" + std::to_string(K) + ": window at z=" + std::to_string(z) + " beyond the bound");
            }
            if (flat && gout != g32) fail("march K=" + std::to_string(K) + ": flat adjoint window at z=" + std::to_string(z));
            if (std::fabs(gout - gref) > (K - 1) * std::ldexp(1.0, -24) * gmag + 1e-30)
                fail("march K=" + std::to_string(K) + ": adjoint window beyond the bound");
        }
    }
    std::printf("march K=%d chain M=%d: %s\n", K, M, g_fail == before ? "ok" : "FAILED");
}

// every split of the previous block's suffix, M = 0 (none) .. K-1
template <int K, int M = 0>
void check_all_splits(std::mt19937& rng) {
    if constexpr (M < K) {
        check_march<K, M>(rng);
        check_all_splits<K, M + 1>(rng);
    }
}

}  // namespace

int main(int argc, char** argv) {
    g_plant = argc > 1 ? std::atoi(argv[1]) : 0;
    std::mt19937 rng(1234);
    // the segment lengths of the kernel: X 20, Y 4, AX 16, AYs 16 (12 at k = 9)
    check_box<1, 20>(rng, "x");
    check_box<2, 20>(rng, "x");
    check_box<3, 20>(rng, "x");
    check_box<4, 20>(rng, "x");
    check_box<1, 4>(rng, "y");
    check_box<2, 4>(rng, "y");
    check_box<3, 4>(rng, "y");
    check_box<4, 4>(rng, "y");
    check_box<1, 16>(rng, "ax/ays");
    check_box<2, 16>(rng, "ax/ays");
    check_box<3, 16>(rng, "ax/ays");
    check_box<4, 16>(rng, "ax");
    check_box<4, 12>(rng, "ays");
    check_all_splits<3>(rng);
    check_all_splits<5>(rng);
    check_all_splits<7>(rng);
    check_all_splits<9>(rng);
    std::printf("%s\n", g_fail ? "FAILED" : "all ok");
    return g_fail ? 1 : 0;
}
