// Window sums of width K = 2H+1 built only from the values inside each window. Plain C++ (host
// and device): the kernel uses these functions, and tests/window_model.cpp checks them on the host.
//
// Why not running sums (acc += v[i+2H] - v[i-1]): the rounding error of every add and subtract
// stays in the accumulator, so a window that has moved from signal into an exactly zero or
// constant region does not sum to exactly 0 or K*c. The reference sums each window directly
// (fused_lncc/csrc/lncc3d.cu:57-92), where such windows give exactly cross = var = 0, and any
// residue there is divided by dr^2 in ncc and in its adjoints. Here each window is the sum of a
// suffix of one block of K values and a prefix of the next (van Herk / Gil-Werman), so it is a sum
// of its own values only, with at most K-1 roundings, as a direct sum: all-zero windows give 0 and
// windows of one representable constant give exactly K*c. The cost is about that of running sums:
// per block of K outputs K-1 suffix adds, K-2 prefix adds and K-1 combining adds.
#pragma once

#if defined(__HIPCC__)
#define FL_WHD __host__ __device__
#else
#define FL_WHD
#endif
// full unrolling where the compiler knows the pragma (hipcc, clang); a host build with gcc
// computes the same sums in the same order without it
#if defined(__clang__)
#define FL_UNROLL _Pragma("unroll")
#else
#define FL_UNROLL
#endif

namespace fl {

// out[i] = v[i] + ... + v[i+2H] for i < S, from v[0 .. S+2H). Blocks of K start at 0, K, 2K, ...:
// a window that starts on a block boundary is that block's suffix from its start (the whole
// block); any other window is the suffix of its first block from i plus the prefix of the next
// block up to i+2H. Unused partial sums are dead code after unrolling.
template <int H, int S>
FL_WHD inline void box_sums(const float (&v)[S + 2 * H], float (&out)[S]) {
    constexpr int K = 2 * H + 1, N = S + 2 * H;
    float suf[N], pre[N];
FL_UNROLL
    for (int b = 0; b < N; b += K) {
        const int e = (b + K < N ? b + K : N) - 1;
        suf[e] = v[e];
FL_UNROLL
        for (int i = e - 1; i >= b; --i) suf[i] = v[i] + suf[i + 1];
        pre[b] = v[b];
FL_UNROLL
        for (int i = b + 1; i <= e; ++i) pre[i] = pre[i - 1] + v[i];
    }
FL_UNROLL
    for (int i = 0; i < S; ++i) out[i] = (i % K == 0) ? suf[i] : suf[i] + pre[i + K - 1];
}

// One step of the march along D for a column of p, t: the five window sums of p, t, p^2, t^2, p*t
// over the K planes ending at this one. The march is unrolled by K and R = the step's position in
// its block of K planes = the ring slot of this plane. pre holds the sums over the current block
// (slots 0..R after this step), the ring p, t of the last K planes: slots 0..R this block's,
// slots R+1..K-1 the previous block's, which complete the window. With M > 0 the previous block's
// sums over slots M..K-1 are kept as one partial sum per field (ch), formed from the ring when a
// block completes (R = K-1): a step R < M adds the ring's slots R+1..M-1 and ch, a step R >= M adds
// slots R+1..K-1. Each window is still a sum of its own K terms (in another order), and a step costs
// M(M+1)/2 + (K-1-M)(K-M)/2 + (K-1-M) adds per block and field instead of K(K-1)/2 (M = 0 or
// K-1: no chain). The ring and ch start at zero.
template <int K, int R, int M = 0>
FL_WHD inline void zstep5(float p, float t, float (&pre)[5], float (&pr)[K], float (&tr)[K], float (&ch)[5],
                          float (&out)[5]) {
    static_assert(M >= 0 && M < K, "chain split");
    constexpr bool CH = M > 0 && M < K - 1;
    if constexpr (R == 0) {
        pre[0] = p;
        pre[1] = t;
        pre[2] = p * p;
        pre[3] = t * t;
        pre[4] = p * t;
    } else {
        pre[0] += p;
        pre[1] += t;
        pre[2] = __builtin_fmaf(p, p, pre[2]);
        pre[3] = __builtin_fmaf(t, t, pre[3]);
        pre[4] = __builtin_fmaf(p, t, pre[4]);
    }
FL_UNROLL
    for (int q = 0; q < 5; ++q) out[q] = pre[q];
    constexpr int E = (CH && R < M) ? M : K;   // ring slots R+1..E-1 are added from the ring
FL_UNROLL
    for (int s = R + 1; s < E; ++s) {
        out[0] += pr[s];
        out[1] += tr[s];
        out[2] = __builtin_fmaf(pr[s], pr[s], out[2]);
        out[3] = __builtin_fmaf(tr[s], tr[s], out[3]);
        out[4] = __builtin_fmaf(pr[s], tr[s], out[4]);
    }
    if constexpr (CH && R < M) {
FL_UNROLL
        for (int q = 0; q < 5; ++q) out[q] += ch[q];
    }
    pr[R] = p;
    tr[R] = t;
    if constexpr (CH && R == K - 1) {
        // the block is complete: its sums over slots M..K-1, from the last slot down
        ch[0] = pr[K - 1];
        ch[1] = tr[K - 1];
        ch[2] = pr[K - 1] * pr[K - 1];
        ch[3] = tr[K - 1] * tr[K - 1];
        ch[4] = pr[K - 1] * tr[K - 1];
FL_UNROLL
        for (int s = K - 2; s >= M; --s) {
            ch[0] += pr[s];
            ch[1] += tr[s];
            ch[2] = __builtin_fmaf(pr[s], pr[s], ch[2]);
            ch[3] = __builtin_fmaf(tr[s], tr[s], ch[3]);
            ch[4] = __builtin_fmaf(pr[s], tr[s], ch[4]);
        }
    }
}

// The same for one field y (the xy-sums of an adjoint coefficient): returns the sum over the K
// planes ending at this one. With the chain (M as above) the previous block's sum over slots
// M..K-1 is formed in ring slot M itself when a block completes (that slot's own value is not read
// again before the next block overwrites it), so the chain costs no register.
template <int K, int R, int M = 0>
FL_WHD inline float zstep1(float y, float& pre, float (&ring)[K]) {
    static_assert(M >= 0 && M < K, "chain split");
    constexpr bool CH = M > 0 && M < K - 1;
    if constexpr (R == 0) {
        pre = y;
    } else {
        pre += y;
    }
    float out = pre;
    constexpr int E = (CH && R < M) ? M + 1 : K;   // slots R+1..E-1 (slot M = the chain when R < M)
FL_UNROLL
    for (int s = R + 1; s < E; ++s) out += ring[s];
    ring[R] = y;
    if constexpr (CH && R == K - 1) {
        float c = ring[K - 1];
FL_UNROLL
        for (int s = K - 2; s > M; --s) c += ring[s];
        ring[M] += c;
    }
    return out;
}

}  // namespace fl
