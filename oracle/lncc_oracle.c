/*
 * CPU oracle for the fused 3D LNCC loss — TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C and float64, the algorithm of the reference's LNCC hot path so
 * that the HIP kernels can be checked against it. Only the tests, the smoke check and the CPU
 * baseline leg of the benchmark load it; the product path never calls it.
 *
 * What it follows (reference files):
 *   - box-sum: zero-padded k^3 window with constant n = k^3
 *       baselines/torch_lncc.py:12-14 (grouped F.conv3d with a ones kernel, padding=k//2),
 *       fused_lncc/csrc/lncc3d.cu:45-54 (zero outside the volume);
 *   - per-voxel squared NCC and its clamp
 *       baselines/torch_lncc.py:25-32 (policy LNCC_POLICY_TORCH: no variance clamp; the autograd of
 *       clamp(max=1) passes the gradient where ncc <= 1),
 *       fused_lncc/csrc/lncc3d.cu:93-107 (policy LNCC_POLICY_KERNEL: raw variances clamped at 0
 *       before adding dr; adjoints zeroed where ncc >= 1; NaN keeps NaN ncc and zero adjoints);
 *   - adjoints A = dncc/dSp, B = dncc/dSpp, C = dncc/dSpt: lncc3d.cu:101-104;
 *   - loss = 1 - mean(ncc) over all N*C*D*H*W voxels: fused_lncc/__init__.py:62;
 *   - gradient wrt pred = -(1/M) * (box(A) + 2 p box(B) + t box(C)): lncc3d.cu:163-165,231-233 and
 *     fused_lncc/__init__.py:73 (box is self-adjoint under zero padding).
 *
 * Pinning (tests/test_oracle.py): golden vectors written from baselines/torch_lncc.py (loss and
 * autograd gradient), brute-force box-sums on tiny volumes, the constant-field closed form,
 * scipy.ndimage.uniform_filter, float64 central finite differences of the loss, and the
 * self-adjoint identity <box a, b> = <a, box b>. The float32 restatement lncc_oracle_ref32 (end of
 * this file): the same golden vectors to float32 accuracy, exact zeros in zero and constant
 * windows, float32-sized errors on offset intensities.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define LNCC_POLICY_TORCH 0
#define LNCC_POLICY_KERNEL 1

/* One pass of a zero-padded window sum of width 2h+1 along an axis of `len` points spaced
 * `stride` apart. The independent lines start at o*ostride + i*istride for o < outer, i < inner. */
static void box_axis(const double* in, double* out, int len, long stride, int h,
                     long outer, long ostride, long inner, long istride) {
    for (long o = 0; o < outer; ++o) {
        for (long i = 0; i < inner; ++i) {
            const double* src = in + o * ostride + i * istride;
            double* dst = out + o * ostride + i * istride;
            for (int x = 0; x < len; ++x) {
                int lo = x - h < 0 ? 0 : x - h;
                int hi = x + h > len - 1 ? len - 1 : x + h;
                double s = 0.0;
                for (int j = lo; j <= hi; ++j) s += src[(long)j * stride];
                dst[(long)x * stride] = s;
            }
        }
    }
}

/* Zero-padded k^3 box-sum of one (D,H,W) volume. `tmp` holds D*H*W doubles. */
static void box_volume(const double* x, double* y, double* tmp, int D, int H, int W, int k) {
    int h = k / 2;
    long HW = (long)H * W;
    box_axis(x, y, W, 1, h, (long)D * H, W, 1, 1);     /* along W */
    box_axis(y, tmp, H, W, h, D, HW, W, 1);            /* along H */
    box_axis(tmp, y, D, HW, h, 1, 0, HW, 1);           /* along D */
}

/* Box-sum of B volumes (float64 in/out). */
void lncc_oracle_box3d(const double* x, double* y, int B, int D, int H, int W, int k) {
    long V = (long)D * H * W;
    double* tmp = (double*)malloc(sizeof(double) * V);
    for (int b = 0; b < B; ++b) box_volume(x + b * V, y + b * V, tmp, D, H, W, k);
    free(tmp);
}

/* Per-voxel ncc and adjoints for one volume from its five box-sums. Returns the ncc sum. */
static double ncc_adjoints(const double* Sp, const double* St, const double* Spp, const double* Stt,
                           const double* Spt, long V, double n, double dr, int policy,
                           double* ncc_out, double* A, double* Bc, double* Cc) {
    double acc = 0.0;
    for (long i = 0; i < V; ++i) {
        double cross = Spt[i] - Sp[i] * St[i] / n;
        double vp = Spp[i] - Sp[i] * Sp[i] / n;
        double vt = Stt[i] - St[i] * St[i] / n;
        if (policy == LNCC_POLICY_KERNEL) {
            vp = vp > 0.0 ? vp : 0.0;
            vt = vt > 0.0 ? vt : 0.0;
        }
        vp += dr;
        vt += dr;
        double ncc = (cross * cross) / (vp * vt);
        int live = policy == LNCC_POLICY_KERNEL ? (ncc < 1.0) : (ncc <= 1.0);
        double a = 0.0, b = 0.0, c = 0.0;
        if (live) {
            c = 2.0 * cross / (vp * vt);
            b = -(cross * cross) / (vp * vp * vt);
            a = -(St[i] * c + 2.0 * Sp[i] * b) / n;
        }
        if (ncc >= 1.0) ncc = 1.0; /* NaN compares false and stays NaN */
        acc += ncc;
        if (ncc_out) ncc_out[i] = ncc;
        A[i] = a;
        Bc[i] = b;
        Cc[i] = c;
    }
    return acc;
}

/* Oracle for one (D,H,W) volume; returns the ncc sum, or NAN with *err set on allocation failure. */
static double oracle_volume(const float* pb, const float* tb, int D, int H, int W, int k, double dr,
                            int policy, double M, float* gb, double* ncc_map, double* a_map,
                            double* b_map, double* c_map, int* err) {
    long V = (long)D * H * W;
    double n = (double)k * k * k;
    double* buf = (double*)malloc(sizeof(double) * V * 13);
    if (!buf) { *err = 1; return NAN; }
    double *p = buf, *t = buf + V, *q = buf + 2 * V, *tmp = buf + 3 * V;
    double *Sp = buf + 4 * V, *St = buf + 5 * V, *Spp = buf + 6 * V, *Stt = buf + 7 * V,
           *Spt = buf + 8 * V;
    double *A = buf + 9 * V, *Bc = buf + 10 * V, *Cc = buf + 11 * V, *box = buf + 12 * V;
    for (long i = 0; i < V; ++i) { p[i] = pb[i]; t[i] = tb[i]; }
    box_volume(p, Sp, tmp, D, H, W, k);
    box_volume(t, St, tmp, D, H, W, k);
    for (long i = 0; i < V; ++i) q[i] = p[i] * p[i];
    box_volume(q, Spp, tmp, D, H, W, k);
    for (long i = 0; i < V; ++i) q[i] = t[i] * t[i];
    box_volume(q, Stt, tmp, D, H, W, k);
    for (long i = 0; i < V; ++i) q[i] = p[i] * t[i];
    box_volume(q, Spt, tmp, D, H, W, k);
    double total = ncc_adjoints(Sp, St, Spp, Stt, Spt, V, n, dr, policy, ncc_map, A, Bc, Cc);
    if (a_map) memcpy(a_map, A, sizeof(double) * V);
    if (b_map) memcpy(b_map, Bc, sizeof(double) * V);
    if (c_map) memcpy(c_map, Cc, sizeof(double) * V);
    if (gb) {
        box_volume(A, box, tmp, D, H, W, k);
        for (long i = 0; i < V; ++i) q[i] = box[i];
        box_volume(Bc, box, tmp, D, H, W, k);
        for (long i = 0; i < V; ++i) q[i] += 2.0 * p[i] * box[i];
        box_volume(Cc, box, tmp, D, H, W, k);
        for (long i = 0; i < V; ++i) gb[i] = (float)(-(q[i] + t[i] * box[i]) / M);
    }
    free(buf);
    return total;
}

/*
 * Full oracle: loss = 1 - mean(ncc), optional gradient wrt pred (float32 out, already multiplied by
 * -1/M) and optional per-voxel maps (float64 out): ncc, A, B, C. Inputs are float32 (bf16 inputs
 * are upcast by the caller). Volumes run in parallel when built with OpenMP. Returns 0, or -1 on
 * allocation failure.
 */
int lncc_oracle(const float* pred, const float* target, int B, int D, int H, int W, int k, double dr,
                int policy, double* loss_out, float* grad, double* ncc_map, double* a_map,
                double* b_map, double* c_map) {
    long V = (long)D * H * W;
    double M = (double)B * V;
    double total = 0.0;
    int err = 0;
#pragma omp parallel for schedule(dynamic) reduction(+ : total) reduction(| : err)
    for (int b = 0; b < B; ++b) {
        long o = (long)b * V;
        total += oracle_volume(pred + o, target + o, D, H, W, k, dr, policy, M,
                               grad ? grad + o : NULL, ncc_map ? ncc_map + o : NULL,
                               a_map ? a_map + o : NULL, b_map ? b_map + o : NULL,
                               c_map ? c_map + o : NULL, &err);
    }
    if (err) return -1;
    *loss_out = 1.0 - total / M;
    return 0;
}

/* Round-to-nearest-even float32 -> bfloat16 -> float32, NaN kept quiet (lncc3d.cu:21). */
float lncc_oracle_round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        u |= 0x00400000u;
        u &= 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    float y;
    memcpy(&y, &u, 4);
    return y;
}

/*
 * The reference kernel's own float32 arithmetic, restated (fused_lncc/csrc/lncc3d.cu): the
 * error level the GPU path is measured against on ill-conditioned inputs (offset intensities,
 * zero and constant regions). Not a second oracle: the float64 functions above are the exact
 * values; this gives what the reference itself returns for the same float32 inputs.
 *   - box-sums as direct k-tap sums in float32, x then y then z, each tap added in order with
 *     the products fused (the CUDA compiler contracts `app += p * p` to an fma):
 *     lncc3d.cu:57-92 (forward), lncc3d.cu:195-227 (backward);
 *   - cross, clamped variances, ncc and the adjoints with IEEE divisions: lncc3d.cu:93-107;
 *   - grad = scale * (box A + 2 p box B + t box C) with scale 1 (lncc3d.cu:231-233), then the
 *     float32 tensor multiply by -1/M of fused_lncc/__init__.py:73.
 * The loss is 1 - mean(ncc) with the mean taken in float64 (torch's float32 mean differs from it
 * by far less than the errors this is used to bound).
 */
static void ref32_axis(const float* in, float* out, int len, long stride, int h, long outer,
                       long ostride, long inner, long istride) {
    for (long o = 0; o < outer; ++o)
        for (long i = 0; i < inner; ++i) {
            const float* src = in + o * ostride + i * istride;
            float* dst = out + o * ostride + i * istride;
            for (int x = 0; x < len; ++x) {
                float s = 0.f;
                for (int d = -h; d <= h; ++d) {
                    int j = x + d;
                    s += (j >= 0 && j < len) ? src[(long)j * stride] : 0.f;
                }
                dst[(long)x * stride] = s;
            }
        }
}

/* One float32 field box-summed in the reference's order; `x` already holds the x-tap input. */
static void ref32_box(const float* x, float* y, float* tmp, int D, int H, int W, int h) {
    long HW = (long)H * W;
    ref32_axis(x, tmp, W, 1, h, (long)D * H, W, 1, 1);
    ref32_axis(tmp, y, H, W, h, D, HW, W, 1);
    ref32_axis(y, tmp, D, HW, h, 1, 0, HW, 1);
    memcpy(y, tmp, sizeof(float) * D * HW);
}

/* x-pass of a product field: s = fma(a_j, b_j, s) over the taps (lncc3d.cu:62-67). */
static void ref32_xprod(const float* a, const float* b, float* out, int D, int H, int W, int h) {
    for (long r = 0; r < (long)D * H; ++r)
        for (int x = 0; x < W; ++x) {
            float s = 0.f;
            for (int d = -h; d <= h; ++d) {
                int j = x + d;
                float u = (j >= 0 && j < W) ? a[r * W + j] : 0.f;
                float v = (j >= 0 && j < W) ? b[r * W + j] : 0.f;
                s = fmaf(u, v, s);
            }
            out[r * W + x] = s;
        }
}

static int ref32_volume(const float* p, const float* t, int D, int H, int W, int k, float dr,
                        double M, float* g, float* ncc_map, double* ncc_sum) {
    long V = (long)D * H * W, HW = (long)H * W;
    int h = k / 2;
    float n = (float)(k * k * k);
    float* buf = (float*)malloc(sizeof(float) * V * 10);
    if (!buf) return 1;
    float *Sp = buf, *St = buf + V, *Spp = buf + 2 * V, *Stt = buf + 3 * V, *Spt = buf + 4 * V;
    float *A = buf + 5 * V, *Bm = buf + 6 * V, *Cm = buf + 7 * V, *tmp = buf + 8 * V, *x = buf + 9 * V;
    /* x-pass of the five fields, then y and z (the reference stages x-sums, y-sums, z-sums) */
    ref32_axis(p, x, W, 1, h, (long)D * H, W, 1, 1);
    ref32_axis(x, tmp, H, W, h, D, HW, W, 1);
    ref32_axis(tmp, Sp, D, HW, h, 1, 0, HW, 1);
    ref32_axis(t, x, W, 1, h, (long)D * H, W, 1, 1);
    ref32_axis(x, tmp, H, W, h, D, HW, W, 1);
    ref32_axis(tmp, St, D, HW, h, 1, 0, HW, 1);
    float* outs[3] = {Spp, Stt, Spt};
    const float* fa[3] = {p, t, p};
    const float* fb[3] = {p, t, t};
    for (int f = 0; f < 3; ++f) {
        ref32_xprod(fa[f], fb[f], x, D, H, W, h);
        ref32_axis(x, tmp, H, W, h, D, HW, W, 1);
        ref32_axis(tmp, outs[f], D, HW, h, 1, 0, HW, 1);
    }
    double acc = 0.0;
    for (long i = 0; i < V; ++i) {
        float cross = Spt[i] - Sp[i] * St[i] / n;
        float vp = fmaxf(Spp[i] - Sp[i] * Sp[i] / n, 0.f) + dr;
        float vt = fmaxf(Stt[i] - St[i] * St[i] / n, 0.f) + dr;
        float ncc = (cross * cross) / (vp * vt);
        float a = 0.f, b = 0.f, c = 0.f;
        if (ncc < 1.0f) {
            c = 2.f * cross / (vp * vt);
            b = -(cross * cross) / (vp * vp * vt);
            a = -fmaf(St[i], c, 2.f * Sp[i] * b) / n;
        } else if (ncc >= 1.0f) {
            ncc = 1.0f;
        }
        acc += ncc;
        if (ncc_map) ncc_map[i] = ncc;
        A[i] = a;
        Bm[i] = b;
        Cm[i] = c;
    }
    *ncc_sum = acc;
    if (g) {
        float* bA = Sp; /* the box-sums are no longer needed */
        float* bB = St;
        float* bC = Spp;
        ref32_box(A, bA, tmp, D, H, W, h);
        ref32_box(Bm, bB, tmp, D, H, W, h);
        ref32_box(Cm, bC, tmp, D, H, W, h);
        float sc = (float)(-1.0 / M);
        for (long i = 0; i < V; ++i) g[i] = fmaf(t[i], bC[i], fmaf(2.f * p[i], bB[i], bA[i])) * sc;
    }
    free(buf);
    return 0;
}

/* Loss, optional gradient wrt pred (float32, times -1/M) and optional ncc map (float32) as the
 * reference kernel computes them in float32. Returns 0, or -1 on allocation failure. */
int lncc_oracle_ref32(const float* pred, const float* target, int B, int D, int H, int W, int k,
                      float dr, double* loss_out, float* grad, float* ncc_map) {
    long V = (long)D * H * W;
    double M = (double)B * V;
    double total = 0.0;
    int err = 0;
#pragma omp parallel for schedule(dynamic) reduction(+ : total) reduction(| : err)
    for (int b = 0; b < B; ++b) {
        long o = (long)b * V;
        double s = 0.0;
        err |= ref32_volume(pred + o, target + o, D, H, W, k, dr, M, grad ? grad + o : NULL,
                            ncc_map ? ncc_map + o : NULL, &s);
        total += s;
    }
    if (err) return -1;
    *loss_out = 1.0 - total / M;
    return 0;
}
