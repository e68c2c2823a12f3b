// Auxiliary gfx950 kernels around the fused LNCC kernel:
//   * box_kernel     zero-padded k^3 box-sum of one fp32 field (the reference's box3d_sep test hook,
//                    fused_lncc/csrc/lncc3d.cu:286-344), or the reference's backward combine
//                    grad = scale (box A + 2p box Bc + t box Cc) from materialized fp32 maps
//                    (lncc3d.cu:163-235). Plane-marching: direct k-tap x/y sums in LDS, z window sums
//                    from a register ring (lncc_window.h), each window a sum of its own values only.
//   * finalize_kernel  loss = 1 - (sum of workgroup partials)/M, summed in a fixed order (float64).
//   * scale_kernel   grad *= grad_out, skipped on the device when grad_out == 1 (no host sync).
#include "lncc_common.h"
#include "lncc_launch.h"
#include "lncc_window.h"

namespace fl {

constexpr int BT = 16;      // box kernel output tile BT x BT, one lane per output column
constexpr int BNT = BT * BT;
static_assert(BNT == kBoxLanes, "box launch shape");

template <int HH, int NF, bool BF16>
__global__ __launch_bounds__(BNT) void box_kernel(BoxArgs a) {
    constexpr int K = 2 * HH + 1;
    constexpr int R = BT + 2 * HH;          // loaded region R x R
    constexpr int RS = odd(R);
    constexpr int XS = odd(BT);
    __shared__ float reg[NF][R][RS];
    __shared__ float xsum[NF][R][XS];

    const int tid = threadIdx.x;
    const int ox = tid % BT, oy = tid / BT;
    uint32_t L = blockIdx.x;
    const int tx = (int)(L % (uint32_t)a.ntx); L /= (uint32_t)a.ntx;
    const int ty = (int)(L % (uint32_t)a.nty); L /= (uint32_t)a.nty;
    const int64_t b = (int64_t)L;
    const int D = a.dimD, Hd = a.dimH, Wd = a.dimW;
    const int64_t HW = (int64_t)Hd * Wd;
    const int x0 = tx * BT, y0 = ty * BT;
    const float* fld[3] = {a.f0, a.f1, a.f2};

    // per field: the xy-sums of the last k planes (ring slot = the plane's position in its block of
    // k) and the prefix sum of the current block; the z-sum of a window is that prefix plus the
    // previous block's suffix from the ring, so a window of zeros sums to exactly zero
    float ring[NF][K], zpre[NF], zsum[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        zpre[f] = 0.f;
#pragma unroll
        for (int r = 0; r < K; ++r) ring[f][r] = 0.f;
    }
    const int zhi = D + HH;
    for (int base = 0; base < zhi; base += K) {
        static_for<0, K>([&](auto rc) __attribute__((always_inline)) {
            constexpr int r = decltype(rc)::value;
            const int zi = base + r;
            if (zi >= zhi) return;
            // load plane zi of the (BT+2h)^2 region (zero outside the volume)
            for (int i = tid; i < R * R; i += BNT) {
                const int ry = i / R, rx = i - ry * R;
                const int gx = x0 - HH + rx, gy = y0 - HH + ry;
                const bool in = zi < D && gx >= 0 && gx < Wd && gy >= 0 && gy < Hd;
                const int64_t o = (b * D + zi) * HW + (int64_t)gy * Wd + gx;
#pragma unroll
                for (int f = 0; f < NF; ++f) reg[f][ry][rx] = in ? fld[f][o] : 0.f;
            }
            __syncthreads();
            for (int i = tid; i < R * BT; i += BNT) {
                const int ry = i / BT, cx = i - ry * BT;
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    float s = 0.f;
#pragma unroll
                    for (int d = 0; d < K; ++d) s += reg[f][ry][cx + d];
                    xsum[f][ry][cx] = s;
                }
            }
            __syncthreads();
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                float s = 0.f;
#pragma unroll
                for (int d = 0; d < K; ++d) s += xsum[f][oy + d][ox];
                zsum[f] = zstep1<K, r>(s, zpre[f], ring[f]);
            }
            const int zo = zi - HH;
            const int gx = x0 + ox, gy = y0 + oy;
            if (zo >= 0 && gx < Wd && gy < Hd) {
                const int64_t o = (b * D + zo) * HW + (int64_t)gy * Wd + gx;
                if constexpr (NF == 1) {
                    reinterpret_cast<float*>(a.out)[o] = zsum[0];
                } else {
                    const float p = load_elem_ptr<BF16>(a.pred, o), t = load_elem_ptr<BF16>(a.target, o);
                    store_elem<BF16>(a.out, o, a.scale * (zsum[0] + 2.f * p * zsum[1] + t * zsum[2]));
                }
            }
        });
    }
}

__global__ __launch_bounds__(256) void finalize_kernel(const double* partials, int nparts, double inv_m,
                                                        float* loss) {
    __shared__ double red[256];
    double s = 0.0;
    for (int i = threadIdx.x; i < nparts; i += 256) s += partials[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) loss[0] = (float)(1.0 - red[0] * inv_m);
}

template <bool BF16>
__global__ __launch_bounds__(256) void scale_kernel(void* grad, int64_t n, const float* grad_out) {
    const float g = *grad_out;
    if (g == 1.0f) return;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        if constexpr (BF16) {
            uint16_t* p = reinterpret_cast<uint16_t*>(grad);
            p[i] = f32_to_bf16_bits(__uint_as_float((uint32_t)p[i] << 16) * g);
        } else {
            reinterpret_cast<float*>(grad)[i] *= g;
        }
    }
}

template <int HH>
static hipError_t launch_box_h(int nfields, bool bf16, const BoxArgs& a, uint32_t nblocks, hipStream_t st) {
    const dim3 grid(nblocks), block(BNT);
    if (nfields == 1) {
        hipLaunchKernelGGL((box_kernel<HH, 1, false>), grid, block, 0, st, a);
    } else if (bf16) {
        hipLaunchKernelGGL((box_kernel<HH, 3, true>), grid, block, 0, st, a);
    } else {
        hipLaunchKernelGGL((box_kernel<HH, 3, false>), grid, block, 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_box(int halo, int nfields, bool bf16, const BoxArgs& a, uint32_t nblocks, hipStream_t st) {
    switch (halo) {
        case 1: return launch_box_h<1>(nfields, bf16, a, nblocks, st);
        case 2: return launch_box_h<2>(nfields, bf16, a, nblocks, st);
        case 3: return launch_box_h<3>(nfields, bf16, a, nblocks, st);
        case 4: return launch_box_h<4>(nfields, bf16, a, nblocks, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_finalize(const double* partials, int nparts, double inv_m, float* loss, hipStream_t st) {
    hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(256), 0, st, partials, nparts, inv_m, loss);
    return hipGetLastError();
}

hipError_t launch_scale(void* grad, bool bf16, int64_t n, const float* grad_out, hipStream_t st) {
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    if (bf16) {
        hipLaunchKernelGGL(scale_kernel<true>, dim3((uint32_t)blocks), dim3(256), 0, st, grad, n, grad_out);
    } else {
        hipLaunchKernelGGL(scale_kernel<false>, dim3((uint32_t)blocks), dim3(256), 0, st, grad, n, grad_out);
    }
    return hipGetLastError();
}

}  // namespace fl
