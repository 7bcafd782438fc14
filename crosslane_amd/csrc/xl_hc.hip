// CDNA4 (gfx950) kernels of the hyper-connection steps on either side of the
// MoE block: the pre + RMS norm that makes its input (below) and the post that
// follows it (hip_backend.cpp:777 `k4::hc_post`; its scalar form
// sycl/hc/core.hpp:81-86, launched per (token, value) by sycl/hc/hc.cpp:107-110):
//   out[t][k][e] = post[t][k] * y[t][e] + sum_j comb[t][j * H + k] * res[t][j][e]
// accumulated over j = 0..H-1 in order, every product and sum one IEEE
// rounding (the library builds with -ffp-contract=off). One thread per (t, e):
// it reads its H residual values before writing, so out may be res itself.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "xl_internal.hpp"

namespace xl::dev {
namespace {

template <int H>
__global__ __launch_bounds__(256) void hc_post_kernel(const float* __restrict__ y, const float* res,
                                                      const float* __restrict__ post, const float* __restrict__ comb,
                                                      int D, int T, float* out) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(T) * D) return;
    const int t = int(i / D), e = int(i - int64_t(t) * D);
    // every load first (independent), then the arithmetic
    float r[H], p[H], c[H * H];
#pragma unroll
    for (int j = 0; j < H; ++j) r[j] = res[(int64_t(t) * H + j) * D + e];
#pragma unroll
    for (int k = 0; k < H; ++k) p[k] = post[t * 8 + k];
#pragma unroll
    for (int m = 0; m < H * H; ++m) c[m] = comb[t * 64 + m];
    const float v = y[i];
#pragma unroll
    for (int k = 0; k < H; ++k) {
        float a = __fmul_rn(p[k], v);
#pragma unroll
        for (int j = 0; j < H; ++j) a = __fadd_rn(a, __fmul_rn(c[j * H + k], r[j]));
        out[(int64_t(t) * H + k) * D + e] = a;
    }
}

// Hyper-connection pre + RMS norm before the MoE block (hip_backend.cpp:629
// `k4::hc_pre_norm`; scalar form sycl/hc/core.hpp:74-80, block_sum :9-17):
//   x[t][e] = sum_j mix[t][j] * h[t][j][e]   (j ascending from 0.0f)
// then, with w, x[t][e] = (x[t][e] * inv) * w[e], inv = 1 / sqrt(S / D + eps),
// where S sums x^2 in the reference's fixed order: 1024 lane sums (lane i over
// e = i, i + 1024, ...), a pairwise XOR tree over each 32 lanes (offsets 16,
// 8, 4, 2, 1), the same tree over the 32 group totals. One 1024-thread
// workgroup per token, thread i = lane i, its R <= 32 values in registers
// (every load issued before the first use: one memory latency, not one per
// value): the butterfly of __shfl_xor gives every lane of a group the same
// sum lane 0 gets in the reference (float addition commutes). Separate IEEE
// roundings, correctly rounded sqrt and division.
template <int H, int R>
__global__ __launch_bounds__(1024) void hc_pre_norm_kernel(const float* __restrict__ h, const float* __restrict__ mix,
                                                           const float* __restrict__ w, int D, float eps,
                                                           float* __restrict__ x) {
    // R > 16 (D > 16,384): the pre values go to x and are read back for the
    // scale (registers would spill)
    constexpr bool KEEP = R <= 16;
    __shared__ float red[32];
    const int t = blockIdx.x, i = threadIdx.x;
    const float* hh = h + int64_t(t) * H * D;
    float* xx = x + int64_t(t) * D;
    float m[H], a[KEEP ? R : 1], wv[KEEP ? R : 1], ss = 0.0f;
#pragma unroll
    for (int j = 0; j < H; ++j) m[j] = mix[t * 8 + j];
    if constexpr (KEEP) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int e = i + 1024 * r;
            a[r] = 0.0f;
#pragma unroll
            for (int j = 0; j < H; ++j) a[r] = __fadd_rn(a[r], __fmul_rn(m[j], e < D ? hh[int64_t(j) * D + e] : 0.0f));
            wv[r] = (w && e < D) ? w[e] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (i + 1024 * r < D) ss = __fadd_rn(ss, __fmul_rn(a[r], a[r]));
        if (!w) {   // uniform: the pre values only
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (i + 1024 * r < D) xx[i + 1024 * r] = a[r];
            return;
        }
    } else {
        for (int e = i; e < D; e += 1024) {
            float v = 0.0f;
#pragma unroll
            for (int j = 0; j < H; ++j) v = __fadd_rn(v, __fmul_rn(m[j], hh[int64_t(j) * D + e]));
            xx[e] = v;
            ss = __fadd_rn(ss, __fmul_rn(v, v));
        }
        if (!w) return;
    }
#pragma unroll
    for (int o = 16; o; o >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, o));   // offsets < 32 stay in the group
    if ((i & 31) == 0) red[i >> 5] = ss;
    __syncthreads();
    if (i < 64) {   // wave 0: the tree over the 32 group totals (lanes 32.. carry copies, unused)
        float u = red[i & 31];
#pragma unroll
        for (int o = 16; o; o >>= 1) u = __fadd_rn(u, __shfl_xor(u, o));
        if (i == 0) red[0] = u;
    }
    __syncthreads();
    // sqrtf is the correctly rounded square root here (__fsqrt_rn is the native
    // 1-ulp one unless the OCML rounded operations are enabled)
    const float inv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(red[0], float(D)), eps)));
    if constexpr (KEEP) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (i + 1024 * r < D) xx[i + 1024 * r] = __fmul_rn(__fmul_rn(a[r], inv), wv[r]);
    } else {
        for (int e = i; e < D; e += 1024) xx[e] = __fmul_rn(__fmul_rn(xx[e], inv), w[e]);   // this thread's own writes
    }
}

template <int H>
void launch_pre_norm_h(const float* h, const float* mix, const float* w, int D, int T, float eps, float* x,
                       hipStream_t s, hipEvent_t stop) {
    const int r = (D + 1023) / 1024;
    const auto go = [&](auto kernel) {
        hipExtLaunchKernelGGL(kernel, dim3(T), dim3(1024), 0, s, nullptr, stop, 0, h, mix, w, D, eps, x);
    };
    if (r <= 1) go(hc_pre_norm_kernel<H, 1>);
    else if (r <= 2) go(hc_pre_norm_kernel<H, 2>);
    else if (r <= 4) go(hc_pre_norm_kernel<H, 4>);
    else if (r <= 8) go(hc_pre_norm_kernel<H, 8>);
    else if (r <= 16) go(hc_pre_norm_kernel<H, 16>);
    else go(hc_pre_norm_kernel<H, 32>);
}

}  // namespace

hipError_t launch_hc_pre_norm(const float* h, const float* mix, const float* w, int D, int H, int T, float eps,
                              float* x, hipStream_t s, hipEvent_t stop) {
    if (D < 1 || D > 32768 || H < 1 || H > 4 || T < 1 || T > 8192) return hipErrorInvalidValue;
    switch (H) {
    case 1: launch_pre_norm_h<1>(h, mix, w, D, T, eps, x, s, stop); break;
    case 2: launch_pre_norm_h<2>(h, mix, w, D, T, eps, x, s, stop); break;
    case 3: launch_pre_norm_h<3>(h, mix, w, D, T, eps, x, s, stop); break;
    default: launch_pre_norm_h<4>(h, mix, w, D, T, eps, x, s, stop); break;
    }
    return hipGetLastError();
}

hipError_t launch_hc_post(const float* y, const float* res, const float* post, const float* comb, int D, int H, int T,
                          float* out, hipStream_t s, hipEvent_t stop) {
    if (D < 1 || D > 32768 || H < 1 || H > 4 || T < 1 || T > 8192) return hipErrorInvalidValue;
    const int64_t n = int64_t(T) * D;
    const dim3 grid(unsigned((n + 255) / 256));
    const auto go = [&](auto kernel) {
        hipExtLaunchKernelGGL(kernel, grid, dim3(256), 0, s, nullptr, stop, 0, y, res, post, comb, D, T, out);
    };
    switch (H) {
    case 1: go(hc_post_kernel<1>); break;
    case 2: go(hc_post_kernel<2>); break;
    case 3: go(hc_post_kernel<3>); break;
    default: go(hc_post_kernel<4>); break;
    }
    return hipGetLastError();
}

}  // namespace xl::dev
