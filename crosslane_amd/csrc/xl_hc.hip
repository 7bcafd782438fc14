// CDNA4 (gfx950) kernel of the hyper-connection post that follows the MoE
// block (hip_backend.cpp:777 `k4::hc_post`; its scalar form sycl/hc/core.hpp:
// 81-86, launched per (token, value) by sycl/hc/hc.cpp:107-110):
//   out[t][k][e] = post[t][k] * y[t][e] + sum_j comb[t][j * H + k] * res[t][j][e]
// accumulated over j = 0..H-1 in order, every product and sum one IEEE
// rounding (the library builds with -ffp-contract=off). One thread per (t, e):
// it reads its H residual values before writing, so out may be res itself.
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

}  // namespace

hipError_t launch_hc_post(const float* y, const float* res, const float* post, const float* comb, int D, int H, int T,
                          float* out, hipStream_t s) {
    if (D < 1 || D > 32768 || H < 1 || H > 4 || T < 1 || T > 8192) return hipErrorInvalidValue;
    const int64_t n = int64_t(T) * D;
    const dim3 grid(unsigned((n + 255) / 256));
    switch (H) {
    case 1: hipLaunchKernelGGL(hc_post_kernel<1>, grid, dim3(256), 0, s, y, res, post, comb, D, T, out); break;
    case 2: hipLaunchKernelGGL(hc_post_kernel<2>, grid, dim3(256), 0, s, y, res, post, comb, D, T, out); break;
    case 3: hipLaunchKernelGGL(hc_post_kernel<3>, grid, dim3(256), 0, s, y, res, post, comb, D, T, out); break;
    default: hipLaunchKernelGGL(hc_post_kernel<4>, grid, dim3(256), 0, s, y, res, post, comb, D, T, out); break;
    }
    return hipGetLastError();
}

}  // namespace xl::dev
