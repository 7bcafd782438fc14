// CDNA4 (gfx950) kernels of the per32 mode: the arithmetic of the reference's
// production HIP lane (engine/strata/warm/hip_experts.hip:17-39 with the
// sub-block decode of hip_experts_core.hpp / sycl/moe/core.hpp:66-88), so that
// this lane reproduces that lane's bits:
//
//   quant32_kernel  activations in blocks of 32: d = max|x| / 127 (IEEE
//                   division), q = round-half-even(x / d), zero block all zero
//   mv32_kernel     rows of the picks' matrices: 32 lanes per row, lane l
//                   takes sub-blocks l, l + 32, ...: dot = (fp16(d) * 0.125) *
//                   float(s0 * a + s1 * b) (a, b: the integer dots of the two
//                   16-weight halves, s: odd sub-scales), acc = fma(xd, dot,
//                   acc); then a 16-8-4-2-1 butterfly and lane 0 + 0
//   swiglu32_kernel g / (1 + exp(-g)) * u (the device's expf; g and u clamped
//                   first when the SwiGLU limit is set)
//
// The bank's planar blocks are decoded directly (xl_format.hpp layout); the
// codebooks come from the context's expanded tables. Build with
// -ffp-contract=off: every float operation above is a separate IEEE rounding.
#include <hip/hip_runtime.h>

#include "xl_dev.hpp"
#include "xl_format.hpp"
#include "xl_internal.hpp"

namespace xl::dev {
namespace {

constexpr int kTabSgn = 0, kTabXXS = 256, kTabXS = 512, kTabIQ1 = 1024;   // u64 row offsets (layer_tables)

// Aligned loads: p is 2- (ld16) or 4-byte (ld32) aligned.
__device__ __forceinline__ uint16_t ld16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Sub-block kb (32 weights) of row `row`: the two half integer dots against the
// 8 activation words q, the odd half scales and the block's d * 0.125.
struct Sub32 {
    int a, b, s0, s1;
    float d8;
};
__device__ __forceinline__ Sub32 sub32(const MatRef& m, int row, int kb, const uint32_t* q, const uint64_t* tab) {
    const size_t blk = size_t(row) * m.nb + (kb >> 3);
    const int ib = kb & 7;
    Sub32 r{0, 0, 1, 1, 0.0f};
    int half[2] = {0, 0};
    if (m.type == kIQ2_XXS || m.type == kIQ2_XS) {
        const uint8_t* p = m.base + blk * 64 + 8 * ib;
        const uint32_t w0 = ld32(p), w1 = ld32(p + 4);
        uint16_t d16;
        if (m.type == kIQ2_XXS) {   // four grid bytes; aux bytes sign7 | (scale bit) << 7
            int s = 0;
#pragma unroll
            for (int l = 0; l < 4; ++l) s |= int((w1 >> (8 * l + 7)) & 1u) << l;
            r.s0 = r.s1 = 2 * s + 1;
            d16 = ld16(m.base + m.off1 + blk * 2);
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const uint64_t g = tab[kTabXXS + ((w0 >> (8 * l)) & 255u)];
                const uint32_t sg = (w1 >> (8 * l)) & 127u;
                const uint64_t M = tab[kTabSgn + 2 * sg], M1 = tab[kTabSgn + 2 * sg + 1];
                half[l >> 1] = sdot4(xad(uint32_t(g), uint32_t(M), uint32_t(M1)), q[2 * l], half[l >> 1]);
                half[l >> 1] = sdot4(xad(uint32_t(g >> 32), uint32_t(M >> 32), uint32_t(M1 >> 32)), q[2 * l + 1], half[l >> 1]);
            }
        } else {   // four u16 codes sign7 | grid9 << 7; a scale byte per sub-block
            const uint32_t sb = m.base[m.off1 + blk * 8 + ib];
            r.s0 = 2 * int(sb & 15u) + 1;
            r.s1 = 2 * int(sb >> 4) + 1;
            d16 = ld16(m.base + m.off2 + blk * 2);
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const uint32_t c = ((l < 2 ? w0 : w1) >> (16 * (l & 1))) & 0xffffu;
                const uint64_t g = tab[kTabXS + (c >> 7)];
                const uint32_t sg = c & 127u;
                const uint64_t M = tab[kTabSgn + 2 * sg], M1 = tab[kTabSgn + 2 * sg + 1];
                half[l >> 1] = sdot4(xad(uint32_t(g), uint32_t(M), uint32_t(M1)), q[2 * l], half[l >> 1]);
                half[l >> 1] = sdot4(xad(uint32_t(g >> 32), uint32_t(M >> 32), uint32_t(M1 >> 32)), q[2 * l + 1], half[l >> 1]);
            }
        }
        r.d8 = __fmul_rn(h2f(d16), 0.125f);
    } else {   // IQ1_M: qs, qh nibbles (3 index bits + delta sign), scale words with the fp16 d in their top nibbles
        const uint8_t* qs = m.base + blk * 32 + 4 * ib;
        const uint8_t* qh = m.base + m.off1 + blk * 16 + 2 * ib;
        const uint8_t* sc = m.base + m.off2 + blk * 8;
        const uint32_t w = ld16(sc + 2 * (ib >> 1));
        r.s0 = 2 * int((w >> (6 * (ib & 1))) & 7u) + 1;
        r.s1 = 2 * int((w >> (6 * (ib & 1) + 3)) & 7u) + 1;
        const uint16_t d16 = uint16_t((ld16(sc) >> 12) | ((ld16(sc + 2) >> 8) & 0xf0u) | ((ld16(sc + 4) >> 4) & 0xf00u) |
                                      (ld16(sc + 6) & 0xf000u));
        r.d8 = __fmul_rn(h2f(d16), 0.125f);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t h = qh[l >> 1], nib = (l & 1) ? (h >> 4) : (h & 15u);
            const uint64_t g = tab[kTabIQ1 + (qs[l] | ((nib & 7u) << 8))];
            const int mdot = sdot4(uint32_t(g >> 32), q[2 * l + 1], sdot4(uint32_t(g), q[2 * l], 0));
            const int qsum = sdot4(0x01010101u, q[2 * l + 1], sdot4(0x01010101u, q[2 * l], 0));
            half[l >> 1] += 8 * mdot + ((nib & 8u) ? -qsum : qsum);   // values 8 * grid + delta
        }
    }
    r.a = half[0];
    r.b = half[1];
    return r;
}

__global__ __launch_bounds__(256) void quant32_kernel(const float* __restrict__ x, int nblk, int8_t* __restrict__ q,
                                                      float* __restrict__ d, int* __restrict__ err) {
    const int i = blockIdx.x * 256 + threadIdx.x;   // value index; 32 lanes per block of 32
    const bool in = (i >> 5) < nblk;
    const float v = in ? x[i] : 0.0f;
    float am = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 32));
    if (__any(in && !(fabsf(v) <= 3.402823466e38f)) && (threadIdx.x & 63) == 0) atomicOr(err, kDevErrNonFinite);
    if (!in) return;
    const float sc = __fdiv_rn(am, 127.0f);
    q[i] = int8_t(am > 0.0f ? __float2int_rn(__fdiv_rn(v, sc)) : 0);
    if ((i & 31) == 0) d[i >> 5] = sc;
}

// Rows of one or two roles of every pick: grid (ceil(n / 8), picks, roles), 8
// rows per 256-thread workgroup, 32 lanes per row. Role role0 + z writes yz.
// Activations: q + pick * q_stride (k int8), d + pick * d_stride (k / 32
// scales); output y + pick * y_stride. ids == nullptr: the one matrix `single`.
__global__ __launch_bounds__(256) void mv32_kernel(const ExpertDesc* __restrict__ descs, const int32_t* __restrict__ ids,
                                                   MatRef single, int n_experts, int role0, int n, int k,
                                                   const int8_t* __restrict__ q, size_t q_stride,
                                                   const float* __restrict__ d, size_t d_stride, float* __restrict__ y0,
                                                   float* __restrict__ y1, size_t y_stride,
                                                   const uint64_t* __restrict__ tab, int* __restrict__ err) {
    const int pick = blockIdx.y;
    MatRef m = single;
    if (ids) {
        const int id = ids[pick];
        if (id < 0 || id >= n_experts) {   // the pick contributes nothing (the combine skips it)
            if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, kDevErrExpertId);
            return;
        }
        m = descs[id].m[role0 + blockIdx.z];
    }
    float* y = blockIdx.z ? y1 : y0;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5), l = threadIdx.x & 31;
    const int8_t* qp = q + pick * q_stride;
    const float* dp = d + pick * d_stride;
    float acc = 0.0f;
    if (row < n)
        for (int kb = l; kb < k / 32; kb += 32) {
            const uint4* qw = reinterpret_cast<const uint4*>(qp + 32 * kb);
            const uint4 lo = qw[0], hi = qw[1];
            const uint32_t a[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            const Sub32 s = sub32(m, row, kb, a, tab);
            const float dot = __fmul_rn(s.d8, float(s.s0 * s.a + s.s1 * s.b));
            acc = fmaf(dp[kb], dot, acc);
        }
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) acc = __fadd_rn(acc, __shfl_xor(acc, o, 32));
    if (row < n && l == 0) y[pick * y_stride + row] = __fadd_rn(acc, 0.0f);
}

__global__ __launch_bounds__(256) void swiglu32_kernel(const float* __restrict__ g, const float* __restrict__ u, int n,
                                                       float lim, float* __restrict__ h) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] = silu_mul3(g[i], u[i], lim);
}

}  // namespace

hipError_t launch_quant32(const float* x, int rows, int k, int8_t* q, float* d, int* err, hipStream_t s) {
    if (rows < 1 || k < 32 || k % 32) return hipErrorInvalidValue;
    const int nblk = rows * (k / 32);
    hipLaunchKernelGGL(quant32_kernel, dim3((nblk * 32 + 255) / 256), dim3(256), 0, s, x, nblk, q, d, err);
    return hipGetLastError();
}

hipError_t launch_mv32(const ExpertDesc* descs, const int32_t* ids, const MatRef& single, int picks, int n_experts,
                       int role0, int roles, int n, int k, const int8_t* q, size_t q_stride, const float* d,
                       size_t d_stride, float* y0, float* y1, size_t y_stride, const uint64_t* tables, int* err,
                       hipStream_t s) {
    if (picks < 1 || roles < 1 || roles > 2 || n < 1 || k < 256 || k % 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mv32_kernel, dim3((n + 7) / 8, picks, roles), dim3(256), 0, s, descs, ids, single, n_experts,
                       role0, n, k, q, q_stride, d, d_stride, y0, y1, y_stride, tables, err);
    return hipGetLastError();
}

hipError_t launch_swiglu32(const float* g, const float* u, int n, float lim, float* h, hipStream_t s) {
    hipLaunchKernelGGL(swiglu32_kernel, dim3((n + 255) / 256), dim3(256), 0, s, g, u, n, lim, h);
    return hipGetLastError();
}

}  // namespace xl::dev
