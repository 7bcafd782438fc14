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
//                   acc); then a 16-8-4-2-1 butterfly and lane 0 + 0.
//                   Persistent workgroups (row groups g, g + G, ...) with the
//                   expanded codebooks staged in LDS once each
//   swiglu_quant32_kernel
//                   h = g / (1 + exp(-g)) * u (the device's expf; g and u
//                   clamped first when the SwiGLU limit is set), quantized per
//                   32 as quant32_kernel does
//
// The bank's planar blocks are decoded directly (xl_format.hpp layout); the
// codebooks come from the context's expanded tables. The dense formats of the
// shared-expert matrices (Q8_0, Q4_K, Q5_K, Q6_K) are read as raw ggml blocks:
// Q4_K / Q5_K subtract the min term as two fmas (corr = fma(m, sum x[0..15],
// m * sum x[16..31]), dot = fma(d, float(s * (a + b)), -corr)); Q6_K values are
// q - 32 with signed per-16 scales; Q8_0 accumulates fma(d * d_x, float(dot)). Build with
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
    float d8;          // the sub-block's d (IQ types: fp16 d * 0.125)
    int sa, sb;        // Q4_K / Q5_K: the two half sums of the activations
    float m;           // Q4_K / Q5_K: fp16 dmin * min (both halves)
};

// 32 bytes at a 2-byte-aligned address as eight words (the Q8_0 / Q6_K rows).
__device__ __forceinline__ void ld32b_a2(const uint8_t* p, uint32_t* w) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = uint32_t(h[2 * j]) | (uint32_t(h[2 * j + 1]) << 16);
}
// 32 bytes at a 2-byte-aligned address as eight words, from the nine aligned
// words that cover them (the last read only when p is not 4-byte aligned) and
// a byte shift: for runs whose covering words stay inside their block (the
// Q6_K rows' low and high bits end at least 16 bytes before the block's end).
__device__ __forceinline__ void ld32b_a2w(const uint8_t* p, uint32_t* w) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
    const uint32_t sh = uint32_t(a & 2u);   // bytes: 0 or 2
    uint32_t d[9];
#pragma unroll
    for (int j = 0; j < 8; ++j) d[j] = q[j];
    d[8] = sh ? q[8] : 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = __builtin_amdgcn_alignbyte(d[j + 1], d[j], sh);
}
// 32 bytes at a 16-byte-aligned address (the Q4_K / Q5_K planes).
__device__ __forceinline__ void ld32b_a16(const uint8_t* p, uint32_t* w) {
    const uint4 lo = reinterpret_cast<const uint4*>(p)[0], hi = reinterpret_cast<const uint4*>(p)[1];
    w[0] = lo.x; w[1] = lo.y; w[2] = lo.z; w[3] = lo.w; w[4] = hi.x; w[5] = hi.y; w[6] = hi.z; w[7] = hi.w;
}

// Dense sub-block kb (32 values) of row `row` (raw ggml blocks).
__device__ __forceinline__ Sub32 sub32_dense(const MatRef& m, int row, int kb, const uint32_t* q) {
    Sub32 r{0, 0, 1, 1, 0.0f, 0, 0, 0.0f};
    uint32_t v[8];
    if (m.type == kQ8_0) {
        const uint8_t* b = m.base + (size_t(row) * m.nb + kb) * 34;
        r.d8 = h2f(ld16(b));
        ld32b_a2(b + 2, v);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r.a = sdot4(v[j], q[j], r.a);
            r.b = sdot4(v[4 + j], q[4 + j], r.b);
        }
        return r;
    }
    const int ib = kb & 7;
    if (m.type == kQ6_K) {
        const uint8_t* b = m.base + (size_t(row) * m.nb + (kb >> 3)) * 210;
        const int h = ib >> 2, quarter = ib & 3;
        uint32_t hi[8];
        ld32b_a2w(b + 64 * h + ((quarter & 1) ? 32 : 0), v);   // ends by byte 128 of 210
        ld32b_a2w(b + 128 + 32 * h, hi);                         // ends by byte 192
        const uint32_t sc = ld16(b + 192 + 8 * h + 2 * quarter);
        r.s0 = int(int8_t(sc & 255u));
        r.s1 = int(int8_t(sc >> 8));
        r.d8 = h2f(ld16(b + 208));
        int sx0 = 0, sx1 = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t w6 = ((v[j] >> (4 * (quarter >> 1))) & 0x0f0f0f0fu) | (((hi[j] >> (2 * quarter)) & 0x03030303u) << 4);
            if (j < 4) { r.a = sdot4(w6, q[j], r.a); sx0 = sdot4(0x01010101u, q[j], sx0); }
            else { r.b = sdot4(w6, q[j], r.b); sx1 = sdot4(0x01010101u, q[j], sx1); }
        }
        r.a -= 32 * sx0;   // values q - 32: exact integer correction
        r.b -= 32 * sx1;
        return r;
    }
    // Q4_K / Q5_K
    const uint8_t* b = m.base + (size_t(row) * m.nb + (kb >> 3)) * (m.type == kQ5_K ? 176 : 144);
    const uint4 hd = *reinterpret_cast<const uint4*>(b);   // d, dmin, 12 scale bytes (blocks of 144 / 176 B: 16-byte aligned)
    const uint32_t dd = hd.x, s03 = hd.y, s47 = hd.z, s8b = hd.w;
    const auto sbyte = [&](int i) -> uint32_t {
        const uint32_t w = i < 4 ? s03 : i < 8 ? s47 : s8b;
        return (w >> (8 * (i & 3))) & 255u;
    };
    int scale, mn;
    if (ib < 4) {
        scale = int(sbyte(ib) & 63u);
        mn = int(sbyte(ib + 4) & 63u);
    } else {
        scale = int((sbyte(ib + 4) & 15u) | ((sbyte(ib - 4) >> 6) << 4));
        mn = int((sbyte(ib + 4) >> 4) | ((sbyte(ib) >> 6) << 4));
    }
    r.s0 = r.s1 = scale;
    r.d8 = h2f(uint16_t(dd & 0xffffu));
    r.m = __fmul_rn(h2f(uint16_t(dd >> 16)), float(mn));
    ld32b_a16(b + (m.type == kQ5_K ? 48 : 16) + 32 * (ib >> 1), v);
    uint32_t hb[8];
    if (m.type == kQ5_K) ld32b_a16(b + 16, hb);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t w = (v[j] >> (4 * (ib & 1))) & 0x0f0f0f0fu;
        if (m.type == kQ5_K) w |= ((hb[j] >> ib) & 0x01010101u) << 4;
        if (j < 4) { r.a = sdot4(w, q[j], r.a); r.sa = sdot4(0x01010101u, q[j], r.sa); }
        else { r.b = sdot4(w, q[j], r.b); r.sb = sdot4(0x01010101u, q[j], r.sb); }
    }
    return r;
}
__device__ __forceinline__ Sub32 sub32(const MatRef& m, int row, int kb, const uint32_t* q, const uint64_t* tab) {
    const size_t blk = size_t(row) * m.nb + (kb >> 3);
    const int ib = kb & 7;
    Sub32 r{0, 0, 1, 1, 0.0f, 0, 0, 0.0f};
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
        const uint32_t qs = ld32(m.base + blk * 32 + 4 * ib);               // four low index bytes
        const uint32_t qh = ld16(m.base + m.off1 + blk * 16 + 2 * ib);      // two high-bit / delta bytes
        const uint8_t* sc = m.base + m.off2 + blk * 8;
        const uint32_t w = ld16(sc + 2 * (ib >> 1));
        r.s0 = 2 * int((w >> (6 * (ib & 1))) & 7u) + 1;
        r.s1 = 2 * int((w >> (6 * (ib & 1) + 3)) & 7u) + 1;
        const uint16_t d16 = uint16_t((ld16(sc) >> 12) | ((ld16(sc + 2) >> 8) & 0xf0u) | ((ld16(sc + 4) >> 4) & 0xf00u) |
                                      (ld16(sc + 6) & 0xf000u));
        r.d8 = __fmul_rn(h2f(d16), 0.125f);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t h = (qh >> (8 * (l >> 1))) & 255u, nib = (l & 1) ? (h >> 4) : (h & 15u);
            const uint64_t g = tab[kTabIQ1 + (((qs >> (8 * l)) & 255u) | ((nib & 7u) << 8))];
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

// One lane's share of a row: sub-blocks l, l + 32, ... in that order, four per
// pass, each pass's loads all issued before its arithmetic (a sub-block past
// the row's end reads sub-block 0 and leaves acc as it is). T fixes the block
// type, so every type test in the decoders folds away.
template <int T>
__device__ __forceinline__ float row_acc(MatRef m, int row, int l, int nk, const int8_t* qp, const float* dp,
                                         const uint64_t* tab) {
    m.type = T;
    float acc = 0.0f;
    for (int k0 = 0; k0 < nk; k0 += 128) {
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int kr = k0 + l + 32 * it;
            const bool ok = kr < nk;
            const int kb = ok ? kr : 0;
            const uint4* qw = reinterpret_cast<const uint4*>(qp + 32 * kb);
            const uint4 lo = qw[0], hi = qw[1];
            const uint32_t a[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            float next;
            if constexpr (T == kQ8_0) {   // core.hpp:80: fma(d * d_x, float(dot), acc)
                const Sub32 s = sub32_dense(m, row, kb, a);
                next = fmaf(__fmul_rn(s.d8, dp[kb]), float(s.a + s.b), acc);
            } else {
                const Sub32 s = dense_type(T) ? sub32_dense(m, row, kb, a) : sub32(m, row, kb, a, tab);
                const int isum = s.s0 * s.a + s.s1 * s.b;
                float dot = __fmul_rn(s.d8, float(isum));
                if constexpr (T == kQ4_K || T == kQ5_K) {   // core.hpp:62-65: the min term as two fmas
                    const float corr = fmaf(s.m, float(s.sa), __fmul_rn(s.m, float(s.sb)));
                    dot = fmaf(s.d8, float(isum), -corr);
                }
                next = fmaf(dp[kb], dot, acc);
            }
            acc = ok ? next : acc;
        }
    }
    return acc;
}

// Rows of one or two roles of every pick: grid (G, 1, roles), 256 threads, 8
// rows per step, 32 lanes per row; workgroup g takes the row groups (pick,
// group) = g, g + G, ... of its role, so that the codebooks it stages in LDS
// once serve many rows. Role role0 + z writes yz. Activations: q + pick *
// q_stride (k int8), d + pick * d_stride (k / 32 scales); output y + pick *
// y_stride. ids == nullptr: the matrices single0 (z = 0) and single1 (z = 1)
// for every pick. stage: the launch has IQ matrices (their codebooks go to LDS).
// FAM: the block types the launch's matrices have (0 the IQ types, 1 the dense
// ones, 2 any), so that each family's decoder gets the registers it needs
// (the dense decoder's wider loads would cost the IQ rows occupancy).
constexpr int kTabBytes = 24576;   // layer_tables: sign masks, IQ2_XXS, IQ2_XS, IQ1 grids
// EPI: the launch's epilogue, 0 none, 1 Mv32Post (the MoE block's shared down
// rows), 2 Mv32Comb (the per32 layer's combine: workgroup g takes row group g
// of every pick, the picks in the combine's order); only those instances carry
// its code, so the others keep their registers.
template <int FAM, int EPI>
__global__ __launch_bounds__(256) void mv32_kernel(const ExpertDesc* __restrict__ descs, const int32_t* __restrict__ ids,
                                                   MatRef single0, MatRef single1, int picks, int n_experts, int role0,
                                                   int n, int k, const int8_t* __restrict__ q, size_t q_stride,
                                                   const float* __restrict__ d, size_t d_stride, float* __restrict__ y0,
                                                   float* __restrict__ y1, size_t y_stride,
                                                   const uint64_t* __restrict__ tab, int stage, int* __restrict__ err,
                                                   Mv32Post ep, Mv32Comb cb) {
    __shared__ __attribute__((aligned(16))) uint64_t stab[kTabBytes / 8];
    __shared__ int s_order[16];
    if (stage) {
        for (int c = threadIdx.x; c < kTabBytes / 16; c += 256)
            reinterpret_cast<uint4*>(stab)[c] = reinterpret_cast<const uint4*>(tab)[c];
    }
    if constexpr (EPI == 2) {
        if (threadIdx.x == 0) {   // combine_one's order: ascending expert id, equal ids in pick order
            for (int i = 0; i < picks; ++i) {
                int j = i;
                for (; j > 0 && ids[s_order[j - 1]] > ids[i]; --j) s_order[j] = s_order[j - 1];
                s_order[j] = i;
            }
        }
    }
    if (stage || EPI == 2) __syncthreads();
    float* y = blockIdx.z ? y1 : y0;
    const int l = threadIdx.x & 31, rgp = (n + 7) / 8, total = picks * rgp;
    float cacc = 0.0f;   // EPI 2, lane 0 of each row: fma(w, y, .) over the picks so far, from +0
    for (int w = blockIdx.x; w < total; w += gridDim.x) {
        const int slot = w / rgp, row = (w - slot * rgp) * 8 + (threadIdx.x >> 5);
        const int pick = EPI == 2 ? s_order[slot] : slot;
        MatRef m = blockIdx.z ? single1 : single0;
        if (ids) {
            const int id = ids[pick];
            if (id < 0 || id >= n_experts) {   // the pick contributes nothing (the combine skips it)
                if (threadIdx.x == 0) atomicOr(err, kDevErrExpertId);
                continue;
            }
            m = descs[id].m[role0 + blockIdx.z];
        }
        const int8_t* qp = q + pick * q_stride;
        const float* dp = d + pick * d_stride;
        const int rr = row < n ? row : n - 1;   // rows past the end compute row n - 1 and store nothing
        float acc = 0.0f;
        if constexpr (FAM == 0) {
            switch (m.type) {   // uniform per workgroup
            case kIQ2_XXS: acc = row_acc<kIQ2_XXS>(m, rr, l, k / 32, qp, dp, stab); break;
            case kIQ2_XS: acc = row_acc<kIQ2_XS>(m, rr, l, k / 32, qp, dp, stab); break;
            default: acc = row_acc<kIQ1_M>(m, rr, l, k / 32, qp, dp, stab); break;
            }
        } else if constexpr (FAM == 1) {
            switch (m.type) {
            case kQ8_0: acc = row_acc<kQ8_0>(m, rr, l, k / 32, qp, dp, stab); break;
            case kQ4_K: acc = row_acc<kQ4_K>(m, rr, l, k / 32, qp, dp, stab); break;
            case kQ5_K: acc = row_acc<kQ5_K>(m, rr, l, k / 32, qp, dp, stab); break;
            default: acc = row_acc<kQ6_K>(m, rr, l, k / 32, qp, dp, stab); break;
            }
        } else {
            switch (m.type) {
            case kIQ2_XXS: acc = row_acc<kIQ2_XXS>(m, rr, l, k / 32, qp, dp, stab); break;
            case kIQ2_XS: acc = row_acc<kIQ2_XS>(m, rr, l, k / 32, qp, dp, stab); break;
            case kIQ1_M: acc = row_acc<kIQ1_M>(m, rr, l, k / 32, qp, dp, stab); break;
            case kQ8_0: acc = row_acc<kQ8_0>(m, rr, l, k / 32, qp, dp, stab); break;
            case kQ4_K: acc = row_acc<kQ4_K>(m, rr, l, k / 32, qp, dp, stab); break;
            case kQ5_K: acc = row_acc<kQ5_K>(m, rr, l, k / 32, qp, dp, stab); break;
            default: acc = row_acc<kQ6_K>(m, rr, l, k / 32, qp, dp, stab); break;
            }
        }
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) acc = __fadd_rn(acc, __shfl_xor(acc, o, 32));
        if (row < n && l == 0) {
            float v = __fadd_rn(acc, 0.0f);
            if constexpr (EPI == 1) {
                if (ep.add) v = __fadd_rn(ep.add[row], v);   // one pick: the routed output, then + this row
            }
            y[pick * y_stride + row] = v;
            if constexpr (EPI == 2) cacc = fmaf(cb.w[pick], v, cacc);
            if (EPI == 1 && ep.res) {   // hc_post of this column, in hc_post_kernel's order (every load first)
                const int H = ep.H;
                float r[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] = i < H ? ep.res[size_t(i) * n + row] : 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (j < H) {
                        float o = __fmul_rn(ep.post[j], v);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (i < H) o = __fadd_rn(o, __fmul_rn(ep.comb[i * H + j], r[i]));
                        ep.out[size_t(j) * n + row] = o;
                    }
                }
            }
        }
    }
    if constexpr (EPI == 2) {   // combine_one: then + shared
        const int row = int(blockIdx.x) * 8 + int(threadIdx.x >> 5);
        if (row < n && l == 0) cb.out[row] = cb.shared ? __fadd_rn(cacc, cb.shared[row]) : cacc;
    }
}

// h = SwiGLU(g, u) (limit applied) quantized per 32 as quant32_kernel does, in
// one pass: the same h values, the same quants and scales, no h round trip.
__global__ __launch_bounds__(256) void swiglu_quant32_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                             int nblk, float lim, int8_t* __restrict__ q,
                                                             float* __restrict__ d) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const bool in = (i >> 5) < nblk;
    const float v = in ? silu_mul3(g[i], u[i], lim) : 0.0f;
    float am = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 32));
    if (!in) return;
    const float sc = __fdiv_rn(am, 127.0f);
    q[i] = int8_t(am > 0.0f ? __float2int_rn(__fdiv_rn(v, sc)) : 0);
    if ((i & 31) == 0) d[i >> 5] = sc;
}

}  // namespace

hipError_t launch_quant32(const float* x, int rows, int k, int8_t* q, float* d, int* err, hipStream_t s) {
    if (rows < 1 || k < 32 || k % 32) return hipErrorInvalidValue;
    const int nblk = rows * (k / 32);
    hipLaunchKernelGGL(quant32_kernel, dim3((nblk * 32 + 255) / 256), dim3(256), 0, s, x, nblk, q, d, err);
    return hipGetLastError();
}

hipError_t launch_mv32(const ExpertDesc* descs, const int32_t* ids, const MatRef& single0, const MatRef& single1,
                       int picks, int n_experts, int role0, int roles, int n, int k, const int8_t* q, size_t q_stride,
                       const float* d, size_t d_stride, float* y0, float* y1, size_t y_stride,
                       const uint64_t* tables, int* err, hipStream_t s, const Mv32Post* epi,
                       const Mv32Comb* comb) {
    if (picks < 1 || roles < 1 || roles > 2 || n < 1 || k < 256 || k % 256) return hipErrorInvalidValue;
    const Mv32Post ep = epi ? *epi : Mv32Post{};
    if ((ep.add || ep.res) && (picks != 1 || roles != 1 || (ep.res && (ep.H < 1 || ep.H > 4 || !ep.out))))
        return hipErrorInvalidValue;
    const Mv32Comb cb = comb ? *comb : Mv32Comb{};
    if (cb.out && (!ids || roles != 1 || picks > 16 || !cb.w || ep.add || ep.res)) return hipErrorInvalidValue;
    // Bank matrices (ids) may be any IQ type; a single pair of dense matrices needs no codebook.
    const int stage = ids || !dense_type(single0.type) || (roles > 1 && !dense_type(single1.type));
    const int total = picks * ((n + 7) / 8);
    // staging workgroups take several row groups; the combine takes one row group
    // per workgroup, every pick of it
    const int G = cb.out ? (n + 7) / 8 : stage ? (total < 512 ? total : 512) : total;
    // bank matrices (ids) are IQ types; single ones are whatever they are
    const bool dense0 = !ids && dense_type(single0.type), dense1 = roles > 1 ? !ids && dense_type(single1.type) : dense0;
    const auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(G, 1, roles), dim3(256), 0, s, descs, ids, single0, single1, picks, n_experts,
                           role0, n, k, q, q_stride, d, d_stride, y0, y1, y_stride, tables, stage, err, ep, cb);
    };
    const bool epi_on = ep.add || ep.res;
    if (cb.out) go(mv32_kernel<0, 2>);   // bank matrices: the IQ family
    else if (dense0 != dense1) epi_on ? go(mv32_kernel<2, 1>) : go(mv32_kernel<2, 0>);
    else if (dense0) epi_on ? go(mv32_kernel<1, 1>) : go(mv32_kernel<1, 0>);
    else epi_on ? go(mv32_kernel<0, 1>) : go(mv32_kernel<0, 0>);
    return hipGetLastError();
}

hipError_t launch_swiglu_quant32(const float* g, const float* u, int rows, int k, float lim, int8_t* q, float* d,
                                 hipStream_t s) {
    if (rows < 1 || k < 32 || k % 32) return hipErrorInvalidValue;
    const int nblk = rows * (k / 32);
    hipLaunchKernelGGL(swiglu_quant32_kernel, dim3((nblk * 32 + 255) / 256), dim3(256), 0, s, g, u, nblk, lim, q, d);
    return hipGetLastError();
}

}  // namespace xl::dev
