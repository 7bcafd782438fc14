// Device-side decode of one "pair" (two 32-weight sub-blocks, 64 weights) of
// an IQ2_XXS / IQ2_XS / IQ1_M super-block against 64 Q8_K activation bytes.
//
// The integers are exact and order-independent, so per-block sums equal the
// reference's Sum over AVX2 lanes of integer_lane (engine/strata/sycl/stage/
// wiring/q8k_core.hpp:43-69): grid magnitudes with ksigns sign masks times odd
// sub-scales 2s+1 (IQ2), and IQ1_M's (main, delta) integer pair.
//
// LDS tables (u64 rows): IQ2_XXS grid 256, IQ2_XS grid 512, IQ1 grid 2048,
// and 128 sign masks (byte j = 0xFF when bit j of ksigns[i] is set).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace xl::dev {

constexpr int kTabXXS = 0;              // u64 index of the IQ2_XXS grid
constexpr int kTabXS = 256;             // IQ2_XS grid
constexpr int kTabIQ1 = 256 + 512;      // IQ1 grid
constexpr int kTabSign = 256 + 512 + 2048;
constexpr int kTabRows = 256 + 512 + 2048 + 128;   // 2944 rows = 23552 bytes

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(int(a), int(b), c, false);
}

// grid bytes (all < 128) with the sign mask m applied: byte -> -byte where m=0xFF.
// (g ^ 0xFF) + 1 = 256 - g never carries into the next byte because g >= 8.
__device__ __forceinline__ uint32_t apply_sign(uint32_t g, uint32_t m) {
    return (g ^ m) + (m & 0x01010101u);
}

// One IQ2 group of 8 weights: grid row gi, sign row si, activations a0/a1.
__device__ __forceinline__ int iq2_group(const uint2* tab, uint32_t gi, uint32_t si, uint32_t a0, uint32_t a1, int acc) {
    const uint2 g = tab[gi];
    const uint2 m = tab[kTabSign + si];
    acc = dot4(apply_sign(g.x, m.x), a0, acc);
    return dot4(apply_sign(g.y, m.y), a1, acc);
}

// IQ2_XXS: w = 16 bytes = two sub-blocks of {u32 grid indices, u32 aux}
// (aux bits 7g..7g+6 = sign index of group g, bits 28..31 = scale s).
__device__ __forceinline__ int pair_iq2xxs(const uint2* tab, uint4 w, const uint32_t* a) {
    int sa = 0, sb = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g)
        sa = iq2_group(tab, kTabXXS + ((w.x >> (8 * g)) & 255u), (w.y >> (7 * g)) & 127u, a[2 * g], a[2 * g + 1], sa);
#pragma unroll
    for (int g = 0; g < 4; ++g)
        sb = iq2_group(tab, kTabXXS + ((w.z >> (8 * g)) & 255u), (w.w >> (7 * g)) & 127u, a[8 + 2 * g], a[9 + 2 * g], sb);
    return sa * int(2u * (w.y >> 28) + 1u) + sb * int(2u * (w.w >> 28) + 1u);
}

// IQ2_XS: w = 8 u16 codes (9-bit grid | 7-bit sign); sc = the two sub-blocks'
// scale bytes (low nibble: weights 0..15, high nibble: 16..31).
__device__ __forceinline__ int pair_iq2xs(const uint2* tab, uint4 w, uint32_t sc, const uint32_t* a) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    int total = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        int lo = 0, hi = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t code = (words[2 * s + g / 2] >> (16 * (g & 1))) & 0xffffu;
            const int r = iq2_group(tab, kTabXS + (code & 511u), code >> 9, a[8 * s + 2 * g], a[8 * s + 2 * g + 1], 0);
            if (g < 2) lo += r; else hi += r;
        }
        const uint32_t byte = (sc >> (8 * s)) & 255u;
        total += lo * int(2u * (byte & 15u) + 1u) + hi * int(2u * (byte >> 4) + 1u);
    }
    return total;
}

// Sum of the 8 activation bytes of one group (for IQ1_M's delta term).
__device__ __forceinline__ int group_sum(uint32_t a0, uint32_t a1) {
    return dot4(0x01010101u, a1, dot4(0x01010101u, a0, 0));
}

// IQ1_M: q = 8 low-index bytes (4 per sub-block), h = 4 high/delta bytes
// (2 per sub-block; nibble = 3 index bits + delta-sign bit), scw = the u16
// scale word shared by the pair (bits 0-2/3-5: first sub-block's halves,
// bits 6-8/9-11: second's). Returns (main, delta) integers.
// s8 holds the precomputed group_sum of the pair's 8 activation groups.
__device__ __forceinline__ int2 pair_iq1m(const uint2* tab, uint2 q, uint32_t h, uint32_t scw, const uint32_t* a,
                                          const int* s8) {
    int2 out = make_int2(0, 0);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const uint32_t qw = s ? q.y : q.x;
        int mlo = 0, mhi = 0, dlo = 0, dhi = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t nib = (h >> (16 * s + 4 * g)) & 15u;
            const uint32_t idx = ((qw >> (8 * g)) & 255u) | ((nib & 7u) << 8);
            const uint2 gr = tab[kTabIQ1 + idx];
            const uint32_t a0 = a[8 * s + 2 * g], a1 = a[8 * s + 2 * g + 1];
            const int m = dot4(gr.y, a1, dot4(gr.x, a0, 0));
            const int sum = s8[4 * s + g];
            const int d = (nib & 8u) ? -sum : sum;
            if (g < 2) { mlo += m; dlo += d; } else { mhi += m; dhi += d; }
        }
        const int slo = int(2u * ((scw >> (6 * s)) & 7u) + 1u);
        const int shi = int(2u * ((scw >> (6 * s + 3)) & 7u) + 1u);
        out.x += slo * mlo + shi * mhi;
        out.y += slo * dlo + shi * dhi;
    }
    return out;
}

// ---- wave helpers -----------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over the 4 lanes of a quad; every lane of the quad gets the sum.
__device__ __forceinline__ int quad_sum(int v) {
    v += dpp_i<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_i<0x4E>(v);   // quad_perm [2,3,0,1]
    return v;
}
// Sum of values that are replicated within quads, over groups of G lanes
// (G = 4, 8, 16, 32, 64, aligned). Every lane of the group gets the sum.
// Fixed data movement, so the float result is run-to-run identical.
template <int G>
__device__ __forceinline__ float group_sum_quads(float v) {
    if constexpr (G >= 8) v += dpp_f<0x141>(v);   // row_half_mirror: lane i <-> 7-i
    if constexpr (G >= 16) v += dpp_f<0x140>(v);  // row_mirror: lane i <-> 15-i
    if constexpr (G >= 32) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // xor 16
    if constexpr (G >= 64)
        v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    return v;
}

}  // namespace xl::dev
