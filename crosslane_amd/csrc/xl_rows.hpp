// Row engine of the decode kernels: LDS codebooks, raw row loads and the
// IQ x Q8_K row dot, for gfx950 wave64.
//
// Lane mapping: a wave covers RPW = 64 / LPR rows at a time; lane l of a row
// group owns the "pairs" {l + LPR*j : j < PPL} of its row, a pair being two
// 32-weight sub-blocks (64 weights). The 4 pairs of one super-block sit in one
// hardware quad.
//
// Integers are exact and order-independent, so per-block sums equal the
// reference's Sum over AVX2 lanes of integer_lane (engine/strata/sycl/stage/
// wiring/q8k_core.hpp:43-69). IQ1_M's (main, delta) pair enters the fast path
// as the single integer 8*main + delta, read from a premultiplied table of
// 8*grid + delta. Each lane scales its pair integer by fp16(d_w) * d_x, the
// row group sums the lanes, and the row is scaled by 1/8 (q8k_core.hpp:87-91
// regrouped; the float order differs from the AVX2 lanes, the integers do not).
//
// Per group of 8 weights the IQ2 decode is one SDWA address op per table, one
// v_xad_u32 per dword to apply the sign mask ((g ^ M) + M1), and two v_dot4.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "xl_format.hpp"
#include "xl_internal.hpp"

namespace xl::dev {

// ---- LDS codebooks (byte offsets) --------------------------------------------
constexpr int kLdsXXS = 0;          // IQ2_XXS grid: 256 rows x 8 B
constexpr int kLdsXS = 2048;        // IQ2_XS grid: 512 rows x 8 B
constexpr int kLdsSign = 6144;      // 256 rows x 16 B: {M.lo, M.hi, M1.lo, M1.hi} of ksigns[b & 127]
constexpr int kLdsIQ1 = 10240;      // 4096 rows x 8 B: row (nib << 8 | idx_lo) = 8*grid[idx] + (nib & 8 ? -1 : 1)
constexpr int kLdsEnd2 = kLdsIQ1;   // bytes needed by IQ2 types only
constexpr int kLdsEnd1 = kLdsIQ1 + 4096 * 8;

// Compact code buffer in device memory: 2-bit symbols, 8 per u16.
constexpr int kCodesXXS = 0, kCodesXS = 256, kCodesIQ1 = 768, kCodesTotal = 768 + 2048;

enum : int { kNeedXXS = 1, kNeedXS = 2, kNeedIQ1 = 4 };

__device__ __forceinline__ int need_mask(int type) {
    return type == kIQ2_XXS ? kNeedXXS : type == kIQ2_XS ? kNeedXS : type == kIQ1_M ? kNeedIQ1 : 0;
}
inline int lds_bytes_for(int need) {
    return (need & kNeedIQ1) ? kLdsEnd1 : kLdsEnd2;
}

__device__ __forceinline__ uint64_t expand_mag(uint32_t code) {
    uint64_t v = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t s = (code >> (2 * j)) & 3u;
        v |= uint64_t(s == 0 ? 8u : s == 1 ? 25u : 43u) << (8 * j);
    }
    return v;
}
__device__ __forceinline__ uint64_t expand_iq1(uint32_t code, int mul, int delta) {
    uint64_t v = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int s = int((code >> (2 * j)) & 3u) - 1;
        v |= uint64_t(uint8_t(int8_t(mul * s + delta))) << (8 * j);
    }
    return v;
}
__device__ __forceinline__ uint4 sign_row(int b) {
    const uint32_t i = uint32_t(b) & 127u;
    const uint32_t s = i | ((__popc(i) & 1u) << 7);   // ggml ksigns: even parity in bit 7
    uint32_t m0 = 0, m1 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (s & (1u << j)) m0 |= 0xffu << (8 * j);
        if (s & (1u << (j + 4))) m1 |= 0xffu << (8 * j);
    }
    return make_uint4(m0, m1, m0 & 0x01010101u, m1 & 0x01010101u);
}

// Each of the 256 threads of a workgroup prefetches its codes before the
// weight loads and fills the LDS rows after them.
struct CodeRegs {
    uint32_t xxs, xs[2], iq1[8];
};
__device__ __forceinline__ void codes_prefetch(CodeRegs& c, const uint16_t* __restrict__ codes, int need, int t) {
    if (need & kNeedXXS) c.xxs = codes[kCodesXXS + t];
    if (need & kNeedXS) { c.xs[0] = codes[kCodesXS + t]; c.xs[1] = codes[kCodesXS + 256 + t]; }
    if (need & kNeedIQ1) {
#pragma unroll
        for (int r = 0; r < 8; ++r) c.iq1[r] = codes[kCodesIQ1 + 256 * r + t];
    }
}
__device__ __forceinline__ void codes_fill(uint8_t* lds, const CodeRegs& c, int need, int t) {
    uint64_t* G = reinterpret_cast<uint64_t*>(lds);
    if (need & kNeedXXS) G[kLdsXXS / 8 + t] = expand_mag(c.xxs);
    if (need & kNeedXS) { G[kLdsXS / 8 + t] = expand_mag(c.xs[0]); G[kLdsXS / 8 + 256 + t] = expand_mag(c.xs[1]); }
    if (need & (kNeedXXS | kNeedXS)) reinterpret_cast<uint4*>(lds + kLdsSign)[t] = sign_row(t);
    if (need & kNeedIQ1) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            // 11-bit grid index idx = r << 8 | t; rows (nib << 8 | t) for nib = r (delta +1) and r | 8 (delta -1)
            G[kLdsIQ1 / 8 + (r << 8) + t] = expand_iq1(c.iq1[r], 8, 1);
            G[kLdsIQ1 / 8 + ((r | 8) << 8) + t] = expand_iq1(c.iq1[r], 8, -1);
        }
    }
}

// ---- small helpers ---------------------------------------------------------------
typedef const __attribute__((address_space(1))) uint8_t* gptr;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 gload16(gptr p) {
    const u32x4 v = *reinterpret_cast<const __attribute__((address_space(1))) u32x4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 gload8(gptr p) {
    const u32x2 v = *reinterpret_cast<const __attribute__((address_space(1))) u32x2*>(p);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t gload4(gptr p) { return *reinterpret_cast<const __attribute__((address_space(1))) uint32_t*>(p); }
__device__ __forceinline__ uint32_t gload2(gptr p) { return *reinterpret_cast<const __attribute__((address_space(1))) uint16_t*>(p); }

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4(int(a), int(b), c, false); }
__device__ __forceinline__ uint32_t xad(uint32_t a, uint32_t b, uint32_t c) { return (a ^ b) + c; }   // v_xad_u32
__device__ __forceinline__ int mul24(int a, int b) { return __mul24(a, b); }
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return float(__builtin_bit_cast(_Float16, uint16_t(h)));   // v_cvt_f32_f16: exact for every finite half
}
__device__ __forceinline__ uint2 lds8(const uint8_t* lds, uint32_t off) { return *reinterpret_cast<const uint2*>(lds + off); }
__device__ __forceinline__ uint4 lds16(const uint8_t* lds, uint32_t off) { return *reinterpret_cast<const uint4*>(lds + off); }

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ int quad_sum(int v) {
    v += dpp_i<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_i<0x4E>(v);   // quad_perm [2,3,0,1]
    return v;
}
// Sum over aligned groups of G lanes (4..64); every lane of the group gets the
// sum. Fixed data movement, so the float result is run-to-run identical.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    if constexpr (G >= 8) v += dpp_f<0x141>(v);   // row_half_mirror (values are quad-replicated by now)
    if constexpr (G >= 16) v += dpp_f<0x140>(v);  // row_mirror
    if constexpr (G >= 32) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // xor 16
    if constexpr (G >= 64)
        v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    return v;
}

// ---- activations -------------------------------------------------------------------
template <int PPL>
struct Act {
    uint32_t a[PPL][16];   // 64 Q8_K bytes of each owned pair
    float d[PPL];          // Q8_K scale of the pair's block
};
// COH: activations produced earlier in the same launch by other workgroups are
// read with agent-scope atomic loads (see coh_ld in xl_kernels.hip).
template <int LPR, int PPL, bool COH = false>
__device__ __forceinline__ void load_act(Act<PPL>& A, const int8_t* __restrict__ qs, const float* __restrict__ dq, int l) {
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int p = l + LPR * j;
        if constexpr (COH) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(qs + 64 * p);
#pragma unroll
            for (int c = 0; c < 16; ++c) A.a[j][c] = __hip_atomic_load(src + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            A.d[j] = __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(dq + (p >> 2)), __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT));
        } else {
            const uint4* src = reinterpret_cast<const uint4*>(qs + 64 * p);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4 t = src[c];
                A.a[j][4 * c + 0] = t.x; A.a[j][4 * c + 1] = t.y;
                A.a[j][4 * c + 2] = t.z; A.a[j][4 * c + 3] = t.w;
            }
            A.d[j] = dq[p >> 2];
        }
    }
}

// ---- raw rows: 6 words per pair, meaning by type --------------------------------------
//   IQ2_XXS: v0..3 = Q (16 B), v4 = d16
//   IQ2_XS : v0..3 = Q (16 B), v4 = scale bytes (u16), v5 = d16
//   IQ1_M  : v0..1 = Q (8 B), v2 = H (4 B), v3..4 = the block's 4 scale words
template <int PPL>
struct Raw {
    uint32_t v[PPL][6];
};

template <int LPR, int PPL>
__device__ __forceinline__ void load_raw(Raw<PPL>& r, int type, const MatRef& m, int row, int l) {
    const gptr base = (gptr)(m.base);   // generic -> global: bank planes are global memory
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int p = l + LPR * j;
        const uint64_t blk = uint64_t(row) * uint64_t(m.nb) + uint64_t(p >> 2);
        const int pp = p & 3;
        if (type == kIQ1_M) {
            const uint2 q = gload8(base + blk * 32 + pp * 8);
            const uint2 sw = gload8(base + m.off2 + blk * 8);
            r.v[j][0] = q.x; r.v[j][1] = q.y;
            r.v[j][2] = gload4(base + m.off1 + blk * 16 + pp * 4);
            r.v[j][3] = sw.x; r.v[j][4] = sw.y;
        } else {
            const uint4 w = gload16(base + blk * 64 + pp * 16);
            r.v[j][0] = w.x; r.v[j][1] = w.y; r.v[j][2] = w.z; r.v[j][3] = w.w;
            if (type == kIQ2_XXS) {
                r.v[j][4] = gload2(base + m.off1 + blk * 2);
            } else {
                r.v[j][4] = gload2(base + m.off1 + blk * 8 + pp * 2);
                r.v[j][5] = gload2(base + m.off2 + blk * 2);
            }
        }
    }
}
template <int PPL>
__device__ __forceinline__ void zero_raw(Raw<PPL>& r) {
#pragma unroll
    for (int j = 0; j < PPL; ++j)
#pragma unroll
        for (int i = 0; i < 6; ++i) r.v[j][i] = 0;
}

// ---- pair integers ------------------------------------------------------------------------
// One IQ2 group: grid row at byte offset goff, sign row selected by byte sb.
__device__ __forceinline__ int iq2_group(const uint8_t* lds, uint32_t goff, uint32_t sb, uint32_t a0, uint32_t a1, int acc) {
    const uint2 g = lds8(lds, goff);
    const uint4 m = lds16(lds, kLdsSign + (sb << 4));
    acc = dot4(xad(g.x, m.x, m.z), a0, acc);
    return dot4(xad(g.y, m.y, m.w), a1, acc);
}
// 2s+1 from the four scale bits stored in bit 7 of each sign byte.
__device__ __forceinline__ int xxs_scale(uint32_t signs) {
    return int(__builtin_amdgcn_udot4((signs >> 7) & 0x01010101u, 0x10080402u, 1u, false));
}
// IQ2_XXS pair: v0/v2 = 4 grid indices, v1/v3 = 4 sign bytes (scale bit 7).
__device__ __forceinline__ int pair_xxs(const uint8_t* lds, const uint32_t* v, const uint32_t* a) {
    int sa = 0, sb = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g)
        sa = iq2_group(lds, kLdsXXS + (((v[0] >> (8 * g)) & 255u) << 3), (v[1] >> (8 * g)) & 255u, a[2 * g], a[2 * g + 1], sa);
#pragma unroll
    for (int g = 0; g < 4; ++g)
        sb = iq2_group(lds, kLdsXXS + (((v[2] >> (8 * g)) & 255u) << 3), (v[3] >> (8 * g)) & 255u, a[8 + 2 * g], a[9 + 2 * g], sb);
    return mul24(sa, xxs_scale(v[1])) + mul24(sb, xxs_scale(v[3]));
}
// IQ2_XS pair: 8 codes {sign7 | grid9 << 7}, two per word; sc = the two scale bytes.
__device__ __forceinline__ int pair_xs(const uint8_t* lds, const uint32_t* v, uint32_t sc, const uint32_t* a) {
    int total = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        int lo = 0, hi = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t w = v[2 * s + g / 2];
            const uint32_t sh = 16 * (g & 1);
            const uint32_t goff = kLdsXS + (((w >> (sh + 7)) & 511u) << 3);
            const uint32_t sbyte = (w >> sh) & 255u;
            if (g < 2) lo = iq2_group(lds, goff, sbyte, a[8 * s + 2 * g], a[8 * s + 2 * g + 1], lo);
            else hi = iq2_group(lds, goff, sbyte, a[8 * s + 2 * g], a[8 * s + 2 * g + 1], hi);
        }
        const uint32_t byte = (sc >> (8 * s)) & 255u;
        total += mul24(lo, int(2u * (byte & 15u) + 1u)) + mul24(hi, int(2u * (byte >> 4) + 1u));
    }
    return total;
}
// IQ1_M pair: q0/q1 = 4 low index bytes per sub-block, h = a nibble per group
// (3 index bits + delta-sign bit), scw = the pair's u16 scale word. 8*main + delta.
__device__ __forceinline__ int pair_iq1(const uint8_t* lds, uint32_t q0, uint32_t q1, uint32_t h, uint32_t scw,
                                        const uint32_t* a) {
    int total = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const uint32_t qw = s ? q1 : q0;
        int lo = 0, hi = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t nib = (h >> (16 * s + 4 * g)) & 15u;
            const uint2 gr = lds8(lds, kLdsIQ1 + (nib << 11) + (((qw >> (8 * g)) & 255u) << 3));
            if (g < 2) lo = dot4(gr.y, a[8 * s + 2 * g + 1], dot4(gr.x, a[8 * s + 2 * g], lo));
            else hi = dot4(gr.y, a[8 * s + 2 * g + 1], dot4(gr.x, a[8 * s + 2 * g], hi));
        }
        total += mul24(lo, int(2u * ((scw >> (6 * s)) & 7u) + 1u)) + mul24(hi, int(2u * ((scw >> (6 * s + 3)) & 7u) + 1u));
    }
    return total;
}
__device__ __forceinline__ uint32_t iq1_scale_word(uint32_t sw0, uint32_t sw1, int pp) {
    return ((pp & 2) ? sw1 : sw0) >> (16 * (pp & 1));
}
__device__ __forceinline__ uint32_t iq1_d(uint32_t sw0, uint32_t sw1) {
    return ((sw0 >> 12) & 0xfu) | ((sw0 >> 24) & 0xf0u) | ((sw1 >> 4) & 0xf00u) | ((sw1 >> 16) & 0xf000u);
}

// Row value, replicated over the row group. With PART, lane 4q of the group
// also writes its block's exact integer (IQ1_M: 8 * main + delta).
template <int T, int LPR, int PPL, bool PART>
__device__ __forceinline__ float dot_raw_t(const Raw<PPL>& r, int row, int nb, int l, const Act<PPL>& A,
                                           const uint8_t* lds, int32_t* __restrict__ partials, bool valid) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int p = l + LPR * j;
        const uint32_t* v = r.v[j];
        int I;
        uint32_t d16;
        if constexpr (T == kIQ2_XXS) {
            I = pair_xxs(lds, v, A.a[j]);
            d16 = v[4];
        } else if constexpr (T == kIQ2_XS) {
            I = pair_xs(lds, v, v[4], A.a[j]);
            d16 = v[5];
        } else {
            I = pair_iq1(lds, v[0], v[1], v[2], iq1_scale_word(v[3], v[4], p & 3), A.a[j]);
            d16 = iq1_d(v[3], v[4]);
        }
        if constexpr (PART) {   // the block's integer as the value path forms it (IQ1_M: 8 * main + delta)
            const uint64_t blk = uint64_t(row) * uint64_t(nb) + uint64_t(p >> 2);
            const int ib = quad_sum(I);
            if (valid && (l & 3) == 0) partials[blk] = ib;
        }
        const float db = __fmul_rn(f16_to_f32(d16), A.d[j]);
        acc = fmaf(db, float(I), acc);
    }
    return __fmul_rn(0.125f, group_sum<LPR>(acc));
}
template <int LPR, int PPL, bool PART>
__device__ __forceinline__ float dot_raw(const Raw<PPL>& r, int type, int row, int nb, int l, const Act<PPL>& A,
                                         const uint8_t* lds, int32_t* __restrict__ partials, bool valid) {
    if (type == kIQ2_XXS) return dot_raw_t<kIQ2_XXS, LPR, PPL, PART>(r, row, nb, l, A, lds, partials, valid);
    if (type == kIQ2_XS) return dot_raw_t<kIQ2_XS, LPR, PPL, PART>(r, row, nb, l, A, lds, partials, valid);
    return dot_raw_t<kIQ1_M, LPR, PPL, PART>(r, row, nb, l, A, lds, partials, valid);
}

}  // namespace xl::dev
