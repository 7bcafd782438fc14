// Row decoding of the streaming layer kernels (xl_stream*.hip),
// gfx950: perm-addressed, bank-interleaved LDS codebook copies, IQ2 sign masks
// applied to the activations or to the grid, IQ1_M value rows, the Q8_K
// quantizer of several blocks at once, and the sentinel h exchange words.
#pragma once
#include <hip/hip_runtime.h>

#include <utility>

#include "xl_dev.hpp"

namespace xl::dev {
namespace {

// f.template operator()<J>() for J = 0 .. N-1: the index is a constant in the
// body, so ring slots indexed by it stay in registers (a runtime loop index,
// even of a loop unrolled later, leaves them to memory).
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    [&]<int... Js>(std::integer_sequence<int, Js...>) { (f.template operator()<Js>(), ...); }(std::make_integer_sequence<int, N>{});
}

// Lane constants of the lookups: byte 0 is the lane's copy offset, byte 2 the
// table base in 64-KB units; v_perm_b32 puts the index byte in byte 1.
__device__ __forceinline__ uint32_t perm(uint32_t idx_word, uint32_t lane_word, uint32_t sel) {
    return __builtin_amdgcn_perm(idx_word, lane_word, sel);
}
// selector: byte0 <- lane_word.byte0, byte1 <- idx_word.byte(q), byte2 <- lane_word.byte2, byte3 <- 0
__device__ __forceinline__ constexpr uint32_t sel_b(int q) { return 0x0C020400u + (uint32_t(q) << 8); }

constexpr uint32_t kSentinel = 0xffffffffu;
constexpr uint32_t kQNaN = 0x7fc00000u;

// Sign row r: M has 0xff in the bytes of negative weights (7 sign bits of r
// plus their parity, as ksigns_iq2xs). Two ways to apply it, one op per dword:
// select between a and -a (v_bfi_b32: the activation takes the sign), or
// (g ^ M) + (M & 0x01010101), which negates exactly those bytes of g (grid
// bytes are 1..127, so no carry crosses a byte).
__device__ __forceinline__ uint2 sign_row(uint32_t r) {
    const uint32_t s7 = r & 127u;
    const uint32_t s8 = s7 | ((__builtin_popcount(s7) & 1u) << 7);
    const uint32_t clo = ((s8 & 15u) * 0x00204081u) & 0x01010101u;
    const uint32_t chi = ((s8 >> 4) * 0x00204081u) & 0x01010101u;
    return make_uint2(clo * 255u, chi * 255u);
}
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t x, uint32_t y) { return (m & x) | (~m & y); }   // v_bfi_b32
// Bytewise two's-complement negation: (~x + 1) per byte = (x ^ 0xff..) + 0x01.. with no
// carry across bytes except for a 0x00 byte, whose carry is masked off byte by byte.
__device__ __forceinline__ uint32_t neg_bytes(uint32_t x) {
    const uint32_t lo = ((x & 0x00ff00ffu) ^ 0x00ff00ffu) + 0x00010001u;   // bytes 0, 2 (a carry lands in 1, 3)
    const uint32_t hi = ((x & 0xff00ff00u) ^ 0xff00ff00u) + 0x01000100u;   // bytes 1, 3
    return (lo & 0x00ff00ffu) | (hi & 0xff00ff00u);
}

// (x ^ y) + z as one v_xad_u32: inside the unrolled decoders the compiler emits
// v_xor_b32 and v_add_u32 for it.
__device__ __forceinline__ uint32_t xad_op(uint32_t x, uint32_t y, uint32_t z) {
    uint32_t r;
    asm("v_xad_u32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(y), "v"(z));
    return r;
}
// The grid bytes with the sign mask M applied: (g ^ M) + (M & 0x01010101).
__device__ __forceinline__ uint32_t signed_grid(uint32_t g, uint32_t m) { return xad_op(g, m, m & 0x01010101u); }
// The first v_dot4 of a chain, in the VOP3P form with a zero accumulator (the
// compiler's v_dot4c ties the accumulator to the result and needs a v_mov of 0).
__device__ __forceinline__ int sdot4_0(uint32_t a, uint32_t b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// ---- pair decoders -------------------------------------------------------------------------
// Codebook rows of one pair: 8 grid rows and 8 sign masks. The decoders are
// split into lookups and arithmetic so that a slot issues both of its rows'
// lookups before either row's arithmetic waits on them.
struct Looks {
    uint2 g[8], m[8];
};
// IQ2_XXS pair (w0..3: two sub-blocks of {4 grid bytes, 4 sign|scale-bit bytes}).
// The *_to forms write the caller's Looks field by field, so that a decoder
// chosen at run time among several leaves every field in a register.
__device__ __forceinline__ void look_xxs_to(Looks& L, const uint8_t* lds, uint32_t lo_g, uint32_t lo_s, const uint32_t* w) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            // sign row first: every *_to form's last write is L.g[7], so that the
            // compiler's merging of the branches' last lookups keeps one destination
            L.m[4 * s + q] = *reinterpret_cast<const uint2*>(lds + perm(w[2 * s + 1], lo_s, sel_b(q)));
            L.g[4 * s + q] = *reinterpret_cast<const uint2*>(lds + perm(w[2 * s], lo_g, sel_b(q)));
        }
}
__device__ __forceinline__ Looks look_xxs(const uint8_t* lds, uint32_t lo_g, uint32_t lo_s, const uint32_t* w) {
    Looks L;
    look_xxs_to(L, lds, lo_g, lo_s, w);
    return L;
}
// Against 64 Q8_K quants a (and their negations na): the exact integer sum of
// (2s+1) * grid * sign * q over the pair (q8k_core.hpp:96-114 regrouped per
// sub-block; the sign is applied to q).
__device__ __forceinline__ int sum_xxs(const Looks& L, const uint32_t* w, const uint32_t* a, const uint32_t* na) {
    int acc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = 4 * s + q, k0 = 8 * s + 2 * q;
            const uint32_t v = bfi(L.m[e].x, na[k0], a[k0]);
            acc[s] = q == 0 ? sdot4_0(L.g[e].x, v) : sdot4(L.g[e].x, v, acc[s]);
            acc[s] = sdot4(L.g[e].y, bfi(L.m[e].y, na[k0 + 1], a[k0 + 1]), acc[s]);
        }
    return __mul24(acc[0], xxs_sc(w[1])) + __mul24(acc[1], xxs_sc(w[3]));
}
// IQ2_XS pair (w0..3: 8 codes {sign7 | grid9 << 7}, sc: the pair's two scale
// bytes): the exact integer sum with the 16-weight scales (q8k_core.hpp:116-140).
// Split like the IQ2_XXS decoder, so that a pass issues the next pair's
// lookups before the current pair's arithmetic waits on its own.
__device__ __forceinline__ void look_xs_to(Looks& L, const uint8_t* lds, uint32_t lo_x, uint32_t lo_s, const uint32_t* w) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t h = e & 1;
        // grid row * 32 = (code >> 7) << 5: one shift and one v_and_or_b32 with the lane's copy
        const uint32_t sh = h ? (w[e >> 1] >> 18) : (w[e >> 1] >> 2);
        L.m[e] = *reinterpret_cast<const uint2*>(lds + perm(w[e >> 1], lo_s, sel_b(2 * h)));
        L.g[e] = *reinterpret_cast<const uint2*>(lds + ((sh & 0x3fe0u) | lo_x));
    }
}
__device__ __forceinline__ Looks look_xs(const uint8_t* lds, uint32_t lo_x, uint32_t lo_s, const uint32_t* w) {
    Looks L;
    look_xs_to(L, lds, lo_x, lo_s, w);
    return L;
}
__device__ __forceinline__ int sum_xs(const Looks& L, uint32_t sc, const uint32_t* a) {
    // the four 16-weight scales 2 n + 1, two per word: byte s of t1 from the low
    // nibble of scale byte s, byte s of t2 from its high nibble (sc < 2^16)
    const uint32_t t1 = ((sc << 1) & 0x1e1eu) | 0x0101u;
    const uint32_t t2 = ((sc >> 3) & 0x1e1eu) | 0x0101u;
    int total = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        int part[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {   // 16 weights: groups 4 s + 2 h and 4 s + 2 h + 1
            const int e = 4 * s + 2 * h, k0 = 8 * s + 4 * h;
            int acc = sdot4_0(signed_grid(L.g[e].x, L.m[e].x), a[k0]);
            acc = sdot4(signed_grid(L.g[e].y, L.m[e].y), a[k0 + 1], acc);
            acc = sdot4(signed_grid(L.g[e + 1].x, L.m[e + 1].x), a[k0 + 2], acc);
            part[h] = sdot4(signed_grid(L.g[e + 1].y, L.m[e + 1].y), a[k0 + 3], acc);
        }
        total += __mul24(part[0], int((t1 >> (8 * s)) & 255u)) + __mul24(part[1], int((t2 >> (8 * s)) & 255u));
    }
    return total;
}

// IQ2_XXS pair with the signs applied to the grid bytes instead of the
// activations ((g ^ M) + (M & 0x01010101), no negated activations needed): the
// same integer as sum_xxs.
__device__ __forceinline__ int sum_xxs_g(const Looks& L, const uint32_t* w, const uint32_t* a) {
    int acc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = 4 * s + q, k0 = 8 * s + 2 * q;
            const uint32_t v = signed_grid(L.g[e].x, L.m[e].x);
            acc[s] = q == 0 ? sdot4_0(v, a[k0]) : sdot4(v, a[k0], acc[s]);
            acc[s] = sdot4(signed_grid(L.g[e].y, L.m[e].y), a[k0 + 1], acc[s]);
        }
    return __mul24(acc[0], xxs_sc(w[1])) + __mul24(acc[1], xxs_sc(w[3]));
}

// IQ1_M. The value rows sit at LDS byte 0: row (nib << 8 | idx_lo) holds the 8
// bytes 8 * grid + delta of the 11-bit grid index (nib & 7) << 8 | idx_lo, delta
// -1 when bit 3 of the group's nibble is set, else +1 (kTableIQ1X). One lookup
// and two v_dot4 give a group's exact 8 * main + delta integer. The lookup
// address (nib << 8 | idx_lo) << 3 is one v_perm_b32 of the index byte and the
// nibble byte, then one shift.
// Pair (Raw3): w0, w1 = the low index bytes of sub-blocks 0 and 1, w2 = the
// eight groups' nibbles (group 4 s + g at bits 16 s + 4 g), w3, w4 = the
// block's scale words.
__device__ __forceinline__ void look_iq1_to(Looks& L, const uint8_t* lds, const uint32_t* w) {
    const uint32_t ne = w[2] & 0x0f0f0f0fu;          // nibbles 0, 2, 4, 6 in bytes 0 .. 3
    const uint32_t no = (w[2] >> 4) & 0x0f0f0f0fu;   // nibbles 1, 3, 5, 7
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = 4 * s + g;
            // byte 0 <- index byte g of w[s], byte 1 <- nibble n, bytes 2, 3 <- 0
            const uint32_t r = __builtin_amdgcn_perm((n & 1) ? no : ne, w[s],
                                                     0x0C0C0000u | (uint32_t(4 + (n >> 1)) << 8) | uint32_t(g));
            L.g[n] = *reinterpret_cast<const uint2*>(lds + (r << 3));
        }
}
// Against 64 Q8_K quants a: the exact pair integer, sum over the four 16-weight
// groups of (2 sc + 1) * (8 * main + delta) (q8k_core.hpp's IQ1_M terms times
// 8); scw = the pair's 16-bit scale word (3 bits per 16 weights).
__device__ __forceinline__ int sum_iq1(const Looks& L, uint32_t scw, const uint32_t* a) {
    int total = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        int lo, hi;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            int& acc = g < 2 ? lo : hi;
            acc = (g & 1) ? sdot4(L.g[4 * s + g].x, a[8 * s + 2 * g], acc) : sdot4_0(L.g[4 * s + g].x, a[8 * s + 2 * g]);
            acc = sdot4(L.g[4 * s + g].y, a[8 * s + 2 * g + 1], acc);
        }
        total += __mul24(lo, int(2u * ((scw >> (6 * s)) & 7u) + 1u)) + __mul24(hi, int(2u * ((scw >> (6 * s + 3)) & 7u) + 1u));
    }
    return total;
}
// The pair's scale word (pair pp of its block) and the block's fp16 scale.
__device__ __forceinline__ uint32_t iq1_scw(const uint32_t* w, int pp) { return ((pp & 2) ? w[4] : w[3]) >> (16 * (pp & 1)); }
__device__ __forceinline__ uint32_t iq1_d16(const uint32_t* w) {
    return ((w[3] >> 12) & 0xfu) | ((w[3] >> 24) & 0xf0u) | ((w[4] >> 4) & 0xf00u) | ((w[4] >> 16) & 0xf000u);
}

template <int P>
struct Act {
    uint32_t a[P][16];
    float d[P];
};
// Activations of pairs lp, lp + L, ... from a Q8_K vector in LDS (quants at
// base, block scales at base + scl).
template <int P>
__device__ __forceinline__ void load_act(Act<P>& A, const uint8_t* lds, int base, int scl, int lp, int L) {
#pragma unroll
    for (int q = 0; q < P; ++q) {
        const int p = lp + L * q;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 v = *reinterpret_cast<const uint4*>(lds + base + qswz(64 * p + 16 * c));
            A.a[q][4 * c] = v.x; A.a[q][4 * c + 1] = v.y; A.a[q][4 * c + 2] = v.z; A.a[q][4 * c + 3] = v.w;
        }
        A.d[q] = reinterpret_cast<const float*>(lds + base + scl)[p >> 2];
    }
}

// Coherent (sc1) 16-byte load of 4 h words; a sentinel word means "not yet".
__device__ __forceinline__ uint4 h_load(const float* hb, uint32_t word) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)hb, (short)0, -1, 0x00020000);
    const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(rs, word * 4, 0, 16);   // per-lane offset: voffset
    return make_uint4(v.x, v.y, v.z, v.w);
}
// The sentinel is the largest 32-bit value: no word holds it iff their maximum is below it.
__device__ __forceinline__ bool h_ready(const uint4& v) {
    return max(max(v.x, v.y), max(v.z, v.w)) != kSentinel;
}

// ---- Q8_K of NB blocks at once ---------------------------------------------------------------
// Block m is held by the wave as v[m] (lane l owns values 4l..4l+3). Bit-exact
// with q8k_core.hpp:30-38 on every finite input: mx is the first value of
// largest magnitude (found as the wave's largest magnitude, then the lowest
// position holding it), is = -127/mx, q = min(127, nearest(is * v)), d = 1/is;
// an all-zero block gives d = 0 and q = 0. The two divisions run once for all
// NB blocks (lane m divides for block m). nearest is the reference's own
// (q8k_core.hpp:25-29): the quant byte is the low byte of the bits of
// is * v + 12582912, and four of them are packed by two v_perm_b32.
// One DPP max step on every block at once: the NB chains are independent, so
// each fills the others' DPP wait states. old = 0 is max's identity, which lets
// the compiler fold the move into v_max_u32_dpp.
template <int CTRL, int RM, int NB>
__device__ __forceinline__ void umax_dpp_n(uint32_t (&a)[NB]) {
#pragma unroll
    for (int m = 0; m < NB; ++m) a[m] = max(a[m], uint32_t(__builtin_amdgcn_update_dpp(0, int(a[m]), CTRL, RM, 0xF, false)));
}
// The wave's largest magnitude of each block, as a bit pattern: magnitudes of
// floats order as their bits do, so integer max needs no NaN canonicalization
// (a NaN or an infinity wins and is caught by the finiteness test on the result).
template <int NB>
__device__ __forceinline__ void wave_umax_n(uint32_t (&a)[NB], uint32_t (&out)[NB]) {
    umax_dpp_n<0xB1, 0xF>(a);
    umax_dpp_n<0x4E, 0xF>(a);
    umax_dpp_n<0x141, 0xF>(a);
    umax_dpp_n<0x140, 0xF>(a);   // every lane: its row's max
    umax_dpp_n<0x142, 0xA>(a);   // rows 1, 3
    umax_dpp_n<0x143, 0xC>(a);   // rows 2, 3
#pragma unroll
    for (int m = 0; m < NB; ++m) out[m] = uint32_t(__builtin_amdgcn_readlane(int(a[m]), 63));
}
// Returns false if a value of blocks 0..nvalid-1 is not finite (the others may hold anything).
// With is finite, |is * v| <= 127 (1 + 2^-24)^2 < 127.5 for every v of the block,
// so nearest(is * v) lies in -127..127, the reference's min(127, .) never applies
// and the low byte is q's two's-complement byte. A block whose largest magnitude
// is below 127 / FLT_MAX (subnormal or tiny) has is = -inf or +inf: is * v is
// infinite (or NaN for v = 0), nearest gives -2^22 (or 0), the reference's int8
// cast keeps the low byte 0, and so does the bit pattern of inf + 12582912 (or
// NaN) here; d = 1/is is then -0 or +0, as the reference's.
template <int NB>
__device__ __forceinline__ bool q8k_blocks(const uint4 (&hv)[NB], int nvalid, int lane, uint32_t (&packed)[NB],
                                           float (&d)[NB]) {
    bool fin = true;
    uint32_t x[NB][4], ab[NB][4], am[NB], mxa[NB];
#pragma unroll
    for (int m = 0; m < NB; ++m) {
        // opaque copies: a select chain over the block's words would otherwise be
        // turned into an indexed load from a stack copy of the block
        x[m][0] = hv[m].x; x[m][1] = hv[m].y; x[m][2] = hv[m].z; x[m][3] = hv[m].w;
        asm volatile("" : "+v"(x[m][0]), "+v"(x[m][1]), "+v"(x[m][2]), "+v"(x[m][3]));
#pragma unroll
        for (int i = 0; i < 4; ++i) ab[m][i] = x[m][i] & 0x7fffffffu;
        mxa[m] = max(max(ab[m][0], ab[m][1]), max(ab[m][2], ab[m][3]));
    }
    wave_umax_n<NB>(mxa, am);
    float mxv = 0.0f;
#pragma unroll
    for (int m = 0; m < NB; ++m) {
        fin = fin & ((m >= nvalid) | (am[m] <= 0x7f7fffffu));
        // mx: the magnitude am[m] with the sign of the block's first value of that
        // magnitude: each lane's first such value (a select chain in reverse
        // order), then the first lane holding one (a ballot); no branch
        uint32_t lv = 0u;
#pragma unroll
        for (int i = 3; i >= 0; --i) lv = ab[m][i] == am[m] ? x[m][i] : lv;
        const uint64_t hit = __builtin_amdgcn_ballot_w64((ab[m][0] == am[m]) | (ab[m][1] == am[m]) |
                                                         (ab[m][2] == am[m]) | (ab[m][3] == am[m]));
        const int first = int(__builtin_ctzll(hit | (uint64_t(1) << 63)));
        const float mx = __uint_as_float(am[m] | (uint32_t(__builtin_amdgcn_readlane(int(lv), first)) & 0x80000000u));
        mxv = lane == m ? mx : mxv;
    }
    const float isv = __fdiv_rn(-127.0f, mxv);
    const float dv = __fdiv_rn(1.0f, isv);
#pragma unroll
    for (int m = 0; m < NB; ++m) {
        const float is = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(isv), m));
        uint32_t f[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) f[j] = __float_as_uint(__fadd_rn(__fmul_rn(is, __uint_as_float(x[m][j])), 12582912.0f));
        // bytes 0, 1 <- low bytes of f0, f1; bytes 2, 3 <- low bytes of f2, f3
        const uint32_t lo = __builtin_amdgcn_perm(f[1], f[0], 0x0C0C0400u);
        const uint32_t hi = __builtin_amdgcn_perm(f[3], f[2], 0x04000C0Cu);
        // an all-zero block: d = 0 and q = 0 as the reference's early return (not
        // 1/is = -0 and the bytes of NaN products). The readlane stays outside the
        // select: a select over it becomes a branch (a convergent call is not
        // speculated), which splits the caller's code
        const float dm = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dv), m));
        const bool zero = am[m] == 0u;
        packed[m] = zero ? 0u : lo | hi;
        d[m] = zero ? 0.0f : dm;
    }
    return fin;
}

}  // namespace
}  // namespace xl::dev
