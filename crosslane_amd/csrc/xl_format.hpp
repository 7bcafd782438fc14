// Block formats, fp16 conversion, the planar bank layout and the seeded block
// generator. Shared by host and device code; no HIP API calls here.
//
// Block formats follow ggml (MIT): IQ2_XXS (type 16, 66 B / 256 weights),
// IQ2_XS (type 17, 74 B), IQ1_M (type 29, 56 B) and the Q8_K activation block
// (292 B). Reference: engine/strata/sycl/moe/format.hpp:36-41,
// engine/strata/sycl/stage/wiring/q8k_core.hpp:13-14.
#pragma once
#include <cstddef>
#include <cstdint>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define XL_HD __host__ __device__ __forceinline__
#else
#define XL_HD inline
#endif

namespace xl {

enum : int { kIQ2_XXS = 16, kIQ2_XS = 17, kIQ1_M = 29 };
constexpr int kQK = 256;          // weights per super-block
constexpr int kSub = 32;          // weights per sub-block
constexpr int kQ8KBytes = 292;    // float d; int8 qs[256]; int16 bsums[16]

struct Q8K {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
};
static_assert(sizeof(Q8K) == 292, "Q8_K block is 292 bytes");
static_assert(offsetof(Q8K, qs) == 4 && offsetof(Q8K, bsums) == 260, "Q8_K field offsets");

XL_HD constexpr bool supported_type(int t) { return t == kIQ2_XXS || t == kIQ2_XS || t == kIQ1_M; }

// Dense formats of the shared-expert matrices (per32 rows only; stored as raw
// ggml blocks, row-major, no planar split): Q8_0 (34 B per 32 values), Q4_K
// (144 B per 256), Q5_K (176 B per 256), Q6_K (210 B per 256).
enum : int { kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14 };
XL_HD constexpr bool dense_type(int t) { return t == kQ8_0 || t == kQ4_K || t == kQ5_K || t == kQ6_K; }
XL_HD constexpr int dense_block_bytes(int t) {
    return t == kQ8_0 ? 34 : t == kQ4_K ? 144 : t == kQ5_K ? 176 : t == kQ6_K ? 210 : 0;
}
XL_HD constexpr int dense_block_values(int t) { return t == kQ8_0 ? 32 : 256; }
XL_HD constexpr int block_bytes(int t) {
    return t == kIQ2_XXS ? 66 : t == kIQ2_XS ? 74 : t == kIQ1_M ? 56 : 0;
}

XL_HD uint32_t f32_bits(float f) {
    union { float f; uint32_t u; } v; v.f = f; return v.u;
}
XL_HD float bits_f32(uint32_t u) {
    union { uint32_t u; float f; } v; v.u = u; return v.f;
}
XL_HD uint16_t rd16(const uint8_t* p) { return uint16_t(p[0] | (uint16_t(p[1]) << 8)); }
XL_HD void wr16(uint8_t* p, uint16_t v) { p[0] = uint8_t(v); p[1] = uint8_t(v >> 8); }

// Exact binary16 -> binary32 (every finite half is representable).
XL_HD float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 0) {
        // m * 2^-24 is exact in binary32; the sign is applied by bit so -0 stays -0.
        return bits_f32(sign | f32_bits(float(m) * 5.9604644775390625e-08f));
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

// binary32 -> binary16, round to nearest even. Subnormal halves are produced
// by one IEEE add against 0.5 (whose ulp is 2^-24), so host and device agree.
XL_HD uint16_t float_to_half(float f) {
    const uint32_t x = f32_bits(f);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return uint16_t(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // rounds to infinity
    if (ax < 0x38800000u) {                                  // below the smallest normal half
        const float r = bits_f32(ax) + 0.5f;                  // a lone add: nothing to contract
        return uint16_t(sign | (f32_bits(r) - 0x3f000000u));
    }
    const uint32_t r = ax - 0x38000000u + 0xfffu + ((ax >> 13) & 1u);
    return uint16_t(sign | (r >> 13));
}

// IQ1_M keeps its fp16 super-block scale in the top nibble of its four u16
// scale words (bytes 48..55). Reference: q8k_core.hpp:70-74.
XL_HD uint16_t iq1m_scale_bits(const uint8_t* sc8) {
    return uint16_t((rd16(sc8) >> 12) | ((rd16(sc8 + 2) >> 8) & 0x00f0u) |
                    ((rd16(sc8 + 4) >> 4) & 0x0f00u) | (rd16(sc8 + 6) & 0xf000u));
}

// ---------------------------------------------------------------------------
// Planar ("pair-planar") resident layout.
//
// A matrix of n rows x k columns holds NB = n*(k/256) blocks. The AoS ggml
// bytes are split into field planes, each row-major over [row][block]:
//   IQ2_XXS: Q = 8 sub-blocks x 8 B (4 grid indices + 4 sign/scale bytes) 64 B
//            D = fp16 scale                                               2 B
//   IQ2_XS : Q = 32 u16 codes (7-bit sign index | 9-bit grid << 7)      64 B
//            S = 8 scale bytes                                            8 B
//            D = fp16 scale                                               2 B
//   IQ1_M  : Q = 32 low index bytes                                      32 B
//            H = 16 high-bit / delta bytes                               16 B
//            M = 4 u16 scale words (scales + fp16 nibbles)                8 B
// Two consecutive sub-blocks (a "pair", 64 weights) are one 16-byte load in Q
// for the IQ2 types. Each plane starts on a 256-byte boundary; for the
// benchmark shapes no padding is needed, so the plane bytes equal the AoS bytes.
// ---------------------------------------------------------------------------
XL_HD constexpr uint64_t align256(uint64_t v) { return (v + 255u) & ~uint64_t(255u); }

struct PlaneLayout {
    uint64_t off[3];    // byte offset of planes 0..2 inside the matrix allocation
    uint32_t width[3];  // bytes per block in each plane (0 = unused)
    uint64_t bytes;     // allocation size (multiple of 256)
};

XL_HD PlaneLayout plane_layout(int type, uint64_t nblocks) {
    PlaneLayout L{};
    uint32_t w0 = 0, w1 = 0, w2 = 0;
    if (type == kIQ2_XXS) { w0 = 64; w1 = 2; w2 = 0; }
    else if (type == kIQ2_XS) { w0 = 64; w1 = 8; w2 = 2; }
    else if (type == kIQ1_M) { w0 = 32; w1 = 16; w2 = 8; }
    L.width[0] = w0; L.width[1] = w1; L.width[2] = w2;
    uint64_t at = 0;
    L.off[0] = at; at = align256(at + w0 * nblocks);
    L.off[1] = at; at = align256(at + w1 * nblocks);
    L.off[2] = at; at = align256(at + w2 * nblocks);
    L.bytes = at;
    return L;
}

// Field re-encodings applied by the repack (lossless, same byte count). They
// put every codebook index of a group where one SDWA byte select reaches it:
//   IQ2_XXS aux word: AoS {sign0..3 at bits 7g..7g+6, scale at 28..31} becomes
//     four bytes, byte g = sign_g | (bit g of scale) << 7.
//   IQ2_XS code u16: AoS {grid9 | sign7 << 9} becomes {sign7 | grid9 << 7}.
// IQ1_M is stored as in ggml.
XL_HD uint32_t xxs_aux_to_planar(uint32_t aux) {
    uint32_t out = 0;
    for (int g = 0; g < 4; ++g)
        out |= (((aux >> (7 * g)) & 127u) | (((aux >> (28 + g)) & 1u) << 7)) << (8 * g);
    return out;
}
XL_HD uint32_t xxs_aux_from_planar(uint32_t v) {
    uint32_t out = 0;
    for (int g = 0; g < 4; ++g) {
        const uint32_t b = (v >> (8 * g)) & 255u;
        out |= ((b & 127u) << (7 * g)) | ((b >> 7) << (28 + g));
    }
    return out;
}
XL_HD uint16_t xs_code_to_planar(uint16_t c) { return uint16_t((c >> 9) | ((c & 511u) << 7)); }
XL_HD uint16_t xs_code_from_planar(uint16_t c) { return uint16_t(((c >> 7) & 511u) | ((c & 127u) << 9)); }
XL_HD uint32_t rd32(const uint8_t* p) { return uint32_t(rd16(p)) | (uint32_t(rd16(p + 2)) << 16); }
XL_HD void wr32(uint8_t* p, uint32_t v) { wr16(p, uint16_t(v)); wr16(p + 2, uint16_t(v >> 16)); }

// Scatter one AoS block (index blk of the matrix) into the planes at base.
XL_HD void block_to_planes(int type, const uint8_t* aos, uint8_t* base, const PlaneLayout& L, uint64_t blk) {
    uint8_t* q = base + L.off[0] + L.width[0] * blk;
    uint8_t* p1 = base + L.off[1] + L.width[1] * blk;
    uint8_t* p2 = base + L.off[2] + L.width[2] * blk;
    if (type == kIQ2_XXS) {
        for (int c = 0; c < 8; ++c) {
            for (int i = 0; i < 4; ++i) q[8 * c + i] = aos[2 + 8 * c + i];
            wr32(q + 8 * c + 4, xxs_aux_to_planar(rd32(aos + 6 + 8 * c)));
        }
        p1[0] = aos[0]; p1[1] = aos[1];
    } else if (type == kIQ2_XS) {
        for (int i = 0; i < 32; ++i) wr16(q + 2 * i, xs_code_to_planar(rd16(aos + 2 + 2 * i)));
        for (int i = 0; i < 8; ++i) p1[i] = aos[66 + i];
        p2[0] = aos[0]; p2[1] = aos[1];
    } else {
        for (int i = 0; i < 32; ++i) q[i] = aos[i];
        for (int i = 0; i < 16; ++i) p1[i] = aos[32 + i];
        for (int i = 0; i < 8; ++i) p2[i] = aos[48 + i];
    }
}

XL_HD void planes_to_block(int type, const uint8_t* base, const PlaneLayout& L, uint64_t blk, uint8_t* aos) {
    const uint8_t* q = base + L.off[0] + L.width[0] * blk;
    const uint8_t* p1 = base + L.off[1] + L.width[1] * blk;
    const uint8_t* p2 = base + L.off[2] + L.width[2] * blk;
    if (type == kIQ2_XXS) {
        aos[0] = p1[0]; aos[1] = p1[1];
        for (int c = 0; c < 8; ++c) {
            for (int i = 0; i < 4; ++i) aos[2 + 8 * c + i] = q[8 * c + i];
            wr32(aos + 6 + 8 * c, xxs_aux_from_planar(rd32(q + 8 * c + 4)));
        }
    } else if (type == kIQ2_XS) {
        aos[0] = p2[0]; aos[1] = p2[1];
        for (int i = 0; i < 32; ++i) wr16(aos + 2 + 2 * i, xs_code_from_planar(rd16(q + 2 * i)));
        for (int i = 0; i < 8; ++i) aos[66 + i] = p1[i];
    } else {
        for (int i = 0; i < 32; ++i) aos[i] = q[i];
        for (int i = 0; i < 16; ++i) aos[32 + i] = p1[i];
        for (int i = 0; i < 8; ++i) aos[48 + i] = p2[i];
    }
}

// ---------------------------------------------------------------------------
// Seeded counter-based block generator: the bytes of block `blk` of matrix
// (layer, expert, role) are a pure function of (seed, layer, expert, role, blk),
// so the device can fill a 100+ GB bank in place while a CPU check regenerates
// any single expert. All bit fields of the three formats span full power-of-two
// ranges, so uniform bytes give uniform grid indices, sign indices, sub-scales
// and delta bits; the fp16 super-block scale d is drawn from U(1e-3, 1e-2).
// Mixing function: the splitmix64 finalizer (Steele, Lea & Flood 2014).
// ---------------------------------------------------------------------------
XL_HD uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
XL_HD uint64_t gen_key(uint64_t seed, uint32_t layer, uint32_t expert, uint32_t role) {
    return mix64(seed ^ mix64((uint64_t(layer) << 40) ^ (uint64_t(expert) << 8) ^ uint64_t(role)));
}
XL_HD uint64_t gen_word(uint64_t key, uint64_t blk, uint32_t j) {
    return mix64(key + (blk * 16u + j) * 0xD1B54A32D192ED03ull);
}
// d = 1e-3 + u * (9e-3 / 2^24), u uniform in [0, 2^24), rounded to fp16.
XL_HD uint16_t gen_scale(uint64_t word) {
    const float u = float(uint32_t(word >> 40));
#if defined(__HIP_DEVICE_COMPILE__)
    const float t = __fmul_rn(u, 9e-3f * 5.9604644775390625e-08f);
    const float v = __fadd_rn(1e-3f, t);
#else
    volatile float t = u * (9e-3f * 5.9604644775390625e-08f);
    const float v = 1e-3f + t;
#endif
    return float_to_half(v);
}
// Writes block_bytes(type) bytes of AoS block `blk` to out.
XL_HD void gen_block(int type, uint64_t key, uint64_t blk, uint8_t* out) {
    const int nbytes = block_bytes(type);
    for (int j = 0; j * 8 < nbytes; ++j) {
        const uint64_t w = gen_word(key, blk, uint32_t(j));
        for (int b = 0; b < 8 && j * 8 + b < nbytes; ++b) out[j * 8 + b] = uint8_t(w >> (8 * b));
    }
    const uint16_t d = gen_scale(gen_word(key, blk, 15));
    if (type != kIQ1_M) {
        wr16(out, d);
    } else {
        for (int q = 0; q < 4; ++q) {
            const uint16_t s = uint16_t((rd16(out + 48 + 2 * q) & 0x0fffu) | (((d >> (4 * q)) & 15u) << 12));
            wr16(out + 48 + 2 * q, s);
        }
    }
}

}  // namespace xl
