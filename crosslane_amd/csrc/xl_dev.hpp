// Device helpers shared by the single-launch layer kernels (xl_layer.hip,
// xl_stream.hip): coherent exchange words, DPP reductions, the Q8_K block
// quantizer, planar pair loads and LDS barriers. gfx950 only.
#pragma once
#include <hip/hip_runtime.h>

#include "xl_format.hpp"
#include "xl_internal.hpp"

namespace xl::dev {

typedef const __attribute__((address_space(1))) uint8_t* g8;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Agent-scope (device-coherent) accesses for data exchanged inside one launch.
__device__ __forceinline__ uint64_t coh_ld64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_st64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t coh_ld32(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coh_st32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tag_word(uint32_t bits, uint32_t epoch) { return uint64_t(bits) | (uint64_t(epoch) << 32); }

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4(int(a), int(b), c, false); }
__device__ __forceinline__ uint32_t xad(uint32_t a, uint32_t b, uint32_t c) { return (a ^ b) + c; }   // v_xad_u32
__device__ __forceinline__ float h2f(uint32_t h) { return float(__builtin_bit_cast(_Float16, uint16_t(h))); }
__device__ __forceinline__ float h2f(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over aligned groups of G lanes (G in 4..64) by DPP adds only (no LDS
// traffic); the group's sum lands in the group's last lane (for G <= 16 in
// every lane of the group). A fixed data movement, so run-to-run identical.
template <int G>
__device__ __forceinline__ float gsum(float v) {
    v += dppf<0xB1>(v);                                            // quad_perm [1,0,3,2]
    v += dppf<0x4E>(v);                                            // quad_perm [2,3,0,1]
    if constexpr (G >= 8) v += dppf<0x141>(v);                     // row_half_mirror
    if constexpr (G >= 16) v += dppf<0x140>(v);                    // row_mirror
    if constexpr (G >= 32)                                         // row_bcast:15 into rows 1 and 3
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    if constexpr (G >= 64)                                         // row_bcast:31 into rows 2 and 3
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
    return v;
}

// s_waitcnt immediate for "vector memory counter <= n" (gfx9 encoding; the
// export and LDS/scalar counters are left unconstrained).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// ---- Q8_K of one 256-value block by one wave (lane l owns values 4l..4l+3).
// Bit-exact restatement of engine/strata/sycl/stage/wiring/q8k_core.hpp:30-38:
// mx is the first value of largest magnitude (strict '>' scan), is = -127/mx,
// q = min(127, nearest(is * v)), d = 1/is; an all-zero block gives d = 0, q = 0.
struct Q8Lane {
    uint32_t packed;   // this lane's 4 quants
    float d;
    bool finite;
};
__device__ __forceinline__ int nearest_rn(float x) {
    const float v = __fadd_rn(x, 12582912.0f);   // q8k_core.hpp:25-29
    return int(__float_as_uint(v) & 0x007fffffu) - 0x00400000;
}
// The block's (value, index) of largest magnitude, lowest index on ties: the
// combine is associative and commutative, so the DPP tree gives the same
// winner as the reference's sequential scan.
__device__ __forceinline__ void amax_pick(float& m, int& i, float m2, int i2) {
    const float a = fabsf(m), a2 = fabsf(m2);
    const bool take = (a2 > a) | ((a2 == a) & (i2 < i));   // bitwise: selects, no branches
    m = take ? m2 : m;
    i = take ? i2 : i;
}
template <int CTRL>
__device__ __forceinline__ void amax_step(float& m, int& i) {
    amax_pick(m, i, dppf<CTRL>(m), __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ Q8Lane q8k_lane(const float v[4], int lane) {
    float mx = 0.0f;
    int idx = 4 * lane;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        finite = finite && (fabsf(v[j]) <= 3.402823466e38f);
        if (fabsf(v[j]) > fabsf(mx)) { mx = v[j]; idx = 4 * lane + j; }
    }
    amax_step<0xB1>(mx, idx);
    amax_step<0x4E>(mx, idx);
    amax_step<0x141>(mx, idx);
    amax_step<0x140>(mx, idx);   // every lane of a 16-lane row holds the row's pick
#pragma unroll
    for (int r = 1; r < 4; ++r)
        amax_pick(mx, idx, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 16 * r)),
                  __builtin_amdgcn_readlane(idx, 16 * r));
    mx = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(mx)));   // row 0's lanes now hold the block's pick
    Q8Lane r{0u, 0.0f, !__any(!finite)};
    if (mx != 0.0f) {
        const float is = __fdiv_rn(-127.0f, mx);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int q = nearest_rn(__fmul_rn(is, v[j]));
            q = q < 127 ? q : 127;
            r.packed |= uint32_t(uint8_t(int8_t(q))) << (8 * j);
        }
        r.d = __fdiv_rn(1.0f, is);
    }
    return r;
}

// Q8_K quants staged in LDS: byte o of a row sits at qswz(o), the 16-byte
// chunk index XORed with bits 1-2 of the pair (64-byte) index, so that lanes
// reading consecutive pairs hit different banks.
__device__ __forceinline__ int qswz(int o) { return o ^ (((o >> 7) & 3) << 4); }

// SwiGLU limit (q8k_core.hpp:92-93, the pack's swiglu_limit): with lim > 0,
// g = min(g, lim) and u = min(max(u, -lim), lim) before the product.
__device__ __forceinline__ void swiglu_clamp(float& g, float& u, float lim) {
    if (lim > 0.0f) {
        g = fminf(g, lim);
        u = fminf(fmaxf(u, -lim), lim);
    }
}

__device__ __forceinline__ float silu_mul3(float g, float u, float lim) {
    // q8k_core.hpp:92-95: (g / (1 + exp(-g))) * u after the limit
    swiglu_clamp(g, u, lim);
    const float e = expf(-g);
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}


// Raw words of one pair (64 weights) of one row, meaning by type:
//   IQ2_XXS: w0..3 = 16 B of Q (2 sub-blocks x {4 grid bytes, 4 sign|scale-bit bytes}), h0 = d16
//   IQ2_XS : w0..3 = 8 codes {sign7 | grid9 << 7}, h0 = the pair's two scale bytes, h1 = d16
//   IQ1_M  : w0..1 = 8 low index bytes, w2 = 8 nibbles (3 index bits + delta sign), w3..4 = block scale words
// The 16-bit loads stay 16-bit until used: widening them where they are loaded
// would make the load's wave wait for it (and for every load before it).
struct Raw3 {
    uint32_t w[7];
    uint16_t h[2];
};
// Plane offsets of a matrix of NB blocks (plane_layout in xl_format.hpp).
__device__ __forceinline__ void plane_offs(int type, uint64_t NB, uint32_t& o1, uint32_t& o2) {
    const uint64_t w0 = type == kIQ1_M ? 32 : 64;
    const uint64_t w1 = type == kIQ2_XXS ? 2 : type == kIQ2_XS ? 8 : 16;
    const uint64_t a1 = align256(w0 * NB);
    o1 = uint32_t(a1);
    o2 = uint32_t(align256(a1 + w1 * NB));
}
// A matrix as the kernel addresses it: planes at base, base + o1, base + o2
// (one matrix is far below 4 GB, so plane and row offsets are 32-bit).
struct MRef {
    const uint8_t* base;
    uint32_t o1, o2;
    int type, nb;
};
// Lane-constant byte offsets of pair p of the lane's row (rG rows below the row
// group's first row) in each plane: weight loads are buffer loads whose
// per-lane offset never changes and whose row-group offset is scalar, so a
// load costs no vector address arithmetic.
struct PairOff {
    uint32_t q, a, b;
};
__device__ __forceinline__ PairOff pair_off(int type, int nb, int rG, int p) {
    const uint32_t e = uint32_t(rG * nb * 4 + p), blk = uint32_t(rG * nb + (p >> 2));
    PairOff o;
    if (type == kIQ1_M) { o.q = e * 8; o.a = e * 4; o.b = blk * 8; }
    else if (type == kIQ2_XS) { o.q = e * 16; o.a = e * 2; o.b = blk * 2; }
    else { o.q = e * 16; o.a = blk * 2; o.b = 0; }
    return o;
}
// VMEM instructions one pair load issues, per type (-1: not fixed at compile time).
template <int TM>
constexpr int loads_per_pair() { return TM == 1 ? 2 : (TM == 2 || TM == 4) ? 3 : -1; }

typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));
constexpr int kNT = 2;   // cache policy: non-temporal (streamed once)
// Pair p of row row0 + rG of matrix m (row0 wave-uniform).
__device__ __forceinline__ void load_pair(Raw3& r, int type, const MRef& m, int row0, const PairOff& po) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)m.base, (short)0, -1, 0x00020000);
    const uint32_t rb = uint32_t(row0) * uint32_t(m.nb);   // blocks before the row group
    if (type == kIQ1_M) {
        const v2u32 q = __builtin_amdgcn_raw_buffer_load_b64(rs, po.q, rb * 32, kNT);
        r.w[2] = __builtin_amdgcn_raw_buffer_load_b32(rs, po.a, m.o1 + rb * 16, kNT);
        const v2u32 sw = __builtin_amdgcn_raw_buffer_load_b64(rs, po.b, m.o2 + rb * 8, kNT);
        r.w[0] = q.x; r.w[1] = q.y;
        r.w[3] = sw.x; r.w[4] = sw.y;
    } else {
        const v4u32 q = __builtin_amdgcn_raw_buffer_load_b128(rs, po.q, rb * 64, kNT);
        r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
        if (type == kIQ2_XXS) {
            r.h[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, po.a, m.o1 + rb * 2, kNT);
        } else {
            r.h[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, po.a, m.o1 + rb * 8, kNT);
            r.h[1] = __builtin_amdgcn_raw_buffer_load_b16(rs, po.b, m.o2 + rb * 2, kNT);
        }
    }
}
template <int TM>
__device__ __forceinline__ void load_pair_t(Raw3& r, const MRef& m, int row0, int rG, int p) {
    if constexpr (TM == 1) load_pair(r, kIQ2_XXS, m, row0, pair_off(kIQ2_XXS, m.nb, rG, p));
    else if constexpr (TM == 2) load_pair(r, kIQ2_XS, m, row0, pair_off(kIQ2_XS, m.nb, rG, p));
    else if constexpr (TM == 4) load_pair(r, kIQ1_M, m, row0, pair_off(kIQ1_M, m.nb, rG, p));
    else load_pair(r, m.type, m, row0, pair_off(m.type, m.nb, rG, p));
}

// 2s+1 from the four scale bits stored in bit 7 of each sign byte.
__device__ __forceinline__ int xxs_sc(uint32_t signs) {
    return int(__builtin_amdgcn_udot4((signs >> 7) & 0x01010101u, 0x10080402u, 1u, false));
}

// Matrix (id, role) of a layer: by arithmetic for regular layers, else from
// the descriptor. Rows x nb blocks give the plane offsets.
template <int TM>
__device__ __forceinline__ MRef mref(const Layer3Args& a, int id, int role, int rows, int nb) {
    MRef m;
    if (a.slab) {
        m.base = a.slab + uint64_t(id) * a.estride + a.roff[role];
        m.type = a.rtype[role];
    } else {
        const MatRef& d = a.descs[id].m[role];
        m.base = d.base;
        m.type = d.type;
    }
    if constexpr (TM == 1) m.type = kIQ2_XXS;
    else if constexpr (TM == 2) m.type = kIQ2_XS;
    else if constexpr (TM == 4) m.type = kIQ1_M;
    m.nb = nb;
    plane_offs(m.type, uint64_t(rows) * uint64_t(nb), m.o1, m.o2);
    return m;
}

// ---- codebooks into LDS -------------------------------------------------------------------
// Direct-to-LDS load of `bytes` (a multiple of 1 KB) from global src to LDS
// dst; wave w issues the 1-KB groups w, w + NW, ...
template <int NW>
__device__ __forceinline__ void lds_dma(uint8_t* lds, int dst, const uint8_t* src, int bytes, int wv, int lane) {
    for (int g = wv; g * 1024 < bytes; g += NW)
        __builtin_amdgcn_global_load_lds((const void*)(src + 1024 * g + 16 * lane),
                                         (__attribute__((address_space(3))) void*)(lds + dst + 1024 * g), 16, 0, 0);
}
// Replicates `rows` rows of rb bytes (8 or 16) held once at LDS src into C
// interleaved copies at dst: consecutive threads write consecutive 16-B chunks.
template <int NT>
__device__ __forceinline__ void lds_replicate(uint8_t* lds, int dst, int src, int rows, int rb, int C, int t) {
    const int chunks = rows * C * rb / 16;
    const int per_row = C * rb / 16;
    for (int c = t; c < chunks; c += NT) {
        const int e = c / per_row;
        uint4 v;
        if (rb == 16) {
            v = *reinterpret_cast<const uint4*>(lds + src + 16 * e);
        } else {
            const uint2 h = *reinterpret_cast<const uint2*>(lds + src + 8 * e);
            v = make_uint4(h.x, h.y, h.x, h.y);
        }
        *reinterpret_cast<uint4*>(lds + dst + 16 * c) = v;
    }
}

// Workgroup barrier for LDS data: the wave's LDS accesses complete, then the
// barrier. Unlike __syncthreads it does not wait for the wave's outstanding
// global loads (a workgroup fence would, as it cannot tell them from
// direct-to-LDS loads). The empty asm statements keep the compiler from moving
// memory accesses across it.
constexpr int kLgkm0 = 15 | (3 << 14) | (7 << 4);   // s_waitcnt lgkmcnt(0) only
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kLgkm0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ---- parity trace ---------------------------------------------------------------------------
// Sum over each aligned quad of lanes (DPP), in every lane of the quad: the four
// pairs a quad holds form one 256-weight block, so this is a row's block integer.
__device__ __forceinline__ int quad_isum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    return v;
}
// One wave writes a 292-byte Q8_K block (q8k_core.hpp:13: d, qs[256], bsums[16])
// from its scale and lane l's four quants (values 4l .. 4l + 3).
__device__ __forceinline__ void trace_q8_block(uint8_t* dst, float d, uint32_t packed, int lane) {
    if (lane == 0) *reinterpret_cast<float*>(dst) = d;
    *reinterpret_cast<uint32_t*>(dst + 4 + 4 * lane) = packed;
    const int s = __builtin_amdgcn_sdot4(int(packed), 0x01010101, 0, false);   // the lane's four quants
    const int b = quad_isum(s);                                                  // values 16 j .. 16 j + 15
    if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(dst + 260 + 2 * (lane >> 2)) = int16_t(b);
}

// ---- bounded waits -------------------------------------------------------------------------
constexpr uint32_t kPollLimit = 1u << 21;   // polls (each a device-memory round trip): about a second

__device__ __forceinline__ void set_err(int* err, int bit) { atomicOr(err, bit); }


}  // namespace xl::dev
