// The routed-expert layer in one streaming launch (gfx950). Instances by the
// block types of the layer's matrices (GT: gate/up, DT: down; bits 1 IQ2_XXS,
// 2 IQ2_XS, 4 IQ1_M): IQ2_XXS gate/up with IQ2_XS down (xl_stream.hip),
// IQ1_M only (xl_stream_iq1.hip), and any mix (xl_stream_mix.hip: each pick's
// three matrices found from its descriptor, their types read per slot).
//
// One workgroup of NW waves per CU. The decode work per 8-weight group is one
// grid lookup, (IQ2) one sign lookup, the sign applied by one op per dword,
// and two v_dot4; everything else is laid out so that nothing more is needed:
//
//   codebooks  bank-interleaved copies whose row stride is 256 bytes, so a
//              lookup address is one v_perm_b32 of the index byte and the
//              lane's copy offset: IQ2_XXS grid 32 copies (16 in the mixed
//              instance, sharing each 256-byte row with 16 sign copies), sign
//              rows likewise, IQ2_XS grid 4 copies. The sign table has 256
//              rows, indexed by the whole byte (bit 7 is ignored: it carries a
//              scale bit for IQ2_XXS and a grid bit for IQ2_XS). IQ1_M: one
//              copy of 4096 value rows (8 * grid + delta) at LDS byte 0.
//   gate/up    slot s of the k*ff rows (pick-major) belongs to wave s mod W;
//              the rows' SiLU runs once per batch of kBatch slots, one lane
//              per slot, and h goes out as plain 32-bit words.
//   h exchange two buffers of k_max*ff_max floats, used by alternate launches
//              of this kernel. A buffer holds the sentinel 0xffffffff (a NaN no
//              arithmetic produces; a computed h with those bits is stored as
//              the canonical NaN) in every word before its launch: each launch
//              refills the other buffer, which the previous launch used.
//              Readers poll for non-sentinel words, so no fence is needed.
//   down       workgroup g owns output row groups {g, g+G, ...} of every pick;
//              its passes (row group, pick) are dealt to its waves in pick
//              order, one pass per wave per step. Before step j the workgroup
//              quantizes the h of the picks that step needs (Q8_K, one block
//              per wave at a time) into LDS, from loads issued one step ahead:
//              early steps need early picks, whose h is complete while later
//              picks are still being produced.
//   combine    fixed order (ascending expert id, sequential fma, then + shared;
//              engine/strata/warm/runtime.cpp:183-188), per workgroup.
//
// Waits only point backwards (down waits on gate/up, which waits on nothing)
// and the grid is at most one workgroup per CU, so every workgroup runs once
// the CUs are free and the grid drains. Every wait is bounded: on expiry the
// kernel raises kDevErrTimeout and finishes.
//
// The launch parity comes from a device word advanced by the last workgroup to
// arrive (an arrival counter), never from the host, so a captured launch can
// be replayed.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <utility>

#include "xl_dev.hpp"
#include "xl_internal.hpp"
#include "xl_iq2.hpp"
#include "xl_route.hpp"

namespace xl::dev {
namespace {

// ---- LDS maps (bytes), by the union M of the gate/up and down type masks -----------------------
// SGN/XXS: sign masks and IQ2_XXS grid, 256 rows of 256 bytes each (lookup
// address = index << 8 | the lane's copy offset | table base); XS: IQ2_XS grid
// (512 rows x 4 copies x 8 B); IQ1: IQ1_M value rows; XQ: Q8_K(x) (dim quants,
// swizzled, then 16 block scales; gate/up phase); HQ: Q8_K(h) of the picks
// (down phase, over a region gate/up no longer reads); Y: y staging; NRM: the
// in-kernel pre-norm's 32 group sums (prologue only, a region nothing writes
// before the prologue's last barrier).
template <int M>
struct SLay;
template <>
struct SLay<3> {   // IQ2_XXS gate/up, IQ2_XS down
    static constexpr int CP = 32;                         // grid and sign copies
    static constexpr int SGN = 0, XXS = 65536;            // two tables of 32 copies
    static constexpr int SGN_IN_ROW = 0;                  // byte of the sign copies in a row
    static constexpr int XS = 131072, IQ1 = -1;
    static constexpr int XQ = 147456, HQ = 65536, Y = 147456;   // HQ over the XXS grid, Y over XQ
    static constexpr int NRM = 152704;                    // pre-norm group sums (32 floats), past XQ
    static constexpr int Bytes = NRM + 256;
    static constexpr int HQBytes = 65536;
};
template <>
struct SLay<4> {   // IQ1_M only
    static constexpr int CP = 0, SGN = -1, XXS = -1, SGN_IN_ROW = 0, XS = -1;
    static constexpr int IQ1 = 0;
    static constexpr int XQ = 32768, HQ = 32768, Y = 98304;   // HQ over XQ
    static constexpr int NRM = XQ + 8192;                     // pre-norm partials: past XQ, under HQ
    static constexpr int Bytes = 102400;
    static constexpr int HQBytes = 65536;
};
template <>
struct SLay<7> {   // any mix: one 256-byte row holds 16 grid copies, then 16 sign copies
    static constexpr int CP = 16;
    static constexpr int XXS = 65536, SGN = 65536, SGN_IN_ROW = 128;
    static constexpr int IQ1 = 0, XS = 32768, Y = 49152;
    static constexpr int XQ = 131072, HQ = 131072;   // HQ over XQ
    static constexpr int NRM = XQ + 8192;            // pre-norm partials: past XQ, under HQ
    static constexpr int Bytes = 163584;
    static constexpr int HQBytes = Bytes - HQ;
};
// Down passes over the flattened (pick, row) list of a workgroup's row band
// (single-type instances whose passes hold more than four pairs per lane).
template <int M, int PD>
constexpr bool stream_xp() { return M != 7 && PD > 4; }
constexpr int kS_YFloats = 1024;
// Q8_K(x) in LDS: kMaxRowK quants (swizzled) at XQ, then the block scales.
constexpr int kXQScl = kMaxRowK;
// Slot and pass metadata words: expert id << 17 | pick << 13 | first row (13 bits).
constexpr uint32_t kMetaRow = 0x1fffu;
constexpr int kMetaPick = 13, kMetaId = 17;

// Global codebooks (layer_tables in xl_api.cpp): IQ2_XXS grid, IQ2_XS grid, IQ1_M value rows.
constexpr int kG_XXS = 2048, kG_XS = 4096;

template <int M>
struct Smem {
    uint8_t b[SLay<M>::Bytes];   // first, so that its LDS address is 0 and table bases fold into offsets
    int ids[16];
    float w[16];
    int order[16];   // picks by ascending expert id (stable: equal ids keep pick order)
    uint32_t parity;
    uint32_t gcnt[8];   // down steps' per-group arrival counts (group sync)
};

// Lanes 0 and 32's sums of a butterfly over each 32-lane half of the wave, xor
// offsets 16, 8, 4, 2, 1 (v += v of lane ^ o): the order in which __shfl_xor
// trees sum, by a row swap and DPP moves instead of LDS permutes. Only the
// lanes that feed lanes 0 and 32 get their xor partners.
__device__ __forceinline__ float xor_sum32(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);   // r[1]: rows 1, 3 in rows 0, 2
    v = __fadd_rn(v, __uint_as_float(r[1]));
#define XL_DPP(x, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), ctrl, 0xF, 0xF, false))
    v = __fadd_rn(v, XL_DPP(v, 0x128));   // row_ror:8: lane ^ 8
    v = __fadd_rn(v, XL_DPP(v, 0x104));   // row_shl:4: lanes 0..3 of a row read lanes 4..7
    v = __fadd_rn(v, XL_DPP(v, 0x4E));    // quad_perm 2,3,0,1: lane ^ 2
    v = __fadd_rn(v, XL_DPP(v, 0xB1));    // quad_perm 1,0,3,2: lane ^ 1
#undef XL_DPP
    return v;
}

// Type of a matrix whose mask has one bit.
template <int TM>
constexpr int single_type() { return TM == 1 ? kIQ2_XXS : TM == 2 ? kIQ2_XS : kIQ1_M; }
template <int TM>
constexpr bool one_type() { return TM == 1 || TM == 2 || TM == 4; }

// Lane constants of the codebook lookups.
struct LoLanes {
    uint32_t g, s, x;
};

// Pair loads of the mixed instance: the same three loads whatever the type
// (no branch: register copies where branches merge, and wait counts made
// inexact by them, would wait for the loads), their offsets chosen by the
// wave-uniform type: b128 of code bytes (IQ2: the pair's 16; IQ1_M: its 8
// index bytes and the next pair's 8), b32 (IQ2_XXS: the aligned word holding
// its block's fp16 scale; IQ2_XS: the word holding the pair's scale bytes;
// IQ1_M: its nibble word) and b64 (IQ2_XS: the aligned 4 block scales holding
// its block's; IQ1_M: the block's scale words; IQ2_XXS: 8 code bytes again,
// unused). Every read stays inside the matrix: the row groups start at a
// multiple of 4 blocks and each plane holds a multiple of 4 blocks.
// The per-(pick, role) constants are packed as (MixLoad):
//   voffsets  e << s1, (e >> r2) << 2, (e >> r3) << 3 (e: the pair's index in its row group)
//   soffsets  rb << t1, c2 + (rb << t2), c3 + (rb << t3) (rb: blocks before the row group)
struct MixLoad {
    uint32_t code;   // s1 | r2 << 4 | r3 << 8 | t1 << 12 | t2 << 16 | t3 << 20
    uint32_t c2, c3;
};
__device__ __forceinline__ MixLoad mix_load(int type, uint32_t o1, uint32_t o2) {
    MixLoad L;
    if (type == kIQ2_XXS) {
        L.code = 4u | (3u << 4) | (4u << 8) | (6u << 12) | (1u << 16) | (6u << 20);
        L.c2 = o1; L.c3 = 0;
    } else if (type == kIQ2_XS) {
        L.code = 4u | (1u << 4) | (4u << 8) | (6u << 12) | (3u << 16) | (1u << 20);
        L.c2 = o1; L.c3 = o2;
    } else {
        L.code = 3u | (0u << 4) | (2u << 8) | (5u << 12) | (4u << 16) | (3u << 20);
        L.c2 = o1; L.c3 = o2;
    }
    return L;
}
__device__ __forceinline__ void load_pair_u(Raw3& r, const uint8_t* base, uint32_t code, uint32_t c2, uint32_t c3,
                                            uint32_t rb, uint32_t e, uint32_t dq) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, -1, 0x00020000);
    const uint32_t s1 = code & 15u, r2 = (code >> 4) & 15u, r3 = (code >> 8) & 15u;
    const uint32_t t1 = (code >> 12) & 15u, t2 = (code >> 16) & 15u, t3 = (code >> 20) & 15u;
    const uint32_t ee = e + dq;   // (dq: pairs past the lane's first)
    const v4u32 q = __builtin_amdgcn_raw_buffer_load_b128(rs, ee << s1, rb << t1, kNT);
    r.w[4] = __builtin_amdgcn_raw_buffer_load_b32(rs, (ee >> r2) << 2, c2 + (rb << t2), kNT);
    const v2u32 v = __builtin_amdgcn_raw_buffer_load_b64(rs, (ee >> r3) << 3, c3 + (rb << t3), kNT);
    r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
    r.w[5] = v.x; r.w[6] = v.y;
}
// The fields of a pair loaded by load_pair_u, as the decoders of type T read
// them: pair p of a row group whose first block is bq mod 4.
template <int T>
__device__ __forceinline__ Raw3 mix_view(const Raw3& r, int bq, int p) {
    Raw3 v = r;
    const uint32_t blk = uint32_t(bq + (p >> 2));   // the block mod 4 (within its aligned group)
    if constexpr (T == 1) {
        v.h[0] = uint16_t(r.w[4] >> ((blk & 1u) << 4));
    } else if constexpr (T == 2) {
        v.h[0] = uint16_t(r.w[4] >> (uint32_t(p & 1) << 4));
        v.h[1] = uint16_t(((blk & 2u) ? r.w[6] : r.w[5]) >> ((blk & 1u) << 4));
    } else {
        v.w[2] = r.w[4];
        v.w[3] = r.w[5]; v.w[4] = r.w[6];
    }
    return v;
}

// Lookups and exact integer of one pair of static type T (1 IQ2_XXS, 2 IQ2_XS,
// 4 IQ1_M); NA: IQ2_XXS takes its signs on the negated activations na, else
// on the grid; pp: the pair's place in its block; d16: its fp16 scale.
template <int T>
__device__ __forceinline__ void look_t(Looks& L, const uint8_t* lds, const LoLanes& lo, const Raw3& r) {
    if constexpr (T == 1) look_xxs_to(L, lds, lo.g, lo.s, r.w);
    else if constexpr (T == 2) look_xs_to(L, lds, lo.x, lo.s, r.w);
    else look_iq1_to(L, lds, r.w);
}
template <int T, bool NA>
__device__ __forceinline__ int sum_t(const Looks& L, const Raw3& r, const uint32_t* a, const uint32_t* na, int pp,
                                     uint32_t& d16) {
    if constexpr (T == 1) {
        d16 = r.h[0];
        if constexpr (NA) return sum_xxs(L, r.w, a, na);
        else return sum_xxs_g(L, r.w, a);
    } else if constexpr (T == 2) {
        d16 = r.h[1];
        return sum_xs(L, r.h[0], a);
    } else {
        d16 = iq1_d16(r.w);
        return sum_iq1(L, iq1_scw(r.w, pp), a);
    }
}
// A pair as the decoders of type T read it (V: loaded by load_pair_u; bq, p as mix_view).
template <int T, bool V>
__device__ __forceinline__ Raw3 pair_view(const Raw3& r, int bq, int p) {
    if constexpr (V) return mix_view<T>(r, bq, p);
    else return r;
}
// Gate and up rows of one slot, static types TG_ / TU_: both rows' lookups
// are issued before either row's arithmetic.
template <int TG_, int TU_, bool V, int PG, int NQ>
__device__ __forceinline__ void decode_slot(int (&Ig)[PG], int (&Iu)[PG], uint32_t (&dg)[PG], uint32_t (&du)[PG],
                                            const Raw3 (&G)[PG], const Raw3 (&U)[PG], const Act<PG>& A,
                                            const uint32_t (&NA)[NQ][16], const uint8_t* lds, const LoLanes& lo,
                                            int lG, int LG, int bq) {
#pragma unroll
    for (int q = 0; q < PG; ++q) {
        const int p = lG + LG * q, pp = p & 3;
        const Raw3 g = pair_view<TG_, V>(G[q], bq, p), u = pair_view<TU_, V>(U[q], bq, p);
        Looks Lg, Lu;
        look_t<TG_>(Lg, lds, lo, g);
        look_t<TU_>(Lu, lds, lo, u);
        Ig[q] = sum_t<TG_, true>(Lg, g, A.a[q], NA[NQ > 1 ? q : 0], pp, dg[q]);
        Iu[q] = sum_t<TU_, true>(Lu, u, A.a[q], NA[NQ > 1 ? q : 0], pp, du[q]);
    }
}
// A down pass (PD pairs per lane) of static type T: the next pair's lookups are
// issued before the current pair's arithmetic.
template <int T, bool V, int PD>
__device__ __forceinline__ void decode_pass(int (&I)[PD], uint32_t (&d)[PD], const Raw3 (&R)[PD], const Act<PD>& B,
                                            const uint8_t* lds, const LoLanes& lo, int lD, int LD, int bq) {
    Looks La, Lb;
    look_t<T>(La, lds, lo, pair_view<T, V>(R[0], bq, lD));
    static_for<PD>([&]<int q>() {
        const Raw3 r = pair_view<T, V>(R[q], bq, lD + LD * q);
        Looks& Lc = (q & 1) ? Lb : La;
        Looks& Ln = (q & 1) ? La : Lb;
        if constexpr (q + 1 < PD) look_t<T>(Ln, lds, lo, pair_view<T, V>(R[q + 1], bq, lD + LD * (q + 1)));
        I[q] = sum_t<T, false>(Lc, r, B.a[q], nullptr, (lD + LD * q) & 3, d[q]);
    });
}

// Instances whose lanes cover more pairs (PG > 2 gate/up pairs, PD > 4 down
// pairs: the 5120 x 2304 expert) read each pair's activations from LDS as the
// pair is decoded, since registers for every pair's activations would not fit;
// the IQ2_XXS signs then go on the grid bytes (no negated activations).
template <int TG_, int TU_, bool V>
__device__ __forceinline__ void decode_pair_al(int& Ig, int& Iu, uint32_t& dg, uint32_t& du, float& dx, const Raw3& G,
                                               const Raw3& U, const uint8_t* lds, int xq, const LoLanes& lo, int p,
                                               int bq) {
    Act<1> A;
    load_act<1>(A, lds, xq, kXQScl, p, 0);
    const Raw3 g = pair_view<TG_, V>(G, bq, p), u = pair_view<TU_, V>(U, bq, p);
    Looks Lg, Lu;
    look_t<TG_>(Lg, lds, lo, g);
    look_t<TU_>(Lu, lds, lo, u);
    Ig = sum_t<TG_, false>(Lg, g, A.a[0], nullptr, p & 3, dg);
    Iu = sum_t<TU_, false>(Lu, u, A.a[0], nullptr, p & 3, du);
    dx = A.d[0];
}
// A down pass of the same kind, one pair at a time (lookahead registers would
// not fit beside the pass's raw words; hq, hs: the pick's Q8_K(h) in LDS).
template <int T, bool V, int PD>
__device__ __forceinline__ void decode_pass_al(int (&I)[PD], uint32_t (&d)[PD], float (&dx)[PD], const Raw3 (&R)[PD],
                                               const uint8_t* lds, int hq, int hs, const LoLanes& lo, int lD, int LD,
                                               int bq) {
    static_for<PD>([&]<int q>() {
        const int p = lD + LD * q;
        const Raw3 r = pair_view<T, V>(R[q], bq, p);
        Looks Lc;
        Act<1> Ac;
        look_t<T>(Lc, lds, lo, r);
        load_act<1>(Ac, lds, hq, hs, p, 0);
        I[q] = sum_t<T, false>(Lc, r, Ac.a[0], nullptr, p & 3, d[q]);
        dx[q] = Ac.d[0];
    });
}

// A down pass's PD pairs (p = lD + LD q) of row `row` of a matrix whose base
// differs per lane (XP passes hold rows of two picks): global loads from 64-bit
// lane addresses, the pair offsets immediates.
template <int TM, int PD, int LD>
__device__ __forceinline__ void load_pass_v(Raw3 (&R)[PD], const uint8_t* base, uint32_t o1, uint32_t o2, int row,
                                            int nb, int lD) {
    static_assert(LD % 4 == 0, "a lane's pairs stay in one block column");
    const uint64_t rb = uint64_t(uint32_t(row) * uint32_t(nb));   // blocks before the row
    const int b0 = lD >> 2;                                       // the lane's first block
    if constexpr (TM == 4) {
        const uint8_t* pq = base + rb * 32 + 8 * lD;
        const uint8_t* pa = base + o1 + rb * 16 + 4 * lD;
        const uint8_t* pb = base + o2 + rb * 8 + 8 * b0;
#pragma unroll
        for (int q = 0; q < PD; ++q) {
            const v2u32 v = __builtin_nontemporal_load(reinterpret_cast<const v2u32*>(pq + 8 * LD * q));
            const v2u32 sw = __builtin_nontemporal_load(reinterpret_cast<const v2u32*>(pb + 8 * (LD / 4) * q));
            R[q].w[0] = v.x; R[q].w[1] = v.y;
            R[q].w[2] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(pa + 4 * LD * q));
            R[q].w[3] = sw.x; R[q].w[4] = sw.y;
        }
    } else {
        const uint8_t* pq = base + rb * 64 + 16 * lD;
#pragma unroll
        for (int q = 0; q < PD; ++q) {
            const v4u32 v = __builtin_nontemporal_load(reinterpret_cast<const v4u32*>(pq + 16 * LD * q));
            R[q].w[0] = v.x; R[q].w[1] = v.y; R[q].w[2] = v.z; R[q].w[3] = v.w;
        }
        if constexpr (TM == 1) {
            const uint8_t* pa = base + o1 + rb * 2 + 2 * b0;
#pragma unroll
            for (int q = 0; q < PD; ++q)
                R[q].h[0] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(pa + 2 * (LD / 4) * q));
        } else {
            const uint8_t* pa = base + o1 + rb * 8 + 2 * lD;
            const uint8_t* pb = base + o2 + rb * 2 + 2 * b0;
#pragma unroll
            for (int q = 0; q < PD; ++q) {
                R[q].h[0] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(pa + 2 * LD * q));
                R[q].h[1] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(pb + 2 * (LD / 4) * q));
            }
        }
    }
}

// ---- the kernel ----------------------------------------------------------------------------
// LG x PG: lanes per gate/up row and pairs per lane (LG * PG * 64 == dim);
// LD x PD: the same for down rows (LD * PD * 64 == ff). MG / MD: most gate/up
// slots / down passes per wave; WIN: gate/up slots in flight per wave; WIND:
// down passes in flight; MQ: most Q8_K(h) blocks one wave quantizes per step.
constexpr int kBatch = 3;   // gate/up slots per SiLU batch
// TR: also write the parity trace (Layer3Args::tq8x ...); the untraced instance
// compiles none of it.
template <int NW, int LG, int PG, int LD, int PD, int MG, int MD, int WIN, int WIND, int MQ, int GT, int DT, bool TR>
__global__ __launch_bounds__(NW * 64, 1) void stream_kernel(Layer3Args a) {
    static_assert(WIN <= MG && WIND <= MD && WIND <= MG && MG <= 32 && MD <= 32, "prefetch depths, metadata lanes");
    constexpr int M = (GT == 1 && DT == 2) ? 3 : (GT == 4 && DT == 4) ? 4 : 7;
    constexpr bool MIX = M == 7;   // matrices from per-(pick, role) lane tables, types at run time
    constexpr bool XP = stream_xp<M, PD>();
    using LY = SLay<M>;
    static_assert(MIX || (one_type<GT>() && one_type<DT>()), "single-type instances");
    __shared__ __attribute__((aligned(16))) Smem<M> sm;
    uint8_t* const lds = sm.b;
    constexpr int RG = 64 / LG, RD = 64 / LD;
    const int t = threadIdx.x, lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int G = gridDim.x, W = G * NW, gw = blockIdx.x * NW + wv;
    const int k = a.k, ff = a.ff, dim = a.dim;
    const int lG = lane % LG, rG = lane / LG, lD = lane % LD, rD = lane / LD;
    const int nbx = dim / 256, nbh = ff / 256;
    auto mark = [&](int n) {
        if (a.trace && lane == 0) a.trace[size_t(gw) * 32 + n] = __builtin_amdgcn_s_memrealtime();
    };
    mark(4);   // entry

    // ---- this wave's work: gate/up slots gs + W*j, down passes wv + NW*j (pick-major)
    // When the slots do not divide evenly over the waves, the slot index runs
    // wave-major (wave wv of workgroup b starts at gs = wv G + b): every
    // workgroup then holds the same share to within one slot, instead of some
    // holding twice the slots of others.
    const int sppG = ff / RG, SG = k * sppG;
    const int gs = SG % W ? wv * G + int(blockIdx.x) : gw;
    const int ng = SG > gs ? min(MG, (SG - gs + W - 1) / W) : 0;
    // Down rows. XP instances: workgroup b owns rows [b R, b R + R) of every pick
    // (R = dim / G), and pass u's RD row groups run over the flattened (pick, row)
    // list, so a pass may hold rows of two picks. Else: row quads b, b + G, ...
    // of each pick, one pick per pass.
    const int quads = dim / RD;
    const int nq_wg = quads > int(blockIdx.x) ? (quads - int(blockIdx.x) + G - 1) / G : 0;
    const int RW = XP ? dim / G : nq_wg * RD;   // rows of one pick in this workgroup
    const int P = XP ? (k * RW + RD - 1) / RD : k * nq_wg;
    const int nd = P > wv ? min(MD, (P - wv + NW - 1) / NW) : 0;
    // Routed in the kernel (a.rlogits): thread t loads expert t's logit and bias
    // here; the routing runs after the x and codebook loads are out. Else the ids.
    const bool routed = a.rlogits != nullptr;   // uniform
    static_assert(NW * 64 >= kStreamRouteMax, "one expert per thread");
    float rl = 0.0f, rb = 0.0f;
    int idl = 0;
    if (routed) {
        const int e = min(t, a.n_experts - 1);   // clamped, unconditional
        rl = a.rlogits[e];
        rb = a.rbias ? a.rbias[e] : 0.0f;
    } else {
        idl = a.ids[lane < k ? lane : k - 1];   // unconditional loads keep the wait counts exact
    }
    // ---- x and the codebook rows: they need no ids, so they go out right after
    // the ids load (the wait for the ids then leaves them in flight) and before the
    // slot loads. The rows come into registers (plain loads: waiting for them does
    // not wait for the slot loads issued after them).
    constexpr int NT = NW * 64;
    constexpr bool HASXXS = (M & 1) != 0 || MIX, HASXS = (M & 2) != 0 || MIX;
    constexpr bool HAS1 = (M & 4) != 0;
    constexpr int NX = (4096 + NT - 1) / NT, NS = (1024 + NT - 1) / NT, N1 = (2048 + NT - 1) / NT;
    // x first: its Q8_K runs while the codebook loads are in flight
    constexpr int NBXM = LG * PG / 4;                       // the instance's Q8_K(x) blocks (dim / 256)
    constexpr int UX = (NBXM + NW - 1) / NW;
    constexpr int PNR = (LG * PG * 64 + 1023) / 1024;       // pre-norm elements per hc_pre_norm thread
    float4 xv[UX];
    // Pre-norm in the kernel (a.pn_h, uniform): xv takes the stream's values,
    // pw the norm weights, pv the values of the two threads of hc_pre_norm_kernel's
    // 1,024 that this thread stands in for (v = t and t + 512: elements v + 1024 r).
    // The arithmetic waits until the codebook loads are out.
    const bool pn = a.pn_h != nullptr;
    static_assert(NW * 64 == 512, "pre-norm: two of hc_pre_norm_kernel's 1,024 threads per thread");
    float4 pw[UX];
    float pv[2][PNR], pm = 0.0f;
#pragma unroll
    for (int u = 0; u < UX; ++u) {
        const int b = wv + NW * u;
        xv[u] = reinterpret_cast<const float4*>((pn ? a.pn_h : a.x) + 256 * (b < nbx ? b : 0))[lane];
    }
    if (pn) {
        pm = a.pn_mix[0];
#pragma unroll
        for (int u = 0; u < UX; ++u) {
            const int b = wv + NW * u;
            pw[u] = a.pn_w ? reinterpret_cast<const float4*>(a.pn_w + 256 * (b < nbx ? b : 0))[lane]
                           : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int r = 0; r < PNR; ++r) pv[s][r] = a.pn_h[min(t + 512 * s + 1024 * r, dim - 1)];
    }
    uint2 vx[HASXXS ? NX : 1], vs[HASXS ? NS : 1];
    uint4 v1[HAS1 ? N1 : 1];
    {
        const uint2* gx = reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(a.tables) + kG_XXS);
        const uint2* gs = reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(a.tables) + kG_XS);
        const uint4* g1 = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.tables) + kTableIQ1X);
        // chunk c of the XXS/sign table: row c / 16, 16-byte piece c % 16
        if constexpr (HASXXS)
#pragma unroll
            for (int i = 0; i < NX; ++i) vx[i] = gx[min(t + NT * i, 4095) >> 4];
        if constexpr (HASXS)
#pragma unroll
            for (int i = 0; i < NS; ++i) vs[i] = gs[min(t + NT * i, 1023) >> 1];   // chunk c: row c / 2, copies 2(c % 2), +1
        if constexpr (HAS1)
#pragma unroll
            for (int i = 0; i < N1; ++i) v1[i] = g1[min(t + NT * i, 2047)];
    }
    // Slot and pass metadata, computed lane-parallel and kept in one register:
    // lane j < 32 holds gate/up slot j, lane 32 + j down pass j, packed as
    // expert << 17 | pick << 13 | first row (bad ids read expert 0 and are
    // masked out). A use reads its lane back (v_readlane), so the scalar
    // registers stay free for the loads' addresses.
    float rw = 0.0f;   // routed: lane i < k's pick weight
    if (routed) {
        // Scores and keys by every thread into LDS (the sign-table region, written
        // only after the second barrier), wave 0 selects (the router kernel's
        // order: expert e in lane e % 64, slot e / 64) into sm.ids / sm.w, which
        // every wave then reads (wave 0 later stores the same values there).
        constexpr int RNPL = kStreamRouteMax / 64;
        float* const rsc = reinterpret_cast<float*>(lds);
        uint32_t* const rkey = reinterpret_cast<uint32_t*>(lds + 4 * kStreamRouteMax);
        bool fin = true;
        float sc;
        uint32_t key;
        route_score(rl, rb, t < a.n_experts, sc, key, fin);
        if (__any(!fin) && lane == 0) set_err(a.err, kDevErrNonFinite);
        if (t < kStreamRouteMax) {
            rsc[t] = sc;
            rkey[t] = key;
        }
        lds_barrier();
        if (wv == 0) {
            float scs[RNPL];
            uint32_t keys[RNPL];
#pragma unroll
            for (int j = 0; j < RNPL; ++j) {
                scs[j] = rsc[lane + 64 * j];
                keys[j] = rkey[lane + 64 * j];
            }
            int id;
            float wt;
            route_select<RNPL>(scs, keys, k, lane, a.rscale, id, wt);
            if (lane < k) {
                sm.ids[lane] = id;
                sm.w[lane] = wt;
            }
        }
        lds_barrier();
        idl = sm.ids[lane < k ? lane : k - 1];
        rw = sm.w[lane < k ? lane : k - 1];
    }
    const int idv = lane < k ? idl : -1;
    uint32_t meta;
    uint64_t okmask;   // bit j: slot j is this wave's with a valid id; bit 32 + j: pass j likewise
    {
        const bool isd = lane >= 32;
        const int j = lane & 31;
        const int n = isd ? nd : ng;
        const int jj = j < n ? j : n > 0 ? n - 1 : 0;   // past the last: a valid row
        const int unit = isd ? wv + NW * jj : gs + W * jj;
        const int per = isd ? nq_wg : sppG;
        const int pick = n > 0 ? unit / per : 0;
        // An idle gate/up slot (and every slot of a wave with none) reads the first
        // rows of its pick: in bounds, and the same lines for every idle wave, so
        // they come from cache instead of re-streaming rows from HBM.
        const int row = isd ? (n > 0 ? (int(blockIdx.x) + G * (unit - pick * nq_wg)) * RD : 0)
                            : (j < n ? (unit - pick * sppG) * RG : 0);
        const int id = __shfl(idv, min(pick, 15));
        const bool ok = n > 0 && id >= 0 && id < a.n_experts;
        meta = (uint32_t(ok ? id : 0) << kMetaId) | (uint32_t(min(pick, 15)) << kMetaPick) | uint32_t(row);
        okmask = __builtin_amdgcn_ballot_w64(ok && j < n);
    }
    auto gsl = [&](int j) { return uint32_t(__builtin_amdgcn_readlane(int(meta), j)); };
    auto dsl = [&](int j) { return uint32_t(__builtin_amdgcn_readlane(int(meta), 32 + j)); };
    auto dpick = [&](int j) { return int((dsl(j) >> kMetaPick) & 15u); };
    // XP: lane group rD's row of pass j (flattened index u = pass * RD + rD over
    // pick-major (pick, row) of the band), its expert (a bad id reads expert 0's
    // rows, masked out) and whether it holds one
    struct XRow {
        int pick, row, e;
        bool ok;
    };
    const float rw_inv = XP ? 1.0f / float(RW) : 0.0f;   // (u + 0.5) / RW floors exactly for u, RW < 2^10
    auto xrow = [&](int j) {
        XRow x;
        const int u = (wv + NW * j) * RD + rD;
        const bool in = u < k * RW;
        x.pick = in ? int((float(u) + 0.5f) * rw_inv) : 0;
        x.row = int(blockIdx.x) * RW + (in ? u - x.pick * RW : 0);
        const int id = __shfl(idv, x.pick);
        x.ok = in && id >= 0 && id < a.n_experts;
        x.e = x.ok ? id : 0;
        return x;
    };
    const uint32_t gok = uint32_t(okmask), dok = uint32_t(okmask >> 32);
    // h word of slot j's first row (pick * ff + row = slot * RG), or -2^30 when the
    // slot is not this wave's
    auto hrow = [&](int j) { return j < ng ? (gs + W * j) * RG : -(1 << 30); };

    // Matrices. Single-type instances (regular layers): matrix (e, role) at
    // slab + e * estride + roff[role], plane offsets shared. Mixed instance: lane
    // 16 role + i holds pick i's matrix of that role (base, type), from the
    // layer's slab or the pick's descriptor (a bad id reads expert 0's).
    uint32_t go1 = 0, go2 = 0, do1 = 0, do2 = 0;
    if constexpr (!MIX) {
        plane_offs(single_type<GT>(), uint64_t(ff) * uint64_t(nbx), go1, go2);
        plane_offs(single_type<DT>(), uint64_t(dim) * uint64_t(nbh), do1, do2);
    }
    auto matrix = [&](int e, int role, uint32_t o1, uint32_t o2, int type, int nb) {
        return MRef{a.slab + uint64_t(e) * a.estride + a.roff[role], o1, o2, type, nb};
    };
    uint32_t tb_lo = 0, tb_hi = 0;
    MixLoad tb_ml{};
    int tb_ty = 0;
    if constexpr (MIX) {
        const int ti = lane & 15, tr = min(lane >> 4, 2);
        const int id = __shfl(idv, ti < k ? ti : k - 1);
        const int e = (id >= 0 && id < a.n_experts) ? id : 0;
        uint64_t base;
        if (a.slab) {
            base = uint64_t(a.slab) + uint64_t(e) * a.estride + (tr == 0 ? a.roff[0] : tr == 1 ? a.roff[1] : a.roff[2]);
            tb_ty = tr == 0 ? a.rtype[0] : tr == 1 ? a.rtype[1] : a.rtype[2];
        } else {
            const MatRef& d = a.descs[e].m[tr];
            base = uint64_t(d.base);
            tb_ty = d.type;
        }
        tb_lo = uint32_t(base);
        tb_hi = uint32_t(base >> 32);
        // plane offsets from the type and the role's shape (gate/up: ff rows of nbx
        // blocks, down: dim rows of nbh blocks), then the load constants, once here
        // rather than per slot
        uint32_t o1, o2;
        plane_offs(tb_ty, tr < 2 ? uint64_t(ff) * uint64_t(nbx) : uint64_t(dim) * uint64_t(nbh), o1, o2);
        tb_ml = mix_load(tb_ty, o1, o2);
    }
    // pick i's matrix of a role (mixed instance), from the lane table: base and load constants
    struct MixRef {
        const uint8_t* base;
        uint32_t code, c2, c3;
    };
    auto mref = [&](int pick, int role) {
        const int L = 16 * role + pick;
        MixRef m;
        m.base = reinterpret_cast<const uint8_t*>((uint64_t(uint32_t(__builtin_amdgcn_readlane(int(tb_hi), L))) << 32) |
                                                  uint32_t(__builtin_amdgcn_readlane(int(tb_lo), L)));
        m.code = uint32_t(__builtin_amdgcn_readlane(int(tb_ml.code), L));
        m.c2 = uint32_t(__builtin_amdgcn_readlane(int(tb_ml.c2), L));
        m.c3 = uint32_t(__builtin_amdgcn_readlane(int(tb_ml.c3), L));
        return m;
    };
    // The lanes' pair indices in their row groups (gate/up; down pass pair 0, the
    // others LD * q further, which enters the scalar offsets) and the first block
    // of their row groups mod 4.
    const uint32_t eg = uint32_t(rG * nbx * 4 + lG), ed = uint32_t(rD * nbh * 4 + lD);
    const int bqg = (rG * nbx) & 3, bqd = (rD * nbh) & 3;
    auto mtype = [&](int pick, int role) { return __builtin_amdgcn_readlane(tb_ty, 16 * role + pick); };

    // ---- the first slots (the codebook rows and x are in flight since the start)
    const float cw = routed ? rw : a.w[lane < k ? lane : k - 1];
    uint32_t* ctl = a.ctl + 2;   // [0] parity source: launches of this kernel so far, [1] arrivals
    const uint32_t e_prev = coh_ld32(ctl);

    Raw3 rg[WIN][PG], ru[WIN][PG];
    // pair q of slot j's gate and up rows
    auto load_slot_pair = [&]<int j, int q>() {
        constexpr int b = j % WIN;
        const uint32_t m = gsl(j);
        const int row0 = int(m & kMetaRow), e = int(m >> kMetaId);
        if constexpr (MIX) {
            const int pk = int((m >> kMetaPick) & 15u);
            const uint32_t rb = uint32_t(row0) * uint32_t(nbx);
            const MixRef mg = mref(pk, 0), mu = mref(pk, 1);
            load_pair_u(rg[b][q], mg.base, mg.code, mg.c2, mg.c3, rb, eg, uint32_t(LG * q));
            load_pair_u(ru[b][q], mu.base, mu.code, mu.c2, mu.c3, rb, eg, uint32_t(LG * q));
        } else {
            load_pair_t<GT>(rg[b][q], matrix(e, 0, go1, go2, single_type<GT>(), nbx), row0, rG, lG + LG * q);
            load_pair_t<GT>(ru[b][q], matrix(e, 1, go1, go2, single_type<GT>(), nbx), row0, rG, lG + LG * q);
        }
    };
    auto load_slot = [&]<int j>() { static_for<PG>([&]<int q>() { load_slot_pair.template operator()<j, q>(); }); };
    // Every wave issues the same loads whatever its share (idle slots and passes
    // re-read valid rows and are discarded), so every wait count is exact.
    static_for<WIN>([&]<int j>() { load_slot.template operator()<j>(); });
    mark(0);
    // Down-phase Q8_K(h) blocks, lane-parallel and kept in one register (the
    // steps read their lanes back, so no scalar division runs between steps;
    // computed once the first loads are out):
    // lane j * MQ + m holds step j's m-th block of this wave as valid << 8 |
    // pick << 4 | block. Step j quantizes the picks its passes are the first to
    // need, [ceil(NW RD j / RW), ceil(NW RD (j + 1) / RW)) clipped to k; wave wv
    // owns blocks wv, wv + NW, ... of them.
    static_assert(MD * MQ <= 64, "Q8_K(h) block table lanes");
    uint32_t hblk = 0;
    // Group sync (4096-row instances, four row quads per pick and workgroup): a
    // step's passes then cover two picks, waves 0-3 one and waves 4-7 the other;
    // each group of four quantizes its own pick's Q8_K(h) blocks (nbh / 4 each)
    // and every step waits for its group only (an LDS arrival count) instead of
    // the whole workgroup (config 3: 26.95 -> 26.2 us).
    const bool gsync = !XP && NW == 8 && nq_wg == 4 && nbh % nq_wg == 0 && nbh / nq_wg <= MQ && MD <= 4;
    {
        const int j = lane / MQ, m = lane - j * MQ;
        if (j < MD) {
            const int plo = min(k, (NW * RD * j + RW - 1) / RW), phi = min(k, (NW * RD * (j + 1) + RW - 1) / RW);
            if (gsync) {
                const int g = wv / nq_wg, per = nbh / nq_wg;
                const int i = plo + g, bb = (wv % nq_wg) * per + m;
                const bool v = i < phi && m < per;
                hblk = (uint32_t(v) << 8) | (uint32_t(v ? i : 0) << 4) | uint32_t(v ? bb : 0);
            } else {
                const int b0 = plo * nbh, nb = phi * nbh - b0, bq = wv + NW * m;
                const int blk = bq < nb ? b0 + bq : 0;
                const int i = blk / nbh;
                hblk = (uint32_t(bq < nb) << 8) | (uint32_t(i) << 4) | uint32_t(blk - i * nbh);
            }
        }
    }

    // ---- pre-norm (a.pn_h): hc_pre_norm_kernel's arithmetic in its order. Pre
    // values a = 0 + m h; each of the 1,024 threads' sum of a^2 over its elements
    // in r order, trees over 32-thread groups (xor offsets 16 .. 1), the same
    // tree over the 32 group sums, then x = (a * inv) * w, inv = 1 / sqrt(S /
    // dim + eps).
    if (pn) {
        const float m = pm;
#pragma unroll
        for (int u = 0; u < UX; ++u) {
            xv[u].x = __fadd_rn(0.0f, __fmul_rn(m, xv[u].x));
            xv[u].y = __fadd_rn(0.0f, __fmul_rn(m, xv[u].y));
            xv[u].z = __fadd_rn(0.0f, __fmul_rn(m, xv[u].z));
            xv[u].w = __fadd_rn(0.0f, __fmul_rn(m, xv[u].w));
        }
        if (a.pn_w) {
            float* const red = reinterpret_cast<float*>(lds + LY::NRM);
            float ss[2] = {0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int r = 0; r < PNR; ++r)
                    if (t + 512 * s + 1024 * r < dim) {
                        const float av = __fadd_rn(0.0f, __fmul_rn(m, pv[s][r]));
                        ss[s] = __fadd_rn(ss[s], __fmul_rn(av, av));
                    }
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                ss[s] = xor_sum32(ss[s]);
                if ((lane & 31) == 0) red[(t + 512 * s) >> 5] = ss[s];
            }
            lds_barrier();
            // every wave sums the 32 group sums itself (NRM is not written again
            // before the prologue's last barrier, so no second barrier)
            const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xor_sum32(red[lane & 31])), 0));
            const float inv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, float(dim)), a.pn_eps)));
#pragma unroll
            for (int u = 0; u < UX; ++u) {
                xv[u].x = __fmul_rn(__fmul_rn(xv[u].x, inv), pw[u].x);
                xv[u].y = __fmul_rn(__fmul_rn(xv[u].y, inv), pw[u].y);
                xv[u].z = __fmul_rn(__fmul_rn(xv[u].z, inv), pw[u].z);
                xv[u].w = __fmul_rn(__fmul_rn(xv[u].w, inv), pw[u].w);
            }
        }
        if (a.pn_x && blockIdx.x == 0)
#pragma unroll
            for (int u = 0; u < UX; ++u) {
                const int b = wv + NW * u;
                if (b < nbx) reinterpret_cast<float4*>(a.pn_x + 256 * b)[lane] = xv[u];
            }
    }

    // ---- Q8_K(x), then codebooks (copies, computed sign rows): LDS writes, one barrier
    {
        uint4 xb[UX];
        uint32_t xp[UX];
        float xd[UX];
#pragma unroll
        for (int u = 0; u < UX; ++u)
            xb[u] = make_uint4(__float_as_uint(xv[u].x), __float_as_uint(xv[u].y), __float_as_uint(xv[u].z),
                               __float_as_uint(xv[u].w));
        const bool fin = q8k_blocks<UX>(xb, nbx > wv ? (nbx - wv + NW - 1) / NW : 0, lane, xp, xd);
        if (!fin && lane == 0) set_err(a.err, kDevErrNonFinite);
#pragma unroll
        for (int u = 0; u < UX; ++u) {
            const int b = wv + NW * u;
            if (b < nbx) {
                *reinterpret_cast<uint32_t*>(lds + LY::XQ + qswz(256 * b + 4 * lane)) = xp[u];
                if (lane == 0) reinterpret_cast<float*>(lds + LY::XQ + kXQScl)[b] = xd[u];
            }
        }
        // x per 32 (a.p32_q): workgroup g quantizes the 32-value chunks g, g + G, ...,
        // each by the wave holding its block (lanes 8 c .. 8 c + 7 of block c / 8), as
        // quant32_kernel: d = max|x| / 127, q = round-half-even(x / d), zero chunk zero.
        // (A non-finite x is flagged by the Q8_K(x) above.)
        if (a.p32_q) {
#pragma unroll
            for (int u = 0; u < UX; ++u) {
                const int b = wv + NW * u;
                for (int c = int(blockIdx.x); c < 8 * nbx; c += G) {   // uniform
                    if ((c >> 3) != b) continue;
                    const float v[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
                    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                    am = fmaxf(am, dppf<0xB1>(am));    // quad_perm [1,0,3,2]
                    am = fmaxf(am, dppf<0x4E>(am));    // quad_perm [2,3,0,1]
                    am = fmaxf(am, dppf<0x141>(am));   // row_half_mirror: the 8-lane chunk's two quads
                    const float sc = __fdiv_rn(am, 127.0f);
                    uint32_t qw = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        qw |= uint32_t(uint8_t(int8_t(am > 0.0f ? __float2int_rn(__fdiv_rn(v[i], sc)) : 0))) << (8 * i);
                    if ((lane >> 3) == (c & 7)) {
                        reinterpret_cast<uint32_t*>(a.p32_q)[64 * b + lane] = qw;
                        if ((lane & 7) == 0) a.p32_d[c] = sc;
                    }
                }
            }
        }
    }
    if constexpr (M == 3) {
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int c = t + NT * i;   // chunk c: sign row c / 16, copies 2(c % 16), +1
            if (c < 4096) {
                const uint2 r = sign_row(uint32_t(c) >> 4);
                *reinterpret_cast<uint4*>(lds + LY::SGN + 16 * c) = make_uint4(r.x, r.y, r.x, r.y);
            }
        }
#pragma unroll
        for (int i = 0; i < NX; ++i)
            if (t + NT * i < 4096)
                *reinterpret_cast<uint4*>(lds + LY::XXS + 16 * (t + NT * i)) = make_uint4(vx[i].x, vx[i].y, vx[i].x, vx[i].y);
    } else if constexpr (MIX) {
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int c = t + NT * i;   // chunk c: row c / 16; pieces 0..7 grid copies, 8..15 sign copies
            if (c < 4096) {
                const uint2 r = (c & 8) ? sign_row(uint32_t(c) >> 4) : vx[i];
                *reinterpret_cast<uint4*>(lds + LY::XXS + 16 * c) = make_uint4(r.x, r.y, r.x, r.y);
            }
        }
    }
    if constexpr (HASXS)
#pragma unroll
        for (int i = 0; i < NS; ++i)
            if (t + NT * i < 1024)
                *reinterpret_cast<uint4*>(lds + LY::XS + 16 * (t + NT * i)) = make_uint4(vs[i].x, vs[i].y, vs[i].x, vs[i].y);
    if constexpr (HAS1)
#pragma unroll
        for (int i = 0; i < N1; ++i)
            if (t + NT * i < 2048)
                *reinterpret_cast<uint4*>(lds + LY::IQ1 + 16 * (t + NT * i)) = make_uint4(v1[i].x, v1[i].y, v1[i].z, v1[i].w);
    mark(1);
    if (wv == 0) {
        int rank = 0;   // the combine order (engine/strata/warm/runtime.cpp:183-188)
        for (int j = 0; j < k; ++j) {
            const int idj = __builtin_amdgcn_readlane(idv, j);
            rank += (idj < idv) | ((idj == idv) & (j < lane));
        }
        if (lane < k) {
            sm.ids[lane] = idv;
            sm.w[lane] = cw;
            sm.order[rank] = lane;
        }
    }
    if (t == 0) sm.parity = (e_prev + 1u) & 1u;
    if (t < 8) sm.gcnt[t] = 0u;
    lds_barrier();
    if constexpr (TR) {   // workgroup 0's staged Q8_K(x), as the gate/up rows read it
        if (blockIdx.x == 0 && a.tq8x)
            for (int b = wv; b < nbx; b += NW)
                trace_q8_block(a.tq8x + 292 * b, reinterpret_cast<const float*>(lds + LY::XQ + kXQScl)[b],
                               *reinterpret_cast<const uint32_t*>(lds + LY::XQ + qswz(256 * b + 4 * lane)), lane);
    }
    const uint32_t parity = __builtin_amdgcn_readfirstlane(sm.parity);   // uniform: keeps buffer bases scalar
    float* const hcur = a.hbuf + size_t(parity) * kHBufWords;
    // Arrival: the last workgroup to arrive advances the launch count at its end.
    uint32_t arrived = 0;
    if (t == 0) arrived = __hip_atomic_fetch_add(ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (gw < k && lane == 0) {
        const int id = sm.ids[gw];
        if (id < 0 || id >= a.n_experts) set_err(a.err, kDevErrExpertId);
    }
    // The other buffer (used by the previous launch) back to the sentinel for the next one.
    {
        float* const hnext = a.hbuf + size_t(parity ^ 1u) * kHBufWords;
        const uint4 s4 = make_uint4(kSentinel, kSentinel, kSentinel, kSentinel);
        for (int c = int(blockIdx.x) * NW * 64 + t; c < kHBufWords / 4; c += G * NW * 64)
            reinterpret_cast<uint4*>(hnext)[c] = s4;
    }
    mark(2);

    LoLanes lo;
    {
        constexpr uint32_t cmask = LY::CP > 0 ? uint32_t(LY::CP - 1) : 0u;
        const uint32_t cp = (uint32_t(lane) & cmask) * 8u;
        lo.g = cp | uint32_t(LY::XXS > 0 ? LY::XXS : 0);                              // table base in byte 2
        lo.s = cp | uint32_t(LY::SGN > 0 ? LY::SGN : 0) | uint32_t(LY::SGN_IN_ROW);
        lo.x = uint32_t(LY::XS > 0 ? LY::XS : 0) + uint32_t(lane & 3) * 8u;
        asm volatile("" : "+v"(lo.x));   // opaque: keeps (x & mask) | lo.x one v_and_or_b32
    }

    Raw3 rd[WIND + 1][PD];
    auto load_pass = [&]<int j>() {
        if constexpr (XP) {
            const XRow x = xrow(j);
            load_pass_v<DT, PD, LD>(rd[j % (WIND + 1)], a.slab + uint64_t(x.e) * a.estride + a.roff[2], do1, do2, x.row,
                                    nbh, lD);
            return;
        }
        const uint32_t m = dsl(j);
#pragma unroll
        for (int q = 0; q < PD; ++q) {
            if constexpr (MIX) {
                const MixRef md = mref(int((m >> kMetaPick) & 15u), 2);
                load_pair_u(rd[j % (WIND + 1)][q], md.base, md.code, md.c2, md.c3, uint32_t(m & kMetaRow) * uint32_t(nbh),
                            ed, uint32_t(LD * q));
            } else
                load_pair_t<DT>(rd[j % (WIND + 1)][q], matrix(int(m >> kMetaId), 2, do1, do2, single_type<DT>(), nbh),
                                int(m & kMetaRow), rD, lD + LD * q);
        }
    };

    // ---- gate/up
    {
        constexpr bool ALG = PG > 2;   // activations per pair from LDS (decode_pair_al)
        Act<ALG ? 1 : PG> A;
        if constexpr (!ALG) load_act<PG>(A, lds, LY::XQ, kXQScl, lG, LG);
        constexpr bool NEEDNA = (GT & 1) != 0 && !ALG;
        uint32_t NA[NEEDNA ? PG : 1][16];   // -q bytewise (q in -127..127, so no overflow); unused without IQ2_XXS
        if constexpr (NEEDNA)
#pragma unroll
            for (int q = 0; q < PG; ++q)
#pragma unroll
                for (int c = 0; c < 16; ++c) NA[q][c] = neg_bytes(A.a[q][c]);
        float bg = 0.0f, bu = 0.0f;   // lane LG-1-b of each row group: slot b of the batch
        int hidx = 0;                 // that slot's h word (pick * ff + row)
        static_for<MG>([&]<int j>() {
            // The SIMD arbiter favours older waves, so the first NW/2 waves of a
            // workgroup would finish gate/up well before their SIMD partners (which
            // then run alone, latency-bound, while the down phase waits for them).
            // The younger half runs at wave priority 1 for the first two thirds of
            // its slots (all of them when a wave has at most two), which evens out
            // the finish times (5120 x 2304, two slots: 26.9 -> 25.9 us).
            if constexpr (j == 0) {
                if (wv >= NW / 2) __builtin_amdgcn_s_setprio(1);
            }
            if constexpr (j == (MG <= 2 ? MG : (2 * MG) / 3)) __builtin_amdgcn_s_setprio(0);
            if constexpr (j >= 1 && j + WIN - 1 < MG && !(ALG && WIN == 1)) load_slot.template operator()<j + WIN - 1>();
            // the down stream starts under the last slots (ALG instances: after gate/up,
            // their slots' raw words and per-pair activations fill the registers)
            if constexpr (!ALG && j >= MG - WIND) load_pass.template operator()<j - (MG - WIND)>();
            // (gate and up share a block type: xl_open rejects a bank where they differ)
            const int tg = MIX ? mtype(int((gsl(j) >> kMetaPick) & 15u), 0) : 0;
            int Ig[PG], Iu[PG];
            uint32_t dg[PG], du[PG];
            float dxs[PG];
            if constexpr (ALG) {
                // (WIN == 1: the next slot's pair q goes into pair q's registers as soon as
                // pair q is decoded, so one slot's raw words are live at a time)
                auto pairs = [&]<int T_, bool V_>(int bq) {
                    static_for<PG>([&]<int q>() {
                        decode_pair_al<T_, T_, V_>(Ig[q], Iu[q], dg[q], du[q], dxs[q], rg[j % WIN][q], ru[j % WIN][q], lds,
                                                   LY::XQ, lo, lG + LG * q, bq);
                        if constexpr (WIN == 1 && j + 1 < MG) load_slot_pair.template operator()<j + 1, q>();
                    });
                };
                if constexpr (!MIX) pairs.template operator()<GT, false>(0);
                else if (tg == kIQ2_XXS) pairs.template operator()<1, true>(bqg);
                else if (tg == kIQ2_XS) pairs.template operator()<2, true>(bqg);
                else pairs.template operator()<4, true>(bqg);
            } else {
                if constexpr (!MIX) {
                    decode_slot<GT, GT, false>(Ig, Iu, dg, du, rg[j % WIN], ru[j % WIN], A, NA, lds, lo, lG, LG, 0);
                } else {   // one branch per slot, static types inside
                    if (tg == kIQ2_XXS) decode_slot<1, 1, true>(Ig, Iu, dg, du, rg[j % WIN], ru[j % WIN], A, NA, lds, lo, lG, LG, bqg);
                    else if (tg == kIQ2_XS) decode_slot<2, 2, true>(Ig, Iu, dg, du, rg[j % WIN], ru[j % WIN], A, NA, lds, lo, lG, LG, bqg);
                    else decode_slot<4, 4, true>(Ig, Iu, dg, du, rg[j % WIN], ru[j % WIN], A, NA, lds, lo, lG, LG, bqg);
                }
#pragma unroll
                for (int q = 0; q < PG; ++q) dxs[q] = A.d[ALG ? 0 : q];
            }
            float fg = 0.0f, fu = 0.0f;
#pragma unroll
            for (int q = 0; q < PG; ++q) {
                if constexpr (TR) {   // the row's block integers: a quad holds one block's four pairs
                    const int bg = quad_isum(Ig[q]), bu = quad_isum(Iu[q]);
                    // (the lane read stays outside the branch: a spilled meta reloaded
                    // inside it would leave lane j, inactive there, stale)
                    const uint32_t m = gsl(j);
                    if (a.tint && ((gok >> j) & 1u) && (lG & 3) == 0) {
                        const size_t rec = size_t((m >> kMetaPick) & 15u) * (2 * size_t(ff) * nbx + size_t(dim) * nbh);
                        const size_t o = rec + size_t(int(m & kMetaRow) + rG) * nbx + size_t((lG + LG * q) >> 2);
                        a.tint[o] = bg;
                        a.tint[o + size_t(ff) * nbx] = bu;
                    }
                }
                fg = fmaf(__fmul_rn(h2f(dg[q]), dxs[q]), float(Ig[q]), fg);
                fu = fmaf(__fmul_rn(h2f(du[q]), dxs[q]), float(Iu[q]), fu);
            }
            // A bad id read expert 0's rows: its h is published as 0 so that readers
            // finish. The mask is applied by an opaque multiply: a select would let the
            // compiler sink each row's whole decode into its own branch, serializing the
            // gate and up rows.
            float okf = ((gok >> j) & 1u) ? 1.0f : 0.0f;
            asm volatile("" : "+v"(okf));
            const float g = gsum<LG>(fg) * okf, u = gsum<LG>(fu) * okf;
            const int b = j % kBatch;
            const bool mine = lG == LG - 1 - b;
            bg = mine ? g : bg;
            bu = mine ? u : bu;
            hidx = mine ? hrow(j) + rG : hidx;
            // a batch's h goes out at its last slot, or at the wave's last valid slot
            // (fewer picks than slots: published a slot or two sooner, fewer polls)
            if (b == kBatch - 1 || j == MG - 1 || j == ng - 1) {
                // (g / (1 + exp(-g))) * u with the device expf and an IEEE division, as
                // q8k_core.hpp:92-95: an approximate exp or reciprocal moves h by an ulp
                // often enough to flip Q8_K(h) quants (a 1e-4-scale output change each)
                const float hv = silu_mul3(__fmul_rn(0.125f, bg), __fmul_rn(0.125f, bu), a.lim);
                const uint32_t hb = __float_as_uint(hv) == kSentinel ? kQNaN : __float_as_uint(hv);
                if (lG >= LG - 1 - b && hidx >= 0)
                    __hip_atomic_store(reinterpret_cast<uint32_t*>(hcur) + hidx, hb, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                if constexpr (TR) {
                    if (a.th && lG >= LG - 1 - b && hidx >= 0) a.th[hidx] = __uint_as_float(hb);
                }
            }
            mark(8 + j);
        });
    }
    mark(3);
    __builtin_amdgcn_s_setprio(0);
    if constexpr (PG > 2) static_for<WIND>([&]<int j>() { load_pass.template operator()<j>(); });

    // ---- down: step j quantizes the h of the picks it needs, then every wave runs pass j
    float* ys = reinterpret_cast<float*>(lds + LY::Y);
    const int hq_stride = ff + 64;
    // step j's m-th Q8_K(h) block of this wave (from the lane table hblk)
    auto hb_of = [&](int j, int m) { return uint32_t(__builtin_amdgcn_readlane(int(hblk), j * MQ + m)); };
    uint4 hv[2][MQ];   // h loads of steps j and j + 1 (issued two steps ahead)
    // loads of step j's blocks owned by this wave; an unused slot still loads (so
    // that every wait count is exact), all its lanes the same 16 bytes
    auto h_issue = [&]<int j>() {
#pragma unroll
        for (int m = 0; m < MQ; ++m) {
            const uint32_t b = hb_of(j, m);
            const uint32_t w = ((b >> 8) & 1u) ? uint32_t(int((b >> 4) & 15u) * ff + 256 * int(b & 15u) + 4 * lane) : 0u;
            hv[j & 1][m] = h_load(hcur, w);
        }
    };
    // The first step's h loads: before the workgroup barrier when its picks were
    // published by an early SiLU batch; after it when every slot is in one batch
    // (then they are published at the end of gate/up, and loads issued before
    // the barrier mostly see sentinels and poll again: one pick 16.7 -> 15.5 us)
    constexpr bool H0LATE = MG <= kBatch;
    if constexpr (!H0LATE) h_issue.template operator()<0>();
    if constexpr (MD > 1) h_issue.template operator()<1>();
    // wait until step j's blocks are complete (all re-polled together; the common
    // case never enters the retry loop)
    auto h_wait = [&]<int j>() {
        auto all_ready = [&]() {
            bool ok = true;
#pragma unroll
            for (int m = 0; m < MQ; ++m) ok = ok & (((hb_of(j, m) >> 8) & 1u) == 0u || h_ready(hv[j & 1][m]));
            return __all(ok);
        };
        uint32_t polls = 0;
        if (!all_ready()) {
            do {
                if (++polls > kPollLimit) {
                    if (lane == 0) set_err(a.err, kDevErrTimeout);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
                h_issue.template operator()<j>();
            } while (!all_ready());
        }
        if (a.trace && lane == 0 && j < 4) a.trace[size_t(gw) * 32 + 20 + j] = polls;
    };
    // Q8_K of step j's blocks owned by this wave (registers), then their LDS stores
    auto h_quant = [&]<int j>(uint32_t (&hp)[MQ], float (&hd)[MQ]) {
        int nvalid = 0;   // the valid blocks are the first ones
#pragma unroll
        for (int m = 0; m < MQ; ++m) nvalid += int((hb_of(j, m) >> 8) & 1u);
        return q8k_blocks<MQ>(hv[j & 1], nvalid, lane, hp, hd);
    };
    auto h_store = [&]<int j>(const uint32_t (&hp)[MQ], const float (&hd)[MQ], bool fin) {
        if (!fin && lane == 0) set_err(a.err, kDevErrNonFinite);
#pragma unroll
        for (int m = 0; m < MQ; ++m) {
            const uint32_t b = hb_of(j, m);
            if ((b >> 8) & 1u) {
                const int i = int((b >> 4) & 15u), bb = int(b & 15u);
                uint8_t* hq = lds + LY::HQ + i * hq_stride;
                *reinterpret_cast<uint32_t*>(hq + qswz(256 * bb + 4 * lane)) = hp[m];
                if (lane == 0) reinterpret_cast<float*>(hq + ff)[bb] = hd[m];
            }
        }
    };
    // Group sync: count this wave in at gcnt[c] (after its LDS stores, in order)
    // and wait until the group's four waves are in; bounded like every wait.
    auto group_wait = [&](int c) {
        uint32_t* const p = &sm.gcnt[c];
        if (lane == 0) __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        uint32_t spins = 0;
        while (__hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < 4u) {
            if (++spins > (1u << 20)) {
                if (lane == 0) set_err(a.err, kDevErrTimeout);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    };
    lds_barrier();   // Q8_K(h) is staged over a region gate/up read: every wave is past gate/up
    if constexpr (H0LATE) h_issue.template operator()<0>();
    {
        h_wait.template operator()<0>();
        mark(24);
        {
            uint32_t hp[MQ];
            float hd[MQ];
            const bool fin = h_quant.template operator()<0>(hp, hd);
            h_store.template operator()<0>(hp, hd, fin);
        }
        mark(17);
        if (gsync) {
            group_wait(6 + wv / 4);   // the group has stored step 0's blocks
        } else {
            lds_barrier();
        }
        mark(25);
        // Step j runs pass j with the next step's Q8_K(h) in the same straight-line
        // code (its quantizer's DPP and division chains fill the pass's LDS waits);
        // the next step's blocks go to LDS after the pass, then one barrier.
        constexpr bool ALD = PD > 4;   // activations per pair from LDS (decode_pass_al)
        Act<ALD ? 1 : PD> B;
        static_for<MD>([&]<int j>() {   // steps past nsteps stage nothing and compute a discarded pass
            // the next step's h first (its loads went out a step ago), then the next
            // pass's weight loads: issued before the check, their texture-unit time
            // would delay it
            if constexpr (j + 1 < MD) {
                h_wait.template operator()<j + 1>();
                mark(24 + 2 * (j + 1));
            }
            if constexpr (j + WIND < MD) load_pass.template operator()<j + WIND>();
            XRow xr{};
            int i;   // the pass's pick (XP: the lane group's)
            if constexpr (XP) {
                xr = xrow(j);
                i = xr.pick;
            } else {
                i = dpick(j);
            }
            if constexpr (!ALD) {
                if (j == 0 || i != dpick(j > 0 ? j - 1 : 0)) load_act<PD>(B, lds, LY::HQ + i * hq_stride, ff, lD, LD);
            }
            uint32_t hp[MQ];
            float hd[MQ];
            bool fin = true;
            if constexpr (j + 1 < MD) fin = h_quant.template operator()<j + 1>(hp, hd);
            const int td = MIX ? mtype(i, 2) : 0;
            int I[PD];
            uint32_t d16[PD];
            float dxs[PD];
            if constexpr (ALD) {
                const int hq = LY::HQ + i * hq_stride;
                if constexpr (!MIX) {
                    decode_pass_al<DT, false>(I, d16, dxs, rd[j % (WIND + 1)], lds, hq, ff, lo, lD, LD, 0);
                } else {
                    if (td == kIQ2_XXS) decode_pass_al<1, true>(I, d16, dxs, rd[j % (WIND + 1)], lds, hq, ff, lo, lD, LD, bqd);
                    else if (td == kIQ2_XS) decode_pass_al<2, true>(I, d16, dxs, rd[j % (WIND + 1)], lds, hq, ff, lo, lD, LD, bqd);
                    else decode_pass_al<4, true>(I, d16, dxs, rd[j % (WIND + 1)], lds, hq, ff, lo, lD, LD, bqd);
                }
            } else {
                if constexpr (!MIX) {
                    decode_pass<DT, false>(I, d16, rd[j % (WIND + 1)], B, lds, lo, lD, LD, 0);
                } else {   // one branch per pass, static type inside
                    if (td == kIQ2_XXS) decode_pass<1, true>(I, d16, rd[j % (WIND + 1)], B, lds, lo, lD, LD, bqd);
                    else if (td == kIQ2_XS) decode_pass<2, true>(I, d16, rd[j % (WIND + 1)], B, lds, lo, lD, LD, bqd);
                    else decode_pass<4, true>(I, d16, rd[j % (WIND + 1)], B, lds, lo, lD, LD, bqd);
                }
#pragma unroll
                for (int q = 0; q < PD; ++q) dxs[q] = B.d[ALD ? 0 : q];
            }
            float f = 0.0f;
#pragma unroll
            for (int q = 0; q < PD; ++q) {
                if constexpr (TR) {
                    const int bi = quad_isum(I[q]);
                    const uint32_t m = dsl(j);   // outside the branch, as in gate/up
                    const bool tok = XP ? xr.ok : ((dok >> j) & 1u) != 0;
                    const int tpick = XP ? xr.pick : int((m >> kMetaPick) & 15u);
                    const int trow = XP ? xr.row : int(m & kMetaRow) + rD;
                    if (a.tint && tok && (lD & 3) == 0) {
                        const size_t rec = size_t(tpick) * (2 * size_t(ff) * nbx + size_t(dim) * nbh);
                        a.tint[rec + 2 * size_t(ff) * nbx + size_t(trow) * nbh + size_t((lD + LD * q) >> 2)] = bi;
                    }
                }
                f = fmaf(__fmul_rn(h2f(d16[q]), dxs[q]), float(I[q]), f);
            }
            float okf = (XP ? xr.ok : ((dok >> j) & 1u) != 0) ? 0.125f : 0.0f;   // opaque, as in gate/up
            asm volatile("" : "+v"(okf));
            const float y = __fmul_rn(okf, gsum<LD>(f));
            // ys[u]: pick-major rows of the band, u = pass * RD + rD (passes past nd
            // have u >= k RW)
            const int u = (wv + NW * j) * RD + rD;
            if (u < k * RW && lD == LD - 1) ys[u] = y;
            if (j == 0) mark(5);
            // the h loads of step j + 2 go out after the pass: later issue, fewer re-polls
            if constexpr (j + 2 < MD) h_issue.template operator()<j + 2>();
            if constexpr (j + 1 < MD) {
                h_store.template operator()<j + 1>(hp, hd, fin);
                if (j + 1 < 3) mark(17 + j + 1);
                if (gsync) {
                    group_wait(2 * j + wv / 4);   // the group has stored the next step's blocks
                } else {
                    lds_barrier();
                }
                mark(25 + 2 * (j + 1));
            }
        });
    }
    mark(6);
    lds_barrier();
    if constexpr (TR) {   // workgroup 0's staged Q8_K(h) of every pick, as its down passes read it
        if (blockIdx.x == 0 && a.tq8h)
            for (int blk = wv; blk < k * nbh; blk += NW) {
                const int i = blk / nbh, bb = blk - i * nbh;
                const uint8_t* hq = lds + LY::HQ + i * hq_stride;
                trace_q8_block(a.tq8h + 292 * blk, reinterpret_cast<const float*>(hq + ff)[bb],
                               *reinterpret_cast<const uint32_t*>(hq + qswz(256 * bb + 4 * lane)), lane);
            }
    }

    // ---- fixed-order combine of this workgroup's rows
    for (int r = t; r < RW; r += NW * 64) {
        const int qq = r / RD, rr = r - qq * RD;
        const int orow = XP ? int(blockIdx.x) * RW + r : (int(blockIdx.x) + G * qq) * RD + rr;
        float acc = 0.0f;
        for (int s2 = 0; s2 < k; ++s2) {
            const int i = sm.order[s2];
            const float yi = ys[i * RW + r];
            if constexpr (TR) {
                if (a.ty) a.ty[size_t(i) * dim + orow] = yi;
            }
            acc = fmaf(sm.w[i], yi, acc);
        }
        if (a.shared) acc = __fadd_rn(acc, a.shared[orow]);
        a.out[orow] = acc;
        if (a.po_out) {   // hc_post of this column, in hc_post_kernel's order (every load first)
            const int H = a.po_H;
            float r[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] = i < H ? a.po_res[size_t(i) * dim + orow] : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (j < H) {
                    float v = __fmul_rn(a.po_post[j], acc);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (i < H) v = __fadd_rn(v, __fmul_rn(a.po_comb[i * H + j], r[i]));
                    a.po_out[size_t(j) * dim + orow] = v;
                }
            }
        }
    }
    mark(7);
    if (t == 0 && arrived == uint32_t(G) - 1u) {   // every workgroup has read the launch count
        coh_st32(ctl, e_prev + 1u);
        coh_st32(ctl + 1, 0u);
    }
}

template <int NW, int LG, int PG, int LD, int PD, int MG, int MD, int WIN, int WIND, int MQ, int GT, int DT>
hipError_t launch_stream_t(const Layer3Args& args, int grid, hipStream_t s, hipEvent_t stop) {
    constexpr int M = (GT == 1 && DT == 2) ? 3 : (GT == 4 && DT == 4) ? 4 : 7;
    const bool tr = args.tq8x || args.tq8h || args.th || args.tint || args.ty;
    constexpr int RG = 64 / LG, RD = 64 / LD;
    const int W = grid * NW;
    const int SG = args.k * (args.ff / RG);
    constexpr bool XP = stream_xp<M, PD>();
    const int quads = args.dim / RD;
    const int nq_wg = (quads + grid - 1) / grid;
    // rows of one pick in a workgroup (XP: its band; else up to nq_wg quads)
    const int RW = XP ? args.dim / grid : nq_wg * RD;
    const int P = (args.k * RW + RD - 1) / RD;
    const int nbh = args.ff / 256;
    // most blocks one step needs: the picks first needed by NW consecutive passes,
    // in workgroups owning RW rows of each pick (else quads / grid and quads / grid + 1 quads)
    int most = 0;
    for (int rw = XP ? RW : (quads / grid) * RD; rw <= RW; rw += RD)
        for (int j = 0; j * NW * RD < args.k * rw; ++j) {
            const int lo = std::min(args.k, (NW * RD * j + rw - 1) / rw);
            const int hi = std::min(args.k, (NW * RD * (j + 1) + rw - 1) / rw);
            most = std::max(most, (hi - lo) * nbh);
        }
    if ((SG + W - 1) / W > MG || args.n_experts > 32768 || args.dim > kMaxRowK || args.ff > 4096 ||
        (P + NW - 1) / NW > MD || (most + NW - 1) / NW > MQ || args.k * RW > kS_YFloats || grid > quads ||
        (XP && args.dim % grid != 0) ||
        args.k * (args.ff + 64) > SLay<M>::HQBytes || args.k * args.ff > kHBufWords || !args.hbuf ||
        (M != 7 && !args.slab) || (M == 7 && !args.slab && !args.descs))
        return hipErrorNotSupported;
    if (tr)
        hipExtLaunchKernelGGL((stream_kernel<NW, LG, PG, LD, PD, MG, MD, WIN, WIND, MQ, GT, DT, true>), dim3(grid),
                              dim3(NW * 64), 0, s, nullptr, stop, 0, args);
    else
        hipExtLaunchKernelGGL((stream_kernel<NW, LG, PG, LD, PD, MG, MD, WIN, WIND, MQ, GT, DT, false>), dim3(grid),
                              dim3(NW * 64), 0, s, nullptr, stop, 0, args);
    return hipGetLastError();
}

// Instances by shape and pick count for one (GT, DT).
template <int GT, int DT>
hipError_t launch_stream_shapes(const Layer3Args& args, int cus, hipStream_t s, hipEvent_t stop) {
    if (args.k < 1 || args.k > 16 || args.dim > kMaxRowK || args.ff > 4096) return hipErrorNotSupported;
    int lg, pg, ld, pd;
    if (!row_shape(args.dim, lg, pg) || !row_shape(args.ff, ld, pd)) return hipErrorNotSupported;
    const int RD = 64 / ld;
    const int grid = std::min(cus, args.dim / RD);
    if (lg == 64 && pg == 1 && ld == 16 && pd == 3) {   // 4096 x 3072: slots and steps sized by the pick count
        // one pick: 3,072 rows over 2,048 waves fill at most two slots per wave (a
        // third, idle slot would re-read rows for nothing)
        if (args.k == 1) return launch_stream_t<8, 64, 1, 16, 3, 2, 1, 2, 1, 3, GT, DT>(args, grid, s, stop);
        if (args.k <= 2) return launch_stream_t<8, 64, 1, 16, 3, 3, 1, 3, 1, 3, GT, DT>(args, grid, s, stop);
        if (args.k <= 4) return launch_stream_t<8, 64, 1, 16, 3, 6, 2, 3, 2, 3, GT, DT>(args, grid, s, stop);
        // one down pass in flight: its weights load under the last gate/up slot and
        // each later pass's under the step before it (three passes in flight under
        // the last three slots: 25.4 us at config 1, one: 24.4 us)
        return launch_stream_t<8, 64, 1, 16, 3, 9, 3, 3, 1, 3, GT, DT>(args, grid, s, stop);
    }
    if (lg == 16 && pg == 5 && ld == 4 && pd == 9) {   // 5120 x 2304, the DeepSeek expert (cpu_lane_fixture.cpp:17)
        if (args.k <= 2) return launch_stream_t<8, 16, 5, 4, 9, 1, 1, 1, 1, 7, GT, DT>(args, grid, s, stop);
        // single-type layers: up to six picks' 20-row bands fill one pass per wave
        if constexpr (GT != 7) return launch_stream_t<8, 16, 5, 4, 9, 2, 1, 1, 1, 7, GT, DT>(args, grid, s, stop);
        else return launch_stream_t<8, 16, 5, 4, 9, 2, 2, 1, 1, 7, GT, DT>(args, grid, s, stop);
    }
    if (lg == 16 && pg == 1 && ld == 8 && pd == 1)    // 1024 x 512
        return launch_stream_t<8, 16, 1, 8, 1, 6, 2, 3, 1, 2, GT, DT>(args, grid, s, stop);
    if (lg == 4 && pg == 1 && ld == 4 && pd == 3)     // 256 x 768
        return launch_stream_t<8, 4, 1, 4, 3, 6, 2, 3, 1, 3, GT, DT>(args, grid, s, stop);
    return hipErrorNotSupported;
}

}  // namespace
}  // namespace xl::dev
