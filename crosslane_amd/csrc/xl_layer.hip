// The routed-expert layer in one launch (gfx950).
//
// One workgroup of NW waves per CU, one launch per layer. The layer's weight
// bytes move as one steady stream (about two items in flight per wave, the
// point where gfx950 HBM reads run fastest), in the order the work needs them:
//
//   prologue  one copy of each codebook and x are loaded first (they need no
//             ids); the first gate/up slots follow; the codebooks are then
//             replicated inside LDS (bank-interleaved copies, see Lay) and x
//             quantized to Q8_K in LDS by every workgroup
//   gate/up   slot s of the k*ff gate/up rows (pick-major) belongs to wave
//             s mod W of the grid; h = silu(gate.x) * (up.x) is published per
//             row as a 64-bit (value, epoch) word
//   Q8_K(h)   block (i, b) is quantized by one designated wave once all of its
//             256 tagged h words carry this launch's epoch, and published as
//             tagged words (4 quants, epoch) plus a tagged scale
//   down      workgroup g owns output row groups {g, g+G, ...} of every pick.
//             Its passes (row group, pick) are dealt to its waves round robin
//             in pick order, so every wave streams early picks first and the
//             last pick's rows arrive last, while that pick's h is still being
//             quantized. The wave holding a workgroup's first pass of a pick
//             stages the pick's Q8_K(h) in LDS; the results go to LDS, and the
//             fixed-order combine (ascending expert id, sequential fma, then
//             + shared; engine/strata/warm/runtime.cpp:183-188) needs nothing
//             from other workgroups
//
// Waits only point backwards (gate/up never waits; quantizers wait on gate/up;
// down waits on quantizers), so the grid drains whether or not all workgroups
// are resident at once. Every wait is bounded: on expiry the kernel raises
// kDevErrTimeout and finishes.
//
// Epoch: each launch reads the device word E and tags its data E + 1 (0 is
// skipped: zero is what unwritten tags hold); the last workgroup to arrive (an
// arrival counter) stores that tag for the next launch. The tag never comes
// from the host, so a captured launch can be replayed.
//
// Cross-workgroup data moves through agent-scope (sc1) atomic loads and stores,
// which are coherent across the XCDs' L2 caches; every published word carries
// its own tag, so no store ordering wait is needed.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "xl_dev.hpp"
#include "xl_format.hpp"
#include "xl_internal.hpp"

namespace xl::dev {

// ---- LDS layout ------------------------------------------------------------------------
// Codebooks are replicated in C bank-interleaved copies: entry e of copy c sits
// at (e * C + c) * row_bytes and lane l reads copy l % C. Random lookups by the
// 16 (b128) or 32 (b64) lanes an LDS cycle serves then fall into distinct banks
// far more often than with one copy (measured on gfx950: random b128 lookups
// from one copy take 2.2x the conflict-free time, from 16 interleaved copies
// 1.0x; random b64 from one copy 1.7x, from 16 copies 1.5x).
constexpr int kYStage = 1024;                 // floats of y staging for the combine
constexpr int kLdsBytes = 160 * 1024 - 512;   // the kernel's LDS array (the rest: small shared words)
// Byte offsets for an instance whose matrices use the block types in TM (bits
// 1 IQ2_XXS, 2 IQ2_XS, 4 IQ1_M): only those codebooks are held. HQ: Q8_K(h)
// of the picks staged once per workgroup (per pick ff quants then 16 scales);
// before the codebooks are replicated it holds their single copies.
template <int TM>
struct Lay {
    static constexpr int CS = 16;                       // sign-row copies (16-byte rows)
    static constexpr int CXXS = 16;                     // IQ2_XXS grid copies (8-byte rows)
    static constexpr int CXS = (TM & 4) ? 8 : 16;       // IQ2_XS grid copies
    static constexpr int SGN = 0;                                            // 128 rows {M.lo, M.hi, M1.lo, M1.hi}
    static constexpr int XXS = SGN + ((TM & 3) ? 128 * CS * 16 : 0);         // 256 rows of 8 magnitudes
    static constexpr int XS = XXS + ((TM & 1) ? 256 * CXXS * 8 : 0);         // 512 rows of 8 magnitudes
    // IQ1 grid copies: only without the IQ2 tables is there room for copies and
    // for staging the single copy (at HQ, where those tables' copies would be staged).
    static constexpr int C1 = TM == 4 ? 4 : 1;
    static_assert(C1 == 1 || (TM & 3) == 0, "the IQ1 single copy is staged where the IQ2 tables' are");
    static constexpr int IQ1 = XS + ((TM & 2) ? 512 * CXS * 8 : 0);          // 2048 rows of 8 values
    static constexpr int XQ = IQ1 + ((TM & 4) ? 2048 * 8 * C1 : 0);          // Q8_K(x) quants (dim <= kMaxRowK)
    static constexpr int XD = XQ + kMaxRowK;                                 // Q8_K(x) scales (kMaxRowK / 256)
    static constexpr int Y = XD + kMaxRowK / 64;                             // y staging
    static constexpr int HQ = Y + kYStage * 4;
    static_assert(HQ + 8192 <= kLdsBytes, "LDS budget");
};
// Global codebooks (uploaded once per context), one copy each, byte offsets:
// sign rows {M.lo, M.hi, M1.lo, M1.hi} x 128 (M: 0xff in the bytes of negative
// weights), IQ2_XXS rows x 256, IQ2_XS rows x 512, IQ1 rows x 2048 (8 B each).
constexpr int kG_SGN = 0, kG_XXS = 2048, kG_XS = 4096, kG_IQ1 = 8192, kG_Bytes = 24576;
static_assert(kG_Bytes == kLayer3TableBytes, "table layout");

// ---- row engine --------------------------------------------------------------------------
struct Lut {
    uint32_t sgn, xxs, xs, iq1;   // per-lane LDS byte address of this lane's copy of each table
};
template <int TM>
__device__ __forceinline__ Lut make_lut(int lane) {
    using LY = Lay<TM>;
    Lut L;
    L.sgn = LY::SGN + uint32_t(lane % LY::CS) * 16;
    L.xxs = LY::XXS + uint32_t(lane % LY::CXXS) * 8;
    L.xs = LY::XS + uint32_t(lane % LY::CXS) * 8;
    L.iq1 = LY::IQ1 + uint32_t(lane % LY::C1) * 8;
    return L;
}

// Activations of the pairs a lane owns: 64 Q8_K bytes per pair, the pair's
// block scale, and (for IQ1_M rows) the sums of its eight groups of 8 quants,
// which every row's delta term reuses.
template <int P>
struct Act3 {
    uint32_t a[P][16];
    float d[P];
    int gs[P][8];
};
template <int TM, int P>
__device__ __forceinline__ void group_sums(Act3<P>& A) {
    if constexpr (TM & 4) {
#pragma unroll
        for (int q = 0; q < P; ++q)
#pragma unroll
            for (int g = 0; g < 8; ++g) A.gs[q][g] = sdot4(0x01010101u, A.a[q][2 * g + 1], sdot4(0x01010101u, A.a[q][2 * g], 0));
    }
}


// The pair decoders issue every codebook lookup of the pair before using any:
// 16 LDS reads in flight per lane hide the LDS latency.
template <int TM>
__device__ __forceinline__ int pair_xxs3(const uint8_t* lds, const Lut& L, const uint32_t* w, const uint32_t* a) {
    constexpr int SX = Lay<TM>::CXXS * 8, SS = Lay<TM>::CS * 16;   // entry strides
    uint2 g[8];
    uint4 m[8];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            g[4 * s + q] = *reinterpret_cast<const uint2*>(lds + L.xxs + ((w[2 * s] >> (8 * q)) & 255u) * SX);
            m[4 * s + q] = *reinterpret_cast<const uint4*>(lds + L.sgn + ((w[2 * s + 1] >> (8 * q)) & 127u) * SS);
        }
    int acc[2] = {0, 0};
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = 4 * s + q;
            acc[s] = sdot4(xad(g[e].x, m[e].x, m[e].z), a[8 * s + 2 * q], acc[s]);
            acc[s] = sdot4(xad(g[e].y, m[e].y, m[e].w), a[8 * s + 2 * q + 1], acc[s]);
        }
    return __mul24(acc[0], xxs_sc(w[1])) + __mul24(acc[1], xxs_sc(w[3]));
}
template <int TM>
__device__ __forceinline__ int pair_xs3(const uint8_t* lds, const Lut& L, const uint32_t* w, uint32_t sc, const uint32_t* a) {
    constexpr int SX = Lay<TM>::CXS * 8, SS = Lay<TM>::CS * 16;
    uint2 g[8];
    uint4 m[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t c = (w[e / 2] >> (16 * (e & 1))) & 0xffffu;
        g[e] = *reinterpret_cast<const uint2*>(lds + L.xs + (c >> 7) * SX);
        m[e] = *reinterpret_cast<const uint4*>(lds + L.sgn + (c & 127u) * SS);
    }
    int total = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        int lo = 0, hi = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = 4 * s + q;
            int& acc = q < 2 ? lo : hi;
            acc = sdot4(xad(g[e].x, m[e].x, m[e].z), a[8 * s + 2 * q], acc);
            acc = sdot4(xad(g[e].y, m[e].y, m[e].w), a[8 * s + 2 * q + 1], acc);
        }
        const uint32_t byte = (sc >> (8 * s)) & 255u;
        total += __mul24(lo, int(2u * (byte & 15u) + 1u)) + __mul24(hi, int(2u * (byte >> 4) + 1u));
    }
    return total;
}
// IQ1_M pair as the single integer sum over its 64 weights of (2s+1)*(8*grid + delta)*q;
// the delta part uses the group sums of the quants (gs, computed once per activation load).
template <int TM>
__device__ __forceinline__ int pair_iq13(const uint8_t* lds, const Lut& L, const uint32_t* w, uint32_t scw, const uint32_t* a,
                                         const int* gs) {
    constexpr int S1 = Lay<TM>::C1 * 8;   // entry stride
    uint2 gr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int s = e / 4, g = e % 4;
        const uint32_t nib = (w[2] >> (16 * s + 4 * g)) & 15u;
        const uint32_t idx = ((w[s] >> (8 * g)) & 255u) | ((nib & 7u) << 8);
        gr[e] = *reinterpret_cast<const uint2*>(lds + L.iq1 + idx * S1);
    }
    int total = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        int m0 = 0, m1 = 0, d0 = 0, d1 = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int e = 4 * s + g;
            const uint32_t nib = (w[2] >> (16 * s + 4 * g)) & 15u;
            const uint32_t a0 = a[8 * s + 2 * g], a1 = a[8 * s + 2 * g + 1];
            const int m = sdot4(gr[e].y, a1, sdot4(gr[e].x, a0, 0));
            const int sg = gs[e];
            const int dl = (nib & 8u) ? -sg : sg;
            if (g < 2) { m0 += m; d0 += dl; } else { m1 += m; d1 += dl; }
        }
        const int c0 = int(2u * ((scw >> (6 * s)) & 7u) + 1u), c1 = int(2u * ((scw >> (6 * s + 3)) & 7u) + 1u);
        total += c0 * (8 * m0 + d0) + c1 * (8 * m1 + d1);
    }
    return total;
}

// One pair's contribution fma(fp16(d_w) * d_x, I, acc); the row is then summed
// over its lanes and scaled by 1/8 (q8k_core.hpp:87-91 regrouped: the integers
// per block are exact, the float order is this kernel's own).
// Io (null outside the parity trace): receives the pair's integer.
template <int T, int TM>
__device__ __forceinline__ float pair_term(const uint8_t* lds, const Lut& L, const Raw3& r, int p, const uint32_t* a,
                                           const int* gs, float dx, float acc, int* Io) {
    int I;
    uint32_t d16;
    if constexpr (T == kIQ2_XXS) {
        I = pair_xxs3<TM>(lds, L, r.w, a);
        d16 = r.h[0];
    } else if constexpr (T == kIQ2_XS) {
        I = pair_xs3<TM>(lds, L, r.w, r.h[0], a);
        d16 = r.h[1];
    } else {
        const uint32_t scw = ((p & 2) ? r.w[4] : r.w[3]) >> (16 * (p & 1));
        I = pair_iq13<TM>(lds, L, r.w, scw, a, gs);
        d16 = ((r.w[3] >> 12) & 0xfu) | ((r.w[3] >> 24) & 0xf0u) | ((r.w[4] >> 4) & 0xf00u) | ((r.w[4] >> 16) & 0xf000u);
    }
    if (Io) *Io = I;
    return fmaf(__fmul_rn(h2f(d16), dx), float(I), acc);
}
template <int T, int TM>
__device__ __forceinline__ bool has_type() {
    return (T == kIQ2_XXS && (TM & 1)) || (T == kIQ2_XS && (TM & 2)) || (T == kIQ1_M && (TM & 4));
}
// Lane partial of one row (TM: types possible for this row; LT: types held in
// LDS). Io (null outside the parity trace): the lane's P pair integers.
template <int TM, int LT, int P>
__device__ __forceinline__ float row_sum(const uint8_t* lds, const Lut& L, int type, const Raw3* r, const Act3<P>& A, int l,
                                         int LPR, int* Io = nullptr) {
    float acc = 0.0f;
    if constexpr (TM == 1 || TM == 2 || TM == 4) {
        constexpr int T = TM == 1 ? kIQ2_XXS : TM == 2 ? kIQ2_XS : kIQ1_M;
#pragma unroll
        for (int j = 0; j < P; ++j)
            acc = pair_term<T, LT>(lds, L, r[j], l + LPR * j, A.a[j], A.gs[j], A.d[j], acc, Io ? Io + j : nullptr);
    } else {
        if (has_type<kIQ2_XXS, TM>() && type == kIQ2_XXS) {
#pragma unroll
            for (int j = 0; j < P; ++j)
                acc = pair_term<kIQ2_XXS, LT>(lds, L, r[j], l + LPR * j, A.a[j], A.gs[j], A.d[j], acc, Io ? Io + j : nullptr);
        } else if (has_type<kIQ2_XS, TM>() && type == kIQ2_XS) {
#pragma unroll
            for (int j = 0; j < P; ++j)
                acc = pair_term<kIQ2_XS, LT>(lds, L, r[j], l + LPR * j, A.a[j], A.gs[j], A.d[j], acc, Io ? Io + j : nullptr);
        } else if (has_type<kIQ1_M, TM>()) {
#pragma unroll
            for (int j = 0; j < P; ++j)
                acc = pair_term<kIQ1_M, LT>(lds, L, r[j], l + LPR * j, A.a[j], A.gs[j], A.d[j], acc, Io ? Io + j : nullptr);
        }
    }
    return acc;
}

// ---- the kernel --------------------------------------------------------------------------------
// NW waves per workgroup. LG x PG: lanes per gate/up row and pairs per lane
// (LG * PG * 64 == dim); LD x PD: the same for down rows (LD * PD * 64 == ff).
// GUT / DNT: block types among the gate/up / down matrices (bits 1 IQ2_XXS,
// 2 IQ2_XS, 4 IQ1_M). MG / MD: most gate/up slots / down passes one wave
// holds; WIN: gate/up slots in flight per wave; WIND: down passes in flight.
// TR: also write the parity trace (Layer3Args::tq8x ...); the untraced instance
// compiles none of it.
// DP: pairs of a down row when LD * PD * 64 exceeds ff (0: exactly LD * PD).
// Lanes past them load the row's last pair (in bounds) against zero activations.
template <int NW, int LG, int PG, int LD, int PD, int MG, int MD, int WIN, int WIND, int GUT, int DNT, bool TR, int DP>
__global__ __launch_bounds__(NW * 64, 1) void layer3_kernel(Layer3Args a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
    __shared__ uint32_t s_epoch;
    __shared__ int s_ids[16];
    __shared__ float s_w[16];
    __shared__ uint32_t s_hq_ready[16];   // epoch once pick i's Q8_K(h) is staged in LDS
    constexpr int TM = GUT | DNT;
    using LY = Lay<TM>;
    constexpr int RG = 64 / LG, RD = 64 / LD;
    constexpr int NPD = DP ? DP : LD * PD;   // live pairs of a down row
    static_assert(NPD <= LD * PD && (LD * PD - NPD) < LD, "only the last pair slot of a lane may be dead");
    const int t = threadIdx.x, lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);   // wave-uniform: keeps slot/pick/matrix math scalar
    const int G = gridDim.x, W = G * NW, gw = blockIdx.x * NW + wv;
    const int k = a.k, ff = a.ff, dim = a.dim;
    const int lG = lane % LG, rG = lane / LG, lD = lane % LD, rD = lane / LD;
    const int nbx = dim / 256, nbh = ff / 256;
    auto mark = [&](int n) {   // optional per-wave timeline (s_memrealtime, 100 MHz)
        if (a.trace && lane == 0) a.trace[size_t(gw) * 32 + n] = __builtin_amdgcn_s_memrealtime();
    };

    // ---- ids and matrix references of this wave's work, read before the
    // kernel's first global store so that they come through the scalar unit.
    // Slots past the wave's last repeat it and bad ids read expert 0, so every
    // path issues the same loads (the waits on them stay exact); gid < 0 marks
    // a slot whose result is not used. Passes likewise.
    const int sppG = ff / RG, SG = k * sppG;
    const int ng = SG > gw ? min(MG, (SG - gw + W - 1) / W) : 0;
    const int quads = dim / RD;
    const int nq_wg = quads > int(blockIdx.x) ? (quads - int(blockIdx.x) + G - 1) / G : 0;
    const int P = k * nq_wg;
    const int nd = P > wv ? min(MD, (P - wv + NW - 1) / NW) : 0;   // passes p = wv + NW*j, pick-major
    // pick indices first, then every id load, then the references: one wait
    int gslot[MG], gpick[MG], dpick[MD], drow[MD], gidr[MG], didr[MD];
#pragma unroll
    for (int j = 0; j < MG; ++j) {
        gslot[j] = gw + W * (j < ng ? j : ng - 1);
        gpick[j] = ng > 0 ? gslot[j] / sppG : 0;
    }
#pragma unroll
    for (int j = 0; j < MD; ++j) {
        const int p = wv + NW * (j < nd ? j : nd - 1);
        dpick[j] = nd > 0 ? p / nq_wg : 0;
        drow[j] = nd > 0 ? (int(blockIdx.x) + G * (p - dpick[j] * nq_wg)) * RD + rD : rD;
    }
    // lane i holds ids[i] (one load); a wave reads the ids it needs by readlane
    const int idv = lane < k ? a.ids[lane] : -1;
#pragma unroll
    for (int j = 0; j < MG; ++j) gidr[j] = __builtin_amdgcn_readlane(idv, gpick[j]);
#pragma unroll
    for (int j = 0; j < MD; ++j) didr[j] = __builtin_amdgcn_readlane(idv, dpick[j]);
    MRef gm[MG], um[MG], dm[MD];
    int gid[MG], did[MD];
#pragma unroll
    for (int j = 0; j < MG; ++j) {
        const bool ok = ng > 0 && gidr[j] >= 0 && gidr[j] < a.n_experts;
        gid[j] = (j < ng && ok) ? gidr[j] : -1;
        gm[j] = mref<GUT>(a, ok ? gidr[j] : 0, 0, ff, nbx);
        um[j] = mref<GUT>(a, ok ? gidr[j] : 0, 1, ff, nbx);
    }
#pragma unroll
    for (int j = 0; j < MD; ++j) {
        const bool ok = nd > 0 && didr[j] >= 0 && didr[j] < a.n_experts;
        did[j] = (j < nd && ok) ? didr[j] : -1;
        dm[j] = mref<DNT>(a, ok ? didr[j] : 0, 2, dim, nbh);
    }
    // ---- codebook single copies and x (issued ahead of the weight loads)
    {
        const uint8_t* gt = reinterpret_cast<const uint8_t*>(a.tables);
        if constexpr (TM & 3) lds_dma<NW>(lds, LY::HQ, gt + kG_SGN, 2048, wv, lane);
        if constexpr (TM & 1) lds_dma<NW>(lds, LY::HQ + 2048, gt + kG_XXS, 2048, wv, lane);
        if constexpr (TM & 2) lds_dma<NW>(lds, LY::HQ + 4096, gt + kG_XS, 4096, wv, lane);
        if constexpr (TM & 4) lds_dma<NW>(lds, LY::C1 > 1 ? LY::HQ : LY::IQ1, gt + kG_IQ1, 16384, wv, lane);
    }
    constexpr int UX = (kMaxRowK / 256 + NW - 1) / NW;
    float4 xv[UX];
#pragma unroll
    for (int u = 0; u < UX; ++u) {
        const int b = wv + NW * u;
        if (b < nbx) xv[u] = reinterpret_cast<const float4*>(a.x + 256 * b)[lane];
    }

    // ids and weights for the combine, and the epoch word: loaded now, used later
    const int cid = idv;
    float cw = 0.0f;
    if (wv == 0 && lane < k) cw = a.w[lane];
    uint32_t* ctl = a.ctl;   // [0] epoch of the last launch, [1] arrivals
    const uint32_t e_prev = coh_ld32(ctl);

    // ---- the first WIN gate/up slots
    Raw3 rg[WIN][PG], ru[WIN][PG];
    auto load_slot = [&](int j, int b) {
        const int row0 = (gslot[j] % sppG) * RG;
#pragma unroll
        for (int q = 0; q < PG; ++q) {
            load_pair_t<GUT>(rg[b][q], gm[j], row0, rG, lG + LG * q);
            load_pair_t<GUT>(ru[b][q], um[j], row0, rG, lG + LG * q);
        }
    };
    if (ng > 0) {
#pragma unroll
        for (int j = 0; j < WIN; ++j) load_slot(j, j);
    }
    mark(0);

    // ---- codebooks replicated, x quantized (LDS), epoch
    constexpr int LPP = loads_per_pair<GUT>();
    if (LPP > 0 && ng > 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPP > 0 ? WIN * PG * 2 * LPP : 0));   // all but the slot loads
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    lds_barrier();   // every wave's codebook chunks are in
    mark(1);
    if constexpr (TM & 3) lds_replicate<NW * 64>(lds, LY::SGN, LY::HQ, 128, 16, LY::CS, t);
    if constexpr (TM & 1) lds_replicate<NW * 64>(lds, LY::XXS, LY::HQ + 2048, 256, 8, LY::CXXS, t);
    if constexpr (TM & 2) lds_replicate<NW * 64>(lds, LY::XS, LY::HQ + 4096, 512, 8, LY::CXS, t);
    if constexpr ((TM & 4) && LY::C1 > 1) lds_replicate<NW * 64>(lds, LY::IQ1, LY::HQ, 2048, 8, LY::C1, t);
#pragma unroll
    for (int u = 0; u < UX; ++u) {
        const int b = wv + NW * u;
        if (b < nbx) {
            const float v[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
            const Q8Lane q = q8k_lane(v, lane);
            if (!q.finite && lane == 0) set_err(a.err, kDevErrNonFinite);
            *reinterpret_cast<uint32_t*>(lds + LY::XQ + qswz(256 * b + 4 * lane)) = q.packed;
            if (lane == 0) reinterpret_cast<float*>(lds + LY::XD)[b] = q.d;
        }
    }
    if (wv == 0 && lane < k) {
        s_ids[lane] = cid;
        s_w[lane] = cw;
    }
    if (t < 16) s_hq_ready[t] = 0u;
    // Epoch 0 is never used: tags start zeroed (and s_hq_ready is zeroed every
    // launch), so a launch tagging with 0 would read words no one has written.
    // After 2^32 - 1 launches the count wraps from 0xffffffff to 1.
    if (t == 0) s_epoch = e_prev + 1u == 0u ? 1u : e_prev + 1u;
    lds_barrier();
    const uint32_t epoch = s_epoch;
    if constexpr (TR) {   // workgroup 0's staged Q8_K(x), as the gate/up rows read it
        if (blockIdx.x == 0 && a.tq8x)
            for (int b = wv; b < nbx; b += NW)
                trace_q8_block(a.tq8x + 292 * b, reinterpret_cast<const float*>(lds + LY::XD)[b],
                               *reinterpret_cast<const uint32_t*>(lds + LY::XQ + qswz(256 * b + 4 * lane)), lane);
    }
    const size_t rec = 2 * size_t(ff) * nbx + size_t(dim) * nbh;   // trace integers per pick
    // Arrival: this workgroup has read the epoch word. Whoever arrives last
    // advances it, at the end of the kernel (the count is not awaited before).
    uint32_t arrived = 0;
    if (t == 0) arrived = __hip_atomic_fetch_add(ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (gw < k && lane == 0) {   // each bad id is reported once
        const int id = s_ids[gw];
        if (id < 0 || id >= a.n_experts) set_err(a.err, kDevErrExpertId);
    }
    mark(2);

    const Lut L = make_lut<TM>(lane);
    Raw3 rd[WIND + 1][PD];   // ring of down passes in flight
    auto load_pass = [&](int j) {
#pragma unroll
        for (int q = 0; q < PD; ++q)
            load_pair_t<DNT>(rd[j % (WIND + 1)][q], dm[j], drow[j] - rD, rD, min(lD + LD * q, NPD - 1));
    };
    int issued = 0;   // down passes issued so far (wave-uniform)

    // ---- gate/up; its last WIND iterations start the down stream
    {
        Act3<PG> A;
#pragma unroll
        for (int q = 0; q < PG; ++q) {
            const int p = lG + LG * q;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4 v = *reinterpret_cast<const uint4*>(lds + LY::XQ + qswz(64 * p + 16 * c));
                A.a[q][4 * c] = v.x; A.a[q][4 * c + 1] = v.y; A.a[q][4 * c + 2] = v.z; A.a[q][4 * c + 3] = v.w;
            }
            A.d[q] = reinterpret_cast<const float*>(lds + LY::XD)[p >> 2];
        }
        group_sums<GUT>(A);
        // Fully unrolled (no break): the per-slot references stay in registers.
#pragma unroll
        for (int j = 0; j < MG; ++j) {
            // Older waves win the SIMD arbiter; the younger half of the workgroup
            // runs at wave priority 1 for two thirds of its slots so that both
            // halves finish gate/up together (the down phase waits for the last).
            if (j == 0 && wv >= NW / 2) __builtin_amdgcn_s_setprio(1);
            if (j == (2 * MG) / 3) __builtin_amdgcn_s_setprio(0);
            if (j < ng) {
                if (j >= 1 && j + WIN - 1 < MG) load_slot(j + WIN - 1, (j + WIN - 1) % WIN);
                if (j >= MG - WIND && nd > 0) {   // static position for the common case ng == MG
                    load_pass(j - (MG - WIND));
                    issued = j - (MG - WIND) + 1;
                }
                const int s = gslot[j];
                const int i = s / sppG, row = (s - i * sppG) * RG + rG;
                float hv = 0.0f;
                if (gid[j] >= 0) {
                    int Ig[PG], Iu[PG];
                    const float g = gsum<LG>(row_sum<GUT, TM, PG>(lds, L, gm[j].type, rg[j % WIN], A, lG, LG, TR ? Ig : nullptr));
                    const float u = gsum<LG>(row_sum<GUT, TM, PG>(lds, L, gm[j].type, ru[j % WIN], A, lG, LG, TR ? Iu : nullptr));
                    hv = silu_mul3(__fmul_rn(0.125f, g), __fmul_rn(0.125f, u), a.lim);
                    if constexpr (TR) {   // the row's block integers: a quad holds one block's four pairs
#pragma unroll
                        for (int q = 0; q < PG; ++q) {
                            const int bg = quad_isum(Ig[q]), bu = quad_isum(Iu[q]);
                            if (a.tint && (lG & 3) == 0) {
                                const size_t o = size_t(i) * rec + size_t(row) * nbx + size_t((lG + LG * q) >> 2);
                                a.tint[o] = bg;
                                a.tint[o + size_t(ff) * nbx] = bu;
                            }
                        }
                    }
                }
                if (lG == LG - 1) coh_st64(a.htag + size_t(i) * ff + row, tag_word(__float_as_uint(hv), epoch));
                if constexpr (TR) {
                    if (a.th && lG == LG - 1 && gid[j] >= 0) a.th[size_t(i) * ff + row] = hv;
                }
                mark(8 + j);
            }
        }
    }
    mark(3);
    __builtin_amdgcn_s_setprio(0);
    // waves with fewer slots start their down stream here
#pragma unroll
    for (int j = 0; j < WIND; ++j)
        if (j < MD && j >= issued && nd > 0) load_pass(j);

    // ---- Q8_K(h): block q of the k*ff/256 blocks belongs to wave q*stride
    const int nqb = k * nbh;
    const int stride = W / nqb;
    if (stride >= 1 && gw % stride == 0 && gw / stride < nqb) {
        const int qb = gw / stride, i = qb / nbh, bb = qb - i * nbh;
        const uint64_t* src = a.htag + size_t(i) * ff + 256 * bb + 4 * lane;
        uint64_t v[4];
        uint32_t polls = 0;
        for (;;) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = coh_ld64(src + j);
            bool ok = true;
#pragma unroll
            for (int j = 0; j < 4; ++j) ok = ok && uint32_t(v[j] >> 32) == epoch;
            if (__all(ok)) break;
            if (++polls > kPollLimit) {
                if (lane == 0) set_err(a.err, kDevErrTimeout);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        const float hv[4] = {__uint_as_float(uint32_t(v[0])), __uint_as_float(uint32_t(v[1])),
                             __uint_as_float(uint32_t(v[2])), __uint_as_float(uint32_t(v[3]))};
        const Q8Lane q = q8k_lane(hv, lane);
        if (!q.finite && lane == 0) set_err(a.err, kDevErrNonFinite);
        coh_st64(a.hqtag + size_t(i) * (ff / 4) + 64 * bb + lane, tag_word(q.packed, epoch));
        if (lane == 0) coh_st64(a.hdtag + qb, tag_word(__float_as_uint(q.d), epoch));
    }
    mark(4);

    // ---- down passes, pick by pick, into LDS
    float* ys = reinterpret_cast<float*>(lds + LY::Y);
    const int hq_stride = ff + 64;
    {
        int cur = -1;
        Act3<PD> B;
#pragma unroll
        for (int j = 0; j < MD; ++j) {
            if (j < nd) {
                if (j + WIND < MD && j + WIND < nd) load_pass(j + WIND);
                const int i = dpick[j];
                float y = 0.0f;
                if (did[j] >= 0) {
                    if (i != cur) {
                        uint8_t* hq = lds + LY::HQ + i * hq_stride;
                        if ((i * nq_wg) % NW == wv) {
                            // this wave holds the workgroup's first pass of pick i: stage the
                            // pick's Q8_K(h) once all its tagged words are in
                            const int per = ff / 256;   // tagged words per lane (ff <= 4096: at most 16)
                            const uint64_t* src = a.hqtag + size_t(i) * (ff / 4) + per * lane;
                            uint64_t w16[16];
                            uint64_t dw = 0;
                            uint32_t polls = 0;
                            for (;;) {
#pragma unroll
                                for (int c = 0; c < 16; ++c)
                                    if (c < per) w16[c] = coh_ld64(src + c);
                                if (lane < nbh) dw = coh_ld64(a.hdtag + size_t(i) * nbh + lane);
                                bool ok = lane >= nbh || uint32_t(dw >> 32) == epoch;
#pragma unroll
                                for (int c = 0; c < 16; ++c)
                                    if (c < per) ok = ok && uint32_t(w16[c] >> 32) == epoch;
                                if (__all(ok)) break;
                                if (++polls > kPollLimit) {
                                    if (lane == 0) set_err(a.err, kDevErrTimeout);
                                    break;
                                }
                                __builtin_amdgcn_s_sleep(2);
                            }
#pragma unroll
                            for (int c = 0; c < 16; ++c)
                                if (c < per) *reinterpret_cast<uint32_t*>(hq + qswz(4 * (per * lane + c))) = uint32_t(w16[c]);
                            if (lane < nbh) reinterpret_cast<uint32_t*>(hq + ff)[lane] = uint32_t(dw);
                            // LDS writes of one wave land in order: the flag goes last
                            if (lane == 0) __hip_atomic_store(&s_hq_ready[i], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        } else {
                            uint32_t polls = 0;
                            while (__hip_atomic_load(&s_hq_ready[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != epoch) {
                                if (++polls > kPollLimit) {
                                    if (lane == 0) set_err(a.err, kDevErrTimeout);
                                    break;
                                }
                                __builtin_amdgcn_s_sleep(1);
                            }
                        }
#pragma unroll
                        for (int q = 0; q < PD; ++q) {
                            const int p = lD + LD * q;
                            const bool live = p < NPD;   // a dead pair slot: zero activations
                            const int pl = live ? p : NPD - 1;
#pragma unroll
                            for (int c = 0; c < 4; ++c) {
                                const uint4 v = *reinterpret_cast<const uint4*>(hq + qswz(64 * pl + 16 * c));
                                B.a[q][4 * c] = live ? v.x : 0u; B.a[q][4 * c + 1] = live ? v.y : 0u;
                                B.a[q][4 * c + 2] = live ? v.z : 0u; B.a[q][4 * c + 3] = live ? v.w : 0u;
                            }
                            B.d[q] = live ? reinterpret_cast<const float*>(hq + ff)[pl >> 2] : 0.0f;
                        }
                        group_sums<DNT>(B);
                        cur = i;
                    }
                    int Id[PD];
                    y = __fmul_rn(0.125f, gsum<LD>(row_sum<DNT, TM, PD>(lds, L, dm[j].type, rd[j % (WIND + 1)], B, lD, LD,
                                                                        TR ? Id : nullptr)));
                    if constexpr (TR) {
#pragma unroll
                        for (int q = 0; q < PD; ++q) {
                            const int bi = quad_isum(Id[q]);
                            if (a.tint && (lD & 3) == 0 && lD + LD * q < NPD)
                                a.tint[size_t(i) * rec + 2 * size_t(ff) * nbx + size_t(drow[j]) * nbh +
                                       size_t((lD + LD * q) >> 2)] = bi;
                        }
                    }
                }
                if (lD == LD - 1) ys[(wv + NW * j) * RD + rD] = y;
                if (j == 0) mark(5);
            }
        }
    }
    mark(6);
    lds_barrier();
    if constexpr (TR) {   // workgroup 0's staged Q8_K(h) of every pick it staged, as its down passes read it
        if (blockIdx.x == 0 && a.tq8h)
            for (int blk = wv; blk < k * nbh; blk += NW) {
                const int i = blk / nbh, bb = blk - i * nbh;
                if (s_hq_ready[i] != epoch) continue;   // a bad id: nothing staged
                const uint8_t* hq = lds + LY::HQ + i * hq_stride;
                trace_q8_block(a.tq8h + 292 * blk, reinterpret_cast<const float*>(hq + ff)[bb],
                               *reinterpret_cast<const uint32_t*>(hq + qswz(256 * bb + 4 * lane)), lane);
            }
    }

    // ---- fixed-order combine of this workgroup's rows
    const int nrows = nq_wg * RD;
    for (int r = t; r < nrows; r += NW * 64) {
        const int qq = r / RD, rr = r - qq * RD;
        const int orow = (int(blockIdx.x) + G * qq) * RD + rr;
        int order[16];
        for (int i = 0; i < k; ++i) order[i] = i;
        for (int i = 1; i < k; ++i)
            for (int j = i; j > 0 && s_ids[order[j]] < s_ids[order[j - 1]]; --j) {
                const int tmp = order[j]; order[j] = order[j - 1]; order[j - 1] = tmp;
            }
        float acc = 0.0f;
        for (int s2 = 0; s2 < k; ++s2) {
            const int i = order[s2];
            const float yi = ys[(i * nq_wg + qq) * RD + rr];
            if constexpr (TR) {
                if (a.ty) a.ty[size_t(i) * dim + orow] = yi;
            }
            acc = fmaf(s_w[i], yi, acc);
        }
        if (a.shared) acc = __fadd_rn(acc, a.shared[orow]);
        a.out[orow] = acc;
    }
    mark(7);
    if (t == 0 && arrived == uint32_t(G) - 1u) {   // every workgroup has read the epoch word
        coh_st32(ctl, epoch);
        coh_st32(ctl + 1, 0u);
    }
}

// ---- launcher ------------------------------------------------------------------------------
template <int NW, int LG, int PG, int LD, int PD, int MG, int MD, int WIN, int WIND, int GUT, int DNT, int DP = 0>
static hipError_t launch3(const Layer3Args& args, int grid, hipStream_t s, hipEvent_t stop) {
    const bool tr = args.tq8x || args.tq8h || args.th || args.tint || args.ty;
    constexpr int RG = 64 / LG, RD = 64 / LD;
    const int W = grid * NW;
    const int SG = args.k * (args.ff / RG);
    const int quads = args.dim / RD;
    const int nq_wg = (quads + grid - 1) / grid;
    const int P = args.k * nq_wg;
    const int nqb = args.k * (args.ff / 256);
    if ((SG + W - 1) / W > MG || (P + NW - 1) / NW > MD || nqb > W || P * RD > kYStage || grid > quads ||
        args.ff > 4096 || Lay<GUT | DNT>::HQ + args.k * (args.ff + 64) > kLdsBytes ||
        Lay<GUT | DNT>::HQ + 16384 > kLdsBytes)   // the codebooks' single copies are staged there
        return hipErrorNotSupported;
    if (tr)
        hipExtLaunchKernelGGL((layer3_kernel<NW, LG, PG, LD, PD, MG, MD, WIN, WIND, GUT, DNT, true, DP>), dim3(grid),
                              dim3(NW * 64), 0, s, nullptr, stop, 0, args);
    else
        hipExtLaunchKernelGGL((layer3_kernel<NW, LG, PG, LD, PD, MG, MD, WIN, WIND, GUT, DNT, false, DP>), dim3(grid),
                              dim3(NW * 64), 0, s, nullptr, stop, 0, args);
    return hipGetLastError();
}

// Instances by block-type set: (gate/up types, down types) exactly ({IQ2_XXS},
// {IQ2_XS}) and ({IQ1_M}, {IQ1_M}) have their own instances; anything else
// takes the all-types one.
template <int NW, int LG, int PG, int LD, int PD, int MG, int MD, int WIN, int WIND, int DP = 0>
static hipError_t launch3_types(const Layer3Args& args, int gu_types, int dn_types, int grid, hipStream_t s,
                                hipEvent_t stop) {
    if (gu_types == 1 && dn_types == 2)
        return launch3<NW, LG, PG, LD, PD, MG, MD, WIN, WIND, 1, 2, DP>(args, grid, s, stop);
    if (gu_types == 4 && dn_types == 4)
        return launch3<NW, LG, PG, LD, PD, MG, MD, WIN, WIND, 4, 4, DP>(args, grid, s, stop);
    return launch3<NW, LG, PG, LD, PD, MG, MD, WIN, WIND, 7, 7, DP>(args, grid, s, stop);
}

hipError_t launch_layer3(const Layer3Args& args, int gu_types, int dn_types, int cus, hipStream_t s, hipEvent_t stop) {
    if (args.k < 1 || args.k > 16 || args.dim > kMaxRowK) return hipErrorNotSupported;
    int lg, pg, ld, pd;
    if (!row_shape(args.dim, lg, pg) || !row_shape(args.ff, ld, pd)) return hipErrorNotSupported;
    if (lg == 16 && pg == 5 && ld == 4 && pd == 9)   // 5120 x 2304 (the real expert), down rows as 16 lanes x 3 pairs
        return launch3_types<8, 16, 5, 16, 3, 3, 5, 1, 1, 36>(args, gu_types, dn_types, std::min(cus, args.dim / 4),
                                                              s, stop);
    const int RD = 64 / ld;
    const int grid = std::min(cus, args.dim / RD);
    if (lg == 64 && pg == 1 && ld == 16 && pd == 3)   // 4096 x 3072
        return launch3_types<8, 64, 1, 16, 3, 9, 3, 3, 1>(args, gu_types, dn_types, grid, s, stop);
    if (lg == 16 && pg == 1 && ld == 8 && pd == 1)    // 1024 x 512
        return launch3<8, 16, 1, 8, 1, 6, 2, 3, 1, 7, 7>(args, grid, s, stop);
    if (lg == 4 && pg == 1 && ld == 4 && pd == 3)     // 256 x 768
        return launch3<8, 4, 1, 4, 3, 6, 2, 3, 1, 7, 7>(args, grid, s, stop);
    if (lg == 8 && pg == 1 && ld == 4 && pd == 1)     // 512 x 256
        return launch3<8, 8, 1, 4, 1, 6, 2, 3, 1, 7, 7>(args, grid, s, stop);
    if (lg == 4 && pg == 1 && ld == 4 && pd == 1)     // 256 x 256
        return launch3<8, 4, 1, 4, 1, 6, 2, 3, 1, 7, 7>(args, grid, s, stop);
    return hipErrorNotSupported;
}

}  // namespace xl::dev
