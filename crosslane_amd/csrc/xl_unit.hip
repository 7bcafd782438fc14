// The routed-expert layer in one launch, organized by units (gfx950), for
// layers whose gate/up matrices are all IQ2_XXS and whose down matrices are all
// IQ2_XS (configs 0 and 1).
//
// A unit is one 256-row block b of one pick i's SwiGLU output h: its gate/up
// rows produce it, and it is one 256-column block of that pick's down matrix.
// The grid's waves form NG groups of WPU = 256 / RG waves (RG gate/up rows per
// wave slot); group g owns units g, g + NG, g + 2 NG, ... (unit u = pick u / nbh,
// block u % nbh). Slot j of a wave computes row w (its place in the group) of
// unit g + NG j, so a unit's h is complete once its group's waves are past that
// slot, long before the layer's last rows are read. LAG slots later (LAG = 5 for
// more than three units per group) every wave of the group computes its 16 rows
// of the unit's down block:
//
//   h exchange  as the streaming kernel's: h goes out as plain 32-bit words into
//               one of two sentinel-filled buffers (launch parity), readers poll
//               for non-sentinel words;
//   Q8_K(h)     per workgroup, one wave (the unit's quantizer, wave j mod NW)
//               loads the unit's 256 h words LAG - 1 slots after they were produced,
//               quantizes them (q8k_core.hpp:30-38) into LDS and raises an LDS
//               flag; the other waves read the staged block one slot later;
//   down        lane l of a wave takes row 16 w + l / 4, pair l mod 4 of the
//               block: the quad's four pair integers sum to the row's exact block
//               integer, which becomes the float partial fp16(d_w) * d_h * int,
//               stored per (unit, row);
//   combine     once every wave has stored its partials (a device counter), each
//               workgroup sums its 16-row groups' partials in a fixed order: per
//               pick 1/8 * (P_0 + P_1 + ...) over ascending blocks, then ascending
//               expert id, out = fma(w, y, out), + shared
//               (engine/strata/warm/runtime.cpp:183-188).
//
// The down weights stream under the gate/up slots (each unit's are loaded LAG
// slots ahead), so HBM reads the layer's bytes as one stream and the down
// arithmetic of early units runs while later gate/up rows arrive. Every wait is
// bounded (kDevErrTimeout on expiry); waits point backwards only (down waits on
// gate/up of earlier slots, the combine on every down), and the grid is one
// workgroup per CU, so the grid drains.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "xl_dev.hpp"
#include "xl_iq2.hpp"

namespace xl::dev {
namespace {

// ---- LDS map (bytes) ---------------------------------------------------------------
constexpr int kU_SGN = 0;          // sign masks: 256 rows x 32 copies x 8 B {M.lo, M.hi}
constexpr int kU_XXS = 65536;      // IQ2_XXS grid: 256 x 32 copies x 8 B
constexpr int kU_XS = 131072;      // IQ2_XS grid: 512 x 4 copies x 8 B
constexpr int kU_XQ = 147456;      // Q8_K(x): dim quants (swizzled), then 16 block scales
constexpr int kU_HQ = kU_XQ + 4096 + 64;   // the group's units' Q8_K(h): 256 quants + scale per unit slot
constexpr int kU_HQStride = 272;
constexpr int kU_MaxSlots = 24;
constexpr int kU_Bytes = kU_HQ + kU_MaxSlots * kU_HQStride;
static_assert(kU_Bytes <= 160 * 1024 - 256, "LDS map");
constexpr int kG_XXS = 2048, kG_XS = 4096;   // expanded codebooks in the context's table buffer

struct USmem {
    uint8_t b[kU_Bytes];   // first, so that its LDS address is 0 and table bases fold into offsets
    int ids[16];
    float w[16];
    int order[16];
    uint32_t parity;
    uint32_t ready[kU_MaxSlots];   // 1 once unit slot j's Q8_K(h) is staged
    float yv[16][17];              // combine: per output row, per pick
};

// Raw words of one down pair (IQ2_XS): 16 B of codes, the pair's two scale bytes, the block's d.
struct DRaw {
    uint32_t w[4];
    uint16_t sc, d;
};

// NW waves per workgroup; LG lanes per gate/up row (RG = 64 / LG rows per wave
// slot, LG * 64 == dim); MG slots per wave; WIN gate/up slots in flight.
// LAG: slots between a unit's gate/up and its down.
template <int NW, int LG, int MG, int WIN, int LAG, bool TR>
__global__ __launch_bounds__(NW * 64, 1) void unit_kernel(Layer3Args a) {
    constexpr int kLag = LAG;
    static_assert(WIN <= MG && MG <= kU_MaxSlots && MG <= 32, "slots");
    __shared__ __attribute__((aligned(16))) USmem sm;
    uint8_t* const lds = sm.b;
    constexpr int RG = 64 / LG;
    constexpr int WPU = 256 / RG;   // waves per unit (a group)
    const int t = threadIdx.x, lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int G = gridDim.x, gw = blockIdx.x * NW + wv;
    const int NG = G * NW / WPU;                 // groups
    const int grp = gw / WPU, wi = gw - grp * WPU;   // this wave's group and place in it
    const int k = a.k, ff = a.ff, dim = a.dim;
    const int nbx = dim / 256, nbh = ff / 256;
    const int U = k * nbh;
    const int lG = lane % LG, rG = lane / LG;
    const int nu = U > grp ? min(MG, (U - grp + NG - 1) / NG) : 0;   // this group's units
    auto unit_of = [&](int j) { return grp + NG * j; };
    // Optional per-wave timeline (s_memrealtime, 100 MHz; xl_profile_timeline):
    // 0 start, 1 LDS staged, 2 + j slot j's gate/up done, 14 + j slot j's down
    // done (j < 12), 26 .. 28 slots 0 .. 2's Q8_K(h) staged (their quantizer
    // waves), 29 partials counted, 30 combine may start, 31 end.
    auto mark = [&](int n) {
        if (a.trace && lane == 0) a.trace[size_t(gw) * 32 + n] = __builtin_amdgcn_s_memrealtime();
    };
    mark(0);

    // ---- ids: lane i < k holds ids[i]; per slot the pick and validity (wave-uniform)
    const int idl = a.ids[lane < k ? lane : k - 1];
    const int idv = lane < k ? idl : -1;
    const float cw = a.w[lane < k ? lane : k - 1];
    // Lane j < MG: slot j's expert (0 for bad ids: read, then discarded), read back
    // by v_readlane so that no per-slot array lives in memory.
    uint32_t ok_mask;   // bit j: slot j is a unit with a valid expert id
    int eidv;
    {
        const int j = lane & 31;
        const int u = j < nu ? unit_of(j) : (nu > 0 ? unit_of(nu - 1) : 0);
        const int id = __shfl(idv, min(u / nbh, 15));
        const bool ok = j < nu && j < MG && id >= 0 && id < a.n_experts;
        eidv = ok ? id : 0;
        ok_mask = uint32_t(__builtin_amdgcn_ballot_w64(ok && lane < 32));
    }
    auto eid = [&](int j) { return __builtin_amdgcn_readlane(eidv, j); };
    uint32_t go1, go2, do1, do2;
    plane_offs(kIQ2_XXS, uint64_t(ff) * uint64_t(nbx), go1, go2);
    plane_offs(kIQ2_XS, uint64_t(dim) * uint64_t(nbh), do1, do2);
    auto matrix = [&](int e, int role, uint32_t o1, uint32_t o2, int type, int nb) {
        return MRef{a.slab + uint64_t(e) * a.estride + a.roff[role], o1, o2, type, nb};
    };
    auto uclamp = [&](int j) { return j < nu ? unit_of(j) : (nu > 0 ? unit_of(nu - 1) : 0); };

    // ---- codebook rows and x first, then the first slots
    constexpr int NT = NW * 64;
    constexpr int NX = (4096 + NT - 1) / NT, NS = (1024 + NT - 1) / NT;
    uint2 vx[NX], vs[NS];
    {
        const uint2* gx = reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(a.tables) + kG_XXS);
        const uint2* gs = reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(a.tables) + kG_XS);
#pragma unroll
        for (int i = 0; i < NX; ++i) vx[i] = gx[min(t + NT * i, 4095) >> 4];
#pragma unroll
        for (int i = 0; i < NS; ++i) vs[i] = gs[min(t + NT * i, 1023) >> 1];
    }
    constexpr int UX = (16 + NW - 1) / NW;
    float4 xv[UX];
#pragma unroll
    for (int u = 0; u < UX; ++u) {
        const int b = wv + NW * u;
        xv[u] = reinterpret_cast<const float4*>(a.x + 256 * (b < nbx ? b : 0))[lane];
    }
    // ctl[2]: launch count, shared with the streaming kernel (its parity picks the
    // h buffer and this launch's set of partial counters); ctl[3]: arrivals.
    uint32_t* ctl = a.ctl + 2;
    const uint32_t e_prev = coh_ld32(ctl);

    Raw3 rg[WIN], ru[WIN];
    auto load_slot = [&]<int j>() {
        const int u = uclamp(j), b = u % nbh;
        const int row0 = 256 * b + wi * RG;   // the wave's first row of the unit
        load_pair_t<1>(rg[j % WIN], matrix(eid(j), 0, go1, go2, kIQ2_XXS, nbx), row0, rG, lG);
        load_pair_t<1>(ru[j % WIN], matrix(eid(j), 1, go1, go2, kIQ2_XXS, nbx), row0, rG, lG);
    };
    static_for<WIN>([&]<int j>() { load_slot.template operator()<j>(); });

    // Down pair of unit slot j: row 16 wi + lane / 4, pair lane % 4 of the unit's block.
    DRaw rd[kLag + 1];
    const int drow = 16 * wi + (lane >> 2);
    auto load_down = [&]<int j>() {
        const int u = uclamp(j), b = u % nbh;
        const MRef m = matrix(eid(j), 2, do1, do2, kIQ2_XS, nbh);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)m.base, (short)0, -1, 0x00020000);
        const uint32_t pe = uint32_t(drow * nbh * 4 + (lane & 3));   // pair index of block 0 in the row
        const v4u32 q = __builtin_amdgcn_raw_buffer_load_b128(rs, pe * 16, uint32_t(b) * 64, kNT);
        DRaw& r = rd[j % (kLag + 1)];
        r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
        r.sc = __builtin_amdgcn_raw_buffer_load_b16(rs, pe * 2, m.o1 + uint32_t(b) * 8, kNT);
        r.d = __builtin_amdgcn_raw_buffer_load_b16(rs, uint32_t(drow * nbh) * 2, m.o2 + uint32_t(b) * 2, kNT);
    };

    // ---- LDS: sign rows (computed), grid copies, Q8_K(x); one barrier
#pragma unroll
    for (int i = 0; i < NX; ++i) {
        const int c = t + NT * i;
        if (c < 4096) {
            const uint2 r = sign_row(uint32_t(c) >> 4);
            *reinterpret_cast<uint4*>(lds + kU_SGN + 16 * c) = make_uint4(r.x, r.y, r.x, r.y);
        }
    }
#pragma unroll
    for (int i = 0; i < NX; ++i)
        if (t + NT * i < 4096)
            *reinterpret_cast<uint4*>(lds + kU_XXS + 16 * (t + NT * i)) = make_uint4(vx[i].x, vx[i].y, vx[i].x, vx[i].y);
#pragma unroll
    for (int i = 0; i < NS; ++i)
        if (t + NT * i < 1024)
            *reinterpret_cast<uint4*>(lds + kU_XS + 16 * (t + NT * i)) = make_uint4(vs[i].x, vs[i].y, vs[i].x, vs[i].y);
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
                *reinterpret_cast<uint32_t*>(lds + kU_XQ + qswz(256 * b + 4 * lane)) = xp[u];
                if (lane == 0) reinterpret_cast<float*>(lds + kU_XQ + 4096)[b] = xd[u];
            }
        }
    }
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
    if (t < kU_MaxSlots) sm.ready[t] = 0u;
    if (t == 0) sm.parity = (e_prev + 1u) & 1u;
    lds_barrier();
    if constexpr (TR) {
        if (blockIdx.x == 0 && a.tq8x)
            for (int b = wv; b < nbx; b += NW)
                trace_q8_block(a.tq8x + 292 * b, reinterpret_cast<const float*>(lds + kU_XQ + 4096)[b],
                               *reinterpret_cast<const uint32_t*>(lds + kU_XQ + qswz(256 * b + 4 * lane)), lane);
    }
    mark(1);
    const uint32_t parity = __builtin_amdgcn_readfirstlane(sm.parity);
    float* const hcur = a.hbuf + size_t(parity) * kHBufWords;
    // Partial counters: eight (workgroups blockIdx mod 8 count into counter
    // blockIdx mod 8, 128 bytes apart, so that their atomics do not queue on one
    // address), one set per launch parity; workgroup 0 clears the other set for
    // the next launch (the previous launch, its user, is over). Every kernel that
    // advances the launch count clears that set (the streaming kernel too), so a
    // launch always finds its own set cleared.
    uint32_t* const pcnt = a.ucnt + size_t(parity) * 256;
    if (blockIdx.x == 0 && t < 8) coh_st32(a.ucnt + size_t(parity ^ 1u) * 256 + 32 * t, 0u);
    // Arrival ticket, awaited only at the end: the last workgroup to arrive (every
    // other one has read the launch count) advances the launch count.
    uint32_t arrived = 0;
    if (t == 0) arrived = __hip_atomic_fetch_add(ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (gw < k && lane == 0) {
        const int id = sm.ids[gw];
        if (id < 0 || id >= a.n_experts) set_err(a.err, kDevErrExpertId);
    }
    {   // the other buffer (used by the previous launch) back to the sentinel for the next one
        float* const hnext = a.hbuf + size_t(parity ^ 1u) * kHBufWords;
        const uint4 s4 = make_uint4(kSentinel, kSentinel, kSentinel, kSentinel);
        for (int c = int(blockIdx.x) * NW * 64 + t; c < kHBufWords / 4; c += G * NW * 64)
            reinterpret_cast<uint4*>(hnext)[c] = s4;
    }

    const uint32_t lo_g = (uint32_t(lane & 31) * 8u) | 0x00010000u;   // kU_XXS = 1 << 16
    const uint32_t lo_s = uint32_t(lane & 31) * 8u;                     // kU_SGN = 0
    uint32_t lo_x = uint32_t(kU_XS) + uint32_t(lane & 3) * 8u;
    asm volatile("" : "+v"(lo_x));
    const size_t rec = 2 * size_t(ff) * nbx + size_t(dim) * nbh;   // trace integers per pick

    Act<1> A;
    load_act<1>(A, lds, kU_XQ, 4096, lG, LG);
    uint32_t NA[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) NA[c] = neg_bytes(A.a[0][c]);

    uint4 hv;   // the quantizer's h load (every wave issues it; the unit's quantizer uses it)
    auto h_issue = [&](int j) {
        const int u = uclamp(j), i = u / nbh, b = u - i * nbh;
        hv = h_load(hcur, uint32_t(i * ff + 256 * b + 4 * lane));
    };
    float* const part = a.part;

    // ---- the slot loop: gate/up of slot j, the quantizer's Q8_K(h) of slot j - 2,
    // the down block of slot j - 3
    static_for<MG + kLag>([&]<int j>() {
        constexpr bool GU = j < MG;
        constexpr int jq = j - (kLag - 1), jd = j - kLag;   // slots quantized / consumed in this iteration
        if constexpr (jq >= 0 && jq < MG) h_issue(jq);
        if constexpr (GU && j >= 1 && j + WIN - 1 < MG) load_slot.template operator()<j + WIN - 1>();
        if constexpr (GU) load_down.template operator()<j>();
        if constexpr (GU) {
            const Raw3& G0 = rg[j % WIN];
            const Raw3& U0 = ru[j % WIN];
            const Looks Lg = look_xxs(lds, lo_g, lo_s, G0.w);
            const Looks Lu = look_xxs(lds, lo_g, lo_s, U0.w);
            const int Ig = sum_xxs(Lg, G0.w, A.a[0], NA);
            const int Iu = sum_xxs(Lu, U0.w, A.a[0], NA);
            const float fg = fmaf(__fmul_rn(h2f(G0.h[0]), A.d[0]), float(Ig), 0.0f);
            const float fu = fmaf(__fmul_rn(h2f(U0.h[0]), A.d[0]), float(Iu), 0.0f);
            const bool okj = (ok_mask >> j) & 1u;
            const int u = uclamp(j), i = u / nbh, b = u - i * nbh;
            const int row = 256 * b + wi * RG + rG;   // pick i's h row
            if constexpr (TR) {
                const int bg = quad_isum(Ig), bu = quad_isum(Iu);
                if (a.tint && okj && (lG & 3) == 0) {
                    const size_t o = size_t(i) * rec + size_t(row) * nbx + size_t(lG >> 2);
                    a.tint[o] = bg;
                    a.tint[o + size_t(ff) * nbx] = bu;
                }
            }
            float okf = okj ? 1.0f : 0.0f;   // a bad id publishes h = 0 (readers finish)
            asm volatile("" : "+v"(okf));
            const float g = gsum<LG>(fg) * okf, uu = gsum<LG>(fu) * okf;
            if (lG == LG - 1 && j < nu) {
                const float hvv = silu_mul3(__fmul_rn(0.125f, g), __fmul_rn(0.125f, uu), a.lim);
                const uint32_t hb = __float_as_uint(hvv) == kSentinel ? kQNaN : __float_as_uint(hvv);
                __hip_atomic_store(reinterpret_cast<uint32_t*>(hcur) + size_t(i) * ff + row, hb, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                if constexpr (TR) {
                    if (a.th) a.th[size_t(i) * ff + row] = __uint_as_float(hb);
                }
            }
        }
        if constexpr (jq >= 0 && jq < MG) {   // the unit's quantizer stages Q8_K(h) in LDS
            if (jq < nu && (jq % NW) == wv) {
                uint32_t polls = 0;
                while (!__all(h_ready(hv))) {   // not yet complete: poll again (the slack normally covers it)
                    if (++polls > kPollLimit) {
                        if (lane == 0) set_err(a.err, kDevErrTimeout);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                    h_issue(jq);
                }
                uint4 h1[1] = {hv};
                uint32_t hp[1];
                float hd[1];
                const bool fin = q8k_blocks<1>(h1, 1, lane, hp, hd);
                if (!fin && lane == 0) set_err(a.err, kDevErrNonFinite);
                uint8_t* hq = lds + kU_HQ + jq * kU_HQStride;
                *reinterpret_cast<uint32_t*>(hq + 4 * lane) = hp[0];
                if (lane == 0) *reinterpret_cast<float*>(hq + 256) = hd[0];
                // A wave's LDS writes land in order: the flag goes last (the empty asm keeps
                // the compiler from moving the block's writes after it)
                asm volatile("" ::: "memory");
                if (lane == 0) __hip_atomic_store(&sm.ready[jq], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                if (jq < 3) mark(26 + jq);
            }
        }
        if constexpr (jd >= 0 && jd < MG) {   // the unit's down block: 16 rows per wave
            if (jd < nu) {
                uint32_t polls = 0;
                while (__hip_atomic_load(&sm.ready[jd], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0u) {
                    if (++polls > kPollLimit) {
                        if (lane == 0) set_err(a.err, kDevErrTimeout);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                asm volatile("" ::: "memory");   // the block's reads stay after the flag
                const uint8_t* hq = lds + kU_HQ + jd * kU_HQStride;
                uint32_t B[16];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const uint4 v = *reinterpret_cast<const uint4*>(hq + 64 * (lane & 3) + 16 * c);
                    B[4 * c] = v.x; B[4 * c + 1] = v.y; B[4 * c + 2] = v.z; B[4 * c + 3] = v.w;
                }
                const float dh = *reinterpret_cast<const float*>(hq + 256);
                const DRaw& D0 = rd[jd % (kLag + 1)];
                const Looks Lx = look_xs(lds, lo_x, lo_s, D0.w);
                const int I = sum_xs(Lx, D0.sc, B);
                const int bi = quad_isum(I);   // the row's exact block integer
                const int u = unit_of(jd), i = u / nbh, b = u - i * nbh;
                if ((lane & 3) == 0) {
                    const float p = ((ok_mask >> jd) & 1u) ? __fmul_rn(__fmul_rn(h2f(D0.d), dh), float(bi)) : 0.0f;
                    __hip_atomic_store(reinterpret_cast<uint32_t*>(part) + size_t(u) * dim + drow, __float_as_uint(p),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if constexpr (TR) {
                        if (a.tint && ((ok_mask >> jd) & 1u))
                            a.tint[size_t(i) * rec + 2 * size_t(ff) * nbx + size_t(drow) * nbh + size_t(b)] = bi;
                    }
                }
            }
        }
        if constexpr (GU && j < 12) mark(2 + j);   // (after the quantizer duty of this iteration)
        if constexpr (jd >= 0 && jd < 12) mark(14 + jd);
    });

    // ---- every partial of this workgroup stored: count it in
    __builtin_amdgcn_s_waitcnt(0);   // the partial stores are acknowledged (device-coherent) before the count
    lds_barrier();
    if (t == 0) __hip_atomic_fetch_add(pcnt + 32 * (blockIdx.x & 7u), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    mark(29);
    if constexpr (TR) {   // the first workgroup of each group: its staged Q8_K(h) of the group's units
        if (a.tq8h && (blockIdx.x * NW) % WPU == 0)
            for (int jj = wv; jj < nu; jj += NW) {
                const int u = unit_of(jj);
                const uint8_t* hq = lds + kU_HQ + jj * kU_HQStride;
                trace_q8_block(a.tq8h + 292 * u, *reinterpret_cast<const float*>(hq + 256),
                               *reinterpret_cast<const uint32_t*>(hq + 4 * lane), lane);
            }
    }

    // ---- fixed-order combine of this workgroup's row groups {blockIdx + G q}, 16 rows each
    if (wv == 0) {   // lane c < 8 waits for counter c to reach its workgroups
        const int c = lane & 7;
        const uint32_t want = uint32_t((G - c + 7) / 8);
        uint32_t polls = 0;
        while (!__all(lane >= 8 || coh_ld32(pcnt + 32 * c) >= want)) {
            if (++polls > kPollLimit) {
                if (lane == 0) set_err(a.err, kDevErrTimeout);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    lds_barrier();
    mark(30);
    // A row group's 16 partials of one unit are 64 contiguous bytes (written by one
    // wave's down block), so thread t = 16 i + r reads one line per block.
    const int ngroups = dim / 16;
    for (int q = int(blockIdx.x); q < ngroups; q += G) {
        if (t < 16 * k) {
            const int i = t >> 4, orow = 16 * q + (t & 15);
            const uint32_t* pp = reinterpret_cast<const uint32_t*>(part) + size_t(i) * nbh * dim + orow;
            uint32_t pv[16];   // all of the row's partials in flight at once, then summed in block order
#pragma unroll
            for (int b = 0; b < 16; ++b) pv[b] = b < nbh ? coh_ld32(pp + size_t(b) * dim) : 0u;
            float y = 0.0f;
#pragma unroll
            for (int b = 0; b < 16; ++b)
                if (b < nbh) y = __fadd_rn(y, __uint_as_float(pv[b]));
            sm.yv[t & 15][i] = __fmul_rn(0.125f, y);
        }
        lds_barrier();
        if (t < 16) {
            const int orow = 16 * q + t;
            float acc = 0.0f;
            for (int s2 = 0; s2 < k; ++s2) {
                const int i = sm.order[s2];
                if constexpr (TR) {
                    if (a.ty) a.ty[size_t(i) * dim + orow] = sm.yv[t][i];
                }
                acc = fmaf(sm.w[i], sm.yv[t][i], acc);
            }
            if (a.shared) acc = __fadd_rn(acc, a.shared[orow]);
            a.out[orow] = acc;
        }
        lds_barrier();
    }
    mark(31);
    if (t == 0 && arrived == uint32_t(G) - 1u) {
        coh_st32(ctl + 1, 0u);
        coh_st32(ctl, e_prev + 1u);
    }
}

template <int NW, int LG, int MG, int WIN, int LAG>
hipError_t launch_unit_t(const Layer3Args& args, int grid, hipStream_t s, hipEvent_t stop) {
    constexpr int RG = 64 / LG, WPU = 256 / RG;
    const int NG = grid * NW / WPU;
    const int U = args.k * (args.ff / 256);
    if (NG < 1 || (grid * NW) % WPU || (U + NG - 1) / NG > MG || args.dim != 16 * WPU || args.k > 16 ||
        args.k * args.ff > kHBufWords || !args.hbuf || !args.slab || !args.part || !args.ucnt || args.n_experts > 65536)
        return hipErrorNotSupported;
    const bool tr = args.tq8x || args.tq8h || args.th || args.tint || args.ty;
    if (tr)
        hipExtLaunchKernelGGL((unit_kernel<NW, LG, MG, WIN, LAG, true>), dim3(grid), dim3(NW * 64), 0, s, nullptr, stop, 0,
                              args);
    else
        hipExtLaunchKernelGGL((unit_kernel<NW, LG, MG, WIN, LAG, false>), dim3(grid), dim3(NW * 64), 0, s, nullptr, stop, 0,
                              args);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_unit(const Layer3Args& args, int cus, hipStream_t s, hipEvent_t stop) {
    if (args.k < 1 || args.k > 16 || args.dim > 4096 || args.ff > 4096) return hipErrorNotSupported;
    int lg, pg, ld, pd;
    if (!row_shape(args.dim, lg, pg) || !row_shape(args.ff, ld, pd) || pg != 1) return hipErrorNotSupported;
    const int U = args.k * (args.ff / 256);
    if (lg == 64) {   // dim 4096: groups of 32 workgroups (256 waves)
        const int grid = (cus / 32) * 32;
        const int per = grid >= 32 ? (U + grid / 32 - 1) / (grid / 32) : 1 << 30;
        if (per <= 3) return launch_unit_t<8, 64, 3, 3, 3>(args, grid, s, stop);
        if (per <= 6) return launch_unit_t<8, 64, 6, 3, 5>(args, grid, s, stop);
        if (per <= 9) return launch_unit_t<8, 64, 9, 3, 5>(args, grid, s, stop);
        if (per <= 12) return launch_unit_t<8, 64, 12, 3, 5>(args, grid, s, stop);
        return hipErrorNotSupported;
    }
    return hipErrorNotSupported;
}

}  // namespace xl::dev
