// CDNA4 (gfx950) kernels of the routed-expert lane.
//
//   q8k_kernel      Q8_K activation quantization, bit-exact to the reference's
//                   quant_block (engine/strata/sycl/stage/wiring/q8k_core.hpp:30-38)
//   matvec_kernel   one IQ matrix x Q8_K vector (+ optional per-block int32
//                   partials); the parity probe for the row core
//   gate_up_kernel  gate and up rows of all picks + SwiGLU, one launch
//   down_kernel     down rows of all picks, one launch
//   combine_kernel  fixed-order weighted combine (engine/strata/warm/runtime.cpp:183-188)
//   generate_kernel seeded planar bank fill
//
// Row core: a wave covers RPW = 64 / LPR rows at a time; lane l of a row group
// owns pairs {l + LPR*j : j < PPL} (a pair = 2 sub-blocks = 64 weights = one
// 16-byte load of the Q plane for IQ2 types). Its 64-byte activation slices stay
// in VGPRs for every row the wave visits. Per-block integers are completed by a
// quad DPP sum (the 4 pairs of a block sit in one quad), converted to float once,
// scaled by fp16(d_w) * d_x and summed over the row group by DPP/swizzle.
// Codebooks and sign masks live in LDS.
//
// Build with -ffp-contract=off: the quantizer and the combine rely on separately
// rounded IEEE operations (explicit __f*_rn below as well).
#include <hip/hip_runtime.h>

#include "xl_decode.hpp"
#include "xl_format.hpp"
#include "xl_internal.hpp"

namespace xl::dev {

// ---------------------------------------------------------------------------
// Q8_K quantization. One wave per 256-value block, lane l owns values 4l..4l+3.
// The block maximum is the first value of largest magnitude (the reference's
// strict '>' scan), found by an argmax that breaks ties toward the lower index.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int nearest_i(float x) {
    const float v = __fadd_rn(x, 12582912.0f);   // q8k_core.hpp:25-29
    return int(__float_as_uint(v) & 0x007fffffu) - 0x00400000;
}

__global__ __launch_bounds__(256) void q8k_kernel(const float* __restrict__ x, int nblocks, int8_t* __restrict__ qs,
                                                  float* __restrict__ dq, uint8_t* __restrict__ std_out,
                                                  int* __restrict__ err) {
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblocks) return;
    const float4 v4 = reinterpret_cast<const float4*>(x + size_t(b) * 256)[lane];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    float am = 0.0f, mx = 0.0f;
    int idx = 1 << 30;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = fabsf(v[j]);
        finite = finite && (a <= 3.402823466e38f);
        if (a > am) { am = a; mx = v[j]; idx = 4 * lane + j; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float am2 = __shfl_xor(am, off);
        const float mx2 = __shfl_xor(mx, off);
        const int idx2 = __shfl_xor(idx, off);
        if (am2 > am || (am2 == am && idx2 < idx)) { am = am2; mx = mx2; idx = idx2; }
    }
    if (__any(!finite) && lane == 0) atomicOr(err, kDevErrNonFinite);
    uint32_t packed = 0;
    int bsum = 0;
    float d = 0.0f;
    if (am != 0.0f) {
        const float is = __fdiv_rn(-127.0f, mx);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int q = nearest_i(__fmul_rn(is, v[j]));
            q = q < 127 ? q : 127;
            packed |= uint32_t(uint8_t(int8_t(q))) << (8 * j);
            bsum += q;
        }
        d = __fdiv_rn(1.0f, is);
    }
    bsum = quad_sum(bsum);
    reinterpret_cast<uint32_t*>(qs + size_t(b) * 256)[lane] = packed;
    if (lane == 0) dq[b] = d;
    if (std_out) {
        uint8_t* o = std_out + size_t(b) * 292;
        if (lane == 0) *reinterpret_cast<float*>(o) = d;
        reinterpret_cast<uint32_t*>(o + 4)[lane] = packed;
        if ((lane & 3) == 0) reinterpret_cast<int16_t*>(o + 260)[lane >> 2] = int16_t(bsum);
    }
}

// ---------------------------------------------------------------------------
// Row core
// ---------------------------------------------------------------------------
template <int PPL>
struct Act {
    uint32_t a[PPL][16];   // 64 Q8_K bytes of each owned pair
    float d[PPL];          // Q8_K scale of the pair's block
    int s8[PPL][8];        // per-8 activation sums (IQ1_M delta term)
};

template <int LPR, int PPL>
__device__ __forceinline__ void load_act(Act<PPL>& A, const int8_t* __restrict__ qs, const float* __restrict__ dq, int l) {
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int p = l + LPR * j;
        const uint4* src = reinterpret_cast<const uint4*>(qs + 64 * p);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 t = src[c];
            A.a[j][4 * c + 0] = t.x; A.a[j][4 * c + 1] = t.y;
            A.a[j][4 * c + 2] = t.z; A.a[j][4 * c + 3] = t.w;
        }
        A.d[j] = dq[p >> 2];
#pragma unroll
        for (int g = 0; g < 8; ++g) A.s8[j][g] = group_sum(A.a[j][2 * g], A.a[j][2 * g + 1]);
    }
}

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld8(const uint8_t* p) { return *reinterpret_cast<const uint2*>(p); }
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ uint32_t ld2(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// Dot of one row against the activation slices. Returns the row value in every
// lane of the row group. With PART, lane 4q of the group writes the per-block
// integer(s) of its quad's block (IQ1_M: main, delta).
template <int TYPE, int LPR, int PPL, bool PART>
__device__ __forceinline__ float row_dot(const MatRef& m, int row, bool valid, int l, const Act<PPL>& A,
                                         const uint2* tab, int32_t* __restrict__ partials) {
    float acc = 0.0f, accd = 0.0f;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int p = l + LPR * j;
        const uint64_t blk = uint64_t(row) * uint64_t(m.nb) + uint64_t(p >> 2);
        const int pp = p & 3;
        if constexpr (TYPE == kIQ2_XXS) {
            uint4 w = make_uint4(0, 0, 0, 0);
            uint32_t d16 = 0;
            if (valid) { w = ld16(m.base + blk * 64 + pp * 16); d16 = ld2(m.base + m.off1 + blk * 2); }
            const int I = quad_sum(pair_iq2xxs(tab, w, A.a[j]));
            const float db = __fmul_rn(half_to_float(uint16_t(d16)), A.d[j]);
            acc = fmaf(db, float(I), acc);
            if constexpr (PART) if (valid && (l & 3) == 0) partials[blk] = I;
        } else if constexpr (TYPE == kIQ2_XS) {
            uint4 w = make_uint4(0, 0, 0, 0);
            uint32_t sc = 0, d16 = 0;
            if (valid) {
                w = ld16(m.base + blk * 64 + pp * 16);
                sc = ld2(m.base + m.off1 + blk * 8 + pp * 2);
                d16 = ld2(m.base + m.off2 + blk * 2);
            }
            const int I = quad_sum(pair_iq2xs(tab, w, sc, A.a[j]));
            const float db = __fmul_rn(half_to_float(uint16_t(d16)), A.d[j]);
            acc = fmaf(db, float(I), acc);
            if constexpr (PART) if (valid && (l & 3) == 0) partials[blk] = I;
        } else {
            uint2 q = make_uint2(0, 0), sw = make_uint2(0, 0);
            uint32_t h = 0;
            if (valid) {
                q = ld8(m.base + blk * 32 + pp * 8);
                h = ld4(m.base + m.off1 + blk * 16 + pp * 4);
                sw = ld8(m.base + m.off2 + blk * 8);
            }
            const uint32_t scw = ((pp & 2) ? sw.y : sw.x) >> (16 * (pp & 1));
            const int2 r = pair_iq1m(tab, q, h, scw, A.a[j], A.s8[j]);
            const int im = quad_sum(r.x), id = quad_sum(r.y);
            const uint16_t dh = uint16_t((sw.x >> 12) & 0xfu) | uint16_t((sw.x >> 24) & 0xf0u) |
                                uint16_t((sw.y >> 4) & 0xf00u) | uint16_t((sw.y >> 16) & 0xf000u);
            const float db = __fmul_rn(half_to_float(dh), A.d[j]);
            acc = fmaf(db, float(im), acc);
            accd = fmaf(db, float(id), accd);
            if constexpr (PART) if (valid && (l & 3) == 0) { partials[2 * blk] = im; partials[2 * blk + 1] = id; }
        }
    }
    const float tm = group_sum_quads<LPR>(acc);
    if constexpr (TYPE == kIQ1_M) {
        const float td = group_sum_quads<LPR>(accd);
        return __fadd_rn(tm, __fmul_rn(0.125f, td));
    } else {
        return __fmul_rn(0.125f, tm);
    }
}

template <int LPR, int PPL, bool PART>
__device__ __forceinline__ float row_dot_any(const MatRef& m, int row, bool valid, int l, const Act<PPL>& A,
                                             const uint2* tab, int32_t* partials, int* err) {
    switch (m.type) {
        case kIQ2_XXS: return row_dot<kIQ2_XXS, LPR, PPL, PART>(m, row, valid, l, A, tab, partials);
        case kIQ2_XS: return row_dot<kIQ2_XS, LPR, PPL, PART>(m, row, valid, l, A, tab, partials);
        case kIQ1_M: return row_dot<kIQ1_M, LPR, PPL, PART>(m, row, valid, l, A, tab, partials);
        default:
            if (l == 0) atomicOr(err, kDevErrType);
            return 0.0f;
    }
}

__device__ __forceinline__ void load_tables(uint2* tab, const uint2* __restrict__ g) {
    for (int i = threadIdx.x; i < kTabRows; i += blockDim.x) tab[i] = g[i];
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Debug/probe matvec: one matrix, one Q8_K vector.
// ---------------------------------------------------------------------------
template <int LPR, int PPL, bool PART>
__global__ __launch_bounds__(256) void matvec_kernel(MatRef m, int n, const int8_t* __restrict__ aq,
                                                     const float* __restrict__ ad, const uint2* __restrict__ tables,
                                                     float* __restrict__ y, int32_t* __restrict__ partials, int* err) {
    __shared__ uint2 tab[kTabRows];
    load_tables(tab, tables);
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, grp = lane / LPR, l = lane % LPR;
    Act<PPL> A;
    load_act<LPR, PPL>(A, aq, ad, l);
    const int waves = gridDim.x * 4;
    for (int s = blockIdx.x * 4 + (threadIdx.x >> 6); s * RPW < n; s += waves) {
        const int row = s * RPW + grp;
        const bool valid = row < n;
        const float v = row_dot_any<LPR, PPL, PART>(m, row, valid, l, A, tab, partials, err);
        if (valid && l == 0) y[row] = v;
    }
}

// ---------------------------------------------------------------------------
// Gate/up + SwiGLU for all picks in one launch. Work = k*ff rows flattened
// (pick-major), split into contiguous per-wave ranges of row slots.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu_mul(float g, float u) {
    // q8k_core.hpp:92-95 with limit 0: (g / (1 + exp(-g))) * u
    const float e = expf(-g);
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

template <int LPR, int PPL>
__global__ __launch_bounds__(256) void gate_up_kernel(const ExpertDesc* __restrict__ descs,
                                                      const int32_t* __restrict__ ids, int k, int n_experts, int ff,
                                                      const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                      const uint2* __restrict__ tables, float* __restrict__ h,
                                                      float* __restrict__ g_dbg, float* __restrict__ u_dbg,
                                                      int* __restrict__ err) {
    __shared__ uint2 tab[kTabRows];
    load_tables(tab, tables);
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, grp = lane / LPR, l = lane % LPR;
    Act<PPL> A;
    load_act<LPR, PPL>(A, xq, xd, l);
    const int slots_per_pick = ff / RPW, total = k * slots_per_pick;
    const int waves = gridDim.x * 4, gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int per = (total + waves - 1) / waves;
    const int first = gw * per, last = min(total, first + per);
    for (int s = first; s < last; ++s) {
        const int i = s / slots_per_pick;
        const int row = (s - i * slots_per_pick) * RPW + grp;
        const int id = ids[i];
        if (id < 0 || id >= n_experts) {
            if (lane == 0) atomicOr(err, kDevErrExpertId);
            continue;
        }
        const ExpertDesc& D = descs[id];
        const float g = row_dot_any<LPR, PPL, false>(D.m[0], row, true, l, A, tab, nullptr, err);
        const float u = row_dot_any<LPR, PPL, false>(D.m[1], row, true, l, A, tab, nullptr, err);
        if (l == 0) {
            h[size_t(i) * ff + row] = silu_mul(g, u);
            if (g_dbg) g_dbg[size_t(i) * ff + row] = g;
            if (u_dbg) u_dbg[size_t(i) * ff + row] = u;
        }
    }
}

// ---------------------------------------------------------------------------
// Down rows of all picks in one launch; activation slices reload when the
// wave's range crosses into the next pick.
// ---------------------------------------------------------------------------
template <int LPR, int PPL>
__global__ __launch_bounds__(256) void down_kernel(const ExpertDesc* __restrict__ descs, const int32_t* __restrict__ ids,
                                                   int k, int n_experts, int dim, int ff, const int8_t* __restrict__ hq,
                                                   const float* __restrict__ hd, const uint2* __restrict__ tables,
                                                   float* __restrict__ y, int* __restrict__ err) {
    __shared__ uint2 tab[kTabRows];
    load_tables(tab, tables);
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, grp = lane / LPR, l = lane % LPR;
    Act<PPL> A;
    const int slots_per_pick = dim / RPW, total = k * slots_per_pick;
    const int waves = gridDim.x * 4, gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int per = (total + waves - 1) / waves;
    const int first = gw * per, last = min(total, first + per);
    int cur = -1;
    for (int s = first; s < last; ++s) {
        const int i = s / slots_per_pick;
        const int row = (s - i * slots_per_pick) * RPW + grp;
        const int id = ids[i];
        if (id < 0 || id >= n_experts) {
            if (lane == 0) atomicOr(err, kDevErrExpertId);
            continue;
        }
        if (i != cur) {
            load_act<LPR, PPL>(A, hq + size_t(i) * ff, hd + size_t(i) * (ff / 256), l);
            cur = i;
        }
        const float v = row_dot_any<LPR, PPL, false>(descs[id].m[2], row, true, l, A, tab, nullptr, err);
        if (l == 0) y[size_t(i) * dim + row] = v;
    }
}

// ---------------------------------------------------------------------------
// Fixed-order combine (runtime.cpp:183-188): ascending expert id, sequential
// fma starting from +0, then + shared. One thread per output coordinate.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void combine_kernel(const int32_t* __restrict__ ids, const float* __restrict__ w,
                                                      int k, const float* __restrict__ y, int dim,
                                                      const float* __restrict__ shared, float* __restrict__ out) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= dim) return;
    int order[16];
    for (int i = 0; i < k; ++i) order[i] = i;
    for (int i = 1; i < k; ++i)
        for (int j = i; j > 0 && ids[order[j]] < ids[order[j - 1]]; --j) {
            const int t = order[j]; order[j] = order[j - 1]; order[j - 1] = t;
        }
    float acc = 0.0f;
    for (int t = 0; t < k; ++t) acc = fmaf(w[order[t]], y[size_t(order[t]) * dim + c], acc);
    if (shared) acc = __fadd_rn(acc, shared[c]);
    out[c] = acc;
}

// ---------------------------------------------------------------------------
// Seeded planar generation: one thread per block, 8-byte stores.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t shift_pair(uint64_t lo, uint64_t hi) { return (lo >> 16) | (hi << 48); }

__global__ __launch_bounds__(256) void generate_kernel(uint8_t* __restrict__ base, int type, uint64_t nblocks,
                                                       uint64_t off1, uint64_t off2, uint64_t key) {
    const uint64_t blk = uint64_t(blockIdx.x) * 256u + threadIdx.x;
    if (blk >= nblocks) return;
    uint64_t w[10];
#pragma unroll
    for (int j = 0; j < 10; ++j) w[j] = gen_word(key, blk, uint32_t(j));
    const uint16_t d = gen_scale(gen_word(key, blk, 15));
    if (type == kIQ2_XXS || type == kIQ2_XS) {
        uint64_t* q = reinterpret_cast<uint64_t*>(base + blk * 64);
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = shift_pair(w[j], w[j + 1]);
        if (type == kIQ2_XXS) {
            *reinterpret_cast<uint16_t*>(base + off1 + blk * 2) = d;
        } else {
            *reinterpret_cast<uint64_t*>(base + off1 + blk * 8) = shift_pair(w[8], w[9]);
            *reinterpret_cast<uint16_t*>(base + off2 + blk * 2) = d;
        }
    } else {
        uint64_t* q = reinterpret_cast<uint64_t*>(base + blk * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = w[j];
        uint64_t* hp = reinterpret_cast<uint64_t*>(base + off1 + blk * 16);
        hp[0] = w[4];
        hp[1] = w[5];
        uint64_t sc = w[6] & 0x0fff0fff0fff0fffull;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) sc |= uint64_t((d >> (4 * q4)) & 15u) << (16 * q4 + 12);
        *reinterpret_cast<uint64_t*>(base + off2 + blk * 8) = sc;
    }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
#define XL_SHAPES(X) X(4, 1) X(8, 1) X(4, 3) X(16, 1) X(32, 1) X(16, 3) X(64, 1)

hipError_t launch_q8k(const float* x, int nblocks, int8_t* qs, float* d, uint8_t* std_out, int* err, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(q8k_kernel, dim3((nblocks + 3) / 4), dim3(256), 0, s, x, nblocks, qs, d, std_out, err);
    return hipGetLastError();
}

hipError_t launch_matvec(const MatRef& m, int n, int k, const int8_t* aq, const float* ad, const uint2* tables,
                         float* y, int32_t* partials, int* err, hipStream_t s) {
    int lpr, ppl;
    if (!row_shape(k, lpr, ppl) || n <= 0) return hipErrorInvalidValue;
    const int rpw = 64 / lpr, slots = (n + rpw - 1) / rpw;
    const int grid = (slots + 3) / 4 < 1024 ? (slots + 3) / 4 : 1024;
#define XL_MV(L, P)                                                                                                   \
    if (lpr == L && ppl == P) {                                                                                       \
        if (partials)                                                                                                 \
            hipLaunchKernelGGL((matvec_kernel<L, P, true>), dim3(grid), dim3(256), 0, s, m, n, aq, ad, tables, y,     \
                               partials, err);                                                                        \
        else                                                                                                          \
            hipLaunchKernelGGL((matvec_kernel<L, P, false>), dim3(grid), dim3(256), 0, s, m, n, aq, ad, tables, y,    \
                               partials, err);                                                                        \
        return hipGetLastError();                                                                                     \
    }
    XL_SHAPES(XL_MV)
#undef XL_MV
    return hipErrorInvalidValue;
}

hipError_t launch_gate_up(const ExpertDesc* descs, const int32_t* ids, int k, int n_experts, int dim, int ff,
                          const int8_t* xq, const float* xd, const uint2* tables, float* h, float* g_dbg, float* u_dbg,
                          int* err, int grid, hipStream_t s) {
    int lpr, ppl;
    if (!row_shape(dim, lpr, ppl)) return hipErrorInvalidValue;
#define XL_GU(L, P)                                                                                                   \
    if (lpr == L && ppl == P) {                                                                                       \
        hipLaunchKernelGGL((gate_up_kernel<L, P>), dim3(grid), dim3(256), 0, s, descs, ids, k, n_experts, ff, xq, xd, \
                           tables, h, g_dbg, u_dbg, err);                                                             \
        return hipGetLastError();                                                                                     \
    }
    XL_SHAPES(XL_GU)
#undef XL_GU
    return hipErrorInvalidValue;
}

hipError_t launch_down(const ExpertDesc* descs, const int32_t* ids, int k, int n_experts, int dim, int ff,
                       const int8_t* hq, const float* hd, const uint2* tables, float* y, int* err, int grid,
                       hipStream_t s) {
    int lpr, ppl;
    if (!row_shape(ff, lpr, ppl)) return hipErrorInvalidValue;
#define XL_DN(L, P)                                                                                                   \
    if (lpr == L && ppl == P) {                                                                                       \
        hipLaunchKernelGGL((down_kernel<L, P>), dim3(grid), dim3(256), 0, s, descs, ids, k, n_experts, dim, ff, hq,   \
                           hd, tables, y, err);                                                                       \
        return hipGetLastError();                                                                                     \
    }
    XL_SHAPES(XL_DN)
#undef XL_DN
    return hipErrorInvalidValue;
}

hipError_t launch_combine(const int32_t* ids, const float* w, int k, const float* y, int dim, const float* shared,
                          float* out, hipStream_t s) {
    if (k < 0 || k > 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(combine_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, ids, w, k, y, dim, shared, out);
    return hipGetLastError();
}

hipError_t launch_generate(uint8_t* base, int type, int n, int k, uint64_t seed, uint32_t layer, uint32_t expert,
                           uint32_t role, hipStream_t s) {
    const uint64_t nblocks = uint64_t(n) * uint64_t(k / 256);
    const PlaneLayout L = plane_layout(type, nblocks);
    const uint64_t key = gen_key(seed, layer, expert, role);
    const uint64_t grid = (nblocks + 255) / 256;
    hipLaunchKernelGGL(generate_kernel, dim3(unsigned(grid)), dim3(256), 0, s, base, type, nblocks, L.off[1], L.off[2],
                       key);
    return hipGetLastError();
}

}  // namespace xl::dev
