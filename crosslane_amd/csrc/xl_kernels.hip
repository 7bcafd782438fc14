// CDNA4 (gfx950) kernels of the routed-expert lane.
//
//   q8k_kernel      Q8_K activation quantization, bit-exact to the reference's
//                   quant_block (engine/strata/sycl/stage/wiring/q8k_core.hpp:30-38)
//   matvec_kernel   one IQ matrix x Q8_K vector (+ optional per-block int32
//                   partials); the parity probe for the row engine
//   gate_up_kernel, down_kernel, combine_kernel
//                   the layer as separate launches (probe / fallback path; the
//                   single launches are in xl_stream.hpp and xl_layer.hip)
//   generate_kernel seeded planar bank fill
//
// Build with -ffp-contract=off: the quantizer and the combine rely on separately
// rounded IEEE operations (explicit __f*_rn below as well).
#include <hip/hip_runtime.h>

#include "xl_format.hpp"
#include "xl_internal.hpp"
#include "xl_route.hpp"
#include "xl_rows.hpp"

namespace xl::dev {

int type_bit(int type) { return type == kIQ2_XXS ? 1 : type == kIQ2_XS ? 2 : type == kIQ1_M ? 4 : 0; }

// ---------------------------------------------------------------------------
// Q8_K of one 256-value block by one wave (lane l owns values 4l..4l+3). The
// block maximum is the first value of largest magnitude (the reference's strict
// '>' scan), found by an argmax that breaks ties toward the lower index.
// Writes the split form (qs, d) and optionally the 292-byte block.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int nearest_i(float x) {
    const float v = __fadd_rn(x, 12582912.0f);   // q8k_core.hpp:25-29
    return int(__float_as_uint(v) & 0x007fffffu) - 0x00400000;
}

__device__ __forceinline__ void q8k_block(const float* __restrict__ x, int8_t* __restrict__ qs, float* __restrict__ dq,
                                          uint8_t* __restrict__ std_out, int* __restrict__ err, int lane) {
    float v[4];
    const float4 v4 = reinterpret_cast<const float4*>(x)[lane];
    v[0] = v4.x; v[1] = v4.y; v[2] = v4.z; v[3] = v4.w;
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
    reinterpret_cast<uint32_t*>(qs)[lane] = packed;
    if (lane == 0) *dq = d;
    if (std_out) {
        if (lane == 0) *reinterpret_cast<float*>(std_out) = d;
        reinterpret_cast<uint32_t*>(std_out + 4)[lane] = packed;
        if ((lane & 3) == 0) reinterpret_cast<int16_t*>(std_out + 260)[lane >> 2] = int16_t(bsum);
    }
}

__global__ __launch_bounds__(256) void q8k_kernel(const float* __restrict__ x, int nblocks, int8_t* __restrict__ qs,
                                                  float* __restrict__ dq, uint8_t* __restrict__ std_out,
                                                  int* __restrict__ err) {
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblocks) return;   // wave-uniform
    q8k_block(x + size_t(b) * 256, qs + size_t(b) * 256, dq + b, std_out ? std_out + size_t(b) * 292 : nullptr, err,
              threadIdx.x & 63);
}

__device__ __forceinline__ float silu_mul(float g, float u, float lim) {
    // q8k_core.hpp:92-95: the limit (lim > 0: g = min(g, lim), u = clamp(u,
    // -lim, lim)), then (g / (1 + exp(-g))) * u
    if (lim > 0.0f) {
        g = fminf(g, lim);
        u = fminf(fmaxf(u, -lim), lim);
    }
    const float e = expf(-g);
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

// ---------------------------------------------------------------------------
// Probe matvec: one matrix, one Q8_K vector, optional per-block partials.
// ---------------------------------------------------------------------------
template <int LPR, int PPL, bool PART>
__global__ __launch_bounds__(256) void matvec_kernel(MatRef m, int n, const int8_t* __restrict__ aq,
                                                     const float* __restrict__ ad, const uint16_t* __restrict__ codes,
                                                     int need, float* __restrict__ y, int32_t* __restrict__ partials) {
    extern __shared__ uint8_t lds[];
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, grp = lane / LPR, l = lane % LPR;
    CodeRegs cr;
    codes_prefetch(cr, codes, need, threadIdx.x);
    Act<PPL> A;
    load_act<LPR, PPL>(A, aq, ad, l);
    codes_fill(lds, cr, need, threadIdx.x);
    __syncthreads();
    const int waves = gridDim.x * 4;
    for (int s = blockIdx.x * 4 + (threadIdx.x >> 6); s * RPW < n; s += waves) {
        const int row = s * RPW + grp;
        const bool valid = row < n;
        Raw<PPL> r;
        if (valid) load_raw<LPR, PPL>(r, m.type, m, row, l); else zero_raw(r);
        const float v = dot_raw<LPR, PPL, PART>(r, m.type, row, m.nb, l, A, lds, partials, valid);
        if (valid && l == 0) y[row] = v;
    }
}

// ---------------------------------------------------------------------------
// Separate-launch layer path: gate/up + SwiGLU, down, combine. Workgroup b
// serves pick b / wgpp; each wave loads all of its (at most U) row slots before
// the LDS codebook fill.
// ---------------------------------------------------------------------------
template <int LPR, int PPL, int U>
__global__ __launch_bounds__(256) void gate_up_kernel(const ExpertDesc* __restrict__ descs,
                                                      const int32_t* __restrict__ ids, int n_experts, int ff, int wgpp,
                                                      const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                      const uint16_t* __restrict__ codes, int need,
                                                      float* __restrict__ h, float* __restrict__ g_dbg,
                                                      float* __restrict__ u_dbg, int* __restrict__ err, float lim) {
    extern __shared__ uint8_t lds[];
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, grp = lane / LPR, l = lane % LPR;
    const int i = blockIdx.x / wgpp;
    const int jw = (blockIdx.x - i * wgpp) * 4 + (threadIdx.x >> 6);
    const int id = ids[i];
    if (id < 0 || id >= n_experts) {   // workgroup-uniform: no barrier is skipped by part of the group
        if (threadIdx.x == 0) atomicOr(err, kDevErrExpertId);
        return;
    }
    const ExpertDesc& D = descs[id];
    const int type = D.m[0].type;
    const int slots = ff / RPW, per = (slots + 4 * wgpp - 1) / (4 * wgpp);
    const int slot0 = jw * per, nslots = max(0, min(per, slots - slot0));
    CodeRegs cr;
    codes_prefetch(cr, codes, need, threadIdx.x);
    Act<PPL> A;
    load_act<LPR, PPL>(A, xq, xd, l);
    Raw<PPL> rg[U], ru[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (u < nslots) {
            load_raw<LPR, PPL>(rg[u], type, D.m[0], (slot0 + u) * RPW + grp, l);
            load_raw<LPR, PPL>(ru[u], type, D.m[1], (slot0 + u) * RPW + grp, l);
        }
    codes_fill(lds, cr, need, threadIdx.x);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (u < nslots) {
            const int row = (slot0 + u) * RPW + grp;
            const float g = dot_raw<LPR, PPL, false>(rg[u], type, row, D.m[0].nb, l, A, lds, nullptr, true);
            const float v = dot_raw<LPR, PPL, false>(ru[u], type, row, D.m[1].nb, l, A, lds, nullptr, true);
            if (l == 0) {
                h[size_t(i) * ff + row] = silu_mul(g, v, lim);
                if (g_dbg) g_dbg[size_t(i) * ff + row] = g;
                if (u_dbg) u_dbg[size_t(i) * ff + row] = v;
            }
        }
}

template <int LPR, int PPL, int U>
__global__ __launch_bounds__(256) void down_kernel(const ExpertDesc* __restrict__ descs, const int32_t* __restrict__ ids,
                                                   int n_experts, int dim, int ff, int wgpp,
                                                   const int8_t* __restrict__ hq, const float* __restrict__ hd,
                                                   const uint16_t* __restrict__ codes, int need, float* __restrict__ y,
                                                   int* __restrict__ err) {
    extern __shared__ uint8_t lds[];
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, grp = lane / LPR, l = lane % LPR;
    const int i = blockIdx.x / wgpp;
    const int jw = (blockIdx.x - i * wgpp) * 4 + (threadIdx.x >> 6);
    const int id = ids[i];
    if (id < 0 || id >= n_experts) {
        if (threadIdx.x == 0) atomicOr(err, kDevErrExpertId);
        return;
    }
    const MatRef& M = descs[id].m[2];
    const int type = M.type;
    const int slots = dim / RPW, per = (slots + 4 * wgpp - 1) / (4 * wgpp);
    const int slot0 = jw * per, nslots = max(0, min(per, slots - slot0));
    CodeRegs cr;
    codes_prefetch(cr, codes, need, threadIdx.x);
    Act<PPL> A;
    load_act<LPR, PPL>(A, hq + size_t(i) * ff, hd + size_t(i) * (ff / 256), l);
    Raw<PPL> r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (u < nslots) load_raw<LPR, PPL>(r[u], type, M, (slot0 + u) * RPW + grp, l);
    codes_fill(lds, cr, need, threadIdx.x);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (u < nslots) {
            const int row = (slot0 + u) * RPW + grp;
            const float v = dot_raw<LPR, PPL, false>(r[u], type, row, M.nb, l, A, lds, nullptr, true);
            if (l == 0) y[size_t(i) * dim + row] = v;
        }
}

// Fixed-order combine (runtime.cpp:183-188) of one output coordinate: ascending
// expert id, out = fma(w, y, out) from +0, then + shared.
__device__ __forceinline__ float combine_one(const int32_t* ids, const float* w, int k, const float* y, int dim, int c,
                                             const float* shared) {
    int order[16];
    for (int i = 0; i < k; ++i) order[i] = i;
    for (int i = 1; i < k; ++i)
        for (int j = i; j > 0 && ids[order[j]] < ids[order[j - 1]]; --j) {
            const int t = order[j]; order[j] = order[j - 1]; order[j - 1] = t;
        }
    float acc = 0.0f;
    for (int t = 0; t < k; ++t) {
        const float* p = y + size_t(order[t]) * dim + c;
        acc = fmaf(w[order[t]], *p, acc);
    }
    if (shared) acc = __fadd_rn(acc, shared[c]);
    return acc;
}

// h = SwiGLU(g, u) with the limit, elementwise (hip_q8k.hip activate_kernel,
// q8k_core.hpp:92-95 per element).
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, int n,
                                                     float lim, float* __restrict__ h) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] = silu_mul(g[i], u[i], lim);
}

__global__ __launch_bounds__(256) void combine_kernel(const int32_t* __restrict__ ids, const float* __restrict__ w,
                                                      int k, const float* __restrict__ y, int dim,
                                                      const float* __restrict__ shared, float* __restrict__ out) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c < dim) out[c] = combine_one(ids, w, k, y, dim, c, shared);
}

// ---------------------------------------------------------------------------
// Router (route.cpp:15-37, route_cpu), one workgroup per token; its arithmetic
// is xl_route.hpp's. Scores and keys by all 512 threads (PT experts each,
// loads first), through LDS to wave 0, which selects: expert e in lane e % 64,
// slot e / 64.
// ---------------------------------------------------------------------------
template <int NPL>   // n <= 64 * NPL
__global__ __launch_bounds__(512) void route_kernel(const float* __restrict__ logits, int stride,
                                                    const float* __restrict__ bias, int n, int k, float scale,
                                                    int32_t* __restrict__ ids, float* __restrict__ w,
                                                    int* __restrict__ err) {
    constexpr int PT = (64 * NPL + 511) / 512;
    __shared__ float s_sc[64 * NPL];
    __shared__ uint32_t s_key[64 * NPL];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* lg = logits + size_t(t) * stride;
    float lv[PT], bv[PT];
#pragma unroll
    for (int j = 0; j < PT; ++j) {   // every load first (clamped, unconditional): one round trip
        const int e = min(tid + 512 * j, n - 1);
        lv[j] = lg[e];
        bv[j] = bias ? bias[e] : 0.0f;
    }
    bool fin = true;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int e = tid + 512 * j;
        float s;
        uint32_t key;
        route_score(lv[j], bv[j], e < n, s, key, fin);
        if (e < 64 * NPL) {
            s_sc[e] = s;
            s_key[e] = key;
        }
    }
    if (__any(!fin) && (tid & 63) == 0) atomicOr(err, kDevErrNonFinite);
    __syncthreads();
    if (tid >= 64) return;
    const int lane = tid;
    float sc[NPL];
    uint32_t key[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        sc[j] = s_sc[lane + 64 * j];
        key[j] = s_key[lane + 64 * j];
    }
    int id;
    float wt;
    route_select<NPL>(sc, key, k, lane, scale, id, wt);
    if (lane < k) {
        ids[size_t(t) * k + lane] = id;
        w[size_t(t) * k + lane] = wt;
    }
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
        for (int j = 0; j < 8; ++j) {
            const uint64_t v = shift_pair(w[j], w[j + 1]);   // AoS bytes 2+8j .. 9+8j
            uint64_t o;
            if (type == kIQ2_XXS) {
                o = (v & 0xffffffffull) | (uint64_t(xxs_aux_to_planar(uint32_t(v >> 32))) << 32);
            } else {
                o = 0;
#pragma unroll
                for (int c = 0; c < 4; ++c) o |= uint64_t(xs_code_to_planar(uint16_t(v >> (16 * c)))) << (16 * c);
            }
            q[j] = o;
        }
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
#define XL_SHAPES(X) X(4, 1) X(8, 1) X(4, 3) X(16, 1) X(32, 1) X(4, 9) X(16, 3) X(64, 1) X(16, 5)
// Row slots a wave holds in flight: fewer for long lanes (PPL pairs each), so
// that the raw words and activations stay within the register file.
constexpr int gu_slots(int ppl) { return ppl >= 9 ? 1 : ppl >= 5 ? 2 : 4; }
constexpr int dn_slots(int ppl) { return ppl >= 5 ? 1 : 2; }

static int need_of(int type_mask) {
    return ((type_mask & 1) ? kNeedXXS : 0) | ((type_mask & 2) ? kNeedXS : 0) | ((type_mask & 4) ? kNeedIQ1 : 0);
}

hipError_t launch_q8k(const float* x, int nblocks, int8_t* qs, float* d, uint8_t* std_out, int* err, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(q8k_kernel, dim3((nblocks + 3) / 4), dim3(256), 0, s, x, nblocks, qs, d, std_out, err);
    return hipGetLastError();
}

hipError_t launch_matvec(const MatRef& m, int n, int k, const int8_t* aq, const float* ad, const uint16_t* codes,
                         float* y, int32_t* partials, int* err, hipStream_t s) {
    (void)err;
    int lpr, ppl;
    if (!row_shape(k, lpr, ppl) || n <= 0 || !supported_type(m.type)) return hipErrorInvalidValue;
    const int rpw = 64 / lpr, slots = (n + rpw - 1) / rpw;
    const int grid = (slots + 3) / 4 < 1024 ? (slots + 3) / 4 : 1024;
    const int need = need_of(type_bit(m.type));
    const size_t lds = size_t(lds_bytes_for(need));
#define XL_MV(L, P)                                                                                                   \
    if (lpr == L && ppl == P) {                                                                                       \
        if (partials)                                                                                                 \
            hipLaunchKernelGGL((matvec_kernel<L, P, true>), dim3(grid), dim3(256), lds, s, m, n, aq, ad, codes, need, \
                               y, partials);                                                                          \
        else                                                                                                          \
            hipLaunchKernelGGL((matvec_kernel<L, P, false>), dim3(grid), dim3(256), lds, s, m, n, aq, ad, codes,      \
                               need, y, partials);                                                                    \
        return hipGetLastError();                                                                                     \
    }
    XL_SHAPES(XL_MV)
#undef XL_MV
    return hipErrorInvalidValue;
}

// Workgroups per pick: enough that no wave owns more than U row slots, and at
// least target_wgs / k so the launch fills the device.
static int wg_per_pick(int slots, int umax, int k, int target_wgs) {
    const int need = (slots + 4 * umax - 1) / (4 * umax);
    const int fill = (target_wgs + k - 1) / k;
    const int cap = (slots + 3) / 4;
    int w = need > fill ? need : fill;
    return w < cap ? w : (need > cap ? need : cap);
}

hipError_t launch_gate_up(const ExpertDesc* descs, const int32_t* ids, int k, int n_experts, int dim, int ff,
                          const int8_t* xq, const float* xd, const uint16_t* codes, float* h, float* g_dbg,
                          float* u_dbg, int* err, int target_wgs, int type_mask, float lim, hipStream_t s) {
    int lpr, ppl;
    if (!row_shape(dim, lpr, ppl) || k <= 0) return hipErrorInvalidValue;
    const int need = need_of(type_mask);
    const size_t lds = size_t(lds_bytes_for(need));
#define XL_GU(L, P)                                                                                                   \
    if (lpr == L && ppl == P) {                                                                                       \
        constexpr int U = gu_slots(P);                                                                                \
        const int wgpp = wg_per_pick(ff / (64 / lpr), U, k, target_wgs);                                             \
        hipLaunchKernelGGL((gate_up_kernel<L, P, U>), dim3(k * wgpp), dim3(256), lds, s, descs, ids, n_experts, ff,   \
                           wgpp, xq, xd, codes, need, h, g_dbg, u_dbg, err, lim);                                     \
        return hipGetLastError();                                                                                     \
    }
    XL_SHAPES(XL_GU)
#undef XL_GU
    return hipErrorInvalidValue;
}

hipError_t launch_down(const ExpertDesc* descs, const int32_t* ids, int k, int n_experts, int dim, int ff,
                       const int8_t* hq, const float* hd, const uint16_t* codes, float* y, int* err, int target_wgs,
                       int type_mask, hipStream_t s) {
    int lpr, ppl;
    if (!row_shape(ff, lpr, ppl) || k <= 0) return hipErrorInvalidValue;
    const int need = need_of(type_mask);
    const size_t lds = size_t(lds_bytes_for(need));
#define XL_DN(L, P)                                                                                                   \
    if (lpr == L && ppl == P) {                                                                                       \
        constexpr int U = dn_slots(P);                                                                                \
        const int wgpp = wg_per_pick(dim / (64 / lpr), U, k, target_wgs);                                            \
        hipLaunchKernelGGL((down_kernel<L, P, U>), dim3(k * wgpp), dim3(256), lds, s, descs, ids, n_experts, dim, ff, \
                           wgpp, hq, hd, codes, need, y, err);                                                        \
        return hipGetLastError();                                                                                     \
    }
    XL_SHAPES(XL_DN)
#undef XL_DN
    return hipErrorInvalidValue;
}

hipError_t launch_route(const float* logits, int T, int stride, const float* bias, int n, int k, float scale,
                        int32_t* ids, float* w, int* err, hipStream_t s) {
    if (T < 1 || n < 1 || n > kRouteMaxExperts || k < 1 || k > 16 || k > n || stride < n) return hipErrorInvalidValue;
    if (n <= 64)
        hipLaunchKernelGGL(route_kernel<1>, dim3(T), dim3(512), 0, s, logits, stride, bias, n, k, scale, ids, w, err);
    else if (n <= 512)
        hipLaunchKernelGGL(route_kernel<8>, dim3(T), dim3(512), 0, s, logits, stride, bias, n, k, scale, ids, w, err);
    else
        hipLaunchKernelGGL(route_kernel<64>, dim3(T), dim3(512), 0, s, logits, stride, bias, n, k, scale, ids, w, err);
    return hipGetLastError();
}

hipError_t launch_combine(const int32_t* ids, const float* w, int k, const float* y, int dim, const float* shared,
                          float* out, hipStream_t s) {
    if (k < 0 || k > 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(combine_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, ids, w, k, y, dim, shared, out);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, int n, float lim, float* h, hipStream_t s) {
    if (n < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, s, g, u, n, lim, h);
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
