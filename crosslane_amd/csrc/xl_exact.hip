// The routed-expert rows in the reference CPU lane's own float order (gfx950).
//
// q8k_core.hpp:76-91 (`dot_lane`, `hsum`, `dot`), the arithmetic of the AVX2
// ggml lane it restates: for each AVX2 lane L (positions 4L..4L+3 of every
// 32-weight sub-block) an exact integer per 256-weight block, then one fmaf
// chain per lane over the blocks in order, acc_L = fmaf(fp16(d_w) * d_a,
// float(int_L), acc_L) (IQ1_M: a main and a delta chain), then the fixed hsum
// ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7)), times 1/8 (IQ1_M: main + 1/8 delta).
// The SwiGLU (q8k_core.hpp:92-95) takes the host C library's expf, restated
// for the device in xl_refexp.hpp.
//
// The fast layer kernels keep the integers exact but sum each row's floats in
// their own order (within ~1e-7 of the reference); this path gives the
// reference's bits, so that a pass over many layers, whose chaotic synthetic
// map amplifies any last-bit difference once a Q8_K rounding flips, can be
// compared with the CPU reference bit for bit.
//
// Layout: a workgroup of 4 waves takes 32 rows of one pick; row r of a wave is
// lanes 8r..8r+7, lane L = AVX2 lane L. Each lane walks the row's blocks in
// order; the codebooks (sign masks, the three grids) and the activation vector
// are staged in LDS. Gate/up rows give h directly (both chains in the same
// lanes); down rows give y.
#include <hip/hip_runtime.h>

#include "xl_dev.hpp"
#include "xl_format.hpp"
#include "xl_internal.hpp"
#include "xl_refexp.hpp"

namespace xl::dev {
namespace {

// LDS map: sign masks (128 x {mask, mask & 0x01..}), IQ2_XXS grid (256 x 8 B),
// IQ2_XS grid (512 x 8 B), IQ1 grid (2048 x 8 int8), then the Q8_K quants and
// block scales of the activation.
constexpr int kXSgn = 0, kXXxs = 2048, kXXs = 4096, kXIq1 = 8192, kXTab = 24576;
constexpr int kXAct = kXTab;   // kMaxRowK quants, then kMaxRowK / 256 floats
constexpr int kXLds = kXAct + kMaxRowK + 4 * (kMaxRowK / 256);

struct ExactArgs {
    const ExpertDesc* descs;   // this layer's descriptors
    const int32_t* ids;        // k expert ids
    int k, n_experts;
    int rows, kdim;            // rows per matrix, contraction length (multiples of 32 and 256)
    int role;                  // 0: gate and up rows (-> h), 2: down rows (-> y)
    const int8_t* aq;          // Q8_K quants (kdim per pick when role 2, else kdim shared)
    const float* ad;           // Q8_K block scales
    const uint64_t* tables;    // expanded codebooks (kLayer3TableBytes)
    float* out;                // h: k x rows, or y: k x rows
    float lim;                 // SwiGLU limit (role 0)
    int* err;
};

// Signed grid bytes: (g ^ m) + (m & 0x01010101) negates the bytes where m is 0xff.
__device__ __forceinline__ uint32_t sgn_bytes(uint32_t g, uint32_t m, uint32_t ones) { return (g ^ m) + ones; }

struct Ints {
    int main, delta;
};

// Lane L's exact integers over block b of a matrix (q8k_core.hpp:43-69,
// `integer_lane`), planar fields (xl_format.hpp). q: the block's 256 quants.
__device__ __forceinline__ Ints lane_ints(const MatRef& m, uint64_t blk, const int8_t* q, const uint8_t* lds, int L) {
    Ints r{0, 0};
    const int g = L >> 1, half = 4 * (L & 1);
    const uint8_t* Q = m.base + uint64_t(m.type == kIQ1_M ? 32 : 64) * blk;
    if (m.type == kIQ2_XXS) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t aux = *reinterpret_cast<const uint32_t*>(Q + 8 * c + 4);   // byte j: sign_j | scale bit j << 7
            const int idx = Q[8 * c + g];
            const int s7 = int((aux >> (8 * g)) & 127u);
            const uint32_t sc4 = ((aux >> 7) & 1u) | ((aux >> 14) & 2u) | ((aux >> 21) & 4u) | ((aux >> 28) & 8u);
            const uint32_t gr = *reinterpret_cast<const uint32_t*>(lds + kXXxs + 8 * idx + half);
            const uint32_t mk = *reinterpret_cast<const uint32_t*>(lds + kXSgn + 16 * s7 + half);
            const uint32_t on = *reinterpret_cast<const uint32_t*>(lds + kXSgn + 16 * s7 + 8 + half);
            const uint32_t qa = *reinterpret_cast<const uint32_t*>(q + 32 * c + 4 * L);
            r.main += int(2 * sc4 + 1) * __builtin_amdgcn_sdot4(int(sgn_bytes(gr, mk, on)), int(qa), 0, false);
        }
    } else if (m.type == kIQ2_XS) {
        const uint8_t* S = m.base + m.off1 + 8 * blk;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t code = *reinterpret_cast<const uint16_t*>(Q + 2 * (4 * c + g));   // sign7 | grid9 << 7
            const int s7 = int(code & 127u), idx = int(code >> 7);
            const int sc = 2 * int((S[c] >> (4 * (L >> 2))) & 15u) + 1;
            const uint32_t gr = *reinterpret_cast<const uint32_t*>(lds + kXXs + 8 * idx + half);
            const uint32_t mk = *reinterpret_cast<const uint32_t*>(lds + kXSgn + 16 * s7 + half);
            const uint32_t on = *reinterpret_cast<const uint32_t*>(lds + kXSgn + 16 * s7 + 8 + half);
            const uint32_t qa = *reinterpret_cast<const uint32_t*>(q + 32 * c + 4 * L);
            r.main += sc * __builtin_amdgcn_sdot4(int(sgn_bytes(gr, mk, on)), int(qa), 0, false);
        }
    } else {   // IQ1_M: qs (Q), qh (off1), scale words (off2)
        const uint8_t* H = m.base + m.off1 + 16 * blk;
        const uint8_t* W = m.base + m.off2 + 8 * blk;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t hi = H[2 * c + (g >> 1)];
            const int idx = int(Q[4 * c + g]) | int(((g & 1) ? (hi >> 4) : hi) & 7u) << 8;
            const int dl = (hi & ((g & 1) ? 0x80u : 0x08u)) ? -1 : 1;
            const uint32_t sw = *reinterpret_cast<const uint16_t*>(W + 2 * (c >> 1));
            const int sc = 2 * int((sw >> (6 * (c & 1) + 3 * (L >> 2))) & 7u) + 1;
            const uint32_t gr = *reinterpret_cast<const uint32_t*>(lds + kXIq1 + 8 * idx + half);
            const uint32_t qa = *reinterpret_cast<const uint32_t*>(q + 32 * c + 4 * L);
            r.main += sc * __builtin_amdgcn_sdot4(int(gr), int(qa), 0, false);
            r.delta += sc * dl * __builtin_amdgcn_sdot4(0x01010101, int(qa), 0, false);
        }
    }
    return r;
}

// fp16 super-block scale of block blk (q8k_core.hpp:70-74 `scale`).
__device__ __forceinline__ float block_scale(const MatRef& m, uint64_t blk) {
    if (m.type == kIQ2_XXS) return half_to_float(*reinterpret_cast<const uint16_t*>(m.base + m.off1 + 2 * blk));
    if (m.type == kIQ2_XS) return half_to_float(*reinterpret_cast<const uint16_t*>(m.base + m.off2 + 2 * blk));
    return half_to_float(iq1m_scale_bits(m.base + m.off2 + 8 * blk));
}

// The hsum of the 8 lanes of each row group, in the reference's order; the
// result is in lane 0 of the group.
__device__ __forceinline__ float row_hsum(float v) {
    v = __fadd_rn(v, __shfl_down(v, 4, 8));   // lanes 0..3: v0+v4, v1+v5, v2+v6, v3+v7
    v = __fadd_rn(v, __shfl_down(v, 2, 8));   // lanes 0, 1: (v0+v4)+(v2+v6), (v1+v5)+(v3+v7)
    return __fadd_rn(v, __shfl_down(v, 1, 8));
}

// One row's dot (q8k_core.hpp:85-91 `dot`) in lane 0 of its 8-lane group.
__device__ __forceinline__ float exact_dot(const MatRef& m, int row, const int8_t* aq, const float* ad, int nb,
                                           const uint8_t* lds, int L) {
    float sm = 0.0f, sd = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint64_t blk = uint64_t(row) * uint64_t(nb) + uint64_t(b);
        const Ints v = lane_ints(m, blk, aq + 256 * b, lds, L);
        const float d = __fmul_rn(block_scale(m, blk), ad[b]);
        sm = fmaf(d, float(v.main), sm);
        if (m.type == kIQ1_M) sd = fmaf(d, float(v.delta), sd);
    }
    const float hm = row_hsum(sm);
    if (m.type == kIQ1_M) return __fadd_rn(hm, __fmul_rn(0.125f, row_hsum(sd)));
    return __fmul_rn(0.125f, hm);
}

__global__ __launch_bounds__(256) void exact_rows_kernel(ExactArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kXLds];
    const int t = threadIdx.x, lane = t & 63, L = lane & 7;
    const int pick = blockIdx.y;
    const int row = blockIdx.x * 32 + (t >> 3);
    const int nb = a.kdim / 256;
    // codebooks
    const uint4* tab = reinterpret_cast<const uint4*>(a.tables);
    for (int i = t; i < kXTab / 16; i += 256) reinterpret_cast<uint4*>(lds)[i] = tab[i];
    // the activation: Q8_K(x) for gate/up, this pick's Q8_K(h) for down
    const size_t ao = a.role == 2 ? size_t(pick) * size_t(a.kdim) : 0;
    const size_t so = a.role == 2 ? size_t(pick) * size_t(nb) : 0;
    for (int i = t; i < a.kdim / 16; i += 256)
        reinterpret_cast<uint4*>(lds + kXAct)[i] = reinterpret_cast<const uint4*>(a.aq + ao)[i];
    float* const sd = reinterpret_cast<float*>(lds + kXAct + kMaxRowK);
    for (int i = t; i < nb; i += 256) sd[i] = a.ad[so + i];
    __syncthreads();
    const int id = a.ids[pick];
    if (id < 0 || id >= a.n_experts) {
        if (t == 0) set_err(a.err, kDevErrExpertId);
        return;   // the whole workgroup: no barrier follows
    }
    if (row >= a.rows) return;
    const int8_t* q = reinterpret_cast<const int8_t*>(lds + kXAct);
    if (a.role == 2) {
        const float y = exact_dot(a.descs[id].m[2], row, q, sd, nb, lds, L);
        if (L == 0) a.out[size_t(pick) * size_t(a.rows) + row] = y;
        return;
    }
    float g = exact_dot(a.descs[id].m[0], row, q, sd, nb, lds, L);
    float u = exact_dot(a.descs[id].m[1], row, q, sd, nb, lds, L);
    if (L == 0) {
        // q8k_core.hpp:92-95: (g / (1 + expf(-g))) * u
        if (a.lim > 0.0f) {
            g = fminf(g, a.lim);
            u = fminf(fmaxf(u, -a.lim), a.lim);
        }
        const float e = ref_expf(-g);
        a.out[size_t(pick) * size_t(a.rows) + row] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
    }
}

}  // namespace

hipError_t launch_exact_rows(const ExpertDesc* descs, const int32_t* ids, int k, int n_experts, int rows, int kdim,
                             int role, const int8_t* aq, const float* ad, const uint64_t* tables, float* out, float lim,
                             int* err, hipStream_t s) {
    if (k < 1 || k > 65535 || rows < 1 || rows % 32 || kdim < 256 || kdim % 256 || kdim > kMaxRowK ||
        (role != 0 && role != 2))
        return hipErrorInvalidValue;
    ExactArgs a{descs, ids, k, n_experts, rows, kdim, role, aq, ad, tables, out, lim, err};
    hipLaunchKernelGGL(exact_rows_kernel, dim3(rows / 32, k), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace xl::dev
