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
// lanes 8r..8r+7, lane L = AVX2 lane L. Each row group loads a block's bytes
// whole (16-byte loads its 8 lanes share) and the next block's before the
// current block's arithmetic, and walks the row's blocks in order; the
// codebooks (sign masks, the three grids) and the activation vector are staged
// in LDS. Gate/up rows give h directly (the gate and up chains side by side in
// the same lanes); down rows give y. 84 us per config-1 layer (five launches),
// 100.6 with per-field loads and one chain at a time.
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

// One block's bytes as a row group loads them (the 8 lanes of a row read the
// same addresses, so each load is one 16-byte access per row): q the 64-byte
// quant plane (IQ1_M: q[0..1] the 32 qs bytes, q[2] the 16 qh bytes), s the
// IQ2_XS scale bytes or the IQ1_M scale words, d the fp16 block scale bits.
struct RawBlk {
    uint4 q[4];
    uint2 s;
    uint32_t d;
};
template <int T>
__device__ __forceinline__ RawBlk load_blk(const MatRef& m, uint64_t blk) {
    RawBlk r{};
    if constexpr (T == kIQ1_M) {
        const uint4* Q = reinterpret_cast<const uint4*>(m.base + 32 * blk);
        r.q[0] = Q[0];
        r.q[1] = Q[1];
        r.q[2] = *reinterpret_cast<const uint4*>(m.base + m.off1 + 16 * blk);
        r.s = *reinterpret_cast<const uint2*>(m.base + m.off2 + 8 * blk);
    } else {
        const uint4* Q = reinterpret_cast<const uint4*>(m.base + 64 * blk);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = Q[i];
        if constexpr (T == kIQ2_XXS) {
            r.d = *reinterpret_cast<const uint16_t*>(m.base + m.off1 + 2 * blk);
        } else {
            r.s = *reinterpret_cast<const uint2*>(m.base + m.off1 + 8 * blk);
            r.d = *reinterpret_cast<const uint16_t*>(m.base + m.off2 + 2 * blk);
        }
    }
    return r;
}
__device__ __forceinline__ uint32_t qword(const RawBlk& r, int w) {   // dword w (compile-time) of q
    const uint4 v = r.q[w >> 2];
    return (w & 3) == 0 ? v.x : (w & 3) == 1 ? v.y : (w & 3) == 2 ? v.z : v.w;
}

// Lane L's exact integers over one block (q8k_core.hpp:43-69, `integer_lane`),
// from the planar fields (xl_format.hpp) of the block's bytes. q: the block's
// 256 activation quants.
template <int T>
__device__ __forceinline__ Ints lane_ints(const RawBlk& r, const int8_t* q, const uint8_t* lds, int L) {
    Ints o{0, 0};
    const int g = L >> 1, half = 4 * (L & 1);
    if constexpr (T == kIQ2_XXS) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t idxw = qword(r, 2 * c), aux = qword(r, 2 * c + 1);   // aux byte j: sign_j | scale bit j << 7
            const int idx = int((idxw >> (8 * g)) & 255u);
            const int s7 = int((aux >> (8 * g)) & 127u);
            const uint32_t sc4 = ((aux >> 7) & 1u) | ((aux >> 14) & 2u) | ((aux >> 21) & 4u) | ((aux >> 28) & 8u);
            const uint32_t gr = *reinterpret_cast<const uint32_t*>(lds + kXXxs + 8 * idx + half);
            const uint32_t mk = *reinterpret_cast<const uint32_t*>(lds + kXSgn + 16 * s7 + half);
            const uint32_t on = *reinterpret_cast<const uint32_t*>(lds + kXSgn + 16 * s7 + 8 + half);
            const uint32_t qa = *reinterpret_cast<const uint32_t*>(q + 32 * c + 4 * L);
            o.main += int(2 * sc4 + 1) * __builtin_amdgcn_sdot4(int(sgn_bytes(gr, mk, on)), int(qa), 0, false);
        }
    } else if constexpr (T == kIQ2_XS) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            // code 4c + g (sign7 | grid9 << 7) sits in dword 2c + g / 2, half g % 2
            const uint32_t w = (g >> 1) ? qword(r, 2 * c + 1) : qword(r, 2 * c);
            const uint32_t code = (w >> (16 * (g & 1))) & 0xffffu;
            const int s7 = int(code & 127u), idx = int(code >> 7);
            const uint32_t sb = ((c < 4 ? r.s.x : r.s.y) >> (8 * (c & 3))) & 255u;
            const int sc = 2 * int((sb >> (4 * (L >> 2))) & 15u) + 1;
            const uint32_t gr = *reinterpret_cast<const uint32_t*>(lds + kXXs + 8 * idx + half);
            const uint32_t mk = *reinterpret_cast<const uint32_t*>(lds + kXSgn + 16 * s7 + half);
            const uint32_t on = *reinterpret_cast<const uint32_t*>(lds + kXSgn + 16 * s7 + 8 + half);
            const uint32_t qa = *reinterpret_cast<const uint32_t*>(q + 32 * c + 4 * L);
            o.main += sc * __builtin_amdgcn_sdot4(int(sgn_bytes(gr, mk, on)), int(qa), 0, false);
        }
    } else {   // IQ1_M: qs bytes 4c + g, qh byte 2c + g / 2, scale word c / 2
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t qs = (qword(r, c) >> (8 * g)) & 255u;
            const uint32_t hi = (qword(r, 8 + (c >> 1)) >> (8 * (2 * (c & 1) + (g >> 1)))) & 255u;
            const int idx = int(qs) | int(((g & 1) ? (hi >> 4) : hi) & 7u) << 8;
            const int dl = (hi & ((g & 1) ? 0x80u : 0x08u)) ? -1 : 1;
            const uint32_t sw = ((c >> 2) ? r.s.y : r.s.x) >> (16 * ((c >> 1) & 1));
            const int sc = 2 * int((sw >> (6 * (c & 1) + 3 * (L >> 2))) & 7u) + 1;
            const uint32_t gr = *reinterpret_cast<const uint32_t*>(lds + kXIq1 + 8 * idx + half);
            const uint32_t qa = *reinterpret_cast<const uint32_t*>(q + 32 * c + 4 * L);
            o.main += sc * __builtin_amdgcn_sdot4(int(gr), int(qa), 0, false);
            o.delta += sc * dl * __builtin_amdgcn_sdot4(0x01010101, int(qa), 0, false);
        }
    }
    return o;
}

// fp16 super-block scale (q8k_core.hpp:70-74 `scale`); IQ1_M's from the top
// nibbles of its four scale words.
template <int T>
__device__ __forceinline__ float block_scale(const RawBlk& r) {
    if constexpr (T == kIQ1_M) {
        const uint32_t w0 = r.s.x & 0xffffu, w1 = r.s.x >> 16, w2 = r.s.y & 0xffffu, w3 = r.s.y >> 16;
        return half_to_float(uint16_t((w0 >> 12) | ((w1 >> 8) & 0x00f0u) | ((w2 >> 4) & 0x0f00u) | (w3 & 0xf000u)));
    } else {
        return half_to_float(uint16_t(r.d));
    }
}

// The hsum of the 8 lanes of each row group, in the reference's order; the
// result is in lane 0 of the group.
__device__ __forceinline__ float row_hsum(float v) {
    v = __fadd_rn(v, __shfl_down(v, 4, 8));   // lanes 0..3: v0+v4, v1+v5, v2+v6, v3+v7
    v = __fadd_rn(v, __shfl_down(v, 2, 8));   // lanes 0, 1: (v0+v4)+(v2+v6), (v1+v5)+(v3+v7)
    return __fadd_rn(v, __shfl_down(v, 1, 8));
}
__device__ __forceinline__ float finish(int type, float sm, float sd) {   // q8k_core.hpp:85-91 `dot`
    const float hm = row_hsum(sm);
    if (type == kIQ1_M) return __fadd_rn(hm, __fmul_rn(0.125f, row_hsum(sd)));
    return __fmul_rn(0.125f, hm);
}

// The dots of row `row` of NM matrices of type T (gate and up, or down) in lane
// 0 of its 8-lane group: one fmaf chain per lane and matrix over the blocks in
// order, the next block's bytes loaded before the current block's arithmetic.
template <int T, int NM>
__device__ __forceinline__ void exact_dots(const MatRef* const (&m)[NM], int row, const int8_t* aq, const float* ad,
                                           int nb, const uint8_t* lds, int L, float (&res)[NM]) {
    float sm[NM], sd[NM];
    RawBlk cur[NM];
    const uint64_t b0 = uint64_t(row) * uint64_t(nb);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
        sm[i] = 0.0f;
        sd[i] = 0.0f;
        cur[i] = load_blk<T>(*m[i], b0);
    }
    for (int b = 0; b < nb; ++b) {
        RawBlk nxt[NM];
        const uint64_t bn = b0 + uint64_t(b + 1 < nb ? b + 1 : b);   // the last block reloads itself
#pragma unroll
        for (int i = 0; i < NM; ++i) nxt[i] = load_blk<T>(*m[i], bn);
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const Ints v = lane_ints<T>(cur[i], aq + 256 * b, lds, L);
            const float d = __fmul_rn(block_scale<T>(cur[i]), ad[b]);
            sm[i] = fmaf(d, float(v.main), sm[i]);
            if constexpr (T == kIQ1_M) sd[i] = fmaf(d, float(v.delta), sd[i]);
            cur[i] = nxt[i];
        }
    }
#pragma unroll
    for (int i = 0; i < NM; ++i) res[i] = finish(T, sm[i], sd[i]);
}
template <int NM>
__device__ __forceinline__ void exact_dots_any(const MatRef* const (&m)[NM], int row, const int8_t* aq,
                                               const float* ad, int nb, const uint8_t* lds, int L,
                                               float (&res)[NM]) {
    // (gate and up share a type: xl_open rejects banks where they differ)
    const int t = m[0]->type;
    if (t == kIQ2_XXS) exact_dots<kIQ2_XXS, NM>(m, row, aq, ad, nb, lds, L, res);
    else if (t == kIQ2_XS) exact_dots<kIQ2_XS, NM>(m, row, aq, ad, nb, lds, L, res);
    else exact_dots<kIQ1_M, NM>(m, row, aq, ad, nb, lds, L, res);
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
    const ExpertDesc& e = a.descs[id];
    if (a.role == 2) {
        const MatRef* const md[1] = {&e.m[2]};
        float y[1];
        exact_dots_any<1>(md, row, q, sd, nb, lds, L, y);
        if (L == 0) a.out[size_t(pick) * size_t(a.rows) + row] = y[0];
        return;
    }
    const MatRef* const mg[2] = {&e.m[0], &e.m[1]};
    float gu[2];
    exact_dots_any<2>(mg, row, q, sd, nb, lds, L, gu);
    float g = gu[0], u = gu[1];
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
