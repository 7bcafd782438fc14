// Internal types shared by the host API (xl_api.cpp) and the kernels
// (xl_kernels.hip). Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace xl {

// Device-side error bits (OR-ed into the context's flag word by kernels).
enum : int {
    kDevErrExpertId = 1,     // an id outside [0, n_experts)
    kDevErrNonFinite = 2,    // non-finite activation seen by a quantizer
    kDevErrType = 4,         // a matrix with an unsupported block type
    kDevErrTimeout = 8,      // a bounded wait of a single-launch layer kernel expired
};

// One planar matrix (see plane_layout in xl_format.hpp).
struct MatRef {
    const uint8_t* base;
    uint64_t off1, off2;     // byte offsets of planes 1 and 2
    int32_t type;            // ggml type id 16 / 17 / 29
    int32_t nb;              // blocks per row (k / 256)
};

// Per (layer, expert) descriptor: gate (w1), up (w3), down (w2).
struct ExpertDesc {
    MatRef m[3];
};

// Shapes accepted by the specialized row kernels: K (the contraction length)
// maps to lanes-per-row LPR and pairs-per-lane PPL with LPR * PPL * 64 == K.
// 2304 and 5120 are the DeepSeek-V4.1 expert's ff and dim
// (engine/strata/fixtures/moe/cpu_lane_fixture.cpp:17).
inline bool row_shape(int k, int& lpr, int& ppl) {
    if (k <= 0 || k % 256) return false;
    const int pairs = k / 64;
    int l = 64;
    while (l > 4 && pairs % l) l >>= 1;
    lpr = l;
    ppl = pairs / l;
    switch (k) {
        case 256: case 512: case 768: case 1024: case 2048: case 2304: case 3072: case 4096: case 5120: return true;
        default: return false;
    }
}
constexpr int kMaxRowK = 5120;   // the longest row any kernel stages

// Arguments of the single-launch layer kernel (xl_layer.hip); device pointers.
struct Layer3Args {
    const ExpertDesc* descs;    // this layer's n_experts descriptors
    const int32_t* ids;
    const float* w;
    const float* x;
    const float* shared;        // may be null
    float* out;
    int k, n_experts, dim, ff;
    uint64_t* htag;             // k * ff words: (h value bits, epoch << 32)
    uint64_t* hqtag;            // k * ff/4 words: (4 Q8_K(h) quants, epoch << 32)
    uint64_t* hdtag;            // k * ff/256 words: (Q8_K(h) block scale bits, epoch << 32)
    uint32_t* ctl;              // [0] epoch of the last launch, [1] arrival counter (zero between launches)
    int* err;
    float lim;                  // SwiGLU limit (> 0: g = min(g, lim), u = clamp(u, -lim, lim))
    const uint64_t* tables;     // expanded codebooks (kTableBytes), see kG_* in xl_layer.hip
    // Regular layers (all experts with the same three block types, each
    // expert's matrices consecutive in the layer slab): matrix (id, role)
    // starts at slab + id * estride + roff[role] and no descriptor is read.
    // slab == nullptr: read the descriptors.
    const uint8_t* slab;
    uint64_t estride;
    uint64_t roff[3];
    int rtype[3];
    uint64_t* trace;            // null, or 32 timestamps (s_memrealtime) per wave of the grid
    float* hbuf;                // streaming kernel: 2 x kHBufWords h words, sentinel-filled (see xl_stream.hip)
    // Parity trace (all null unless traced; xl_layer_trace_async): the launch's own
    // Q8_K(x) and Q8_K(h) as 292-byte blocks (q8x: dim/256, q8h: k * ff/256, as
    // staged in workgroup 0's LDS), its h (k * ff floats) and every row's integer
    // per 256-weight block (tint: per pick, gate ff x dim/256, up ff x dim/256,
    // down dim x ff/256; IQ1_M rows: 8 * main + delta).
    uint8_t* tq8x;
    uint8_t* tq8h;
    float* th;
    int32_t* tint;
    float* ty;                  // trace: every pick's row before the combine (k x dim, ids order)
    // Routed in the kernel (streaming kernel; null: ids and w are read): every
    // wave routes the token from its n_experts <= kStreamRouteMax logits (bias
    // may be null) as the router kernel does; ids and w are then not read.
    const float* rlogits;
    const float* rbias;
    float rscale;
    // Pre-norm in the kernel (streaming kernel; null: x is read as is): x is the
    // hyper-connection pre + RMS norm of one token's single stream pn_h (dim
    // floats), mix weight pn_mix[0], norm weights pn_w (null: the pre values
    // only), as hc_pre_norm_kernel computes it; workgroup 0 writes it to pn_x.
    const float* pn_h;
    const float* pn_mix;
    const float* pn_w;
    float* pn_x;
    float pn_eps;
    // Hyper-connection post in the kernel (streaming kernel; null: none): each
    // output row e of the layer also gives po_out[j][e] = po_post[j] * out[e] +
    // sum_i po_comb[i * po_H + j] * po_res[i][e], as hc_post_kernel computes it
    // for one token (po_res and po_out po_H x dim; po_out may be po_res).
    const float* po_res;
    const float* po_post;
    const float* po_comb;
    float* po_out;
    int po_H;
    // x quantized per 32 as quant32_kernel does (streaming kernel; null: not
    // written): dim int8 quants in x order and dim / 32 scales, for a per32
    // shared-expert FFN that runs after the layer.
    int8_t* p32_q;
    float* p32_d;
};
constexpr int kHBufWords = 16 * 4096;      // k_max * ff_max
constexpr int kStreamRouteMax = 512;       // experts a streaming kernel routes itself (8 per lane)

// Arguments of the grouped path (xl_grouped.hip): T tokens with k picks each,
// P = T * k (token, pick) pairs, pair p = token p / k. Device pointers.
struct GroupArgs {
    const ExpertDesc* descs;    // this layer's n_experts descriptors
    const int32_t* ids;         // P expert ids
    const float* w;             // P route weights
    const float* x;             // T * dim
    const float* shared;        // T * dim, or null
    float* out;                 // T * dim
    int T, k, n_experts, dim, ff;
    // Slots: task i owns slots 16 i .. 16 i + 15, its pairs in the first ones.
    int8_t* xq; float* xd;      // Q8_K(x): quants per slot (16 * max tasks * dim, the MFMA order), scales per token
    int32_t* order;             // pair of each used slot (16 * max tasks)
    int32_t* pos;               // slot of each pair (P; -1 for a bad id)
    int4* tasks;                // (expert, first slot, pairs <= 16, 0) per task
    int32_t* n_tasks;           // tasks written by the bucket kernel
    float* h;                   // P * ff
    int8_t* hq; float* hd;      // Q8_K(h): quants per slot (16 * max tasks * ff), scales per pair
    float* y;                   // P * dim
    const uint64_t* tables;     // expanded codebooks (kLayer3TableBytes)
    int* err;
    float lim;                  // SwiGLU limit (> 0: g = min(g, lim), u = clamp(u, -lim, lim))
    // Parity trace (all null unless traced; xl_grouped_trace_async): Q8_K(x) per
    // token (T x dim/256 blocks of 292 bytes), Q8_K(h) per pair (P x ff/256), h
    // per pair (P x ff floats) and the block integers per pair (layout as
    // Layer3Args::tint, one record per pair).
    uint8_t* tq8x;
    uint8_t* tq8h;
    float* th;
    int32_t* tint;
};
constexpr int kGroupMaxExperts = 8192;
constexpr int kRouteMaxExperts = 4096;   // router: scores and keys of one token in LDS   // experts per layer the bucket kernel counts in LDS
// Tasks the bucket kernel can write for P pairs: one per started tile of 16 pairs of an expert.
inline int64_t group_max_tasks(int64_t P, int64_t n_experts) { return P / 16 + (P < n_experts ? P : n_experts) + 1; }
constexpr int kLayer3TableBytes = 24576;   // expanded codebooks of the single-launch kernel
// Then the IQ1_M value rows of the streaming kernels: 4096 rows of 8 int8,
// row (nib << 8 | idx_lo) = 8 * grid[(nib & 7) << 8 | idx_lo] + (nib & 8 ? -1 : 1).
constexpr int kTableIQ1X = kLayer3TableBytes;
constexpr int kTableBytes = kTableIQ1X + 4096 * 8;

// Size of the no-allocation entry point's static device scratch (xl_noalloc.hip).
constexpr uint64_t kNoAllocScratchBytes = uint64_t(8) << 20;

namespace dev {
// Device address of this GPU's copy of the no-allocation scratch (looked up
// once per device by hipGetSymbolAddress, with `device` current; then cached).
hipError_t noalloc_scratch(int device, void** out);
// Single-launch layer: hipErrorNotSupported when (dim, ff, k) has no instance.
// gu_types / dn_types: block types among the layer's gate/up / down matrices
// (bits 1 IQ2_XXS, 2 IQ2_XS, 4 IQ1_M) select the kernel instance.
// `stop` (may be null) is recorded as the launch completes (hipExtLaunchKernel's
// stop event: no extra packet on the stream).
hipError_t launch_layer3(const Layer3Args& args, int gu_types, int dn_types, int cus, hipStream_t s,
                         hipEvent_t stop = nullptr);
// Streaming layer (xl_stream*.hip): instances for IQ2_XXS gate/up + IQ2_XS down,
// IQ1_M only, and any mix of the three types (per matrix, read from each
// pick's descriptor); hipErrorNotSupported when (dim, ff, k, types) has none.
hipError_t launch_stream(const Layer3Args& args, int gu_types, int dn_types, int cus, hipStream_t s,
                         hipEvent_t stop = nullptr);
hipError_t launch_stream_iq1(const Layer3Args& args, int cus, hipStream_t s, hipEvent_t stop);
hipError_t launch_stream_mix(const Layer3Args& args, int cus, hipStream_t s, hipEvent_t stop);
// Grouped path: hipErrorNotSupported unless gate/up are IQ2_XXS, down IQ2_XS and
// the shapes fit (dim, ff multiples of 128; n_experts <= kGroupMaxExperts).
hipError_t launch_grouped(const GroupArgs& args, int cus, hipStream_t s);
hipError_t launch_q8k(const float* x, int nblocks, int8_t* qs, float* d, uint8_t* std_out, int* err, hipStream_t s);
// Rows in the reference CPU lane's float order (xl_exact.hip): role 0 gives
// h = SwiGLU(gate . a, up . a) of every pick (out: k x rows), role 2 the down
// rows against each pick's own activation (aq + pick * kdim; out: k x rows).
hipError_t launch_exact_rows(const ExpertDesc* descs, const int32_t* ids, int k, int n_experts, int rows, int kdim,
                             int role, const int8_t* aq, const float* ad, const uint64_t* tables, float* out, float lim,
                             int* err, hipStream_t s);
// `codes` is the compact codebook buffer (2-bit symbols, see xl_rows.hpp);
// `target_wgs` is the workgroup count the row launches aim for.
hipError_t launch_matvec(const MatRef& m, int n, int k, const int8_t* aq, const float* ad, const uint16_t* codes,
                         float* y, int32_t* partials, int* err, hipStream_t s);
// Gate/up + SwiGLU for k picks: h[i*ff + r] = silu(gate_i . x) * (up_i . x).
hipError_t launch_gate_up(const ExpertDesc* descs, const int32_t* ids, int k, int n_experts, int dim, int ff,
                          const int8_t* xq, const float* xd, const uint16_t* codes, float* h, float* g_dbg,
                          float* u_dbg, int* err, int target_wgs, int type_mask, float lim, hipStream_t s);
// Down for k picks: y[i*dim + r] = down_i . Q8_K(h_i).
hipError_t launch_down(const ExpertDesc* descs, const int32_t* ids, int k, int n_experts, int dim, int ff,
                       const int8_t* hq, const float* hd, const uint16_t* codes, float* y, int* err, int target_wgs,
                       int type_mask, hipStream_t s);
// type_mask bits (1 IQ2_XXS, 2 IQ2_XS, 4 IQ1_M): block types present among the
// launch's matrices; sizes the LDS codebook region.
int type_bit(int type);
// Fixed-order combine: ascending id, out = fma(w, y, out), then + shared.
// Router (route.cpp:15-37) of T tokens of n <= kRouteMaxExperts logits.
hipError_t launch_route(const float* logits, int T, int stride, const float* bias, int n, int k, float scale,
                        int32_t* ids, float* w, int* err, hipStream_t s);
hipError_t launch_combine(const int32_t* ids, const float* w, int k, const float* y, int dim, const float* shared,
                          float* out, hipStream_t s);
// per32 mode (xl_per32.hip): per-32 activation quantization of rows x k values
// (k a multiple of 32) into q (int8) and d (one float per 32).
hipError_t launch_quant32(const float* x, int rows, int k, int8_t* q, float* d, int* err, hipStream_t s);
// per32 rows of roles role0 .. role0 + roles - 1 (at most 2) of every pick's
// expert (ids == nullptr: the matrices single0 / single1 for roles 0 / 1):
// y_r[pick * y_stride + row] from q + pick * q_stride (16-byte aligned) and
// d + pick * d_stride. Matrices: planar IQ types or raw dense blocks (Q8_0,
// Q4_K, Q5_K, Q6_K, base 16-byte aligned).
// Epilogue of a one-pick, one-role row launch (the MoE block's shared down
// rows): y[row] = add[row] + the row's value (the layer combine's order,
// routed + shared), then, if res is set, the hyper-connection post of that
// column as hc_post_kernel computes it for one token: out[j][row] = post[j] *
// y[row] + sum_i comb[i * H + j] * res[i][row] (out H x n, may equal res).
struct Mv32Post {
    const float* add;
    const float* res;
    const float* post;
    const float* comb;
    float* out;
    int H;
};
// The per32 layer's fixed-order combine in a bank row launch (ids, one role,
// picks <= 16): out[row] = fma(w, y, .) over the picks by ascending expert id
// (equal ids in pick order) from +0, then + shared[row] when shared is set;
// y is written as well.
struct Mv32Comb {
    const float* w;
    const float* shared;
    float* out;
};
hipError_t launch_mv32(const ExpertDesc* descs, const int32_t* ids, const MatRef& single0, const MatRef& single1,
                       int picks, int n_experts, int role0, int roles, int n, int k, const int8_t* q, size_t q_stride,
                       const float* d, size_t d_stride, float* y0, float* y1, size_t y_stride,
                       const uint64_t* tables, int* err, hipStream_t s, const Mv32Post* epi = nullptr,
                       const Mv32Comb* comb = nullptr);
// Hyper-connection post (sycl/hc/core.hpp:81-86) of T tokens, H <= 4 streams
// of D: out[t][k][e] = post[t][k] * y[t][e] + sum_j comb[t][j * H + k] *
// res[t][j][e]; out may equal res (in place).
// stop: recorded as the launch completes (the caller's ordering event)
hipError_t launch_hc_pre_norm(const float* h, const float* mix, const float* w, int D, int H, int T, float eps,
                              float* x, hipStream_t s, hipEvent_t stop);
hipError_t launch_hc_post(const float* y, const float* res, const float* post, const float* comb, int D, int H, int T,
                          float* out, hipStream_t s, hipEvent_t stop);
// h = g / (1 + exp(-g)) * u (lim > 0: g, u clamped first) of rows x k values,
// quantized per 32 into q, d exactly as launch_quant32 would quantize h.
hipError_t launch_swiglu_quant32(const float* g, const float* u, int rows, int k, float lim, int8_t* q, float* d,
                                 hipStream_t s);
// h = SwiGLU(g, u) elementwise over n values, with the limit (lim <= 0: none).
hipError_t launch_swiglu(const float* g, const float* u, int n, float lim, float* h, hipStream_t s);
// Seeded generation of one planar matrix (role 0 gate, 1 up, 2 down).
hipError_t launch_generate(uint8_t* base, int type, int n, int k, uint64_t seed, uint32_t layer, uint32_t expert,
                           uint32_t role, hipStream_t s);
}  // namespace dev
}  // namespace xl
