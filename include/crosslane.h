/* crosslane MI355X routed-expert lane: C ABI.
 *
 * One resident expert bank on one GPU; per token and layer, "compute these
 * top-k experts for this vector, then join them in a fixed order". Plain
 * pointers and sizes only. Every call returns int32 status (XL_OK = 0) and,
 * when `err` is non-null, fills it; the context also keeps the last error.
 * A context is driven by one caller thread at a time (the reference drives its
 * HIP lane from one dedicated worker thread, engine/strata/warm/worker.hpp:9-18).
 * Its device work is ordered: every call that enqueues work waits (on the GPU,
 * hipStreamWaitEvent) for the context's previous call when that one named
 * another stream, so calls on one context never overlap, whatever streams they
 * name (they share the context's workspace, exchange buffers and counters).
 * The single-launch layer kernels spin on data other workgroups of the same
 * launch produce: they need all their workgroups resident at once (one per CU)
 * and make progress only while no other kernel holds the CUs they wait for.
 * Two contexts, or another persistent kernel, launched concurrently on other
 * streams can starve them; such a wait ends in the device error flag
 * (XL_E_DEVICE, "layer wait timeout") after about a second, not in a hang.
 * No call allocates device memory after xl_bank_create (the workspace is sized
 * at xl_open, like the reference's arena reservation,
 * engine/strata/sycl/stage/wiring/hip_resident_bank.hpp:63-94).
 *
 * Conventions mirror the reference's DSO ABI (engine/strata/sycl/stage/wiring/
 * abi_v2.h:28-68, abi_backend_plugin.cpp:31-39): a version + struct-size check
 * before anything is written, an int32 code plus a 512-byte message, every
 * exception caught at the boundary, and a context poisoned by a device error
 * (all later compute calls fail until xl_close).
 */
#ifndef CROSSLANE_H
#define CROSSLANE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define XL_ABI_VERSION 3u

enum {
    XL_OK = 0,
    XL_E_ARG = 1,        /* invalid argument (shape, id, pointer, finiteness) */
    XL_E_STATE = 2,      /* wrong call order, or a poisoned context */
    XL_E_HIP = 3,        /* HIP runtime error */
    XL_E_DEVICE = 4,     /* a kernel reported an error flag (bad id, non-finite) */
    XL_E_VERSION = 5,    /* ABI version or struct size mismatch */
    XL_E_MEMORY = 6      /* device or host allocation failed */
};

/* ggml block type ids accepted for expert matrices */
enum { XL_IQ2_XXS = 16, XL_IQ2_XS = 17, XL_IQ1_M = 29 };

typedef struct xl_error {
    int32_t code;
    char message[512];
} xl_error;

typedef struct xl_config {
    uint32_t struct_bytes; /* sizeof(xl_config) */
    int32_t device;        /* HIP device ordinal */
    int32_t dim;           /* d_model and d_ff: 256, 512, 768, 1024, 2048, 2304, */
    int32_t ff;            /* 3072, 4096 or 5120 (the real expert: dim 5120, ff 2304) */
    int32_t n_layers;      /* layers in the bank */
    int32_t n_experts;     /* routed experts per layer */
    int32_t max_picks;     /* top-k bound, 1..16 (reference kPicks = 8, model_meta.hpp:18) */
    int32_t max_tokens;    /* grouped-path token bound (0 = grouped path unused). Its
                              workspace, with P = max_tokens * max_picks: about
                              16 * (P / 16 + min(P, n_experts) + 1) * (dim + ff) bytes
                              of per-slot quants plus 4 * P * (dim + ff) bytes of h
                              and per-pick rows (~200 MB at 512 tokens, 8 picks,
                              384 experts, 4096 x 3072) */
    float swiglu_limit;    /* SwiGLU limit (model_meta.hpp:34 `lim`, the pack's swiglu_limit):
                              > 0 clamps g to <= lim and u to [-lim, lim] before
                              SiLU(g) * u (q8k_core.hpp:92-95); <= 0: no clamp */
} xl_config;

typedef struct xl_bank_info {
    uint64_t payload_bytes;    /* ggml bytes of every resident matrix */
    uint64_t allocated_bytes;  /* device bytes held by the bank (256-B aligned planes) */
    uint64_t workspace_bytes;  /* device bytes of the per-call workspace */
    int32_t n_layers, n_experts;
    int32_t generated;         /* 1 after xl_bank_generate */
    int32_t reserved;
} xl_bank_info;

typedef struct xl_context xl_context;

uint32_t xl_abi_version(void);

/* Opens a context on cfg->device and sizes its workspace. */
int32_t xl_open(uint32_t abi_version, const xl_config* cfg, xl_context** out, xl_error* err);
/* Drains the context stream, then frees every device allocation. */
void xl_close(xl_context* ctx);
int32_t xl_last_error(const xl_context* ctx, xl_error* err);

/* ---- bank ---------------------------------------------------------------
 * types: n_layers * n_experts * 3 ggml type ids, roles (gate w1, up w3,
 * down w2) fastest; gate and up must share a type (the reference requires the
 * same, hip_resident.hpp:114). Replaces HipResidentBank::load's slab sizing
 * (hip_resident_bank.hpp:38-142, hip_resident.hpp:54-97). */
int32_t xl_bank_create(xl_context* ctx, const int32_t* types, xl_error* err);
/* Fills every matrix on the device from the seeded generator. */
int32_t xl_bank_generate(xl_context* ctx, uint64_t seed, xl_error* err);
/* Uploads / downloads one matrix as raw ggml AoS blocks (host memory); the
 * bank stores it repacked into planes. role: 0 gate, 1 up, 2 down. */
int32_t xl_bank_upload(xl_context* ctx, int32_t layer, int32_t expert, int32_t role, const void* aos, uint64_t bytes,
                       xl_error* err);
int32_t xl_bank_download(xl_context* ctx, int32_t layer, int32_t expert, int32_t role, void* aos, uint64_t bytes,
                         xl_error* err);
int32_t xl_bank_info_get(const xl_context* ctx, xl_bank_info* out);
/* 1 when (layer, expert) is resident (WarmRedirect::warm_contains,
 * engine/strata/warm/runtime.hpp:14). */
int32_t xl_contains(const xl_context* ctx, int32_t layer, int32_t expert);

/* ---- weight pack -------------------------------------------------------------
 * The reference's pack directory (engine/strata/sycl/stage/wiring/
 * pack_source.cpp:144-186): ds4.txt (model_dir, format gguf, hidden_size,
 * moe_intermediate_size, num_hidden_layers, n_routed_experts,
 * num_experts_per_tok, ...) and tensors.txt over shard files; routed experts
 * are layers.<l>.ffn.experts.<e>.w1 / w3 / w2 .weight (gate / up / down) in
 * raw ggml blocks. Host only: xl_pack_meta_get reads the shape, xl_pack_types
 * the block types of a layer window (layout as xl_bank_create takes them);
 * xl_bank_load_pack uploads every expert of the context's n_layers, pack
 * layers first_layer.. (dim, ff and n_experts must match the pack). */
typedef struct xl_pack_meta {
    uint32_t struct_bytes; /* sizeof(xl_pack_meta) */
    int32_t dim, ff, n_layers, n_experts, top_k;
    float swiglu_limit;    /* ds4.txt swiglu_limit, 0 when absent (pack_source.cpp:99) */
} xl_pack_meta;
int32_t xl_pack_meta_get(const char* pack_dir, xl_pack_meta* out, xl_error* err);
int32_t xl_pack_types(const char* pack_dir, int32_t first_layer, int32_t n_layers, int32_t n_experts, int32_t* types,
                      xl_error* err);
int32_t xl_bank_load_pack(xl_context* ctx, const char* pack_dir, int32_t first_layer, xl_error* err);

/* ---- lane calls, host memory, synchronous --------------------------------
 * xl_expert_forward   = WarmRedirect::warm_compute        (runtime.hpp:15)
 * xl_experts_forward  = WarmRedirect::warm_compute_many   (runtime.hpp:13):
 *                       ys is k rows of dim floats in `ids` order
 * xl_layer_forward    = the lane plus the caller's fixed-order combine
 *                       (warm_execute, runtime.cpp:180-188): ascending id,
 *                       out = fma(w, y, out), then out += shared when given.
 * ids must be unique and in [0, n_experts); k in 1..max_picks; x finite. */
int32_t xl_expert_forward(xl_context* ctx, int32_t layer, int32_t expert, const float* x, float* y, xl_error* err);
int32_t xl_experts_forward(xl_context* ctx, int32_t layer, const int32_t* ids, int32_t k, const float* x, float* ys,
                           xl_error* err);
int32_t xl_layer_forward(xl_context* ctx, int32_t layer, const int32_t* ids, const float* w, int32_t k, const float* x,
                         const float* shared_or_null, float* out, xl_error* err);
/* Expert chain with its intermediates (the reference's probe snapshot,
 * parity/hip_resident_check.cpp:56-62,93-104); any output may be null.
 * q8h receives ff/256 Q8_K blocks of 292 bytes. */
int32_t xl_expert_trace(xl_context* ctx, int32_t layer, int32_t expert, const float* x, float* g, float* u, float* h,
                        void* q8h, float* y, xl_error* err);

/* ---- device-resident calls (device pointers, ordered on `stream`; a null
 * stream means the context stream, created non-blocking: it does not wait
 * for work on the legacy default stream). Results are valid after the stream
 * drains; xl_sync drains and reports kernel error flags. Every buffer passed
 * must stay allocated and unwritten by other streams until then: a caching
 * allocator (PyTorch's) that reuses a freed input's memory for work on its own
 * stream races with the call. ids are checked on the device: a bad id sets the flag and
 * that pick contributes nothing. */
int32_t xl_layer_forward_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                               const float* d_x, const float* d_shared_or_null, float* d_out, void* stream,
                               xl_error* err);
int32_t xl_sync(xl_context* ctx, void* stream, xl_error* err);

/* ---- grouped tokens (prefill / batched decode) ------------------------------
 * T tokens, each with its own k picks: ids and w are T x k (token-major), x,
 * shared and out T x dim. The result is that of T xl_layer_forward calls (per
 * token: WarmRedirect::warm_compute_many, engine/strata/warm/runtime.hpp:13,
 * then warm_execute's fixed-order combine, runtime.cpp:180-188), with every
 * touched expert's weights read once per 16 of its (token, pick) pairs on
 * int8 MFMA for IQ2_XXS gate/up + IQ2_XS down layers (other layers run one
 * layer call per token). Needs a context opened with max_tokens >= T; picks
 * of one token unique. The async form takes device pointers and checks ids on
 * the device (a bad id sets the flag; that pick contributes nothing). */
int32_t xl_grouped_forward(xl_context* ctx, int32_t layer, int32_t T, int32_t k, const int32_t* ids, const float* w,
                           const float* x, const float* shared_or_null, float* out, xl_error* err);
int32_t xl_grouped_forward_async(xl_context* ctx, int32_t layer, int32_t T, int32_t k, const int32_t* d_ids,
                                 const float* d_w, const float* d_x, const float* d_shared_or_null, float* d_out,
                                 void* stream, xl_error* err);

/* The layer call of xl_layer_forward_async with every float computed in the
 * reference CPU lane's own order: q8k_core.hpp:76-91 (`dot_lane`, `hsum`,
 * `dot`: one exact integer per AVX2 lane and block, one fmaf chain per lane
 * over the blocks, the fixed hsum, IQ1_M's main and delta chains apart) and
 * :92-95 (`swiglu`, whose expf is the host C library's, restated for the
 * device), then the fixed-order combine of runtime.cpp:183-188. Its output
 * equals the CPU reference's bit for bit, so that a pass over many layers can
 * be held to the reference end to end. Separate launches, slower than
 * xl_layer_forward_async; same contract and device pointers. */
int32_t xl_layer_forward_exact_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w,
                                     int32_t k, const float* d_x, const float* d_shared_or_null, float* d_out,
                                     void* stream, xl_error* err);

/* ---- parity trace (device pointers) -------------------------------------------
 * The layer call's own intermediates, written by the kernel that computes it
 * (the reference's probe dumps its lane's Q8_K bytes the same way,
 * parity/hip_resident_check.cpp:91-127): the same single launch
 * xl_layer_forward_async would make, plus
 *   q8x  dim/256 Q8_K blocks (292 bytes: d, qs[256], bsums[16]; q8k_core.hpp:13)
 *        of x, as the launch staged them for its gate/up rows;
 *   q8h  k * ff/256 blocks, pick i's Q8_K(h) as staged for its down rows;
 *   h    k * ff floats, the SwiGLU output the launch quantized;
 *   ints per pick (ids order): gate ff x dim/256, up ff x dim/256, down
 *        dim x ff/256 int32, each row's exact integer per 256-weight block (as
 *        xl_matvec_async's partials; IQ1_M: 8 * main + delta);
 *   y    k * dim floats, every pick's row (ids order) as the launch's own
 *        fixed-order combine read it (so that out can be checked bit for bit
 *        against the combine of these rows);
 * kernel_out (host, may be null): 1 the streaming kernel ran, 3 the all-types
 * kernel. Any of q8x, q8h, h, ints, y may be null (not all).
 * XL_E_ARG when the
 * layer does not run as a single launch. A diagnostic aid (no counterpart in
 * the reference beyond its probe); it runs the traced kernel instances. */
int32_t xl_layer_trace_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                             const float* d_x, const float* d_shared_or_null, float* d_out, void* d_q8x, void* d_q8h,
                             float* d_h, int32_t* d_ints, float* d_y, int32_t* kernel_out, void* stream,
                             xl_error* err);
/* The same for the grouped MFMA path (XL_E_ARG when the layer does not run on
 * it): q8x per token (T x dim/256 blocks), q8h, h, ints and y per pair (P =
 * T * k, token-major), layouts as above. */
int32_t xl_grouped_trace_async(xl_context* ctx, int32_t layer, int32_t T, int32_t k, const int32_t* d_ids,
                               const float* d_w, const float* d_x, const float* d_shared_or_null, float* d_out,
                               void* d_q8x, void* d_q8h, float* d_h, int32_t* d_ints, float* d_y, void* stream,
                               xl_error* err);

/* Fixed-order combine of k per-pick rows on the device (engine/strata/warm/
 * runtime.cpp:183-188; other_combine.hpp:51-73 other_combine): out[c] =
 * fma(w_i, rows[i][c], .) over the picks in ascending expert id (equal ids in
 * pick order) from +0, then + shared[c]. d_rows: k x dim floats (ids order);
 * k in 1..16, dim in 1..2^24; d_shared_or_null may be null. Ordered with the
 * context's other calls; for rows computed elsewhere (xl_experts_forward, the
 * per32 rows). */
int32_t xl_combine_async(xl_context* ctx, const int32_t* d_ids, const float* d_w, int32_t k, const float* d_rows,
                         int32_t dim, const float* d_shared_or_null, float* d_out, void* stream, xl_error* err);

/* ---- router (device pointers) -----------------------------------------------
 * route.cpp:15-37 (route_cpu) on the device, per token: score =
 * sqrt(softplus(logit)) (the logit itself above 20), key = score + bias (a null
 * bias is zeros); k rounds of the first largest key (ties: lower index), each
 * taking the expert out; weight = score / (sum of the picked scores + 1e-20) *
 * scale. logits T x stride (n used, n <= 4096), ids and w T x k (k <= 16).
 * A non-finite logit or key sets the device flag (the reference throws). */
int32_t xl_route_async(xl_context* ctx, const float* d_logits, int32_t T, int32_t stride, const float* d_bias_or_null,
                       int32_t n, int32_t k, float scale, int32_t* d_ids, float* d_w, void* stream, xl_error* err);
/* The router over the layer's n_experts logits, then the layer call on its ids
 * and weights, both on `stream` (no host round trip). Where the streaming
 * kernel has the layer and n_experts <= 512 this is one launch that routes in
 * its prologue, bit-identical to the router followed by the layer call;
 * otherwise the route result lives in the context's workspace (routed calls on
 * one context are stream-ordered). */
int32_t xl_layer_forward_routed_async(xl_context* ctx, int32_t layer, const float* d_logits, const float* d_bias_or_null,
                                      int32_t k, float scale, const float* d_x, const float* d_shared_or_null,
                                      float* d_out, void* stream, xl_error* err);
/* The same for T tokens (logits T x n_experts) into xl_grouped_forward_async. */
int32_t xl_grouped_forward_routed_async(xl_context* ctx, int32_t layer, int32_t T, const float* d_logits,
                                        const float* d_bias_or_null, int32_t k, float scale, const float* d_x,
                                        const float* d_shared_or_null, float* d_out, void* stream, xl_error* err);

/* ---- primitives (device pointers) -----------------------------------------
 * q8k_* : Q8_K quantization of rows x k floats (k a multiple of 256) into
 * rows*k/256 blocks of 292 bytes (q8k_core.hpp:13-38, hip_q8k.hpp:9). */
int32_t xl_quantize_q8k_async(xl_context* ctx, const float* d_x, int32_t rows, int32_t k, void* d_q8k, void* stream,
                              xl_error* err);
/* h[n] = SwiGLU(g, u) with the limit (q8k::activate, hip_q8k.hpp:10;
 * q8k_core.hpp:92-95): limit > 0 clamps g to <= limit and u to [-limit,
 * limit], then g / (1 + exp(-g)) * u on the device's expf. */
int32_t xl_swiglu_async(xl_context* ctx, const float* d_g, const float* d_u, int32_t n, float limit, float* d_h,
                        void* stream, xl_error* err);
/* One planar matrix (n x k) times Q8_K(x): y[n] and, when non-null, the
 * per-block int32 partials (n*k/256 ints: each row's exact integer per
 * 256-weight block, sum of (2s+1) * grid * sign * q over the block; IQ1_M:
 * 8 * main + delta, the integer the decoder forms). Replaces q8k::mv
 * (hip_q8k.hpp:10). d_x is the f32 input vector. */
int32_t xl_matvec_async(xl_context* ctx, int32_t type, const void* d_planar, int32_t n, int32_t k, const float* d_x,
                        float* d_y, int32_t* d_partials, void* stream, xl_error* err);

/* ---- per32 mode (the reference's production HIP lane arithmetic) ----------
 * Replaces hipex::quantize / hipex::project (engine/strata/warm/hip_experts.hpp,
 * hip_experts.hip:43-64) and the SoA branch of enqueue_layer
 * (hip_resident_bank.hpp:185-200), bit for bit: activations quantized per 32
 * values (d = max|x| / 127, q = round-half-even(x / d)); a row is 32 lanes,
 * lane l taking sub-blocks l, l + 32, ...: acc = fma(d_x, (fp16(d) * 0.125) *
 * float(s0 * a + s1 * b), acc), then an xor butterfly 16..1 and lane 0 + 0.
 * SwiGLU g / (1 + exp(-g)) * u on the device's expf (the reference's upstream
 * swiglu kernel is not in its tree).
 * xl_layer_forward_per32: y (k x dim, may be null) the per-pick down outputs
 * (the reference's batch_y), out (dim, may be null, needs w) their fixed-order
 * combine (+ shared). The async form takes device pointers (d_y required). */
int32_t xl_layer_forward_per32(xl_context* ctx, int32_t layer, const int32_t* ids, const float* w, int32_t k,
                               const float* x, const float* shared_or_null, float* y_or_null, float* out_or_null,
                               xl_error* err);
int32_t xl_layer_forward_per32_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                                     const float* d_x, const float* d_shared_or_null, float* d_y,
                                     float* d_out_or_null, void* stream, xl_error* err);
/* rows x k floats (k a multiple of 32) into rows*k int8 d_q and rows*k/32 d_d
 * (hip_experts.hip:17-26, hipex::quantize). */
int32_t xl_quantize_per32_async(xl_context* ctx, const float* d_x, int32_t rows, int32_t k, int8_t* d_q, float* d_d,
                                void* stream, xl_error* err);
/* One matrix (n x k) times per32 activations (d_q 16-byte aligned, k int8;
 * d_d k/32 scales): y[n] (dot_kernel<Type>, hip_experts.hip:27-41; the lane<>
 * of sycl/moe/core.hpp:69-84 for the dense formats). d_planar (16-byte
 * aligned): an IQ matrix in the planar layout of xl_repack, or raw ggml blocks
 * of the dense formats Q8_0 (8), Q4_K (12), Q5_K (13), Q6_K (14). */
int32_t xl_matvec_per32_async(xl_context* ctx, int32_t type, const void* d_planar, int32_t n, int32_t k,
                              const int8_t* d_q, const float* d_d, float* d_y, void* stream, xl_error* err);

/* ---- around the routed experts (device pointers) ----------------------------
 * Shared-expert FFN (hip_backend.cpp:664-666: mv(w1, w3), swiglu, mv(w2), the
 * per32 arithmetic of the production GEMV, SwiGLU with the context's limit)
 * for T tokens: out[T x dim] from x[T x dim]. Matrices: gate and up ff x dim,
 * down dim x ff, each raw ggml blocks of a dense format (Q8_0, Q4_K, Q5_K,
 * Q6_K: the pack's ffn.shared_experts.w1 / w3 / w2 bytes) or planar IQ. The
 * caller's workspace (256-byte aligned, xl_shared_work_bytes(dim, ff, T)
 * bytes) holds the intermediates; nothing is allocated. The result is what
 * xl_layer_forward takes as its shared row. */
uint64_t xl_shared_work_bytes(int32_t dim, int32_t ff, int32_t T);
int32_t xl_shared_forward_async(xl_context* ctx, int32_t type_gate, const void* d_gate, int32_t type_up,
                                const void* d_up, int32_t type_down, const void* d_down, int32_t ff, int32_t T,
                                const float* d_x, float* d_out, void* d_work, uint64_t work_bytes, void* stream,
                                xl_error* err);
/* The shared-expert FFN without a caller workspace: the same kernels and
 * result as xl_shared_forward_async, its intermediates in a static device
 * array of 8 MiB (the library's own, held by every GPU it runs on until the
 * process ends). No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). It calls no hipMalloc / hipFree.
 * XL_E_ARG when xl_shared_work_bytes(dim, ff, T) exceeds 8 MiB (T up to 250 at
 * dim 4096 x ff 3072). Every call on one GPU shares that GPU's array: calls
 * that overlap on a GPU (through any context or stream) race. */
int32_t xl_shared_forward_noalloc(xl_context* ctx, int32_t type_gate, const void* d_gate, int32_t type_up,
                                  const void* d_up, int32_t type_down, const void* d_down, int32_t ff, int32_t T,
                                  const float* d_x, float* d_out, void* stream, xl_error* err);
/* Hyper-connection pre + RMS norm that makes the MoE block's input
 * (hip_backend.cpp:629 k4::hc_pre_norm with the layer's ffn_norm; sycl/hc/
 * hc.cpp:89-106, core.hpp:74-80): for T tokens of H <= 4 streams of D,
 * x[t][e] = sum_j mix[t][j] * h[t][j][e] (j ascending), then, when w is not
 * null, x[t][e] = x[t][e] * inv * w[e] with inv = 1 / sqrt(S / D + eps) and S
 * the sum of x^2 in the reference's fixed order (1024 lane sums, 32-lane XOR
 * trees). h T x H x D, mix T x 8, w D, x T x D; bit-identical to the
 * reference. x may not overlap h, mix or w; eps finite and positive. */
int32_t xl_hc_pre_norm_async(xl_context* ctx, const float* d_h, const float* d_mix, const float* d_w_or_null,
                             int32_t D, int32_t H, int32_t T, float eps, float* d_x, void* stream, xl_error* err);
/* The pre-norm and the MoE layer of one token as one call (hip_backend.cpp:629
 * k4::hc_pre_norm, then the routed-expert layer of :635-711): x =
 * xl_hc_pre_norm_async(h, mix, norm_w, D = dim, H, T = 1) is written to d_x
 * and is the layer's input, as xl_layer_forward_async(d_ids, d_w, k, d_x)
 * takes it; out and x bit-identical to those two calls. With H == 1 and a
 * layer the streaming kernel runs, one launch: every workgroup normalizes h
 * in its prologue. h H x dim, mix 8, norm_w dim (null: the pre values only).
 * x may not overlap h, mix or norm_w; out may not overlap h or x. */
int32_t xl_layer_forward_prenorm_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w,
                                       int32_t k, const float* d_h, int32_t H, const float* d_mix,
                                       const float* d_norm_w_or_null, float eps, float* d_x,
                                       const float* d_shared_or_null, float* d_out, void* stream, xl_error* err);
/* Hyper-connection post after the MoE block (hip_backend.cpp:777 k4::hc_post;
 * sycl/hc/hc.cpp:107-115, core.hpp:81-86): for T tokens and H <= 4 streams of
 * D, out[t][k][e] = post[t][k] * y[t][e] + sum_j comb[t][j * H + k] *
 * res[t][j][e] (j ascending, separate roundings). y T x D, res and out T x H x
 * D, post T x 8, comb T x 64. out may be res (in place); other overlaps are
 * rejected. */
int32_t xl_hc_post_async(xl_context* ctx, const float* d_y, const float* d_res, const float* d_post,
                         const float* d_comb, int32_t D, int32_t H, int32_t T, float* d_out, void* stream,
                         xl_error* err);
/* The MoE layer of one token and the hyper-connection post after it as one
 * call (the routed-expert layer of hip_backend.cpp:635-711, then :777
 * k4::hc_post): xl_layer_forward_async(d_ids, d_w, k, d_x, d_shared) writes
 * d_out, and xl_hc_post_async(y = d_out, res, post, comb, D = dim, H, T = 1)
 * writes d_post_out; both bit-identical to those two calls. With a layer the
 * streaming kernel runs, one launch: each workgroup applies hc_post to the
 * output rows it combines. res and post_out H x dim, post 8, comb 64;
 * post_out may be res (in place) and overlaps nothing else. */
int32_t xl_layer_forward_post_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w,
                                    int32_t k, const float* d_x, const float* d_shared_or_null, float* d_out,
                                    const float* d_res, const float* d_post, const float* d_comb, int32_t H,
                                    float* d_post_out, void* stream, xl_error* err);
/* The MoE block of one token as one call (hip_backend.cpp:635-711 with the
 * shared expert of :664-666 added last, then :777 k4::hc_post): d_out and
 * d_post_out bit-identical to xl_shared_forward_async(gate, up, down, ff,
 * T = 1, d_x) into a row s, then xl_layer_forward_post_async(d_ids, d_w, k,
 * d_x, s, d_out, res, post, comb, H, d_post_out). The routed layer runs first
 * and writes d_out; with a layer the streaming kernel runs, that launch also
 * quantizes x per 32 for the shared FFN (no quant32 launch); the shared down
 * rows then add themselves to d_out and apply hc_post in their epilogue.
 * Workspace: xl_shared_work_bytes(dim, ff, 1) bytes, 256-byte aligned,
 * overlapping nothing else. res and post_out H x dim, post 8, comb 64;
 * post_out may be res (in place) and overlaps nothing else; out overlaps no
 * input. */
int32_t xl_moe_block_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                           const float* d_x, int32_t type_gate, const void* d_gate, int32_t type_up, const void* d_up,
                           int32_t type_down, const void* d_down, int32_t ff, void* d_work, uint64_t work_bytes,
                           const float* d_res, const float* d_post, const float* d_comb, int32_t H, float* d_out,
                           float* d_post_out, void* stream, xl_error* err);

/* ---- stage profiling --------------------------------------------------------
 * Between xl_profile_begin and xl_profile_end, the first max_calls layer calls
 * record a HIP event before and after each kernel on the stream it runs on
 * (the reference's phase marks, hip_experts.hpp:13-20). xl_profile_end drains
 * and returns per-stage totals in ms, the stage and call counts and the stage
 * names (comma separated). Event creation happens in xl_profile_begin. */
int32_t xl_profile_begin(xl_context* ctx, int32_t max_calls, xl_error* err);
int32_t xl_profile_end(xl_context* ctx, float* stage_ms, int32_t max_stages, int32_t* n_stages, int32_t* n_calls,
                       char* names, int32_t names_bytes, xl_error* err);

/* Per-wave timeline of the last single-launch layer call made while profiling
 * was active: 32 words per wave, wave-major over the grid, holding
 * s_memrealtime stamps (100 MHz; zero where a wave did not reach a phase).
 * Words: 0 prologue loads issued, 1 codebooks written, 2 x quantized
 * (barrier), 3 gate/up done, 4 quantizer duty done (all-types kernel),
 * 5 first down pass done, 6 all down passes done, 7 combine done, 8 + j
 * gate/up slot j done; streaming kernel only: 20 + j re-polls of down step j
 * (a count, not a stamp), 24 + 2j step j's h complete, 25 + 2j step j's
 * Q8_K(h) staged. A diagnostic aid: it has no counterpart in the reference. */
int32_t xl_profile_timeline(xl_context* ctx, uint64_t* out, int32_t max_words, int32_t* n_words, xl_error* err);

/* Sets the single-launch kernels' device launch counters (the all-types
 * kernel's epoch and the streaming kernel's launch count, whose parity picks
 * its h exchange buffer) to `launches`, as if that many launches had run. A
 * diagnostic aid for testing the counters' wrap at 2^32; it has no
 * counterpart in the reference. The exchange buffers are reset as at
 * xl_open (h words to the sentinel, tags to zero), so that any count, of
 * either parity and any epoch, leaves the next launch correct. */
int32_t xl_debug_set_launch_count(xl_context* ctx, uint32_t launches, xl_error* err);

/* Layer calls made on the context so far, by how they ran: counts[i] for
 * i < n (kinds past XL_LAUNCH_KINDS read 0). A diagnostic aid (no counterpart
 * in the reference): it shows which launch served a call, e.g. that a routed
 * or pre-normed call ran as one launch rather than as its two-call fallback. */
enum {
    XL_LAUNCH_STREAM = 0,     /* xl_layer_* calls served by the streaming kernel */
    XL_LAUNCH_ALLTYPES = 1,   /* ... by the all-types single launch */
    XL_LAUNCH_SEPARATE = 2,   /* ... by separate launches */
    XL_LAUNCH_ROUTED = 3,     /* routed layer calls that routed inside the streaming launch */
    XL_LAUNCH_PRENORM = 4,    /* pre-normed layer calls that normalized inside the streaming launch */
    XL_LAUNCH_EXACT = 5,      /* xl_layer_forward_exact_async calls */
    XL_LAUNCH_POST = 6,       /* layer + hc_post calls that applied hc_post inside the streaming launch */
    XL_LAUNCH_BLOCK = 7,      /* xl_moe_block_async calls whose streaming launch quantized x for the shared FFN */
    XL_LAUNCH_KINDS = 8
};
int32_t xl_debug_launch_counts(xl_context* ctx, int64_t* counts, int32_t n, xl_error* err);

/* ---- host utilities (no device needed) ------------------------------------ */
uint64_t xl_planar_bytes(int32_t type, int32_t n, int32_t k);
int32_t xl_repack(int32_t type, int32_t n, int32_t k, const void* aos, void* planar);
int32_t xl_restore(int32_t type, int32_t n, int32_t k, const void* planar, void* aos);
/* The generator's AoS bytes of matrix (layer, expert, role), host-side. */
int32_t xl_generate_host(int32_t type, uint64_t seed, int32_t layer, int32_t expert, int32_t role, int32_t n, int32_t k,
                         void* aos);
/* Expanded codebooks: 0 IQ2_XXS grid (256 u64), 1 IQ2_XS grid (512),
 * 2 IQ1 grid (2048), 3 ksigns (128 values widened to u64). */
int32_t xl_codebook(int32_t which, uint64_t* out);

#ifdef __cplusplus
}
#endif
#endif
