/* CPU oracle for the routed-expert path. TEST INFRASTRUCTURE ONLY.
 *
 * A scalar C restatement of the reference's CPU arithmetic for the expert
 * lane: Q8_K activation quantization, the IQ2_XXS / IQ2_XS / IQ1_M x Q8_K dot
 * in ggml's x86 AVX2 lane and FMA order, SwiGLU, the fixed-order combine, and
 * this build's seeded block generator. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Reference files followed (paths under engine/strata/):
 *   sycl/stage/wiring/q8k_core.hpp:17-95   half, nearest, quant_block,
 *                                           integer_lane, scale, dot_lane,
 *                                           hsum, dot, swiglu
 *   sycl/moe/core.hpp:66-105                 per-32 decode (brute-force check) and
 *                                           the per32 row dot of the production
 *                                           HIP lane (with hip_experts.hip:17-39)
 *   warm/runtime.cpp:183-188                 fixed-order combine
 *   sycl/route/route.cpp:15-37               router: sqrt(softplus) scores,
 *                                           biased top-k, normalized weights
 *   sycl/moe/cpu_lane.cpp:70-81              64-row jobs over worker threads
 *   sycl/moe/core.hpp:9-12,17,47-65,80       per32 rows of the dense shared-expert
 *                                           formats (Q8_0, Q4_K, Q5_K, Q6_K)
 *   sycl/hc/core.hpp:81-86                   hyper-connection post
 *   sycl/moe/cpu_lane.cpp:70-81,157-170      the AVX2 CPU lane (cpu_lane.c): 64-row
 *                                           jobs, phases q1 / gate_up / q2 / down
 *
 * Parity pins (see tests/): every function here is checked against
 * oracle/_ref (the reference's own q8k_core.hpp / core.hpp / other_combine.hpp
 * and route.cpp compiled from /root/reference) where that builds, against closed forms
 * (zero and one-hot Q8_K blocks, round-half-even ties, ksigns parity) and
 * against a brute-force dequantize-and-multiply integer dot.
 */
#ifndef XL_ORACLE_H
#define XL_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_q8k { float d; int8_t qs[256]; int16_t bsums[16]; } orc_q8k;

int orc_block_bytes(int type);
float orc_half(uint16_t h);
int orc_nearest(float x);

/* Q8_K */
void orc_quant_block(const float* x, orc_q8k* y);
void orc_quantize_row(const float* x, int k, orc_q8k* y);

/* IQ x Q8_K dot, AVX2 order. w = one row of k/256 AoS blocks. */
void orc_integer_lane(int type, const uint8_t* w, const orc_q8k* a, int lane, int32_t* main_out, int32_t* delta_out);
float orc_dot(int type, const uint8_t* w, const orc_q8k* a, int nb);
/* Per-block integer partials: Sum over the 8 AVX2 lanes of integer_lane.
 * IQ2 types write one int per block; IQ1_M writes (main, delta) pairs. */
void orc_block_partials(int type, const uint8_t* w, const orc_q8k* a, int nb, int32_t* out);
/* Block integers of an n x k matrix (AoS rows) against one Q8_K vector of
 * k/256 blocks: n * k/256 ints, row-major; IQ1_M: 8 * main + delta. */
void orc_matrix_ints(int type, const uint8_t* w, int n, int k, const orc_q8k* a, int32_t* out, int threads);
/* Brute force: dequantize to signed ints with per-16 scales and multiply.
 * IQ2: returns Sum (2s+1)*sign*grid*q; IQ1_M: returns 8*main + delta. */
int64_t orc_brute_block(int type, const uint8_t* blk, const orc_q8k* a);

void orc_matvec(int type, const uint8_t* w, int n, int k, const orc_q8k* a, float* y, int threads);
float orc_swiglu(float g, float u, float limit);

/* One expert: y = down(SwiGLU(gate x, up x)), SwiGLU with the limit (0: none).
 * Optional intermediates. */
void orc_expert(const int types[3], const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                int dim, int ff, const float* x, float* y, float* g_out, float* u_out, float* h_out,
                int threads, float limit);
/* Down half only, from a given hidden vector h (used to compare with the
 * device's own SwiGLU output). */
void orc_down_from_hidden(int type, const uint8_t* down, int dim, int ff, const float* h, float* y, int threads);

/* Fixed-order combine: ascending expert id, out = fma(w, y, out), then +shared. */
void orc_combine(const int32_t* ids, const float* w, int k, const float* rows, int dim,
                 const float* shared_or_null, float* out);

/* Generator restated: one AoS block, and one whole matrix (n x k). */
uint64_t orc_gen_key(uint64_t seed, uint32_t layer, uint32_t expert, uint32_t role);
/* per32 arithmetic of the reference's production HIP lane (hip_experts.hip:
 * 17-39, sycl/moe/core.hpp:66-88, warm/expert_check.cpp:44-55): activation
 * blocks of 32 (q int8, one f32 scale each), per-sub-block float dots summed by
 * 32 strided lanes and a butterfly. */
void orc_quant32(const float* x, int k, int8_t* q, float* d);
/* Row bytes of a per32 matrix: IQ types (16, 17, 29) and the dense formats
 * Q8_0 (8), Q4_K (12), Q5_K (13), Q6_K (14) of the shared-expert matrices. */
int orc_row_bytes32(int type, int k);
void orc_dequant32(int type, const uint8_t* row, int kb, double* out);
float orc_row32(int type, const uint8_t* row, int k, const int8_t* xq, const float* xd);
void orc_matvec32(int type, const uint8_t* w, int n, int k, const int8_t* xq, const float* xd, float* y);
void orc_expert32(const int types[3], const uint8_t* gate, const uint8_t* up, const uint8_t* down, int dim, int ff,
                  const float* x, float* y, float* g, float* u, float* h, float limit);

/* Router of route.cpp:15-37 (route_cpu) for T tokens: logits T x stride (the
 * first n used), bias n (NULL = zeros); ids / w: T x k. */
void orc_route(const float* logits, int stride, const float* bias, int n, int T, int k, float scale, int32_t* ids,
               float* w);

void orc_gen_block(int type, uint64_t key, uint64_t blk, uint8_t* out);
void orc_gen_matrix(int type, uint64_t seed, uint32_t layer, uint32_t expert, uint32_t role, int n, int k, uint8_t* out);

/* Expanded codebooks (u64 rows) and the ksigns table, for table checks. */
void orc_codebook(int which, uint64_t* out); /* 0: iq2xxs[256] 1: iq2xs[512] 2: iq1s[2048] */
uint8_t orc_ksigns(int i);

/* AVX2 CPU lane (cpu_lane.c, the CPU baseline): 1 when the host has AVX2 and
 * FMA; one row dot bit-identical to orc_dot; one routed layer in the reference
 * CPU lane's phases (q1, gate_up, q2, down, combine nanoseconds added to
 * phase_ns[0..4]) over `threads` workers in 64-row jobs. */
int orc_lane_avx2(void);
float orc_lane_dot(int type, const uint8_t* w, const orc_q8k* a, int nb);
void orc_lane_layer(int k, const int* types, const uint8_t* const* mats, int dim, int ff, const float* x,
                    const int32_t* ids, const float* w, float* out, float limit, int threads, double* phase_ns);

/* Hyper-connection post (sycl/hc/core.hpp:81-86) of T tokens, H streams of D. */
void orc_hc_post(const float* y, const float* res, const float* post, const float* comb, int D, int H, int T, float* out);
void orc_hc_pre_norm(const float* h, const float* mix, const float* w, int D, int H, int T, float eps, float* x);

#ifdef __cplusplus
}
#endif
#endif
