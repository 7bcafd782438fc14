/* AVX2 CPU lane: the CPU baseline bench.py times beside the GPU. TEST AND
 * BASELINE INFRASTRUCTURE ONLY (loaded by tests/ and bench.py's cpu_baseline
 * leg, never by the product).
 *
 * The reference's CPU lane runs ggml's vec_dot_iq*_q8_K (upstream, absent
 * here; engine/strata/sycl/stage/wiring/cpu_lane.hpp:1-7) in the x86 AVX2
 * order that q8k_core.hpp:43-91 restates: per 256-weight block, eight 32-bit
 * lanes, lane L the exact integer over bytes 4L..4L+3 of every 32-value chunk
 * (what _mm256_maddubs_epi16 then _mm256_madd_epi16 produce), one fused
 * multiply-add per block into eight float accumulators, the AVX2 horizontal
 * sum ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7)), then x 1/8 (IQ2) or main + 1/8 delta
 * (IQ1_M). This file computes exactly that with AVX2 intrinsics, so its rows
 * are bit-identical to the scalar oracle (orc_dot); tests/test_oracle.py checks
 * it.
 *
 * The layer follows the reference lane's structure (engine/strata/sycl/moe/
 * cpu_lane.cpp:70-81,157-170): per expert, quantize x (q1), gate and up rows
 * with the SwiGLU in 64-row jobs over a worker pool (gate_up), quantize h (q2),
 * down rows in 64-row jobs (down); then the fixed-order combine
 * (warm/runtime.cpp:183-188). Phase times are steady-clock nanoseconds.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "xl_oracle.h"

static uint64_t L_xxs[256], L_xs[512], L_iq1[2048], L_sgn[128];
static pthread_once_t L_once = PTHREAD_ONCE_INIT;
static void lane_tables(void) {
    orc_codebook(0, L_xxs);
    orc_codebook(1, L_xs);
    orc_codebook(2, L_iq1);
    for (int i = 0; i < 128; ++i) {   /* byte j = 0xff where sign bit j of ksigns[i] is set */
        const uint8_t s = orc_ksigns(i);
        uint64_t m = 0;
        for (int j = 0; j < 8; ++j)
            if (s & (1u << j)) m |= (uint64_t)0xff << (8 * j);
        L_sgn[i] = m;
    }
}

int orc_lane_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) { return (uint32_t)rd16(p) | ((uint32_t)rd16(p + 2) << 16); }
static inline float hsum8v(__m256 acc) {
    float v[8];
    _mm256_storeu_ps(v, acc);
    return ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
}
/* q with the bytes of mask m negated (m byte 0xff or 0): (q ^ m) - m */
static inline __m256i neg_where(__m256i q, __m256i m) { return _mm256_sub_epi8(_mm256_xor_si256(q, m), m); }

static float dot_xxs(const uint8_t* w, const orc_q8k* a, int nb) {
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = w + (size_t)b * 66;
        const float d = orc_half(rd16(blk)) * a[b].d;
        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < 8; ++c) {
            const uint8_t* ch = blk + 2 + 8 * c;
            const uint32_t aux = rd32(ch + 4);
            const __m256i g = _mm256_set_epi64x((long long)L_xxs[ch[3]], (long long)L_xxs[ch[2]],
                                                (long long)L_xxs[ch[1]], (long long)L_xxs[ch[0]]);
            const __m256i m = _mm256_set_epi64x((long long)L_sgn[(aux >> 21) & 127], (long long)L_sgn[(aux >> 14) & 127],
                                                (long long)L_sgn[(aux >> 7) & 127], (long long)L_sgn[aux & 127]);
            const __m256i q = _mm256_loadu_si256((const __m256i*)(a[b].qs + 32 * c));
            const __m256i p16 = _mm256_maddubs_epi16(g, neg_where(q, m));
            sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(p16, _mm256_set1_epi16((short)(2 * (aux >> 28) + 1))));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return 0.125f * hsum8v(acc);
}

static float dot_xs(const uint8_t* w, const orc_q8k* a, int nb) {
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = w + (size_t)b * 74;
        const float d = orc_half(rd16(blk)) * a[b].d;
        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < 8; ++c) {
            const uint8_t* ch = blk + 2 + 8 * c;
            const uint16_t q0 = rd16(ch), q1 = rd16(ch + 2), q2 = rd16(ch + 4), q3 = rd16(ch + 6);
            const __m256i g = _mm256_set_epi64x((long long)L_xs[q3 & 511], (long long)L_xs[q2 & 511],
                                                (long long)L_xs[q1 & 511], (long long)L_xs[q0 & 511]);
            const __m256i m = _mm256_set_epi64x((long long)L_sgn[q3 >> 9], (long long)L_sgn[q2 >> 9],
                                                (long long)L_sgn[q1 >> 9], (long long)L_sgn[q0 >> 9]);
            const uint8_t sc = blk[66 + c];   /* low nibble: values 0..15 of the chunk, high: 16..31 */
            const __m256i s16 = _mm256_set_m128i(_mm_set1_epi16((short)(2 * (sc >> 4) + 1)),
                                                 _mm_set1_epi16((short)(2 * (sc & 15) + 1)));
            const __m256i q = _mm256_loadu_si256((const __m256i*)(a[b].qs + 32 * c));
            sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(_mm256_maddubs_epi16(g, neg_where(q, m)), s16));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return 0.125f * hsum8v(acc);
}

static float dot_iq1m(const uint8_t* w, const orc_q8k* a, int nb) {
    const __m256i ones = _mm256_set1_epi8(1);
    __m256 accm = _mm256_setzero_ps(), accd = _mm256_setzero_ps();
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = w + (size_t)b * 56;
        const uint16_t dh = (uint16_t)((rd16(blk + 48) >> 12) | ((rd16(blk + 50) >> 8) & 0xf0) |
                                       ((rd16(blk + 52) >> 4) & 0xf00) | (rd16(blk + 54) & 0xf000));
        const float d = orc_half(dh) * a[b].d;
        __m256i summ = _mm256_setzero_si256(), sumd = _mm256_setzero_si256();
        for (int c = 0; c < 8; ++c) {
            uint64_t gv[4], dv[4];
            for (int l = 0; l < 4; ++l) {   /* 8-value group l of chunk c */
                const uint8_t hi = blk[32 + 2 * c + l / 2];
                const int idx = blk[4 * c + l] | (((int)hi << (8 - 4 * (l % 2))) & 0x700);
                gv[l] = L_iq1[idx];
                dv[l] = (hi & (l % 2 ? 128 : 8)) ? 0xffffffffffffffffull : 0x0101010101010101ull;
            }
            const uint16_t sw = rd16(blk + 48 + 2 * (c / 2));
            const int sh = 6 * (c % 2);
            const __m256i s16 = _mm256_set_m128i(_mm_set1_epi16((short)(2 * ((sw >> (sh + 3)) & 7) + 1)),
                                                 _mm_set1_epi16((short)(2 * ((sw >> sh) & 7) + 1)));
            const __m256i g = _mm256_set_epi64x((long long)gv[3], (long long)gv[2], (long long)gv[1], (long long)gv[0]);
            const __m256i dl = _mm256_set_epi64x((long long)dv[3], (long long)dv[2], (long long)dv[1], (long long)dv[0]);
            const __m256i q = _mm256_loadu_si256((const __m256i*)(a[b].qs + 32 * c));
            /* sign_epi8(q, g) = g * q for g in {-1, 0, 1}; maddubs with ones sums byte pairs */
            summ = _mm256_add_epi32(summ, _mm256_madd_epi16(_mm256_maddubs_epi16(ones, _mm256_sign_epi8(q, g)), s16));
            sumd = _mm256_add_epi32(sumd, _mm256_madd_epi16(_mm256_maddubs_epi16(ones, _mm256_sign_epi8(q, dl)), s16));
        }
        accm = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(summ), accm);
        accd = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumd), accd);
    }
    const float mainv = hsum8v(accm);
    return mainv + 0.125f * hsum8v(accd);
}

float orc_lane_dot(int t, const uint8_t* w, const orc_q8k* a, int nb) {
    pthread_once(&L_once, lane_tables);
    return t == 16 ? dot_xxs(w, a, nb) : t == 17 ? dot_xs(w, a, nb) : dot_iq1m(w, a, nb);
}

static double now_ns(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e9 + (double)ts.tv_nsec;
}

/* One routed layer: k experts (types[3 i .. 3 i + 2], matrices mats[3 i .. 3 i + 2]
 * as AoS ggml rows), fixed-order combine into out. phase_ns (5 doubles, added
 * to): q1, gate_up, q2, down, combine. */
void orc_lane_layer(int k, const int* types, const uint8_t* const* mats, int dim, int ff, const float* x,
                    const int32_t* ids, const float* w, float* out, float limit, int threads, double* phase_ns) {
    pthread_once(&L_once, lane_tables);
    if (threads < 1) threads = 1;
    const int nbx = dim / 256, nbh = ff / 256;
    orc_q8k* xq = (orc_q8k*)malloc(sizeof(orc_q8k) * (size_t)nbx);
    orc_q8k* hq = (orc_q8k*)malloc(sizeof(orc_q8k) * (size_t)nbh);
    float* h = (float*)malloc(sizeof(float) * (size_t)ff);
    float* ys = (float*)malloc(sizeof(float) * (size_t)k * dim);
    for (int i = 0; i < k; ++i) {
        const int tg = types[3 * i], tu = types[3 * i + 1], td = types[3 * i + 2];
        const uint8_t *G = mats[3 * i], *U = mats[3 * i + 1], *D = mats[3 * i + 2];
        const size_t rbg = (size_t)nbx * orc_block_bytes(tg), rbu = (size_t)nbx * orc_block_bytes(tu);
        const size_t rbd = (size_t)nbh * orc_block_bytes(td);
        double t0 = now_ns();
        orc_quantize_row(x, dim, xq);
        double t1 = now_ns();
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (int j = 0; j < (ff + 63) / 64; ++j)
            for (int r = 64 * j; r < 64 * j + 64 && r < ff; ++r) {
                const float g = orc_lane_dot(tg, G + (size_t)r * rbg, xq, nbx);
                const float u = orc_lane_dot(tu, U + (size_t)r * rbu, xq, nbx);
                h[r] = orc_swiglu(g, u, limit);
            }
        double t2 = now_ns();
        orc_quantize_row(h, ff, hq);
        double t3 = now_ns();
        float* y = ys + (size_t)i * dim;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (int j = 0; j < (dim + 63) / 64; ++j)
            for (int r = 64 * j; r < 64 * j + 64 && r < dim; ++r) y[r] = orc_lane_dot(td, D + (size_t)r * rbd, hq, nbh);
        double t4 = now_ns();
        if (phase_ns) {
            phase_ns[0] += t1 - t0;
            phase_ns[1] += t2 - t1;
            phase_ns[2] += t3 - t2;
            phase_ns[3] += t4 - t3;
        }
    }
    double t5 = now_ns();
    orc_combine(ids, w, k, ys, dim, NULL, out);
    if (phase_ns) phase_ns[4] += now_ns() - t5;
    free(xq);
    free(hq);
    free(h);
    free(ys);
}
