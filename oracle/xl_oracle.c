/* CPU oracle for the routed-expert path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
 * product. Build: oracle/Makefile (gcc -O2 -mfma -ffp-contract=off). Every
 * floating-point step is written out; nothing is contracted implicitly.
 * Citations are to the reference tree (engine/strata/...). */
#include "xl_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <pthread.h>
#include <stdatomic.h>
#include <string.h>

#include "orc_codebooks.inc"

/* ---- tables ------------------------------------------------------------- */
static uint64_t g_iq2xxs[256], g_iq2xs[512], g_iq1s[2048];
static uint8_t g_ksigns[128];
static pthread_once_t g_once = PTHREAD_ONCE_INIT;

static uint64_t expand_b3(unsigned v, int iq1) {
    static const uint8_t mag[3] = {8, 25, 43};
    static const uint8_t tri[3] = {0xff, 0x00, 0x01};
    uint64_t out = 0;
    for (int j = 0; j < 8; ++j) {
        const unsigned s = v % 3u;
        v /= 3u;
        out |= (uint64_t)(iq1 ? tri[s] : mag[s]) << (8 * j);
    }
    return out;
}
static void init_tables(void) {
    for (int i = 0; i < 256; ++i) g_iq2xxs[i] = expand_b3(orc_iq2xxs_b3[i], 0);
    for (int i = 0; i < 512; ++i) g_iq2xs[i] = expand_b3(orc_iq2xs_b3[i], 0);
    for (int i = 0; i < 2048; ++i) g_iq1s[i] = expand_b3(orc_iq1s_b3[i], 1);
    /* ggml ksigns_iq2xs: 7 stored sign bits plus an even-parity 8th bit
     * (sycl/moe/core.hpp:67; values tabulated at q8k_tables.inc:713). */
    for (int i = 0; i < 128; ++i) g_ksigns[i] = (uint8_t)(i | ((__builtin_popcount((unsigned)i) & 1) << 7));
}
static void tables(void) { pthread_once(&g_once, init_tables); }

void orc_codebook(int which, uint64_t* out) {
    tables();
    if (which == 0) memcpy(out, g_iq2xxs, sizeof g_iq2xxs);
    else if (which == 1) memcpy(out, g_iq2xs, sizeof g_iq2xs);
    else memcpy(out, g_iq1s, sizeof g_iq1s);
}
uint8_t orc_ksigns(int i) { tables(); return g_ksigns[i & 127]; }

/* ---- scalars ------------------------------------------------------------ */
int orc_block_bytes(int type) { return type == 29 ? 56 : type == 17 ? 74 : type == 16 ? 66 : 0; }
static uint16_t u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t u32(const uint8_t* p) { return (uint32_t)u16(p) | ((uint32_t)u16(p + 2) << 16); }

/* q8k_core.hpp:17-24 */
float orc_half(uint16_t h) {
    const int e = (h >> 10) & 31;
    float v;
    if (!e) v = ldexpf((float)(h & 1023), -24);
    else if (e == 31) v = (h & 1023) ? NAN : INFINITY;
    else v = ldexpf((float)(1024 + (h & 1023)), e - 25);
    return (h & 32768) ? -v : v;
}

/* q8k_core.hpp:25-29: ggml nearest_int via the 1.5*2^23 bias. */
int orc_nearest(float x) {
    union { float f; uint32_t u; } v;
    v.f = x + 12582912.0f;
    return (int)(v.u & 0x007fffffu) - 0x00400000;
}

/* q8k_core.hpp:30-38 */
void orc_quant_block(const float* x, orc_q8k* y) {
    float mx = 0, am = 0;
    for (int j = 0; j < 256; ++j) {
        const float a = fabsf(x[j]);
        if (a > am) { am = a; mx = x[j]; }
    }
    if (am == 0) {
        memset(y, 0, sizeof *y);
        return;
    }
    const float is = -127.0f / mx;
    for (int j = 0; j < 256; ++j) {
        const float p = is * x[j];
        const int v = orc_nearest(p);
        y->qs[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int j = 0; j < 16; ++j) {
        int s = 0;
        for (int z = 0; z < 16; ++z) s += y->qs[16 * j + z];
        y->bsums[j] = (int16_t)s;
    }
    y->d = 1.0f / is;
}
void orc_quantize_row(const float* x, int k, orc_q8k* y) {
    for (int b = 0; b < k / 256; ++b) orc_quant_block(x + 256 * b, y + b);
}

/* q8k_core.hpp:43-69. Lane L covers bytes 4L..4L+3 of every 32-value chunk. */
void orc_integer_lane(int t, const uint8_t* w, const orc_q8k* a, int lane, int32_t* main_out, int32_t* delta_out) {
    tables();
    int32_t mainv = 0, deltav = 0;
    for (int c = 0; c < 8; ++c) {
        const int local = 4 * lane, group = local / 8;
        int sign = 0, scale = 0, delta = 0;
        uint64_t tab = 0;
        if (t == 29) {
            const uint8_t hi = w[32 + 2 * c + group / 2];
            const int grid = w[4 * c + group] | (((int)hi << (8 - 4 * (group % 2))) & 0x700);
            tab = g_iq1s[grid];
            delta = (hi & (group % 2 ? 128 : 8)) ? -1 : 1;
            const uint16_t sc = u16(w + 48 + 2 * (c / 2));
            scale = 2 * ((sc >> (6 * (c % 2) + 3 * (local / 16))) & 7) + 1;
        } else if (t == 17) {
            const uint16_t q = u16(w + 2 + 8 * c + 2 * group);
            tab = g_iq2xs[q & 511];
            sign = g_ksigns[q >> 9];
            scale = 2 * ((w[66 + c] >> (4 * (local / 16))) & 15) + 1;
        } else {
            const uint8_t* chunk = w + 2 + 8 * c;
            const uint32_t hi = u32(chunk + 4);
            tab = g_iq2xxs[chunk[group]];
            sign = g_ksigns[(hi >> (7 * group)) & 127];
            scale = 2 * (int)(hi >> 28) + 1;
        }
        for (int j = local % 8; j < local % 8 + 4; ++j) {
            const int q = a->qs[32 * c + 8 * group + j];
            const int code = t == 29 ? (int)(int8_t)(uint8_t)(tab >> (8 * j))
                                     : (int)(uint8_t)(tab >> (8 * j)) * ((sign & (1 << j)) ? -1 : 1);
            mainv += scale * code * q;
            if (t == 29) deltav += scale * delta * q;
        }
    }
    *main_out = mainv;
    *delta_out = deltav;
}

/* q8k_core.hpp:70-74 */
static float block_scale(int t, const uint8_t* w) {
    if (t != 29) return orc_half(u16(w));
    const uint16_t h = (uint16_t)((u16(w + 48) >> 12) | ((u16(w + 50) >> 8) & 0xf0) |
                                  ((u16(w + 52) >> 4) & 0xf00) | (u16(w + 54) & 0xf000));
    return orc_half(h);
}

/* q8k_core.hpp:86: AVX2 horizontal-sum order. */
static float hsum8(const float* v) { return ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7])); }

/* q8k_core.hpp:76-91 */
float orc_dot(int t, const uint8_t* w, const orc_q8k* a, int nb) {
    float m[8], dd[8];
    const int bb = orc_block_bytes(t);
    for (int l = 0; l < 8; ++l) {
        float sm = 0, sd = 0;
        for (int b = 0; b < nb; ++b) {
            const uint8_t* p = w + (size_t)b * bb;
            int32_t vm, vd;
            orc_integer_lane(t, p, a + b, l, &vm, &vd);
            const float d = block_scale(t, p) * a[b].d;
            sm = fmaf(d, (float)vm, sm);
            if (t == 29) sd = fmaf(d, (float)vd, sd);
        }
        m[l] = sm;
        dd[l] = sd;
    }
    const float mainv = hsum8(m);
    if (t == 29) {
        const float dl = 0.125f * hsum8(dd);
        return mainv + dl;
    }
    return 0.125f * mainv;
}

void orc_block_partials(int t, const uint8_t* w, const orc_q8k* a, int nb, int32_t* out) {
    const int bb = orc_block_bytes(t);
    for (int b = 0; b < nb; ++b) {
        int32_t sm = 0, sd = 0;
        for (int l = 0; l < 8; ++l) {
            int32_t vm, vd;
            orc_integer_lane(t, w + (size_t)b * bb, a + b, l, &vm, &vd);
            sm += vm;
            sd += vd;
        }
        if (t == 29) { out[2 * b] = sm; out[2 * b + 1] = sd; }
        else out[b] = sm;
    }
}

/* Block integers of n rows of k/256 blocks against one Q8_K vector: one int
 * per (row, block), the sum over the 8 AVX2 lanes of integer_lane; IQ1_M
 * folds (main, delta) to 8 * main + delta. Rows split over `threads`. */
typedef struct { int t, n, nb, r0, r1; const uint8_t* w; const orc_q8k* a; int32_t* out; } MiJob;
static void* mi_run(void* p) {
    const MiJob* j = (const MiJob*)p;
    const size_t rb = (size_t)j->nb * (size_t)orc_block_bytes(j->t);
    int32_t tmp[2 * 64];
    for (int r = j->r0; r < j->r1; ++r) {
        for (int b0 = 0; b0 < j->nb; b0 += 64) {
            const int nb = j->nb - b0 < 64 ? j->nb - b0 : 64;
            orc_block_partials(j->t, j->w + (size_t)r * rb + (size_t)b0 * orc_block_bytes(j->t), j->a + b0, nb, tmp);
            for (int b = 0; b < nb; ++b)
                j->out[(size_t)r * j->nb + b0 + b] = j->t == 29 ? 8 * tmp[2 * b] + tmp[2 * b + 1] : tmp[b];
        }
    }
    return NULL;
}
void orc_matrix_ints(int t, const uint8_t* w, int n, int k, const orc_q8k* a, int32_t* out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    MiJob jobs[64];
    const int per = (n + threads - 1) / threads;
    int used = 0;
    for (int i = 0; i < threads; ++i) {
        const int r0 = i * per, r1 = r0 + per < n ? r0 + per : n;
        if (r0 >= r1) break;
        jobs[i] = (MiJob){t, n, k / 256, r0, r1, w, a, out};
        pthread_create(&th[i], NULL, mi_run, &jobs[i]);
        ++used;
    }
    for (int i = 0; i < used; ++i) pthread_join(th[i], NULL);
}

/* Per-32 decode of sub-block ib of a 256-weight block, written from
 * sycl/moe/core.hpp:78-105: natural value order, per-16 odd sub-scales (sc),
 * IQ2 values +-grid, IQ1_M values 8*grid + delta. */
static void p32_decode(int t, const uint8_t* blk, int ib, int val[32], int sc[2]) {
    tables();
    if (t == 16 || t == 17) {
        const uint8_t* p = blk + 2 + 8 * ib;
        const uint32_t aux = u32(p + 4);
        for (int l = 0; l < 4; ++l) {
            const unsigned code = u16(p + 2 * l);
            const uint64_t grid = t == 16 ? g_iq2xxs[p[l]] : g_iq2xs[code & 511];
            const unsigned sg = g_ksigns[(t == 16 ? (aux >> (7 * l)) : (code >> 9)) & 127];
            for (int j = 0; j < 8; ++j) {
                const int q = (int)((grid >> (8 * j)) & 255);
                val[8 * l + j] = ((sg >> j) & 1) ? -q : q;
            }
        }
        if (t == 16) sc[0] = sc[1] = 2 * (int)(aux >> 28) + 1;
        else { sc[0] = 2 * (blk[66 + ib] & 15) + 1; sc[1] = 2 * (blk[66 + ib] >> 4) + 1; }
    } else {
        const unsigned word = u16(blk + 48 + 2 * (ib >> 1));
        sc[0] = 2 * (int)((word >> (6 * (ib & 1))) & 7) + 1;
        sc[1] = 2 * (int)((word >> (6 * (ib & 1) + 3)) & 7) + 1;
        for (int l = 0; l < 4; ++l) {
            const unsigned h = blk[32 + 2 * ib + l / 2];
            const unsigned nib = (l & 1) ? (h >> 4) : (h & 15);
            const unsigned idx = blk[4 * ib + l] | ((nib & 7) << 8);
            const int delta = (nib & 8) ? -1 : 1;
            for (int j = 0; j < 8; ++j) {
                const int g = (int)(int8_t)(uint8_t)(g_iq1s[idx] >> (8 * j));
                val[8 * l + j] = 8 * g + delta;
            }
        }
    }
}
/* The block's super-scale as core.hpp:86,99 take it: half(d) * 0.125 (IQ1_M's
 * fp16 d is spread over the top nibbles of its four scale words). */
static float p32_scale(int t, const uint8_t* blk) {
    if (t == 29) {
        const uint16_t d = (uint16_t)((u16(blk + 48) >> 12) | ((u16(blk + 50) >> 8) & 0xf0) | ((u16(blk + 52) >> 4) & 0xf00) |
                                      (u16(blk + 54) & 0xf000));
        return orc_half(d) * 0.125f;
    }
    return orc_half(u16(blk)) * 0.125f;
}

/* Brute force over the per-32 decode, against a Q8_K activation block. */
int64_t orc_brute_block(int t, const uint8_t* blk, const orc_q8k* a) {
    int64_t total = 0;
    for (int ib = 0; ib < 8; ++ib) {
        int val[32], sc[2];
        p32_decode(t, blk, ib, val, sc);
        for (int j = 0; j < 32; ++j) total += (int64_t)sc[j / 16] * val[j] * a->qs[32 * ib + j];
    }
    return total;
}

/* ---- per32 arithmetic (the reference's production HIP lane) ---------------
 * Activation quantization per 32 values (hip_experts.hip:17-26,
 * expert_check.cpp:44-47): d = max|x| / 127, q = round-half-even(x / d), a
 * zero block all zero. */
void orc_quant32(const float* x, int k, int8_t* q, float* d) {
    for (int b = 0; b < k / 32; ++b) {
        float am = 0.0f;
        for (int j = 0; j < 32; ++j) am = fmaxf(am, fabsf(x[32 * b + j]));
        d[b] = am / 127.0f;
        for (int j = 0; j < 32; ++j) q[32 * b + j] = (int8_t)(am > 0.0f ? (int)nearbyintf(x[32 * b + j] / d[b]) : 0);
    }
}
/* ---- per32 dense formats (the shared-expert matrices) ---------------------
 * ggml block layouts (sycl/moe/format.hpp:10-45 names and sizes; sub-block
 * decode as sycl/moe/core.hpp:17,47-58 reads them):
 *   Q8_0 (8)  34 B per 32: fp16 d, int8 q[32]; value d * q.
 *   Q4_K (12) 144 B per 256: fp16 d, fp16 dmin, 12 packed 6-bit (scale, min)
 *             pairs, 128 B of nibbles (sub-blocks 2i, 2i+1 = low, high nibbles
 *             of bytes 32i..32i+31); value d * sc * q - dmin * m.
 *   Q5_K (13) 176 B: as Q4_K plus 32 B of fifth bits before the nibbles (bit
 *             ib of byte j is the fifth bit of value j of sub-block ib).
 *   Q6_K (14) 210 B: 128 B low nibbles, 64 B of 2-bit highs, 16 int8 scales
 *             (one per 16 values), fp16 d last; value d * sc * (q - 32). */
typedef struct { int q[32]; int s[2]; float d; float m[2]; int has_min; } p32_sub;

static int p32_block_bytes(int t) {
    switch (t) { case 8: return 34; case 12: return 144; case 13: return 176; case 14: return 210; default: return orc_block_bytes(t); }
}
static int p32_subs_per_block(int t) { return t == 8 ? 1 : 8; }
int orc_row_bytes32(int t, int k) { return (k / (32 * p32_subs_per_block(t))) * p32_block_bytes(t); }

/* ggml's 6-bit (scale, min) unpacking of K-quant sub-block j from 12 bytes. */
static void kq_scale_min(const uint8_t* sc, int j, int* scale, int* mn) {
    if (j < 4) { *scale = sc[j] & 63; *mn = sc[j + 4] & 63; }
    else { *scale = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4); *mn = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4); }
}

static void p32_sub_get(int t, const uint8_t* row, int kb, p32_sub* s) {
    const uint8_t* blk = row + (size_t)(kb / p32_subs_per_block(t)) * p32_block_bytes(t);
    const int ib = kb & 7;
    memset(s, 0, sizeof *s);
    s->s[0] = s->s[1] = 1;
    if (t == 8) {
        s->d = orc_half(u16(blk));
        for (int j = 0; j < 32; ++j) s->q[j] = (int8_t)blk[2 + j];
    } else if (t == 12 || t == 13) {
        int sc, mn;
        kq_scale_min(blk + 4, ib, &sc, &mn);
        s->s[0] = s->s[1] = sc;
        s->d = orc_half(u16(blk));
        s->m[0] = s->m[1] = orc_half(u16(blk + 2)) * (float)mn;
        s->has_min = 1;
        const uint8_t* nib = blk + (t == 13 ? 48 : 16) + 32 * (ib >> 1);
        for (int j = 0; j < 32; ++j) {
            int q = (nib[j] >> (4 * (ib & 1))) & 15;
            if (t == 13) q |= ((blk[16 + j] >> ib) & 1) << 4;
            s->q[j] = q;
        }
    } else if (t == 14) {
        const int h = ib >> 2, quarter = ib & 3;
        const uint8_t* lo = blk + 64 * h + ((quarter & 1) ? 32 : 0);
        const uint8_t* hi = blk + 128 + 32 * h;
        for (int j = 0; j < 32; ++j)
            s->q[j] = (((lo[j] >> (4 * (quarter >> 1))) & 15) | (((hi[j] >> (2 * quarter)) & 3) << 4)) - 32;
        s->s[0] = (int8_t)blk[192 + 8 * h + 2 * quarter];
        s->s[1] = (int8_t)blk[193 + 8 * h + 2 * quarter];
        s->d = orc_half(u16(blk + 208));
    } else {
        p32_decode(t, blk, ib, s->q, s->s);
        s->d = p32_scale(t, blk);
    }
}

/* One row (core.hpp:66-87 lane<> + sub_dot<>, expert_check.cpp:50-55): lane
 * l of 32 takes sub-blocks l, l + 32, ...: dot = d * float(s0 * a + s1 * b)
 * (a, b: the integer dots of the two 16-value halves; IQ types d = fp16 d *
 * 0.125), for Q4_K / Q5_K minus the min term as two fmas (corr = fma(m0,
 * float(sum x[0..15]), m1 * float(sum x[16..31])), dot = fma(d, float(s0 * a +
 * s1 * b), -corr)), acc = fma(xd, dot, acc); Q8_0: acc = fma(d * xd,
 * float(dot32), acc). Then lane[l] = old[l] + old[l ^ o] for o = 16, 8, 4, 2,
 * 1, and lane 0 + 0. */
float orc_row32(int t, const uint8_t* row, int k, const int8_t* xq, const float* xd) {
    float lane[32];
    for (int l = 0; l < 32; ++l) {
        float acc = 0.0f;
        for (int kb = l; kb < k / 32; kb += 32) {
            p32_sub s;
            p32_sub_get(t, row, kb, &s);
            const int8_t* x = xq + 32 * kb;
            int a = 0, b = 0, sa = 0, sb = 0;
            for (int j = 0; j < 16; ++j) { a += s.q[j] * x[j]; b += s.q[16 + j] * x[16 + j]; sa += x[j]; sb += x[16 + j]; }
            if (t == 8) {
                acc = fmaf(s.d * xd[kb], (float)(a + b), acc);
                continue;
            }
            float dot = s.d * (float)(s.s[0] * a + s.s[1] * b);
            if (s.has_min) {
                const float corr = fmaf(s.m[0], (float)sa, s.m[1] * (float)sb);
                dot = fmaf(s.d, (float)(s.s[0] * a + s.s[1] * b), -corr);
            }
            acc = fmaf(xd[kb], dot, acc);
        }
        lane[l] = acc;
    }
    for (int o = 16; o; o >>= 1) {
        float old[32];
        memcpy(old, lane, sizeof old);
        for (int l = 0; l < 32; ++l) lane[l] = old[l] + old[l ^ o];
    }
    return 1.0f * lane[0] + 0.0f;
}
void orc_matvec32(int t, const uint8_t* w, int n, int k, const int8_t* xq, const float* xd, float* y) {
    const size_t rb = (size_t)orc_row_bytes32(t, k);
    for (int r = 0; r < n; ++r) y[r] = orc_row32(t, w + (size_t)r * rb, k, xq, xd);
}
/* Dequantized sub-block kb of one row, in double: (value_j)_j with the per-16
 * scales and mins applied (for the independent float64 checks). */
void orc_dequant32(int t, const uint8_t* row, int kb, double* out) {
    p32_sub s;
    p32_sub_get(t, row, kb, &s);
    for (int j = 0; j < 32; ++j) {
        const int h = j / 16;
        out[j] = t == 8 ? (double)s.d * s.q[j] : (double)s.d * s.s[h] * s.q[j] - (s.has_min ? (double)s.m[h] : 0.0);
    }
}
/* The per32 expert chain: Q32(x), gate and up rows, SwiGLU (core.hpp:88, the
 * same form as q8k_core.hpp:92-95), Q32(h), down rows. g, u, h may be NULL. */
void orc_expert32(const int types[3], const uint8_t* gate, const uint8_t* up, const uint8_t* down, int dim, int ff,
                  const float* x, float* y, float* g, float* u, float* h, float limit) {
    int8_t* q = (int8_t*)malloc((size_t)(dim > ff ? dim : ff));
    float* d = (float*)malloc(sizeof(float) * (size_t)((dim > ff ? dim : ff) / 32));
    float* gg = (float*)malloc(sizeof(float) * (size_t)ff * 3);
    float *uu = gg + ff, *hh = gg + 2 * ff;
    orc_quant32(x, dim, q, d);
    orc_matvec32(types[0], gate, ff, dim, q, d, gg);
    orc_matvec32(types[1], up, ff, dim, q, d, uu);
    for (int i = 0; i < ff; ++i) hh[i] = orc_swiglu(gg[i], uu[i], limit);
    orc_quant32(hh, ff, q, d);
    orc_matvec32(types[2], down, dim, ff, q, d, y);
    if (g) memcpy(g, gg, sizeof(float) * (size_t)ff);
    if (u) memcpy(u, uu, sizeof(float) * (size_t)ff);
    if (h) memcpy(h, hh, sizeof(float) * (size_t)ff);
    free(q); free(d); free(gg);
}

/* q8k_core.hpp:92-95 */
float orc_swiglu(float g, float u, float limit) {
    if (limit > 0) { g = fminf(g, limit); u = fminf(fmaxf(u, -limit), limit); }
    const float den = 1.0f + expf(-g);
    const float s = g / den;
    return s * u;
}

/* ---- row jobs (cpu_lane.cpp:70-81: 64-row jobs pulled by workers) ------ */
typedef struct {
    int type, n, nb;
    const uint8_t* w;
    const orc_q8k* a;
    float* y;
    atomic_int next;
} mv_job;

static void* mv_worker(void* arg) {
    mv_job* j = (mv_job*)arg;
    const size_t row_bytes = (size_t)j->nb * orc_block_bytes(j->type);
    for (;;) {
        const int job = atomic_fetch_add(&j->next, 1);
        const int lo = job * 64;
        if (lo >= j->n) break;
        const int hi = lo + 64 < j->n ? lo + 64 : j->n;
        for (int r = lo; r < hi; ++r) j->y[r] = orc_dot(j->type, j->w + (size_t)r * row_bytes, j->a, j->nb);
    }
    return NULL;
}

void orc_matvec(int type, const uint8_t* w, int n, int k, const orc_q8k* a, float* y, int threads) {
    tables();
    mv_job job;
    job.type = type; job.n = n; job.nb = k / 256; job.w = w; job.a = a; job.y = y;
    atomic_init(&job.next, 0);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    int started = 0;
    for (int i = 1; i < threads; ++i)
        if (pthread_create(&tid[started], NULL, mv_worker, &job) == 0) ++started;
    mv_worker(&job);
    for (int i = 0; i < started; ++i) pthread_join(tid[i], NULL);
}

void orc_down_from_hidden(int type, const uint8_t* down, int dim, int ff, const float* h, float* y, int threads) {
    orc_q8k hq[64];
    orc_quantize_row(h, ff, hq);
    orc_matvec(type, down, dim, ff, hq, y, threads);
}

/* Expert chain, as the CPU lane runs it (cpu_lane.cpp:157-168). */
void orc_expert(const int types[3], const uint8_t* gate, const uint8_t* up, const uint8_t* down, int dim, int ff,
                const float* x, float* y, float* g_out, float* u_out, float* h_out, int threads, float limit) {
    orc_q8k xq[64];
    float g[16384], u[16384], h[16384];
    orc_quantize_row(x, dim, xq);
    orc_matvec(types[0], gate, ff, dim, xq, g, threads);
    orc_matvec(types[1], up, ff, dim, xq, u, threads);
    for (int i = 0; i < ff; ++i) h[i] = orc_swiglu(g[i], u[i], limit);
    orc_down_from_hidden(types[2], down, dim, ff, h, y, threads);
    if (g_out) memcpy(g_out, g, sizeof(float) * (size_t)ff);
    if (u_out) memcpy(u_out, u, sizeof(float) * (size_t)ff);
    if (h_out) memcpy(h_out, h, sizeof(float) * (size_t)ff);
}

/* warm/runtime.cpp:183-188 */
void orc_combine(const int32_t* ids, const float* w, int k, const float* rows, int dim, const float* shared, float* out) {
    int order[64];
    for (int i = 0; i < k; ++i) order[i] = i;
    for (int i = 1; i < k; ++i) /* insertion sort by id (ids are unique) */
        for (int j = i; j > 0 && ids[order[j]] < ids[order[j - 1]]; --j) {
            const int t = order[j]; order[j] = order[j - 1]; order[j - 1] = t;
        }
    for (int c = 0; c < dim; ++c) out[c] = 0.0f;
    for (int i = 0; i < k; ++i) {
        const int p = order[i];
        for (int c = 0; c < dim; ++c) out[c] = fmaf(w[p], rows[(size_t)p * dim + c], out[c]);
    }
    if (shared)
        for (int c = 0; c < dim; ++c) out[c] += shared[c];
}

/* ---- hyper-connection post (sycl/hc/core.hpp:81-86, hc.cpp:107-110) --------
 * T tokens, H <= 4 residual streams of D: out[t][k][e] = post[t][k] * y[t][e]
 * + comb[t][j][k] * res[t][j][e] for j = 0..H-1, accumulated in that order with
 * separate roundings. post: T x 8 floats, comb: T x 64 (row j, column k at
 * j * H + k). */
void orc_hc_post(const float* y, const float* res, const float* post, const float* comb, int D, int H, int T, float* out) {
    for (int t = 0; t < T; ++t)
        for (int e = 0; e < D; ++e) {
            const float v = y[(size_t)t * D + e];
            for (int k = 0; k < H; ++k) {
                float a = post[t * 8 + k] * v;
                for (int j = 0; j < H; ++j) a += comb[t * 64 + j * H + k] * res[((size_t)t * H + j) * D + e];
                out[((size_t)t * H + k) * D + e] = a;
            }
        }
}

/* ---- hyper-connection pre + RMS norm (sycl/hc/core.hpp:74-80 pre_norm,
 * block_sum core.hpp:9-17; hc.cpp:89-106) -----------------------------------
 * Per token t: x[e] = sum_j mix[t][j] * h[t][j][e] (j ascending from 0.0f,
 * separate roundings); 1024 lane sums, lane i over e = i, i + 1024, ... of
 * x[e] * x[e]; their total by a pairwise XOR tree over each 32 lanes
 * (offsets 16, 8, 4, 2, 1, lane 0's result), then the same tree over the 32
 * group totals; with w, x[e] = (x[e] * inv) * w[e], inv = 1 / sqrtf(total / D
 * + eps). mix: T x 8 floats. */
static float orc_xor32(const float* p) {
    float v[32];
    for (int i = 0; i < 32; ++i) v[i] = p[i];
    for (int o = 16; o; o >>= 1)
        for (int i = 0; i < 32; ++i)
            if (!(i & o)) v[i] += v[i ^ o];
    return v[0];
}
void orc_hc_pre_norm(const float* h, const float* mix, const float* w, int D, int H, int T, float eps, float* x) {
    for (int t = 0; t < T; ++t) {
        const float* hh = h + (size_t)t * H * D;
        const float* mm = mix + (size_t)t * 8;
        float* xx = x + (size_t)t * D;
        float lanes[1024], red[32];
        for (int i = 0; i < 1024; ++i) {
            float ss = 0.0f;
            for (int e = i; e < D; e += 1024) {
                float a = 0.0f;
                for (int j = 0; j < H; ++j) a += mm[j] * hh[(size_t)j * D + e];
                xx[e] = a;
                ss += a * a;
            }
            lanes[i] = ss;
        }
        if (!w) continue;
        for (int g = 0; g < 32; ++g) red[g] = orc_xor32(lanes + 32 * g);
        const float inv = 1.0f / sqrtf(orc_xor32(red) / (float)D + eps);
        for (int e = 0; e < D; ++e) xx[e] = xx[e] * inv * w[e];
    }
}

/* ---- router: route.cpp:15-37 ---------------------------------------------
 * Per token: softplus(l) (l itself above 20), its square root as the score,
 * the score plus the expert's bias as the selection key; k rounds of "first
 * largest key" (strict >), each taking the expert out; the scores of the picks
 * summed in pick order; weight = score / (sum + 1e-20) * scale. Every step in
 * single precision with separate roundings (this file is built without FMA
 * contraction). */
void orc_route(const float* logits, int stride, const float* bias, int n, int T, int k, float scale, int32_t* ids,
               float* w) {
    float* sc = (float*)malloc(sizeof(float) * (size_t)n);
    float* key = (float*)malloc(sizeof(float) * (size_t)n);
    for (int t = 0; t < T; ++t) {
        const float* lg = logits + (size_t)t * stride;
        for (int e = 0; e < n; ++e) {
            const float l = lg[e];
            const float sp = l > 20.0f ? l : log1pf(expf(l));
            sc[e] = sqrtf(sp);
            key[e] = sc[e] + (bias ? bias[e] : 0.0f);
        }
        float sum = 0.0f;
        for (int i = 0; i < k; ++i) {
            int best = 0;
            for (int e = 1; e < n; ++e)
                if (key[e] > key[best]) best = e;
            ids[(size_t)t * k + i] = best;
            sum += sc[best];
            key[best] = -FLT_MAX;
        }
        for (int i = 0; i < k; ++i) {
            const float q = sc[ids[(size_t)t * k + i]] / (sum + 1e-20f);
            w[(size_t)t * k + i] = q * scale;
        }
    }
    free(sc);
    free(key);
}

/* ---- generator (this build's spec; restated independently) ------------- */
static uint64_t splitmix_out(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
uint64_t orc_gen_key(uint64_t seed, uint32_t layer, uint32_t expert, uint32_t role) {
    return splitmix_out(seed ^ splitmix_out(((uint64_t)layer << 40) ^ ((uint64_t)expert << 8) ^ role));
}
static uint64_t gen_word(uint64_t key, uint64_t blk, unsigned j) {
    return splitmix_out(key + (blk * 16u + j) * 0xD1B54A32D192ED03ull);
}
/* float -> fp16 round-to-nearest-even through frexp/rint (normal range only:
 * the generator's d lies in [1e-3, 1e-2]). */
static uint16_t to_half_normal(float v) {
    int e;
    const double m = frexp((double)v, &e);       /* v = m * 2^e, 0.5 <= m < 1 */
    double mant = rint(m * 2048.0);              /* 11 significant bits, RNE */
    if (mant == 2048.0) { mant = 1024.0; ++e; }
    const int he = e - 1 + 15;                   /* biased half exponent */
    return (uint16_t)((he << 10) | ((int)mant - 1024));
}
void orc_gen_block(int type, uint64_t key, uint64_t blk, uint8_t* out) {
    const int nbytes = orc_block_bytes(type);
    for (int i = 0; i < nbytes; ++i) out[i] = (uint8_t)(gen_word(key, blk, (unsigned)(i / 8)) >> (8 * (i % 8)));
    const float u = (float)(uint32_t)(gen_word(key, blk, 15) >> 40);
    const float t = u * (9e-3f * 5.9604644775390625e-08f);
    const float v = 1e-3f + t;
    const uint16_t d = to_half_normal(v);
    if (type != 29) {
        out[0] = (uint8_t)d; out[1] = (uint8_t)(d >> 8);
    } else {
        for (int q = 0; q < 4; ++q) {
            const uint16_t s = (uint16_t)((u16(out + 48 + 2 * q) & 0x0fff) | (((d >> (4 * q)) & 15) << 12));
            out[48 + 2 * q] = (uint8_t)s; out[49 + 2 * q] = (uint8_t)(s >> 8);
        }
    }
}
void orc_gen_matrix(int type, uint64_t seed, uint32_t layer, uint32_t expert, uint32_t role, int n, int k, uint8_t* out) {
    const uint64_t key = orc_gen_key(seed, layer, expert, role);
    const int bb = orc_block_bytes(type);
    const uint64_t nblk = (uint64_t)n * (uint64_t)(k / 256);
    for (uint64_t b = 0; b < nblk; ++b) orc_gen_block(type, key, b, out + b * bb);
}
