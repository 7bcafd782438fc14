// Thin extern "C" wrapper that compiles the reference's own CPU arithmetic from
// its sources under /root/reference (include paths set by oracle/Makefile) into
// oracle/_ref/libxlref.so. TEST INFRASTRUCTURE ONLY: it lets the tests compare
// the oracle restatement with the reference code itself, and serves as the
// "reference" CPU baseline. Nothing here is copied; the headers are included
// where they lie.
//   sycl/stage/wiring/q8k_core.hpp (+ q8k_tables.inc): Q8_K quant and IQ dots
//   sycl/moe/core.hpp (+ format.hpp, tables.hpp):     per-32 decoder
//   warm/other_combine.hpp:                             fixed-order combine
//   sycl/route/route.hpp, route.cpp (compiled alongside): route_cpu
//   sycl/hc/core.hpp:                                   hyper-connection post
#include <array>
#include <cmath>
#include <atomic>
#include <cstring>
#include <span>
#include <thread>
#include <utility>
#include <vector>
#include "q8k_core.hpp"
#include "core.hpp"
#include "other_combine.hpp"
#include "route.hpp"
#include "hc/core.hpp"

namespace q = strata::wiring::q8k;
namespace m = strata::ds4::moe;

extern "C" {
void ref_quant_block(const float* x, void* out) { q::quant_block(x, *static_cast<q::Block*>(out)); }
float ref_dot(int t, const uint8_t* w, const void* a, int nb) { return q::dot(t, w, static_cast<const q::Block*>(a), nb); }
void ref_integer_lane(int t, const uint8_t* w, const void* a, int lane, int* main_out, int* delta_out) {
    const auto v = q::integer_lane(t, w, *static_cast<const q::Block*>(a), lane);
    *main_out = v.main; *delta_out = v.delta;
}
float ref_swiglu(float g, float u, float lim) { return q::swiglu(g, u, lim); }
float ref_half(uint16_t h) { return q::half(h); }
int ref_nearest(float x) { return q::nearest(x); }
void ref_table(int which, uint64_t* out) {
    if (which == 0) std::memcpy(out, q::iq2xxs_grid, sizeof q::iq2xxs_grid);
    else if (which == 1) std::memcpy(out, q::iq2xs_grid, sizeof q::iq2xs_grid);
    else if (which == 2) std::memcpy(out, q::iq1s_grid, sizeof q::iq1s_grid);
    else for (int i = 0; i < 128; ++i) out[i] = q::ksigns_iq2xs[i];
}
static m::Type ref_type(int t) {
    switch (t) {
    case 16: return m::Type::iq2_xxs;
    case 17: return m::Type::iq2_xs;
    case 8: return m::Type::q8_0;
    case 12: return m::Type::q4_k;
    case 13: return m::Type::q5_k;
    case 14: return m::Type::q6_k;
    default: return m::Type::iq1_m;
    }
}
// Per-32 decode of sub-block kb of one row (types 16, 17, 29, 8, 12, 13, 14);
// m2 (may be null) receives the two per-16 min terms.
void ref_decode(int t, const uint8_t* row, int kb, int* q32, int* s2, float* d, float* m2) {
    const auto s = m::decode(ref_type(t), row, kb);
    for (int j = 0; j < 32; ++j) q32[j] = s.q[j];
    s2[0] = s.s[0]; s2[1] = s.s[1]; *d = s.d;
    if (m2) { m2[0] = s.m[0]; m2[1] = s.m[1]; }
}
// hc_scalar::pre_norm over T tokens.
void ref_hc_pre_norm(const float* h, const float* mix, const float* w, int D, int H, int T, float eps, float* x) {
    for (int t = 0; t < T; ++t) strata::ds4::hc_scalar::pre_norm(h, mix, w, D, H, t, eps, x);
}
// hc_scalar::post over T tokens x D values.
void ref_hc_post(const float* y, const float* res, const float* post, const float* comb, int D, int H, int T, float* out) {
    for (int t = 0; t < T; ++t)
        for (int e = 0; e < D; ++e) strata::ds4::hc_scalar::post(y, res, post, comb, D, H, t, e, out);
}
// Matvec over threads with the reference's dot, rows split in 64-row jobs.
void ref_matvec(int t, const uint8_t* w, int n, int k, const void* a, float* y, int threads) {
    const int nb = k / 256; const size_t rb = size_t(nb) * q::block_bytes(t);
    const auto* act = static_cast<const q::Block*>(a);
    std::atomic<int> next{0};
    auto run = [&] { for (int j; (j = next.fetch_add(1)) * 64 < n;) for (int r = j * 64; r < n && r < j * 64 + 64; ++r) y[r] = q::dot(t, w + size_t(r) * rb, act, nb); };
    std::vector<std::thread> pool; for (int i = 1; i < threads; ++i) pool.emplace_back(run);
    run(); for (auto& th : pool) th.join();
}
// One expert chain with the reference's functions: Q8_K(x), gate/up rows,
// SwiGLU (with the limit), Q8_K(h), down rows (the CPU lane order, cpu_lane.cpp:157-168).
void ref_expert(const int* types, const uint8_t* gate, const uint8_t* up, const uint8_t* down, int dim, int ff,
                const float* x, float* y, int threads, float lim) {
    std::vector<q::Block> xq(static_cast<size_t>(dim / 256)), hq(static_cast<size_t>(ff / 256));
    for (int b = 0; b < dim / 256; ++b) q::quant_block(x + 256 * b, xq[size_t(b)]);
    const size_t nff = static_cast<size_t>(ff);
    std::vector<float> g(nff), u(nff), h(nff);
    ref_matvec(types[0], gate, ff, dim, xq.data(), g.data(), threads);
    ref_matvec(types[1], up, ff, dim, xq.data(), u.data(), threads);
    for (int i = 0; i < ff; ++i) h[size_t(i)] = q::swiglu(g[size_t(i)], u[size_t(i)], lim);
    for (int b = 0; b < ff / 256; ++b) q::quant_block(h.data() + 256 * b, hq[size_t(b)]);
    ref_matvec(types[2], down, dim, ff, hq.data(), y, threads);
}
// One row through the reference's per-32 lane<> and the butterfly of
// warm/expert_check.cpp:50-55 (the CPU control of the production HIP lane).
struct RefMath {
    static float fma(float a, float b, float c) { return std::fma(a, b, c); }
    static float exp(float a) { return std::exp(a); }
    static float min(float a, float b) { return std::fmin(a, b); }
    static float max(float a, float b) { return std::fmax(a, b); }
};
float ref_row32(int t, const uint8_t* row, int k, const int8_t* xq, const float* xd) {
    const m::Type ty = ref_type(t);
    std::array<float, 32> lane;
    for (int l = 0; l < 32; ++l) lane[size_t(l)] = m::lane<RefMath>(ty, row, k, nullptr, xq, xd, l, true);
    for (int o = 16; o; o >>= 1) {
        const auto old = lane;
        for (int l = 0; l < 32; ++l) lane[size_t(l)] = old[size_t(l)] + old[size_t(l ^ o)];
    }
    return 1.0f * lane[0] + 0.0f;
}
void ref_route(const float* logits, int stride, const float* bias, int n, int T, int k, float scale, int* ids, float* w) {
    const auto r = strata::ds4::route_port::route_cpu(std::span<const float>(logits, size_t(T) * size_t(stride)),
                                                      size_t(stride), std::span<const float>(bias, size_t(n)),
                                                      size_t(T), size_t(k), scale);
    for (size_t i = 0; i < r.ids.size(); ++i) { ids[i] = r.ids[i]; w[i] = r.weights[i]; }
}
void ref_combine(const int* ids, const float* w, int k, const float* rows, int dim, const float* shared, float* out) {
    std::array<std::vector<std::pair<size_t, std::vector<float>>>, 1> results;
    for (int i = 0; i < k; ++i) results[0].emplace_back(size_t(i), std::vector<float>(rows + size_t(i) * dim, rows + size_t(i + 1) * dim));
    auto y = strata::wiring::other_combine(std::span<const int>(ids, size_t(k)), std::span<const float>(w, size_t(k)),
                                           std::span<const float>(shared, size_t(dim)), results, strata::wiring::OtherOptions{});
    std::memcpy(out, y.data(), sizeof(float) * size_t(dim));
}
}
