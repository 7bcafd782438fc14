// expf as the reference CPU lane evaluates it: the host C library's expf
// (q8k_core.hpp:94 calls expf; glibc on x86-64 resolves it to the FMA build of
// sysdeps/ieee754/flt-32/e_expf.c). That is the published Arm Optimized
// Routines method (Szabolcs Nagy, 2017): x / ln2 = k/32 + r in double with
// k rounded to nearest by the 1.5 * 2^52 shift, 2^(k/32) from a 32-entry
// table whose entry i is the bits of 2^(i/32) (rounded to double) minus
// i << 47, and a degree-3 polynomial in r; one rounding to float at the end.
// The reduction's multiply-adds are fused, as in that build. The table is
// 2^(i/32) itself; the polynomial coefficients are the method's published
// minimax values. Checked against the host's expf on every float input in
// (-130, 100) (tests/test_refexp.py runs a sampled check).
//
// Host and device: the device evaluates it in fp64 (v_fma_f64).
#pragma once
#include <cstdint>
#include <cstring>
#include <cmath>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define XL_RX_HD __host__ __device__ __forceinline__
#define XL_RX_TABLE __device__ __constant__
#else
#define XL_RX_HD inline
#define XL_RX_TABLE
#endif

namespace xl {

// bits(2^(i/32)) - (i << 47), i = 0..31
XL_RX_TABLE static const uint64_t kRefExpTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

XL_RX_HD double rx_asdouble(uint64_t u) {
    double d;
    std::memcpy(&d, &u, sizeof d);
    return d;
}
XL_RX_HD uint64_t rx_asuint64(double d) {
    uint64_t u;
    std::memcpy(&u, &d, sizeof u);
    return u;
}

XL_RX_HD float ref_expf(float x) {
    if (x != x) return x + x;                       // NaN
    if (x > 0x1.62e42ep6f) return INFINITY;         // overflow (and +inf)
    if (x < -0x1.9fe368p6f) return 0.0f;            // underflow (and -inf)
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    constexpr double kShift = 0x1.8p+52;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = double(x);
    double kd = fma(kInvLn2N, xd, kShift);     // k rounded to nearest in the low bits
    const uint64_t ki = rx_asuint64(kd);
    kd -= kShift;
    const double r = fma(kInvLn2N, xd, -kd);   // x / ln2 * 32 - k
    const double s = rx_asdouble(kRefExpTab[ki % 32] + (ki << 47));
    const double z = fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma(kC2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return float(y);
}

}  // namespace xl
