// The router of route.cpp:15-37 (route_cpu) as wave-level device code, shared
// by the router kernel (xl_kernels.hip) and the streaming layer kernel's
// routed prologue (xl_stream.hpp): score = sqrt(softplus(l)) (l itself above
// 20), key = score + bias; k rounds of the first largest key (strict '>' in
// index order: ties go to the lower index), each round taking the expert out
// (key -FLT_MAX); the picked scores summed in pick order; weight = score /
// (sum + 1e-20) * scale. Separate IEEE roundings throughout (no contraction);
// expf / log1pf are the device library's.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace xl::dev {

// Keys as unsigned integers that order as the floats do (-FLT_MAX, the taken
// mark, above 0, which pads lanes past n).
__device__ __forceinline__ uint32_t ordered(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
template <bool MAX>
__device__ __forceinline__ uint32_t wave_ext(uint32_t a) {   // wave max / min by DPP, result in every lane
    auto f = [](uint32_t x, uint32_t y) { return MAX ? max(x, y) : min(x, y); };
    const int id = MAX ? 0 : -1;
    a = f(a, uint32_t(__builtin_amdgcn_update_dpp(int(a), int(a), 0xB1, 0xF, 0xF, false)));   // quad_perm 1,0,3,2
    a = f(a, uint32_t(__builtin_amdgcn_update_dpp(int(a), int(a), 0x4E, 0xF, 0xF, false)));   // quad_perm 2,3,0,1
    a = f(a, uint32_t(__builtin_amdgcn_update_dpp(int(a), int(a), 0x141, 0xF, 0xF, false)));  // row_half_mirror
    a = f(a, uint32_t(__builtin_amdgcn_update_dpp(int(a), int(a), 0x140, 0xF, 0xF, false)));  // row_mirror
    a = f(a, uint32_t(__builtin_amdgcn_update_dpp(id, int(a), 0x142, 0xA, 0xF, false)));       // row_bcast:15
    a = f(a, uint32_t(__builtin_amdgcn_update_dpp(id, int(a), 0x143, 0xC, 0xF, false)));       // row_bcast:31
    return uint32_t(__builtin_amdgcn_readlane(int(a), 63));
}

// Expert e's score and key (e < n; past n: score 0, key 0). fin: l and the key finite.
__device__ __forceinline__ void route_score(float l, float b, bool in, float& sc, uint32_t& key, bool& fin) {
    const float sp = l > 20.0f ? l : log1pf(expf(l));
    const float s = sqrtf(sp);
    const float kk = __fadd_rn(s, b);
    fin = fin && (!in || ((fabsf(l) <= 3.402823466e38f) && (fabsf(kk) <= 3.402823466e38f)));
    sc = in ? s : 0.0f;
    key = in ? ordered(kk) : 0u;
}

// The k picks from one wave's keys (expert lane + 64 j in slot j of lane
// `lane`): lane i < k gets pick i's id and weight. The keys are consumed.
template <int NPL>
__device__ __forceinline__ void route_select(const float (&sc)[NPL], uint32_t (&key)[NPL], int k, int lane, float scale,
                                             int& id_out, float& w_out) {
    const uint32_t taken = ordered(-3.402823466e38f);
    float sum = 0.0f, mine = 0.0f;   // lane i < k keeps pick i's score
    int myid = 0;
    for (int i = 0; i < k; ++i) {
        uint32_t bk = 0u;
        int bj = 0;
#pragma unroll
        for (int j = 0; j < NPL; ++j)   // this lane's first largest key (strict '>')
            if (key[j] > bk) { bk = key[j]; bj = j; }
        const uint32_t top = wave_ext<true>(bk);
        const int e = int(wave_ext<false>(bk == top ? uint32_t(lane + 64 * bj) : 0xffffffffu));   // lowest index
        float se = 0.0f;
#pragma unroll
        for (int j = 0; j < NPL; ++j)
            if (lane + 64 * j == e) { se = sc[j]; key[j] = taken; }
        se = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(se), e & 63));
        sum = __fadd_rn(sum, se);
        mine = lane == i ? se : mine;
        myid = lane == i ? e : myid;
    }
    id_out = myid;
    w_out = __fmul_rn(__fdiv_rn(mine, __fadd_rn(sum, 1e-20f)), scale);
}

}  // namespace xl::dev
