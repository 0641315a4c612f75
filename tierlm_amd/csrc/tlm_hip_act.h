/* tlm_hip_act.h - the activation quantiser's per-block rule on wave lanes
 * (src/lib/tlm_quant.c:458-478: amax / 127, IEEE reciprocal, magic-constant
 * RNE codes clamped to +-127, NaN / Inf poisoning, the double path below
 * 2^-100), shared by the quantiser kernels and the fused kernels that
 * quantise what they produce.  Included by .hip files. */
#ifndef TLM_HIP_ACT_H
#define TLM_HIP_ACT_H

#include "tlm_hip_internal.h"

namespace {

/* Flags and amax of the lanes in a group of `width` lanes (power of two,
 * aligned); every lane of the group receives the result. */
template <int WIDTH>
__device__ __forceinline__ void group_amax(float &amax, int &nan, int &inf) {
#pragma unroll
    for (int m = 1; m < WIDTH; m <<= 1) {
        float o = __shfl_xor(amax, m, 64);
        amax = o > amax ? o : amax;
        nan |= __shfl_xor(nan, m, 64);
        inf |= __shfl_xor(inf, m, 64);
    }
}

/* The shared per-block rule (src/lib/tlm_quant.c:458-478) for this lane's 4
 * values; returns the block scale d and writes 4 codes packed in a dword. */
template <int WIDTH>
__device__ __forceinline__ float act_rule(const float v[4], const bool ok[4], uint32_t &codes) {
    float amax = 0.0f;
    int nan = 0, inf = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (!ok[j]) continue;
        float a = fabsf(v[j]);
        if (a != a) nan = 1;
        else if (a == INFINITY) inf = 1;
        else if (a > amax) amax = a;
    }
    group_amax<WIDTH>(amax, nan, inf);
    codes = 0;
    if (nan || inf) return nan ? __uint_as_float(0x7FC00000u) : INFINITY;
    if (!(amax > 0.0f)) return 0.0f;
    float d = amax / 127.0f;
    if (amax >= 0x1p-100f) {
        float id = 127.0f / amax;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (ok[j]) codes |= (uint32_t)(uint8_t)(int8_t)rne_clamp(v[j] * id, -127, 127) << (8 * j);
    } else {
        double id = 127.0 / (double)amax;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (ok[j]) codes |= (uint32_t)(uint8_t)(int8_t)rne_clamp((float)((double)v[j] * id), -127, 127) << (8 * j);
    }
    return d;
}

__device__ __forceinline__ int byte_sum(uint32_t c) {
    return (int)(int8_t)(c & 0xFF) + (int)(int8_t)((c >> 8) & 0xFF) + (int)(int8_t)((c >> 16) & 0xFF) +
           (int)(int8_t)(c >> 24);
}

}  // namespace

#endif
