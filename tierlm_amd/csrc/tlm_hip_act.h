/* tlm_hip_act.h - the activation quantiser's per-block rule on wave lanes
 * (src/lib/tlm_quant.c:458-478: amax / 127, IEEE reciprocal, magic-constant
 * RNE codes clamped to +-127, NaN / Inf poisoning, the double path below
 * 2^-100), shared by the quantiser kernels and the fused kernels that
 * quantise what they produce: 4 values per lane (act_rule), or 16 contiguous
 * values per lane (act_rule16 / quant16_to: a Q8_K block over 16 lanes, an
 * a8 block over 2, so the per-block work is shared by fewer lanes).
 * Included by .hip files. */
#ifndef TLM_HIP_ACT_H
#define TLM_HIP_ACT_H

#include "tlm_hip_internal.h"

namespace {

/* Flags and amax of the lanes in a group of `width` lanes (power of two,
 * aligned; every lane of the group active); every lane of the group
 * receives the result.  amax >= +0, so its bits order as its values: a DPP
 * maximum over the bits, the flags OR-ed the same way. */
template <int WIDTH>
__device__ __forceinline__ void group_amax(float &amax, int &nan, int &inf) {
    amax = __uint_as_float(group_max_u32<WIDTH>(__float_as_uint(amax)));
    const uint32_t fl = group_or_u32<WIDTH>((nan ? 1u : 0u) | (inf ? 2u : 0u));
    nan = (int)(fl & 1u);
    inf = (int)((fl >> 1) & 1u);
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

/* Codes of 16 values for a block whose amax is below 2^-100, where 127/amax
 * is taken in double (src/lib/tlm_quant.c:466-471).  Out of line: it is never
 * reached by ordinary activations, and a call waits for every load in flight. */
__device__ __attribute__((noinline)) u32x4 tiny_codes16(f32x4 v0, f32x4 v1, f32x4 v2, f32x4 v3, float amax) {
    const double id = 127.0 / (double)amax;
    const f32x4 v[4] = {v0, v1, v2, v3};
    u32x4 c = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int t = 0; t < 16; t++)
        c[t >> 2] |= (uint32_t)(uint8_t)(int8_t)rne_clamp((float)((double)v[t >> 2][t & 3] * id), -127, 127)
                     << (8 * (t & 3));
    return c;
}

/* The activation rule with 16 contiguous values per lane and a block spread
 * over WIDTH lanes of one DPP row (16 for Q8_K, 2 for a8).  Returns d and
 * the 16 codes packed in c[0..3]. */
template <int WIDTH>
__device__ __forceinline__ float act_rule16(const f32x4 (&v)[4], bool ok, u32x4 &c) {
    uint32_t am = 0, fl = 0;
#pragma unroll
    for (int t = 0; t < 16; t++) {
        const uint32_t b = ok ? (__float_as_uint(v[t >> 2][t & 3]) & 0x7FFFFFFFu) : 0u;
        fl |= (b > 0x7F800000u ? 1u : 0u) | (b == 0x7F800000u ? 2u : 0u);
        const uint32_t f = b < 0x7F800000u ? b : 0u;
        am = f > am ? f : am;
    }
    am = group_max_u32<WIDTH>(am);
    fl = group_or_u32<WIDTH>(fl);
    const float amax = __uint_as_float(am);
    c = u32x4{0u, 0u, 0u, 0u};
    if (fl) return (fl & 1u) ? __uint_as_float(0x7FC00000u) : INFINITY;
    if (!(amax > 0.0f) || !ok) return amax > 0.0f ? amax / 127.0f : 0.0f;
    const float d = amax / 127.0f;
    if (amax >= 0x1p-100f) {
        const float id = 127.0f / amax;
#pragma unroll
        for (int t = 0; t < 16; t++)
            c[t >> 2] |= (uint32_t)(uint8_t)(int8_t)rne_clamp(v[t >> 2][t & 3] * id, -127, 127) << (8 * (t & 3));
    } else {
        c = tiny_codes16(v[0], v[1], v[2], v[3], amax);
    }
    return d;
}

__device__ __forceinline__ void st16(LAS uint8_t *p, u32x4 v) { *(LAS u32x4 *)p = v; }
__device__ __forceinline__ void st16(GAS uint8_t *p, u32x4 v) { *(GAS u32x4 *)p = v; }

/* Quantise block b (this lane: values 16*sub..16*sub+15) into the split
 * layout (q codes, bs bsums, dd scales; LDS or global).  Q8_K: 16 lanes per
 * block, and a lane's 16 codes are exactly bsum group sub; a8: 2 lanes per
 * block. */
template <class QP, class BP, class DP>
__device__ __forceinline__ void quant16_to(int kind, const f32x4 (&v)[4], bool ok, int sub, QP q, BP bs, DP dd,
                                           int b) {
    u32x4 c;
    if (kind == DT_Q8_K) {
        const float d = act_rule16<16>(v, ok, c);
        if (ok) {
            st16(q + b * 256 + 16 * sub, c);
            bs[b * 16 + sub] = (int16_t)(byte_sum(c.x) + byte_sum(c.y) + byte_sum(c.z) + byte_sum(c.w));
            if (sub == 0) dd[b] = d;
        }
    } else {
        const float d = act_rule16<2>(v, ok, c);
        if (ok) {
            st16(q + b * 32 + 16 * sub, c);
            if (sub == 0) dd[b] = d;
        }
    }
}

__device__ __attribute__((noinline)) void quant16_to_ool(int kind, f32x4 v0, f32x4 v1, f32x4 v2, f32x4 v3, bool ok,
                                                        int sub, LAS uint8_t *q, LAS int16_t *bs, LAS float *dd,
                                                        int b) {
    const f32x4 v[4] = {v0, v1, v2, v3};
    quant16_to(kind, v, ok, sub, q, bs, dd, b);
}

}  // namespace

#endif
