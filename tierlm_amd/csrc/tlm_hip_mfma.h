/* tlm_hip_mfma.h - the token-batched Q6_K tile on int8 MFMA, shared by the
 * public token matmul and the prefill MoE kernels.  Included by .hip files.
 *
 * The reference's prefill runs the decode step once per token
 * (src/lib/tlm_model.c:1105-1113), so every (token, row) output is the decode
 * dot - per super-block an exact int32 sum, then the row's fma chain in
 * ascending block order (src/lib/tlm_quant.c:853-882 for Q6_K).  A tile
 * streams 32 weight rows once for 32 tokens and takes the int32 sums from
 * v_mfma_i32_32x32x16_i8 (K = 16 = one Q6_K scale group); the chain is the
 * same, so the results are the decode kernel's bits.
 *
 * MFMA roles: srcA = activations (lane l: token l%32, codes 8*(l/32)..+7 of
 * the group), srcB = weights (lane l: weight row l%32, the same 8 positions),
 * D[token][row] in lane l, element v: token 8*(v/4) + 4*(l/32) + v%4, row
 * l%32.  Every accumulator of a lane belongs to one weight row, so the row's
 * group scale is one value per lane.
 *
 * Q6_K codes u in [0, 63] enter as u - 32 (int8): sum((u - 32) x) equals the
 * reference's gs - 32 * bsum exactly. */
#ifndef TLM_HIP_MFMA_H
#define TLM_HIP_MFMA_H

#include "tlm_hip_internal.h"

namespace tokmm {

constexpr int TM_ROWS = 32;      /* weight rows per wave */
constexpr int TM_TOK = 32;       /* tokens per wave */

typedef int v16i __attribute__((ext_vector_type(16)));


/* 4 Q6_K codes (ql nibbles + qh 2-bit fields, selected) -> 4 int8 of u - 32 */
__device__ __forceinline__ uint32_t q6_signed4(uint32_t ql, uint32_t qh, int nib, int sh) {
    const uint32_t u = ((ql >> (4 * nib)) & 0x0F0F0F0Fu) | (((qh >> sh) & 0x03030303u) << 4);
    const uint32_t t = u ^ 0x20202020u;            /* u - 32 for u >= 32; u + 32 otherwise */
    const uint32_t s = t & 0x20202020u;            /* sign bit 5 -> extend into bits 6, 7 */
    return t | (s << 1) | (s << 2);
}

/* One Q6_K block of one weight row, this lane's half (positions 8h..8h+7 of
 * every group): ql pieces [h][qq&1][g&1], qh pieces [h][g&1], scales, d. */
struct Q6Raw {
    u32x2 ql[8], qh[4];
    u32x4 sc;
    uint32_t dw;
};

__device__ __forceinline__ Q6Raw q6_load(const GAS uint8_t *unit, const GAS uint16_t *dp, int half) {
    Q6Raw r;
#pragma unroll
    for (int p = 0; p < 8; p++) {          /* p = 4h + 2(qq&1) + gl */
        const int h = p >> 2, q1 = (p >> 1) & 1, gl = p & 1;
        r.ql[p] = *(const GAS u32x2 *)(unit + 64 * h + 32 * q1 + 16 * gl + 8 * half);
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {          /* p = 2h + gl */
        const int h = p >> 1, gl = p & 1;
        r.qh[p] = *(const GAS u32x2 *)(unit + 128 + 32 * h + 16 * gl + 8 * half);
    }
    r.sc = *(const GAS u32x4 *)(unit + 192);
    r.dw = *dp;
    return r;
}

/* A operand of one Q8_K block of this lane's token: codes 16g + 8*half + 0..7
 * for g = 0..15, and the block's d. */
struct ActRaw {
    uint32_t c[32];
    float d;
};

__device__ __forceinline__ ActRaw act_load_codes(const GAS uint8_t *codes, const GAS float *d, int half) {
    ActRaw a;
    const GAS uint32_t *q = (const GAS uint32_t *)codes;
#pragma unroll
    for (int g = 0; g < 16; g++) {
        a.c[2 * g] = q[4 * g + 2 * half];
        a.c[2 * g + 1] = q[4 * g + 2 * half + 1];
    }
    a.d = *d;
    return a;
}

/* A token's Q8_K activation, block b: the reference layout (292-byte blocks:
 * d, codes, bsums) or the split layout of the MoE kernels (all codes, then
 * all bsums, then all d). */
template <bool SPLIT>
__device__ __forceinline__ ActRaw act_load(const GAS uint8_t *x, int nb, int b, int half) {
    if (SPLIT) return act_load_codes(x + b * 256, (const GAS float *)(x + nb * 288) + b, half);
    return act_load_codes(x + b * 292 + 4, (const GAS float *)(x + b * 292), half);
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return (long)(((unsigned long long)hi << 32) | lo);
}

/* acc[v] = row (l%32) . token (8*(v/4) + 4*half + v%4) of one 32 x 32 tile.
 * Wp / units: the packed matrix; ubase: unit of this lane's row in block 0
 * (valid row); arow: this lane's token (row l%32 of the tile), Q8_K blocks in
 * the reference (SPLIT false) or split layout; sda: 32 floats of wave-private
 * LDS. */
template <bool SPLIT>
__device__ __forceinline__ void tile_q6k(const uint8_t *__restrict__ Wp, int64_t units, int64_t ubase, int nb,
                                         const GAS uint8_t *arow, LAS float *sda, int j, int half,
                                         float (&acc)[16]) {
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;

    /* block b of this row: unit ubase + 16 b (208 bytes each), its d at
     * units * 208 + 2 (ubase + 16 b); the token's block b at arow + 292 b */
    const GAS uint8_t *unit = (const GAS uint8_t *)Wp + ubase * 208;
    const GAS uint16_t *dp = (const GAS uint16_t *)((const GAS uint8_t *)Wp + units * 208) + ubase;
    auto block = [&](const Q6Raw &w, const ActRaw &a) {
        int isum[16];
#pragma unroll
        for (int v = 0; v < 16; v++) isum[v] = 0;
        const uint32_t scw[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
#pragma unroll
        for (int g = 0; g < 16; g++) {
            const int h = g >> 3, qq = (g >> 1) & 3, gl = g & 1;
            const u32x2 qlp = w.ql[4 * h + 2 * (qq & 1) + gl], qhp = w.qh[2 * h + gl];
            const long bw = pack2(q6_signed4(qlp.x, qhp.x, qq >> 1, 2 * qq), q6_signed4(qlp.y, qhp.y, qq >> 1, 2 * qq));
            const long aw = pack2(a.c[2 * g], a.c[2 * g + 1]);
            v16i p = {};
            p = __builtin_amdgcn_mfma_i32_32x32x16_i8(aw, bw, p, 0, 0, 0);
            const int sg = (int)(int8_t)((scw[g >> 2] >> (8 * (g & 3))) & 0xFF);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                isum[v] = __mul24(sg, p[v]) + isum[v];   /* |p| <= 65024, |sg| <= 128: 24-bit exact */
                /* materialise the running sum here: otherwise the integer sums
                 * are reassociated across groups and all sixteen MFMA results
                 * stay live (and spill) */
                asm volatile("" : "+v"(isum[v]));
            }
        }
        /* the chain: acc = fmaf(d_w * d_a, (float)isum, acc), block order */
        if (half == 0) sda[j] = a.d;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float dwf = f16_to_f32(w.dw);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const f32x4 da4 = *(const LAS f32x4 *)(sda + 8 * q + 4 * half);
#pragma unroll
            for (int t = 0; t < 4; t++) acc[4 * q + t] = fmaf(dwf * da4[t], (float)isum[4 * q + t], acc[4 * q + t]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    /* ping-pong: the next block's loads are in flight while one computes */
    Q6Raw w0 = q6_load(unit, dp, half), w1;
    ActRaw a0 = act_load<SPLIT>(arow, nb, 0, half), a1;
    for (int b = 0; b < nb; b += 2) {
        if (b + 1 < nb) {
            w1 = q6_load(unit + (b + 1) * (TILE_ROWS * 208), dp + (b + 1) * TILE_ROWS, half);
            a1 = act_load<SPLIT>(arow, nb, b + 1, half);
        }
        block(w0, a0);
        if (b + 1 >= nb) break;
        if (b + 2 < nb) {
            w0 = q6_load(unit + (b + 2) * (TILE_ROWS * 208), dp + (b + 2) * TILE_ROWS, half);
            a0 = act_load<SPLIT>(arow, nb, b + 2, half);
        }
        block(w1, a1);
    }
}

}  // namespace tokmm

#endif
