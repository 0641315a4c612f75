/* hip_model.hip - the whole decode step on the device (tlm_hip_model_*):
 * src/lib/tlm_model.c:1058-1103 (tlm_model_step) with attention()
 * :730-763, attn_heads :683-719, the f32 KV cache :646-664, rmsnorm
 * :164-169, RoPE :721-728 with the tables of :529-545 and :1069-1073, the
 * MoE block of hip_moe.hip, the final norm + lm_head :1087-1095 and the
 * greedy sampler's argmax :1139-1146.  The model is loaded from a compiled
 * store (host_packet.cpp) into HBM: every weight packed once, every expert
 * resident.
 *
 * Numerics (against the reference's scalar C): the integer-format GEMVs,
 * router, routing, combine and quantisers are bit-exact (hip_gemv.hip,
 * hip_moe.hip); RoPE and the attention dot products, the softmax scaling and
 * the P.V sums run in the reference's order with separate roundings (one
 * thread per dot product, positions in ascending order).  What may differ in
 * the last bit: sums of squares and the softmax sum are double trees instead
 * of sequential double sums, and e^x is exp in double rounded to float; the
 * reference's greedy tokens are reproduced exactly. */
#include "tlm_hip_internal.h"
#include <hip/hip_fp16.h>
#include "tlm_hip_act.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

int tlmh_current_device(void);

namespace {

constexpr int NT = 256;

/* ---- block reductions ------------------------------------------------------ */
__device__ double block_sum_f64(double v, double *red) {
    v = wave_sum_f64(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

/* ---- embedding row (tlm_dequantize_row, src/lib/tlm_quant.c:629-660) -------- */
/* The step's position and token live in device memory (st[0] = pos, seq[pos]
 * = the token), so one captured graph serves every position. */
__global__ __launch_bounds__(NT) void k_embed(const uint8_t *__restrict__ embd, size_t row_bytes, int dt,
                                              const int32_t *__restrict__ seq, const int32_t *__restrict__ st, int D,
                                              float *__restrict__ h) {
    const uint8_t *row = embd + (size_t)seq[st[0]] * row_bytes;
    for (int i = threadIdx.x + blockIdx.x * blockDim.x; i < D; i += blockDim.x * gridDim.x) {
        if (dt == DT_F32) {
            h[i] = ((const float *)row)[i];
        } else {   /* Q8_0: y = f16(d) * (float)q */
            const uint8_t *b = row + (size_t)(i >> 5) * 34;
            const float dd = f16_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
            h[i] = dd * (float)(int8_t)b[2 + (i & 31)];
        }
    }
}

/* ---- attention for one query head, everything it needs fused ---------------
 * (src/lib/tlm_model.c:743-756 with attn_heads :683-719): the head's q-norm
 * and RoPE, the k-norm and RoPE of its key head and the KV append (written by
 * the first query head of each key head; the others take the new key and
 * value from their own copy), scores, softmax and P.V in the reference's
 * order, the output stored to att.  Each score is one thread's dot product in
 * ascending i, each output element one thread's sum over positions in
 * ascending t.
 *
 * Cache layout (per layer and key head): keys dimension-major, K[i][t] at
 * i * max_ctx + t, so that the lanes of a score pass (one position each)
 * read consecutive words for every i; values position-major, V[t][i], so
 * that a chunk of positions is one contiguous run.
 *
 * Latency, not bandwidth, sets this kernel's time (one group per head), so
 * it is arranged around the memory counter, which retires loads in issue
 * order: the loads go out unconditionally (indices clamped) in the order the
 * values are consumed - head vectors, norm weights and RoPE factors and the
 * first pass's key columns per thread at entry (HD <= 128; later passes load
 * theirs at once too), the first two V chunks (ATT_VF floats each) once the
 * scores are done - and no global store precedes a barrier (a barrier waits
 * for the group's stores): the KV append goes last.  The
 * probabilities stay in LDS (dynamic, max_ctx floats) when SPL, else in the
 * head's global scratch row; they are scaled by 1/sum in place (the
 * reference's p = s[t] * inv).  P.V is a pipeline inside the group: waves
 * 2-3 hold V chunks two ahead in registers and store each chunk to one of
 * two LDS buffers as the products p_t * v_t[i]; waves 0-1 (one output
 * element per lane) sum the previous chunk meanwhile, 16 positions per group
 * of LDS reads, the last group of a chunk read whole (a chunk holds a
 * multiple of 16 positions) and its adds masked.  q_norm / k_norm are read
 * only when has_qn / has_kn. */
constexpr int ATT_VF = 8192;                 /* floats of V per LDS chunk (32 KB) */
constexpr int ATT_PF = ATT_VF / 4 / 128;     /* 16-byte V loads per producer thread per chunk */
constexpr int ATT_LDS_POS = 4096;            /* contexts whose probabilities fit in LDS */
constexpr int ATT_PU = 16;                   /* positions per group in the ordered sums */
constexpr int ATT_SPLIT_MIN = 2 * NT;         /* longest context scored inside the fused launch */

/* max over non-NaN values (a NaN never compares greater), -inf if none */
__device__ float block_max_dpp(float v, float *red) {
    v = wave_max_f32(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float m = -INFINITY;
    for (int i = 0; i < nw; i++) m = red[i] > m ? red[i] : m;
    return m;
}

/* Scores of one query head over one slice of NT positions (grid: heads x
 * max_ctx / NT slices; slices past the current position return): the head's
 * q (wave 0) and the new key (wave 1) normalised and rotated exactly as the
 * fused launch does it, then one position per thread - the dot in ascending
 * i, scaled after the dot - into the head's score row, and the slice's
 * maximum (non-NaN values, -inf if none) into smax[h * nslice + slice]. */
template <int HD>
__global__ __launch_bounds__(NT) void k_attn_scores(const float *__restrict__ q, const float *__restrict__ kx,
                                                    const float *__restrict__ q_norm, const float *__restrict__ k_norm,
                                                    int has_qn, int has_kn, const float *__restrict__ cs_all,
                                                    const float *__restrict__ sn_all, const float *__restrict__ kc,
                                                    float *__restrict__ scores, float *__restrict__ smax, int H,
                                                    int KV, int max_ctx, const int32_t *__restrict__ st, float eps) {
    constexpr int HALF = HD / 2, H4 = HD / 4;
    constexpr int KE = (HD + 63) / 64, KH = (HALF + 63) / 64;
    constexpr bool KPRE = HD <= 128;
    __shared__ __align__(16) float s_q[HD], s_k[HD];
    __shared__ float s_redf[NT / 64];
    const int pos = st[0], T = pos + 1;
    const int p0 = (int)blockIdx.y * NT;
    if (p0 >= T) return;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = h / (H / KV);
    const float *K = kc + (size_t)kvh * max_ctx * HD;
    const int t = p0 + tid;
    const float *hv = wave == 1 ? kx + (size_t)kvh * HD : q + (size_t)h * HD;
    const float *nwp = wave == 1 ? k_norm : q_norm;
    float e[KE], nw[KE], cv[KH], sv[KH];
#pragma unroll
    for (int k = 0; k < KE; k++) e[k] = hv[min(lane + 64 * k, HD - 1)];
#pragma unroll
    for (int k = 0; k < KE; k++) nw[k] = nwp[min(lane + 64 * k, HD - 1)];
#pragma unroll
    for (int k = 0; k < KH; k++) {
        cv[k] = cs_all[(size_t)pos * HALF + min(lane + 64 * k, HALF - 1)];
        sv[k] = sn_all[(size_t)pos * HALF + min(lane + 64 * k, HALF - 1)];
    }
    float kr[KPRE ? HD : 1];
    if constexpr (KPRE) {   /* this slice's key columns, all at once (rows clamped to pos) */
        const float *kt = K + min(t, pos);
#pragma unroll
        for (int i = 0; i < HD; i++) kr[i] = kt[(size_t)i * max_ctx];
    }
    if (wave < 2) {   /* norm (tlm_model.c:743-746) and RoPE (rope(), :721-728: pairs (j, j + HD/2)) */
        float *v = wave == 0 ? s_q : s_k;
        if (wave == 0 ? has_qn : has_kn) {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < KE; k++)
                if (lane + 64 * k < HD) ss += (double)e[k] * (double)e[k];
            ss = wave_sum_f64(ss);
            const float r = 1.0f / sqrtf((float)(ss / (double)HD) + eps);
#pragma unroll
            for (int k = 0; k < KE; k++) e[k] = e[k] * r * nw[k];
        }
#pragma unroll
        for (int k = 0; k < KE; k++)
            if (lane + 64 * k < HD) v[lane + 64 * k] = e[k];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int k = 0; k < KH; k++) {
            const int j = lane + 64 * k;
            if (j < HALF) {
                const float a = v[j], c = v[j + HALF];
                v[j] = a * cv[k] - c * sv[k];
                v[j + HALF] = c * cv[k] + a * sv[k];
            }
        }
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    const f32x4 *q4 = (const f32x4 *)s_q;
    float d = 0.0f, mx = -INFINITY;
    if (KPRE) {
        if (t == pos) {   /* the new key, from this group's copy */
#pragma unroll
            for (int i4 = 0; i4 < H4; i4++) {
                const f32x4 k4 = ((const f32x4 *)s_k)[i4];
                kr[4 * i4] = k4.x;
                kr[4 * i4 + 1] = k4.y;
                kr[4 * i4 + 2] = k4.z;
                kr[4 * i4 + 3] = k4.w;
            }
        }
#pragma unroll
        for (int c = 0; c < HD / 16; c++) {   /* q in batches of 16 */
            f32x4 qb[4];
#pragma unroll
            for (int u = 0; u < 4; u++) qb[u] = q4[4 * c + u];
#pragma unroll
            for (int u = 0; u < 16; u++) d += qb[u / 4][u % 4] * kr[16 * c + u];
        }
    } else if (t == pos) {
#pragma unroll
        for (int i = 0; i < HD; i++) d += s_q[i] * s_k[i];
    } else if (t < T) {
        const float *kt = K + t;
#pragma unroll 16
        for (int i = 0; i < HD; i++) d += s_q[i] * kt[(size_t)i * max_ctx];
    }
    if (t < T) {
        d *= scale;
        scores[(size_t)h * max_ctx + t] = d;
        if (d > mx) mx = d;
    }
    mx = block_max_dpp(mx, s_redf);
    if (tid == 0) smax[(size_t)h * gridDim.y + blockIdx.y] = mx;
}

template <int HD, bool SPL, bool SPLIT>
__global__ __launch_bounds__(NT) void k_attn_fused(const float *__restrict__ q, const float *__restrict__ kx,
                                                   const float *__restrict__ vx, const float *__restrict__ q_norm,
                                                   const float *__restrict__ k_norm, int has_qn, int has_kn,
                                                   const float *__restrict__ cs_all, const float *__restrict__ sn_all,
                                                   float *__restrict__ kc, float *__restrict__ vc,
                                                   float *__restrict__ scores, const float *__restrict__ smax,
                                                   float *__restrict__ att, int H, int KV, int max_ctx,
                                                   const int32_t *__restrict__ st, float eps) {
    constexpr int HALF = HD / 2, H4 = HD / 4;
    constexpr int VC = (ATT_VF / HD) & ~(ATT_PU - 1);   /* V positions per chunk */
    constexpr int KE = (HD + 63) / 64, KH = (HALF + 63) / 64;     /* elements / pairs per lane */
    constexpr bool KPRE = HD <= 128 && !SPLIT;
    extern __shared__ __align__(16) float s_dyn[];
    __shared__ __align__(16) float s_q[HD], s_k[HD], s_vn[HD];
    __shared__ __align__(16) float s_v[2 * ATT_VF];
    __shared__ double s_red[NT / 64];
    __shared__ float s_redf[NT / 64];
    const int pos = st[0], T = pos + 1;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = h / (H / KV);
    const float *K = kc + (size_t)kvh * max_ctx * HD, *V = vc + (size_t)kvh * max_ctx * HD;

    /* 1. wave 0: the query head, wave 1: the key head, wave 2: the value
     *    head (the others load the query head too and drop it) */
    const float *hv = wave == 1 ? kx + (size_t)kvh * HD : wave == 2 ? vx + (size_t)kvh * HD : q + (size_t)h * HD;
    const float *nwp = wave == 1 ? k_norm : q_norm;
    float e[KE], nw[KE], cv[KH], sv[KH];
#pragma unroll
    for (int k = 0; k < KE; k++) e[k] = hv[min(lane + 64 * k, HD - 1)];
#pragma unroll
    for (int k = 0; k < KE; k++) nw[k] = nwp[min(lane + 64 * k, HD - 1)];
#pragma unroll
    for (int k = 0; k < KH; k++) {
        cv[k] = cs_all[(size_t)pos * HALF + min(lane + 64 * k, HALF - 1)];
        sv[k] = sn_all[(size_t)pos * HALF + min(lane + 64 * k, HALF - 1)];
    }
    /* 2. without the split launch: the first pass's key columns */
    float kr[KPRE ? HD : 1];
    if constexpr (KPRE) {
        const float *kt = K + min(tid, pos);
#pragma unroll
        for (int i = 0; i < HD; i++) kr[i] = kt[(size_t)i * max_ctx];
    }
    /* V chunks (VC positions): the producer threads (tid >= 128, waves 2-3)
     * hold two in registers, loaded two chunks ahead */
    const int ptid = tid - 128, nch = (T + VC - 1) / VC;
    f32x4 va[ATT_PF], vb[ATT_PF];
    auto vload = [&](int c, f32x4 (&pv)[ATT_PF]) {
        const int t0 = c * VC;
        const int n4 = (T - t0 < VC ? T - t0 : VC) * H4;
        const f32x4 *src = (const f32x4 *)(V + (size_t)t0 * HD);
#pragma unroll
        for (int j = 0; j < ATT_PF; j++) pv[j] = src[min(ptid + 128 * j, n4 - 1)];
    };

    /* norm (tlm_model.c:743-746) and RoPE (rope(), :721-728: pairs (j, j + HD/2)) */
    if (wave < 3) {
        float *v = wave == 0 ? s_q : wave == 1 ? s_k : s_vn;
        if (wave < 2 && (wave == 0 ? has_qn : has_kn)) {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < KE; k++)
                if (lane + 64 * k < HD) ss += (double)e[k] * (double)e[k];
            ss = wave_sum_f64(ss);
            const float r = 1.0f / sqrtf((float)(ss / (double)HD) + eps);
#pragma unroll
            for (int k = 0; k < KE; k++) e[k] = e[k] * r * nw[k];
        }
#pragma unroll
        for (int k = 0; k < KE; k++)
            if (lane + 64 * k < HD) v[lane + 64 * k] = e[k];
        if (wave < 2) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int k = 0; k < KH; k++) {
                const int j = lane + 64 * k;
                if (j < HALF) {
                    const float a = v[j], c = v[j + HALF];
                    v[j] = a * cv[k] - c * sv[k];
                    v[j + HALF] = c * cv[k] + a * sv[k];
                }
            }
        }
    }
    __syncthreads();

    /* scores (scale after the dot, before the max): from the split launch
     * (the head's row and its slices' maxima), or here, a pass of NT
     * positions at a time */
    float *sp;
    if constexpr (SPL) sp = s_dyn;
    else sp = scores + (size_t)h * max_ctx;
    const float *sg = SPLIT ? (const float *)(scores + (size_t)h * max_ctx) : (const float *)sp;
    float mx = -INFINITY;   /* the maximum of non-NaN values, -inf if none */
    if constexpr (SPLIT) {
        if (tid >= 128) {   /* the first V chunks go out before the maximum, exp and sum */
            vload(0, va);
            if (nch > 1) vload(1, vb);
        }
        const int nslice = (max_ctx + NT - 1) / NT, nsl = (T + NT - 1) / NT;
        for (int i = 0; i < nsl; i++) {
            const float m = smax[(size_t)h * nslice + i];
            mx = m > mx ? m : mx;
        }
    } else {
        const float scale = 1.0f / sqrtf((float)HD);
        const f32x4 *q4 = (const f32x4 *)s_q;
        for (int p0 = 0; p0 < T; p0 += NT) {   /* passes of NT positions, uniform over the group */
            const int t = p0 + tid;
            float d = 0.0f;
            if (KPRE) {
                if (p0 > 0) {   /* this pass's key columns, all at once (rows clamped to pos) */
                    const float *kt = K + min(t, pos);
#pragma unroll
                    for (int i = 0; i < HD; i++) kr[i] = kt[(size_t)i * max_ctx];
                }
                if (t == pos) {   /* the new key, from this group's copy */
#pragma unroll
                    for (int i4 = 0; i4 < H4; i4++) {
                        const f32x4 k4 = ((const f32x4 *)s_k)[i4];
                        kr[4 * i4] = k4.x;
                        kr[4 * i4 + 1] = k4.y;
                        kr[4 * i4 + 2] = k4.z;
                        kr[4 * i4 + 3] = k4.w;
                    }
                }
#pragma unroll
                for (int c = 0; c < HD / 16; c++) {   /* q in batches of 16 */
                    f32x4 qb[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) qb[u] = q4[4 * c + u];
#pragma unroll
                    for (int u = 0; u < 16; u++) d += qb[u / 4][u % 4] * kr[16 * c + u];
                }
            } else if (t == pos) {
#pragma unroll
                for (int i = 0; i < HD; i++) d += s_q[i] * s_k[i];
            } else if (t < T) {
                const float *kt = K + t;
#pragma unroll 16
                for (int i = 0; i < HD; i++) d += s_q[i] * kt[(size_t)i * max_ctx];
            }
            if (t < T) {
                d *= scale;
                sp[t] = d;
                if (d > mx) mx = d;
            }
        }
        if (tid >= 128) {   /* the key registers are free now; max, exp and sum cover the latency */
            vload(0, va);
            if (nch > 1) vload(1, vb);
        }
        mx = block_max_dpp(mx, s_redf);
    }
    double sum = 0.0;
    for (int t = tid; t < T; t += NT) {
        const float p = exp_rn(sg[t] - mx);
        sp[t] = p;
        sum += (double)p;
    }
    sum = block_sum_f64(sum, s_red);
    const float inv = (float)(1.0 / sum);
    for (int t = tid; t < T; t += NT) sp[t] = sp[t] * inv;
    __syncthreads();   /* every p stored before the producers read them */

    /* P.V, chunk by chunk, as a pipeline inside the group: the producers
     * store chunk c + 1 to LDS as the products c = p_t * v_t[i] (the
     * reference's product, bit for bit) while the consumers (tid < 128, lane
     * = output element i, and i + 128 when HD = 256) run the ordered sums over
     * chunk c - one add per position; two LDS buffers, one barrier per chunk.
     * A producer reads its chunk's probabilities at once (one wait), and the
     * new row only in the last chunk. */
    constexpr int CD = (HD + 127) / 128;
    float o[CD];
#pragma unroll
    for (int m = 0; m < CD; m++) o[m] = 0.0f;
    float *buf0 = s_v, *buf1 = s_v + ATT_VF;
    auto produce = [&](int c, const f32x4 (&pv)[ATT_PF], float *buf) {
        const int t0 = c * VC, tn = T - t0 < VC ? T - t0 : VC;
        float pt[ATT_PF];
#pragma unroll
        for (int j = 0; j < ATT_PF; j++) {
            const int tl = (ptid + 128 * j) / H4;
            pt[j] = sp[t0 + min(tl, tn - 1)];
        }
        if (c == nch - 1) {   /* the chunk holding row pos: this group's copy, and nothing past T */
#pragma unroll
            for (int j = 0; j < ATT_PF; j++) {
                const int e4 = ptid + 128 * j, tl = e4 / H4;
                f32x4 v4 = t0 + tl == pos ? ((const f32x4 *)s_vn)[e4 % H4] : pv[j];
                const float q = tl < tn ? pt[j] : 0.0f;
                f32x4 cc;
#pragma unroll
                for (int k = 0; k < 4; k++) cc[k] = q * v4[k];
                ((f32x4 *)buf)[e4] = cc;
            }
        } else {
#pragma unroll
            for (int j = 0; j < ATT_PF; j++) {
                f32x4 cc;
#pragma unroll
                for (int k = 0; k < 4; k++) cc[k] = pt[j] * pv[j][k];
                ((f32x4 *)buf)[ptid + 128 * j] = cc;
            }
        }
    };
    auto consume = [&](int c, const float *buf) {
        const int t0 = c * VC, tn = T - t0 < VC ? T - t0 : VC;
        const int ng = (tn + ATT_PU - 1) / ATT_PU;
        /* group g + 1's products load while group g's ordered sums run;
         * reads past the chunk's last position stay inside the buffer and
         * are masked in the last group */
        float ra[CD][ATT_PU], rb[CD][ATT_PU];
        auto ld = [&](int g, float (&r)[CD][ATT_PU]) {
#pragma unroll
            for (int m = 0; m < CD; m++)
#pragma unroll
                for (int u = 0; u < ATT_PU; u++) r[m][u] = buf[(g * ATT_PU + u) * HD + min(tid + 128 * m, HD - 1)];
        };
        auto add = [&](int g, const float (&r)[CD][ATT_PU]) {
            if (g + 1 < ng) {
#pragma unroll
                for (int u = 0; u < ATT_PU; u++)
#pragma unroll
                    for (int m = 0; m < CD; m++) o[m] += r[m][u];
            } else {
                const int lim = tn - g * ATT_PU;
#pragma unroll
                for (int u = 0; u < ATT_PU; u++)
#pragma unroll
                    for (int m = 0; m < CD; m++) {
                        const float a = o[m] + r[m][u];
                        o[m] = u < lim ? a : o[m];
                    }
            }
        };
        ld(0, ra);
#pragma unroll 1
        for (int g = 0; g < ng; g += 2) {
            if (g + 1 < ng) ld(g + 1, rb);
            add(g, ra);
            if (g + 1 >= ng) break;
            if (g + 2 < ng) ld(g + 2, ra);
            add(g + 1, rb);
        }
    };
    if (tid >= 128) {
        produce(0, va, buf0);
        if (nch > 2) vload(2, va);
    }
    __syncthreads();
    for (int c = 0; c < nch; c += 2) {   /* uniform over the group; even chunks in va / buf0, odd in vb / buf1 */
        if (tid < 128) consume(c, buf0);
        else if (c + 1 < nch) {
            produce(c + 1, vb, buf1);
            if (c + 3 < nch) vload(c + 3, vb);
        }
        __syncthreads();
        if (c + 1 >= nch) break;
        if (tid < 128) consume(c + 1, buf1);
        else if (c + 2 < nch) {
            produce(c + 2, va, buf0);
            if (c + 4 < nch) vload(c + 4, va);
        }
        __syncthreads();
    }
#pragma unroll
    for (int m = 0; m < CD; m++)
        if (tid < 128 && tid + 128 * m < HD) att[(size_t)h * HD + tid + 128 * m] = o[m];
    if (h % (H / KV) == 0)   /* the KV append, after the last barrier */
        for (int i = tid; i < HD; i += NT) {
            kc[((size_t)kvh * HD + i) * max_ctx + pos] = s_k[i];
            vc[((size_t)kvh * max_ctx + pos) * HD + i] = s_vn[i];
        }
}

/* host: launch for the model's head width (a multiple of 32, at most 256) */
int launch_attn(int hd, int H, int KV, int max_ctx, const float *q, const float *kx, const float *vx,
                const float *q_norm, const float *k_norm, const float *cs, const float *sn, float *kc, float *vc,
                float *scores, float *smax, float *att, const int32_t *st, float eps, hipStream_t s) {
    const bool spl = max_ctx <= ATT_LDS_POS;
    const int has_qn = q_norm != nullptr, has_kn = k_norm != nullptr;
    if (!q_norm) q_norm = q;   /* read (clamped) and dropped */
    if (!k_norm) k_norm = q;
    const size_t dyn = spl ? (size_t)(max_ctx + ATT_PU) * 4 : 0;   /* the last group reads whole */
    const unsigned nslice = (unsigned)((max_ctx + NT - 1) / NT);
    /* contexts of at most ATT_SPLIT_MIN positions score inside the fused launch (one or two
     * passes); longer ones in the split launch, a group per (head, NT positions) */
    const bool split = max_ctx > ATT_SPLIT_MIN;
#define TLM_ATT(W)                                                                                                \
    case W:                                                                                                       \
        if (!split)                                                                                               \
            hipLaunchKernelGGL((k_attn_fused<W, true, false>), dim3(H), dim3(NT), dyn, s, q, kx, vx, q_norm,      \
                               k_norm, has_qn, has_kn, cs, sn, kc, vc, scores, smax, att, H, KV, max_ctx, st,     \
                               eps);                                                                              \
        else {                                                                                                    \
            hipLaunchKernelGGL((k_attn_scores<W>), dim3(H, nslice), dim3(NT), 0, s, q, kx, q_norm, k_norm,       \
                               has_qn, has_kn, cs, sn, kc, scores, smax, H, KV, max_ctx, st, eps);                \
            if (spl)                                                                                              \
                hipLaunchKernelGGL((k_attn_fused<W, true, true>), dim3(H), dim3(NT), dyn, s, q, kx, vx, q_norm,   \
                                   k_norm, has_qn, has_kn, cs, sn, kc, vc, scores, smax, att, H, KV, max_ctx, st, \
                                   eps);                                                                          \
            else                                                                                                  \
                hipLaunchKernelGGL((k_attn_fused<W, false, true>), dim3(H), dim3(NT), 0, s, q, kx, vx, q_norm,   \
                                   k_norm, has_qn, has_kn, cs, sn, kc, vc, scores, smax, att, H, KV, max_ctx, st, \
                                   eps);                                                                          \
        }                                                                                                         \
        break;
    switch (hd) {
        TLM_ATT(32) TLM_ATT(64) TLM_ATT(96) TLM_ATT(128) TLM_ATT(160) TLM_ATT(192) TLM_ATT(224) TLM_ATT(256)
    default: return tlmh_seterr(TLM_HIP_EUNSUP, "model: head width %d", hd);
    }
#undef TLM_ATT
    return tlmh_check(hipGetLastError(), "model: attention");
}

/* end of a step: with the lm_head tiles' greedy keys (argmax_key of their
 * rows), the maximum decodes to the reference's argmax (src/lib/tlm_model.c:
 * 1139-1146: first maximum, NaN skipped, 0 if none), the next step's token,
 * stored at seq[pos + 1]; the position advances. */
__global__ __launch_bounds__(1024) void k_advance(int32_t *st, int32_t *seq, const unsigned long long *keys,
                                                  int nkeys) {
    __shared__ unsigned long long red[16];
    const int pos = st[0];
    if (keys) {
        unsigned long long k = 0ull;
        for (int i = threadIdx.x; i < nkeys; i += blockDim.x) k = keys[i] > k ? keys[i] : k;
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(k, o, 64);
            k = other > k ? other : k;
        }
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < (int)(blockDim.x >> 6); w++) k = red[w] > k ? red[w] : k;
            seq[pos + 1] = argmax_index(k);
        }
    }
    if (threadIdx.x == 0) st[0] = pos + 1;
}

struct DevMat {
    int dt = -1;
    int64_t rows = 0, n = 0;
    void *p = nullptr;   /* packed */
};

struct Layer {
    const float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    DevMat q, k, v, o;
    tlm_hip_moe_desc moe{};
};

}  // namespace

struct tlm_hip_model {
    tlm_hip_model_geom g{};
    int max_ctx = 0, kv_len = 0;
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;
    std::vector<Layer> L;
    const uint8_t *embd = nullptr;
    int embd_dt = 0;
    size_t embd_row = 0;
    const float *out_norm = nullptr;
    DevMat lm_head;
    float *kc = nullptr, *vc = nullptr, *cs = nullptr, *sn = nullptr, *scores = nullptr, *smax = nullptr;
    float *h = nullptr, *q = nullptr, *kx = nullptr, *vx = nullptr, *att = nullptr;
    float *logits = nullptr;
    uint8_t *moe_ws = nullptr;
    int32_t *st = nullptr, *seq = nullptr, *ids = nullptr;   /* st[0] = position; seq[max_ctx + 1] tokens */
    unsigned long long *keys = nullptr;                      /* greedy key per lm_head tile */
    float *w = nullptr;
    int32_t *host_tok = nullptr;   /* pinned */
    hipGraphExec_t graph[2] = {nullptr, nullptr};   /* step without / with logits, captured at first use */
    bool graph_failed[2] = {false, false};

    void *dalloc(size_t n) {
        void *p = nullptr;
        if (hipMalloc(&p, n ? n : 16) != hipSuccess) return nullptr;
        allocs.push_back(p);
        return p;
    }
    ~tlm_hip_model() {
        if (stream) (void)hipStreamSynchronize(stream);
        for (hipGraphExec_t g : graph)
            if (g) (void)hipGraphExecDestroy(g);
        for (void *p : allocs) (void)hipFree(p);
        if (host_tok) (void)hipHostFree(host_tok);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

int dev_upload(tlm_hip_model *M, const void *src, size_t n, void **out) {
    *out = M->dalloc(n);
    if (!*out) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory (%zu bytes)", n);
    return tlmh_check(hipMemcpy(*out, src, n, hipMemcpyHostToDevice), "model: upload");
}

/* rows x n matrix of a payload in the reference's row layout -> packed on device */
int dev_matrix(tlm_hip_model *M, int dt, const uint8_t *rows_src, int64_t rows, int64_t n, DevMat *out) {
    const int bv = dt_block_values(dt);
    if (bv == 0 || !dt_int_ok(dt) || dt == DT_Q8_K || n % bv)
        return tlmh_seterr(TLM_HIP_EUNSUP, "model: matrix dtype %d, %lld columns", dt, (long long)n);
    const size_t rb = (size_t)(n / bv) * dt_block_bytes(dt), raw = rb * (size_t)rows;
    void *tmp = nullptr;
    if (hipMalloc(&tmp, raw) != hipSuccess) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory");
    int rc = tlmh_check(hipMemcpy(tmp, rows_src, raw, hipMemcpyHostToDevice), "model: upload");
    out->dt = dt;
    out->rows = rows;
    out->n = n;
    out->p = rc ? nullptr : M->dalloc(packed_bytes(dt, rows, n));
    if (!rc && !out->p) rc = tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory");
    if (!rc) rc = launch_pack(dt, tmp, rb, rows, n, out->p, M->stream);
    if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model: pack");
    (void)hipFree(tmp);
    return rc;
}

struct Packet {
    std::vector<uint8_t> buf;
    uint64_t off = 0, len = 0;
    const uint8_t *payload() const { return buf.data() + off; }
};

int read_packet(tlm_hip_manifest *m, int type, int layer, uint32_t id, Packet &p) {
    const tlm_hip_packet_loc *loc = tlm_hip_manifest_find(m, type, layer, id);
    if (!loc) return tlmh_seterr(TLM_HIP_ENOTFOUND, "model: no packet type %d layer %d id %u", type, layer, id);
    p.buf.resize(loc->total_len);
    return tlm_hip_packet_read(m, loc, p.buf.data(), &p.off, &p.len);
}

/* tensor `name` of a directory payload as an f32 vector on device (NULL if
 * absent and not required) - dir_vec, src/lib/tlm_model.c:274-292 */
int dev_vec(tlm_hip_model *M, const Packet &pk, const char *name, int64_t n, bool required, const float **out) {
    *out = nullptr;
    tlm_hip_tensor_ref t;
    int rc = tlm_hip_dir_find(pk.payload(), pk.len, name, &t);
    if (rc == TLM_HIP_ENOTFOUND)
        return required ? tlmh_seterr(TLM_HIP_ENOTFOUND, "model: tensor '%s' missing", name) : TLM_HIP_OK;
    if (rc) return rc;
    if (t.dtype != DT_F32 || t.shape[0] * t.shape[1] != (uint64_t)n || t.nbytes != (uint64_t)n * 4)
        return tlmh_seterr(TLM_HIP_EUNSUP, "model: tensor '%s' is not an f32 vector of %lld", name, (long long)n);
    void *p;
    if ((rc = dev_upload(M, pk.payload() + t.offset, (size_t)t.nbytes, &p))) return rc;
    *out = (const float *)p;
    return TLM_HIP_OK;
}

/* dir_mat, src/lib/tlm_model.c:246-272 */
int dir_mat(tlm_hip_model *M, const Packet &pk, const char *name, int64_t rows, int64_t cols, DevMat *out) {
    tlm_hip_tensor_ref t;
    int rc = tlm_hip_dir_find(pk.payload(), pk.len, name, &t);
    if (rc == TLM_HIP_ENOTFOUND) return tlmh_seterr(TLM_HIP_ENOTFOUND, "model: tensor '%s' missing", name);
    if (rc) return rc;
    const int dt = (int)t.dtype, bv = dt_block_values(dt);
    if ((int64_t)t.shape[0] != rows || (int64_t)t.shape[1] != cols || bv == 0 || cols % bv)
        return tlmh_seterr(TLM_HIP_EFORMAT, "model: tensor '%s' shape [%llu, %llu], expected [%lld, %lld]", name,
                           (unsigned long long)t.shape[0], (unsigned long long)t.shape[1], (long long)rows,
                           (long long)cols);
    if (t.nbytes != (uint64_t)rows * (uint64_t)(cols / bv) * (uint64_t)dt_block_bytes(dt))
        return tlmh_seterr(TLM_HIP_EFORMAT, "model: tensor '%s' byte count", name);
    return dev_matrix(M, dt, pk.payload() + t.offset, rows, cols, out);
}

/* tlm_yarn_transform, src/lib/tlm_model.c:453-484 (HF YaRN, f32 ramp) */
int yarn(std::vector<float> &inv_freq, uint32_t head_dim, double theta, double factor, double beta_fast,
         double beta_slow, uint32_t orig_len, bool truncate, float *attn_factor) {
    const int half = (int)head_dim / 2;
    if (head_dim < 2 || (head_dim & 1) || !(theta > 0.0) || !(factor > 0.0) || !(beta_fast > 0.0) ||
        beta_fast < beta_slow || orig_len == 0)
        return tlmh_seterr(TLM_HIP_EINVAL, "model: invalid rope scaling parameters");
    const double two_pi = 6.283185307179586;
    double low = (double)head_dim * log((double)orig_len / (beta_fast * two_pi)) / (2.0 * log(theta));
    double high = (double)head_dim * log((double)orig_len / (beta_slow * two_pi)) / (2.0 * log(theta));
    if (truncate) {
        low = floor(low);
        high = ceil(high);
    }
    if (low < 0.0) low = 0.0;
    if (high > (double)head_dim - 1.0) high = (double)head_dim - 1.0;
    if (low == high) high += 0.001;
    const double af = factor > 1.0 ? 0.1 * log(factor) + 1.0 : 1.0;
    for (int j = 0; j < half; j++) {
        const float extrap = inv_freq[j];
        const float pos_freq = 1.0f / extrap;
        const float interp = 1.0f / ((float)factor * pos_freq);
        float ramp = ((float)j - (float)low) / (float)(high - low);
        if (ramp < 0.0f) ramp = 0.0f;
        if (ramp > 1.0f) ramp = 1.0f;
        inv_freq[j] = interp * ramp + extrap * (1.0f - ramp);
    }
    *attn_factor = (float)af;
    return TLM_HIP_OK;
}

/* geometry checks and defaults, context, stream, RoPE tables (M->g set) */
int prepare(tlm_hip_model *M, const tlm_hip_model_opts *o) {
    tlm_hip_model_geom &g = M->g;
    /* tlm_model.c:490-498 */
    if (g.n_layers == 0 || g.d_model == 0 || g.n_heads == 0 || g.n_kv_heads == 0 || g.head_dim == 0 ||
        (g.head_dim & 1) || g.n_heads % g.n_kv_heads || g.vocab == 0 || g.top_k > g.n_experts ||
        (g.n_experts > 0 && g.top_k == 0) || g.router > 2 || g.rope_scale > 2)
        return tlmh_seterr(TLM_HIP_EFORMAT, "model: unsupported geometry");
    if (g.n_experts == 0 || g.head_dim > 256 || g.head_dim % 32 || g.top_k > 32)
        return tlmh_seterr(TLM_HIP_EUNSUP, "model: needs routed experts (top_k <= 32) and head_dim a multiple of 32 "
                           "up to 256");
    if (!(g.routed_scale > 0.0f)) g.routed_scale = 1.0f;   /* tlm_model.c:503-505 */
    if (!(g.norm_eps > 0.0f)) g.norm_eps = 1e-6f;
    if (!(g.rope_theta > 0.0f)) g.rope_theta = 10000.0f;
    /* tlm_kv_new, tlm_model.c:646-650 */
    int max_ctx = o && o->max_ctx > 0 ? o->max_ctx : 0;
    if (max_ctx <= 0) max_ctx = g.max_ctx > 0 ? (int)g.max_ctx : 4096;
    if (g.max_ctx > 0 && max_ctx > (int)g.max_ctx) max_ctx = (int)g.max_ctx;
    M->max_ctx = max_ctx;
    M->graph_failed[0] = M->graph_failed[1] = o && o->eager;
    const int64_t hd = g.head_dim;

    int rc = tlmh_check(hipStreamCreateWithFlags(&M->stream, hipStreamNonBlocking), "model: stream");
    if (rc) return rc;
    /* RoPE tables for every position, in double as tlm_model.c:535, 1069-1073 */
    {
        const int half = (int)hd / 2;
        std::vector<float> inv(half);
        for (int j = 0; j < half; j++) inv[j] = (float)pow((double)g.rope_theta, -2.0 * (double)j / (double)hd);
        float attn_scale = 1.0f;
        if (g.rope_scale != 0 &&
            (rc = yarn(inv, g.head_dim, g.rope_theta, g.rope_factor, g.rope_beta_fast, g.rope_beta_slow,
                       g.rope_orig_len, g.rope_scale == 1, &attn_scale)))
            return rc;
        std::vector<float> cs((size_t)max_ctx * half), sn((size_t)max_ctx * half);
        for (int p = 0; p < max_ctx; p++)
            for (int j = 0; j < half; j++) {
                const double a = (double)p * (double)inv[j];
                cs[(size_t)p * half + j] = (float)cos(a) * attn_scale;
                sn[(size_t)p * half + j] = (float)sin(a) * attn_scale;
            }
        void *a, *b;
        if ((rc = dev_upload(M, cs.data(), cs.size() * 4, &a)) || (rc = dev_upload(M, sn.data(), sn.size() * 4, &b)))
            return rc;
        M->cs = (float *)a;
        M->sn = (float *)b;
    }
    M->L.resize(g.n_layers);
    return TLM_HIP_OK;
}

/* KV cache and the step's device state (alloc_scratch, tlm_model.c:402-446) */
int finish(tlm_hip_model *M) {
    const tlm_hip_model_geom &g = M->g;
    const int64_t D = g.d_model, hd = g.head_dim, H = g.n_heads, KV = g.n_kv_heads;
    const int max_ctx = M->max_ctx;
    int rc;
    const size_t per = (size_t)g.n_layers * KV * (size_t)max_ctx * hd;
    M->kc = (float *)M->dalloc(per * 4);
    M->vc = (float *)M->dalloc(per * 4);
    M->scores = (float *)M->dalloc(((size_t)H * max_ctx + 16) * 4);   /* attention reads a row in groups of 16 */
    M->smax = (float *)M->dalloc((size_t)H * ((max_ctx + NT - 1) / NT) * 4);   /* per (head, slice) score maxima */
    M->h = (float *)M->dalloc((size_t)D * 4);
    M->q = (float *)M->dalloc((size_t)H * hd * 4);
    M->kx = (float *)M->dalloc((size_t)KV * hd * 4);
    M->vx = (float *)M->dalloc((size_t)KV * hd * 4);
    M->att = (float *)M->dalloc((size_t)H * hd * 4);
    M->logits = (float *)M->dalloc((size_t)g.vocab * 4);
    size_t ws = 0;
    for (const Layer &Ly : M->L) ws = std::max(ws, tlm_hip_moe_workspace_bytes(&Ly.moe));
    M->moe_ws = (uint8_t *)M->dalloc(ws + 256);
    M->st = (int32_t *)M->dalloc(16);
    M->seq = (int32_t *)M->dalloc(((size_t)max_ctx + 1) * 4);
    M->ids = (int32_t *)M->dalloc(32 * 4);
    M->w = (float *)M->dalloc(32 * 4);
    M->keys = (unsigned long long *)M->dalloc(((size_t)g.vocab + TILE_ROWS - 1) / TILE_ROWS * 8);
    for (void *p : {(void *)M->kc, (void *)M->vc, (void *)M->scores, (void *)M->smax, (void *)M->h,
                    (void *)M->q, (void *)M->kx, (void *)M->vx, (void *)M->att, (void *)M->logits,
                    (void *)M->moe_ws, (void *)M->st, (void *)M->seq, (void *)M->ids,
                    (void *)M->w, (void *)M->keys})
        if (!p) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory for the KV cache / scratch");
    if ((rc = tlmh_check(hipHostMalloc((void **)&M->host_tok, 64, hipHostMallocDefault), "model: pinned scratch")))
        return rc;
    if ((rc = tlmh_check(hipMemset(M->st, 0, 16), "model: position"))) return rc;
    return tlmh_check(hipStreamSynchronize(M->stream), "model: load");
}

int load(tlm_hip_model *M, tlm_hip_manifest *m, const tlm_hip_model_opts *o) {
    M->g = *tlm_hip_manifest_geom(m);
    int rc = prepare(M, o);
    if (rc) return rc;
    const tlm_hip_model_geom &g = M->g;
    const int64_t D = g.d_model, hd = g.head_dim, H = g.n_heads, KV = g.n_kv_heads, E = g.n_experts;
    const int64_t de = g.d_expert, ds = g.n_shared > 0 ? g.d_shared : 0;
    for (uint32_t l = 0; l < g.n_layers; l++) {   /* load_layer, tlm_model.c:294-341 */
        Packet pk;
        if ((rc = read_packet(m, TLM_HIP_PK_DENSE, (int)l, 0, pk))) return rc;
        Layer &Ly = M->L[l];
        tlm_hip_tensor_ref t;
        if (tlm_hip_dir_find(pk.payload(), pk.len, "ffn_gate", &t) == TLM_HIP_OK)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: layer %u has a dense FFN", l);
        if ((rc = dev_vec(M, pk, "attn_norm", D, true, &Ly.attn_norm)) ||
            (rc = dev_vec(M, pk, "ffn_norm", D, true, &Ly.ffn_norm)) ||
            (rc = dev_vec(M, pk, "q_norm", hd, false, &Ly.q_norm)) ||
            (rc = dev_vec(M, pk, "k_norm", hd, false, &Ly.k_norm)) ||
            (rc = dir_mat(M, pk, "attn_q", H * hd, D, &Ly.q)) || (rc = dir_mat(M, pk, "attn_k", KV * hd, D, &Ly.k)) ||
            (rc = dir_mat(M, pk, "attn_v", KV * hd, D, &Ly.v)) || (rc = dir_mat(M, pk, "attn_o", D, H * hd, &Ly.o)))
            return rc;
        if (dt_act_kind(Ly.q.dt) != dt_act_kind(Ly.k.dt) || dt_act_kind(Ly.q.dt) != dt_act_kind(Ly.v.dt))
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: q / k / v of layer %u take different activation kinds", l);
        tlm_hip_moe_desc &d = Ly.moe;
        d.D = D;
        d.de = de;
        d.E = (int32_t)E;
        d.k = (int32_t)g.top_k;
        d.router = (int32_t)g.router;
        d.routed_scale = g.routed_scale;
        d.eps = g.norm_eps;
        d.ffn_norm = Ly.ffn_norm;
        if ((rc = tlm_hip_dir_find(pk.payload(), pk.len, "router", &t))) return rc;
        if (t.dtype != DT_F32 || t.shape[0] != (uint64_t)E || t.shape[1] != (uint64_t)D)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: router of layer %u is not f32 [%lld x %lld]", l, (long long)E,
                               (long long)D);
        void *p;
        if ((rc = dev_upload(M, pk.payload() + t.offset, (size_t)t.nbytes, &p))) return rc;
        d.router_w = (const float *)p;
        if ((rc = dev_vec(M, pk, "router_bias", E, false, &d.router_bias))) return rc;
        if (ds > 0) {
            DevMat sg, su, sd;
            if ((rc = dir_mat(M, pk, "shared_gate", ds, D, &sg)) || (rc = dir_mat(M, pk, "shared_up", ds, D, &su)) ||
                (rc = dir_mat(M, pk, "shared_down", D, ds, &sd)) ||
                (rc = dev_vec(M, pk, "shared_gate_inp", D, false, &d.shared_gate_inp)))
                return rc;
            if (sg.dt != su.dt || sg.dt != sd.dt)
                return tlmh_seterr(TLM_HIP_EUNSUP, "model: shared expert matrices of mixed dtypes");
            d.ds = ds;
            d.shared_dt = sg.dt;
            d.sg = sg.p;
            d.su = su.p;
            d.sd = sd.p;
        }
    }
    /* experts (load_experts, tlm_model.c:343-392): every one resident, packed */
    std::vector<std::vector<const void *>> tables(g.n_layers, std::vector<const void *>(3 * E, nullptr));
    std::vector<std::vector<uint8_t>> masks(g.n_layers, std::vector<uint8_t>(E, 1));
    std::vector<int> edt(g.n_layers, -1);
    for (int i = 0; i < tlm_hip_manifest_n_packets(m); i++) {
        const tlm_hip_packet_loc *loc = tlm_hip_manifest_packet(m, i);
        if (loc->type != TLM_HIP_PK_EXPERT) continue;
        if (loc->layer >= g.n_layers || loc->id >= E)
            return tlmh_seterr(TLM_HIP_EFORMAT, "model: EXPERT packet %u:%u out of range", loc->layer, loc->id);
        if (loc->flags & 2u) continue;   /* pruned: never routable */
        Packet pk;
        pk.buf.resize(loc->total_len);
        if ((rc = tlm_hip_packet_read(m, loc, pk.buf.data(), &pk.off, &pk.len))) return rc;
        uint32_t dt32, off[3];
        tlm_hip_packet_header(pk.buf.data(), &dt32, off);
        const int dt = (int)dt32;
        if (edt[loc->layer] >= 0 && edt[loc->layer] != dt)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: layer %u mixes expert dtypes", loc->layer);
        edt[loc->layer] = dt;
        const int64_t shapes[3][2] = {{de, D}, {de, D}, {D, de}};
        for (int k = 0; k < 3; k++) {
            const int bv = dt_block_values(dt);
            if (bv == 0 || shapes[k][1] % bv) return tlmh_seterr(TLM_HIP_EUNSUP, "model: expert dtype %d", dt);
            const uint64_t raw = (uint64_t)shapes[k][0] * (uint64_t)(shapes[k][1] / bv) * (uint64_t)dt_block_bytes(dt);
            if ((uint64_t)off[k] + raw > pk.len)
                return tlmh_seterr(TLM_HIP_EFORMAT, "model: expert %u:%u item %d overruns", loc->layer, loc->id, k);
            DevMat dm;
            if ((rc = dev_matrix(M, dt, pk.payload() + off[k], shapes[k][0], shapes[k][1], &dm))) return rc;
            tables[loc->layer][3 * loc->id + k] = dm.p;
        }
        masks[loc->layer][loc->id] = 0;
    }
    for (uint32_t l = 0; l < g.n_layers; l++) {
        int live = 0;
        for (int64_t e = 0; e < E; e++) live += !masks[l][e];
        if (live < (int)g.top_k)   /* tlm_model.c:597-600 */
            return tlmh_seterr(TLM_HIP_EFORMAT, "model: layer %u has %d routable experts, needs top_k=%u", l, live,
                               g.top_k);
        /* absent experts point at a present one: never routed (masked), never read */
        const void *any[3] = {nullptr, nullptr, nullptr};
        for (int64_t e = 0; e < E && !any[0]; e++)
            if (!masks[l][e])
                for (int k = 0; k < 3; k++) any[k] = tables[l][3 * e + k];
        for (int64_t e = 0; e < E; e++)
            if (masks[l][e])
                for (int k = 0; k < 3; k++) tables[l][3 * e + k] = any[k];
        void *tp, *mp;
        if ((rc = dev_upload(M, tables[l].data(), tables[l].size() * sizeof(void *), &tp)) ||
            (rc = dev_upload(M, masks[l].data(), masks[l].size(), &mp)))
            return rc;
        Layer &Ly = M->L[l];
        Ly.moe.experts = (const void *const *)tp;
        Ly.moe.mask = (const uint8_t *)mp;
        Ly.moe.expert_dt = edt[l];
    }
    {   /* META: output_norm + lm_head */
        Packet pk;
        if ((rc = read_packet(m, TLM_HIP_PK_META, TLM_HIP_LAYER_NONE, 0, pk)) ||
            (rc = dev_vec(M, pk, "output_norm", D, true, &M->out_norm)) ||
            (rc = dir_mat(M, pk, "lm_head", g.vocab, D, &M->lm_head)))
            return rc;
    }
    {   /* EMBED: tok_embd rows stay in the reference layout (gathered per token) */
        Packet pk;
        if ((rc = read_packet(m, TLM_HIP_PK_EMBED, TLM_HIP_LAYER_NONE, 0, pk))) return rc;
        tlm_hip_tensor_ref t;
        if ((rc = tlm_hip_dir_find(pk.payload(), pk.len, "tok_embd", &t))) return rc;
        const int dt = (int)t.dtype;
        if ((dt != DT_F32 && dt != DT_Q8_0) || t.shape[0] != g.vocab || t.shape[1] != (uint64_t)D || D % 32)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: embedding dtype %d", dt);
        M->embd_dt = dt;
        M->embd_row = dt == DT_F32 ? (size_t)D * 4 : (size_t)(D / 32) * 34;
        if (t.nbytes != (uint64_t)M->embd_row * g.vocab) return tlmh_seterr(TLM_HIP_EFORMAT, "model: embedding bytes");
        void *p;
        if ((rc = dev_upload(M, pk.payload() + t.offset, (size_t)t.nbytes, &p))) return rc;
        M->embd = (const uint8_t *)p;
    }
    return finish(M);
}

/* tlm_model_step, src/lib/tlm_model.c:1058-1103, enqueued: the token is
 * seq[pos], pos = st[0]; with logits, the greedy next token goes to
 * seq[pos + 1]; st[0] advances.  Every argument is the same at every position
 * (the step is captured once as a graph). */
int enqueue_step(tlm_hip_model *M, bool want_logits) {
    const tlm_hip_model_geom &g = M->g;
    const int D = (int)g.d_model, hd = (int)g.head_dim, H = (int)g.n_heads, KV = (int)g.n_kv_heads;
    hipStream_t s = M->stream;
    hipLaunchKernelGGL(k_embed, dim3((D + NT - 1) / NT), dim3(NT), 0, s, M->embd, M->embd_row, M->embd_dt,
                       (const int32_t *)M->seq, (const int32_t *)M->st, D, M->h);
    int rc = tlmh_check(hipGetLastError(), "model: embed");
    for (uint32_t l = 0; l < g.n_layers && !rc; l++) {
        const Layer &Ly = M->L[l];
        /* attention(), tlm_model.c:730-763: q | k | v in one launch whose
         * groups each normalise and quantise h themselves, the fused head
         * kernel, o added into h */
        const MvNorm an{M->h, Ly.attn_norm, g.norm_eps};
        const void *W3[3] = {Ly.q.p, Ly.k.p, Ly.v.p};
        const int64_t R3[3] = {Ly.q.rows, Ly.k.rows, Ly.v.rows};
        float *const Y3[3] = {M->q, M->kx, M->vx};
        if (Ly.q.dt == Ly.k.dt && Ly.q.dt == Ly.v.dt) {
            rc = launch_mv_segs(Ly.q.dt, D, W3, R3, Y3, 3, 0, nullptr, s, &an);
        } else {
            for (int m = 0; m < 3 && !rc; m++) {
                const DevMat &Wm = m == 0 ? Ly.q : m == 1 ? Ly.k : Ly.v;
                rc = launch_mv_segs(Wm.dt, D, &W3[m], &R3[m], &Y3[m], 1, 0, nullptr, s, &an);
            }
        }
        if (rc) break;
        const size_t lbase = (size_t)l * KV * M->max_ctx * hd;
        rc = launch_attn(hd, H, KV, M->max_ctx, M->q, M->kx, M->vx, Ly.q_norm, Ly.k_norm, M->cs, M->sn,
                         M->kc + lbase, M->vc + lbase, M->scores, M->smax, M->att, (const int32_t *)M->st, g.norm_eps, s);
        /* o: every group quantises the attention output itself */
        const MvNorm ao{M->att, nullptr, 0.0f};
        const void *Wo = Ly.o.p;
        const int64_t Ro = Ly.o.rows;
        float *const Yo = M->h;
        if (!rc) rc = launch_mv_segs(Ly.o.dt, (int64_t)H * hd, &Wo, &Ro, &Yo, 1, 1, nullptr, s, &ao);
        /* moe(), tlm_model.c:940-1055 */
        if (!rc) rc = launch_moe_layer(&Ly.moe, M->h, M->ids, M->w, M->moe_ws, s);
    }
    if (rc) return rc;
    const int nkeys = (int)((g.vocab + TILE_ROWS - 1) / TILE_ROWS);
    if (want_logits) {   /* tlm_model.c:1087-1095 (norm in the lm_head's groups), the greedy key */
        const MvNorm on{M->h, M->out_norm, g.norm_eps};
        const void *Wl = M->lm_head.p;
        const int64_t Rl = M->lm_head.rows;
        float *const Yl = M->logits;
        rc = launch_mv_segs(M->lm_head.dt, D, &Wl, &Rl, &Yl, 1, 0, nullptr, s, &on, M->keys);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(want_logits ? 1024 : 64), 0, s, M->st, M->seq,
                       want_logits ? (const unsigned long long *)M->keys : nullptr, nkeys);
    return tlmh_check(hipGetLastError(), "model: step");
}

/* One step (the caller checked the context): the captured graph of the kind,
 * captured at first use; eager launches if capture is unavailable. */
int step(tlm_hip_model *M, bool want_logits) {
    const int k = want_logits ? 1 : 0;
    if (!M->graph[k] && !M->graph_failed[k]) {
        hipGraph_t gr = nullptr;
        int rc = tlmh_check(hipStreamBeginCapture(M->stream, hipStreamCaptureModeThreadLocal), "model: capture");
        if (!rc) {
            const int rc_enq = enqueue_step(M, want_logits);
            rc = tlmh_check(hipStreamEndCapture(M->stream, &gr), "model: capture");
            if (!rc) rc = rc_enq;
        }
        if (!rc) rc = tlmh_check(hipGraphInstantiate(&M->graph[k], gr, nullptr, nullptr, 0), "model: instantiate");
        if (gr) (void)hipGraphDestroy(gr);
        if (rc) {
            M->graph[k] = nullptr;
            M->graph_failed[k] = true;
            (void)hipGetLastError();
        }
    }
    int rc = M->graph[k] ? tlmh_check(hipGraphLaunch(M->graph[k], M->stream), "model: step graph")
                         : enqueue_step(M, want_logits);
    if (!rc) M->kv_len++;
    return rc;
}

/* ---- random-init models (tlm_hip_model_synth) -----------------------------
 * Counter-based: every byte is a function of (seed, tensor, index), through
 * the splitmix64 output function (Steele, Lea, Flood, "Fast splittable
 * pseudorandom number generators", OOPSLA 2014). */
__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* n16 x 16 random bytes */
__global__ __launch_bounds__(NT) void k_synth_bytes(uint8_t *__restrict__ dst, int64_t n16, uint64_t seed) {
    const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (i >= n16) return;
    const uint64_t a = mix64(seed + 2 * (uint64_t)i), b = mix64(seed + 2 * (uint64_t)i + 1);
    ((u32x4 *)dst)[i] = u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

/* the f16 field at byte off of each bb-byte block: scale * (0.5 + u), u in [0, 1) */
__global__ __launch_bounds__(NT) void k_synth_scale(uint8_t *__restrict__ rows, int64_t nblocks, int bb, int off,
                                                    float scale, uint64_t seed) {
    const int64_t b = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (b >= nblocks) return;
    const float u = (float)(mix64(seed ^ (uint64_t)b) >> 40) * 0x1p-24f;
    const __half hv = __float2half(scale * (0.5f + u));
    *(uint16_t *)(rows + b * bb + off) = *(const uint16_t *)&hv;
}

/* f32 values bias + scale * U(-sqrt(3), sqrt(3)) (standard deviation scale) */
__global__ __launch_bounds__(NT) void k_synth_f32(float *__restrict__ dst, int64_t n, uint64_t seed, float scale,
                                                  float bias) {
    const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (i >= n) return;
    const float u = (float)(mix64(seed ^ (uint64_t)i) >> 40) * 0x1p-24f;
    dst[i] = bias + scale * 1.7320508f * (2.0f * u - 1.0f);
}

/* rows of dtype dt in the reference layout: random code bytes, scale fields
 * giving weights of about the spread of N(0, 0.02) */
int synth_rows(hipStream_t s, int dt, uint8_t *dst, int64_t rows, int64_t n, uint64_t seed) {
    const int64_t nb = rows * (n / dt_block_values(dt));
    const int bb = dt_block_bytes(dt);
    const int64_t n16 = (nb * bb + 15) / 16;
    hipLaunchKernelGGL(k_synth_bytes, dim3((unsigned)((n16 + NT - 1) / NT)), dim3(NT), 0, s, dst, n16, seed);
    const dim3 gb((unsigned)((nb + NT - 1) / NT));
    const uint64_t s2 = mix64(seed ^ 0x5CA1Eull);
    switch (dt) {   /* codes uniform: |int8| rms 74, Q6_K code-32 rms 18.5 x int8 scale rms 74, K-quant 6-bit scales */
    case DT_Q8_0: hipLaunchKernelGGL(k_synth_scale, gb, dim3(NT), 0, s, dst, nb, bb, 0, 2.7e-4f, s2); break;
    case DT_Q6_K: hipLaunchKernelGGL(k_synth_scale, gb, dim3(NT), 0, s, dst, nb, bb, 208, 1.5e-5f, s2); break;
    case DT_Q4_K:
    case DT_Q5_K: {
        const float sc = dt == DT_Q4_K ? 6.2e-5f : 3.1e-5f;
        hipLaunchKernelGGL(k_synth_scale, gb, dim3(NT), 0, s, dst, nb, bb, 0, sc, s2);
        hipLaunchKernelGGL(k_synth_scale, gb, dim3(NT), 0, s, dst, nb, bb, 2, sc, mix64(s2));
        break;
    }
    default: return tlmh_seterr(TLM_HIP_EUNSUP, "model synth: dtype %d", dt);
    }
    return tlmh_check(hipGetLastError(), "model synth: rows");
}

/* a synthetic matrix packed at dst (allocated when null); tmp holds the rows */
int synth_matrix(tlm_hip_model *M, int dt, int64_t rows, int64_t n, uint64_t seed, uint8_t *tmp, void *dst,
                 DevMat *out) {
    const int bv = dt_block_values(dt);
    if (bv == 0 || !dt_int_ok(dt) || dt == DT_Q8_K || n % bv)
        return tlmh_seterr(TLM_HIP_EUNSUP, "model synth: matrix dtype %d, %lld columns", dt, (long long)n);
    out->dt = dt;
    out->rows = rows;
    out->n = n;
    out->p = dst ? dst : M->dalloc(packed_bytes(dt, rows, n));
    if (!out->p) return tlmh_seterr(TLM_HIP_ENOMEM, "model synth: out of device memory");
    int rc = synth_rows(M->stream, dt, tmp, rows, n, seed);
    if (!rc) rc = launch_pack(dt, tmp, (size_t)(n / bv) * dt_block_bytes(dt), rows, n, out->p, M->stream);
    return rc;
}

float *synth_vec(tlm_hip_model *M, int64_t n, uint64_t seed, float scale, float bias) {
    float *p = (float *)M->dalloc((size_t)n * 4);
    if (p)
        hipLaunchKernelGGL(k_synth_f32, dim3((unsigned)((n + NT - 1) / NT)), dim3(NT), 0, M->stream, p, n, seed,
                           scale, bias);
    return p;
}

int synth(tlm_hip_model *M, const tlm_hip_model_synth_opts *so, const tlm_hip_model_opts *o) {
    int rc = prepare(M, o);
    if (rc) return rc;
    const tlm_hip_model_geom &g = M->g;
    const int64_t D = g.d_model, hd = g.head_dim, H = g.n_heads, KV = g.n_kv_heads, E = g.n_experts;
    const int64_t de = g.d_expert, ds = g.n_shared > 0 ? g.d_shared : 0, V = g.vocab;
    const int edt = so->expert_dt, ddt = so->dense_dt;
    if (D % 32) return tlmh_seterr(TLM_HIP_EUNSUP, "model synth: d_model %lld", (long long)D);
    /* one scratch for the largest matrix's rows */
    const int64_t mats[][3] = {{ddt, H * hd, D}, {ddt, D, H * hd}, {edt, de, D}, {edt, D, de}, {ddt, V, D},
                               {edt, ds, D}, {edt, D, ds}};
    size_t tmpb = (size_t)V * (D / 32) * 34;   /* the embedding rows (Q8_0) */
    for (const auto &m : mats) {
        const int bv = dt_block_values((int)m[0]);
        if (bv == 0 || m[2] % bv)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model synth: dtype %lld with %lld columns", (long long)m[0],
                               (long long)m[2]);
        tmpb = std::max(tmpb, (size_t)m[1] * (size_t)(m[2] / bv) * dt_block_bytes((int)m[0]));
    }
    uint8_t *tmp = (uint8_t *)M->dalloc((tmpb + 15) & ~(size_t)15);
    if (!tmp) return tlmh_seterr(TLM_HIP_ENOMEM, "model synth: out of device memory");
    uint64_t tensor = 0;
    auto next = [&]() { return mix64(so->seed * 0x100000001B3ull + ++tensor); };
    /* experts: one arena, 256-byte aligned matrices */
    const size_t pg = (packed_bytes(edt, de, D) + 255) & ~(size_t)255, pd = (packed_bytes(edt, D, de) + 255) & ~(size_t)255;
    uint8_t *arena = (uint8_t *)M->dalloc((size_t)g.n_layers * E * (2 * pg + pd));
    if (!arena) return tlmh_seterr(TLM_HIP_ENOMEM, "model synth: out of device memory for the experts");
    std::vector<const void *> table(3 * E);
    for (uint32_t l = 0; l < g.n_layers && !rc; l++) {
        Layer &Ly = M->L[l];
        Ly.attn_norm = synth_vec(M, D, next(), 0.0f, 1.0f);
        Ly.ffn_norm = synth_vec(M, D, next(), 0.0f, 1.0f);
        if (so->qk_norm) {
            Ly.q_norm = synth_vec(M, hd, next(), 0.0f, 1.0f);
            Ly.k_norm = synth_vec(M, hd, next(), 0.0f, 1.0f);
        }
        if (!Ly.attn_norm || !Ly.ffn_norm || (so->qk_norm && (!Ly.q_norm || !Ly.k_norm)))
            return tlmh_seterr(TLM_HIP_ENOMEM, "model synth: out of device memory");
        if ((rc = synth_matrix(M, ddt, H * hd, D, next(), tmp, nullptr, &Ly.q)) ||
            (rc = synth_matrix(M, ddt, KV * hd, D, next(), tmp, nullptr, &Ly.k)) ||
            (rc = synth_matrix(M, ddt, KV * hd, D, next(), tmp, nullptr, &Ly.v)) ||
            (rc = synth_matrix(M, ddt, D, H * hd, next(), tmp, nullptr, &Ly.o)))
            return rc;
        tlm_hip_moe_desc &d = Ly.moe;
        d.D = D;
        d.de = de;
        d.E = (int32_t)E;
        d.k = (int32_t)g.top_k;
        d.router = (int32_t)g.router;
        d.routed_scale = g.routed_scale;
        d.eps = g.norm_eps;
        d.ffn_norm = Ly.ffn_norm;
        d.router_w = synth_vec(M, E * D, next(), 1.0f / sqrtf((float)D), 0.0f);
        if (!d.router_w) return tlmh_seterr(TLM_HIP_ENOMEM, "model synth: out of device memory");
        d.expert_dt = edt;
        for (int64_t e = 0; e < E && !rc; e++) {
            uint8_t *base = arena + ((size_t)l * E + e) * (2 * pg + pd);
            DevMat dm;
            if ((rc = synth_matrix(M, edt, de, D, next(), tmp, base, &dm)) ||
                (rc = synth_matrix(M, edt, de, D, next(), tmp, base + pg, &dm)) ||
                (rc = synth_matrix(M, edt, D, de, next(), tmp, base + 2 * pg, &dm)))
                return rc;
            table[3 * e] = base;
            table[3 * e + 1] = base + pg;
            table[3 * e + 2] = base + 2 * pg;
        }
        void *tp;
        if ((rc = dev_upload(M, table.data(), table.size() * sizeof(void *), &tp))) return rc;
        d.experts = (const void *const *)tp;
        if (ds > 0) {
            DevMat sg, su, sd;
            if ((rc = synth_matrix(M, edt, ds, D, next(), tmp, nullptr, &sg)) ||
                (rc = synth_matrix(M, edt, ds, D, next(), tmp, nullptr, &su)) ||
                (rc = synth_matrix(M, edt, D, ds, next(), tmp, nullptr, &sd)))
                return rc;
            d.ds = ds;
            d.shared_dt = edt;
            d.sg = sg.p;
            d.su = su.p;
            d.sd = sd.p;
        }
    }
    M->out_norm = synth_vec(M, D, next(), 0.0f, 1.0f);
    if (!M->out_norm) return tlmh_seterr(TLM_HIP_ENOMEM, "model synth: out of device memory");
    if ((rc = synth_matrix(M, ddt, V, D, next(), tmp, nullptr, &M->lm_head))) return rc;
    /* embedding rows stay in the reference layout (Q8_0), gathered per token */
    M->embd_dt = DT_Q8_0;
    M->embd_row = (size_t)(D / 32) * 34;
    uint8_t *embd = (uint8_t *)M->dalloc(((size_t)V * M->embd_row + 15) & ~(size_t)15);
    if (!embd) return tlmh_seterr(TLM_HIP_ENOMEM, "model synth: out of device memory");
    if ((rc = synth_rows(M->stream, DT_Q8_0, embd, V, D, next()))) return rc;
    M->embd = embd;
    return finish(M);
}

}  // namespace

extern "C" {

int tlm_hip_model_open(const char *manifest_path, const tlm_hip_model_opts *o, tlm_hip_model **out) {
    if (!manifest_path || !out) return tlmh_seterr(TLM_HIP_EINVAL, "model open: NULL argument");
    *out = nullptr;
    if (tlmh_current_device() < 0) return tlmh_seterr(TLM_HIP_EUNSUP, "model open: tlm_hip_init has not run");
    tlm_hip_manifest *m = nullptr;
    int rc = tlm_hip_manifest_load(manifest_path, &m);
    if (rc) return rc;
    tlm_hip_model *M = new tlm_hip_model;
    rc = load(M, m, o);
    tlm_hip_manifest_free(m);
    if (rc) {
        delete M;
        return rc;
    }
    *out = M;
    return TLM_HIP_OK;
}

int tlm_hip_model_synth(const tlm_hip_model_geom *g, const tlm_hip_model_synth_opts *so, const tlm_hip_model_opts *o,
                        tlm_hip_model **out) {
    if (!g || !so || !out) return tlmh_seterr(TLM_HIP_EINVAL, "model synth: NULL argument");
    *out = nullptr;
    if (tlmh_current_device() < 0) return tlmh_seterr(TLM_HIP_EUNSUP, "model synth: tlm_hip_init has not run");
    tlm_hip_model *M = new tlm_hip_model;
    M->g = *g;
    const int rc = synth(M, so, o);
    if (rc) {
        delete M;
        return rc;
    }
    *out = M;
    return TLM_HIP_OK;
}

void tlm_hip_model_close(tlm_hip_model *M) { delete M; }

const tlm_hip_model_geom *tlm_hip_model_geom_of(const tlm_hip_model *M) { return M ? &M->g : nullptr; }
int tlm_hip_model_kv_len(const tlm_hip_model *M) { return M ? M->kv_len : 0; }
int tlm_hip_model_kv_capacity(const tlm_hip_model *M) { return M ? M->max_ctx : 0; }
void tlm_hip_model_reset(tlm_hip_model *M) {
    if (!M) return;
    M->kv_len = 0;
    M->host_tok[2] = 0;
    (void)hipMemcpyAsync(M->st, M->host_tok + 2, 4, hipMemcpyHostToDevice, M->stream);
    (void)hipStreamSynchronize(M->stream);
}

/* tlm_model_step: one token; logits (host, vocab floats) and the greedy next
 * token (argmax) when asked for. */
int tlm_hip_model_step(tlm_hip_model *M, int token, float *logits, int32_t *next) {
    if (!M) return tlmh_seterr(TLM_HIP_EINVAL, "model step: NULL");
    if (token < 0 || (uint32_t)token >= M->g.vocab) return tlmh_seterr(TLM_HIP_EINVAL, "token %d out of range", token);
    if (M->kv_len >= M->max_ctx) return tlmh_seterr(TLM_HIP_ERANGE, "context full (%d tokens)", M->max_ctx);
    const int pos = M->kv_len;
    M->host_tok[0] = token;
    int rc = tlmh_check(hipMemcpyAsync(M->seq + pos, M->host_tok, 4, hipMemcpyHostToDevice, M->stream), "model: token");
    if (!rc) rc = step(M, logits || next);
    if (!rc && logits)
        rc = tlmh_check(hipMemcpyAsync(logits, M->logits, (size_t)M->g.vocab * 4, hipMemcpyDeviceToHost, M->stream),
                        "model: logits");
    if (!rc && next)
        rc = tlmh_check(hipMemcpyAsync(M->host_tok + 1, M->seq + pos + 1, 4, hipMemcpyDeviceToHost, M->stream),
                        "model: next token");
    if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model: step");
    if (!rc && next) *next = M->host_tok[1];
    return rc;
}

/* tlm_model_prefill (src/lib/tlm_model.c:1105-1113) then n_gen greedy tokens
 * (tierlm bench's loop, src/bin/tierlm.c:720-729): the prompt is written to
 * the device once, each step's token is read there and each greedy token is
 * written there by the previous step; out receives the n_gen tokens. */
int tlm_hip_model_generate(tlm_hip_model *M, const int32_t *prompt, int n_prompt, int n_gen, int32_t *out) {
    if (!M || !prompt || n_prompt <= 0 || n_gen < 0 || (n_gen > 0 && !out))
        return tlmh_seterr(TLM_HIP_EINVAL, "model generate: bad arguments");
    const int pos0 = M->kv_len;
    if ((int64_t)pos0 + n_prompt + (n_gen > 0 ? n_gen - 1 : 0) > M->max_ctx)
        return tlmh_seterr(TLM_HIP_ERANGE, "model generate: %d + %d tokens exceed the context (%d)", n_prompt, n_gen,
                           M->max_ctx);
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || (uint32_t)prompt[i] >= M->g.vocab)
            return tlmh_seterr(TLM_HIP_EINVAL, "token %d out of range", prompt[i]);
    int rc = tlmh_check(hipMemcpy(M->seq + pos0, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice), "model: prompt");
    for (int i = 0; i < n_prompt && !rc; i++) rc = step(M, i == n_prompt - 1);
    for (int gi = 1; gi < n_gen && !rc; gi++) rc = step(M, true);
    if (!rc && n_gen > 0)
        rc = tlmh_check(hipMemcpyAsync(out, M->seq + pos0 + n_prompt, (size_t)n_gen * 4, hipMemcpyDeviceToHost,
                                       M->stream), "model: out");
    if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model: generate");
    return rc;
}

}  // extern "C"
