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
 * thread per dot product, positions in ascending order) and e^x is libm's
 * expf bit for bit (expf_ref).  What may differ in the last bit: sums of
 * squares and the softmax sum are double trees instead of sequential double
 * sums (a float rounding of them moves only when the double sum lies within a
 * few double ulps of a float rounding boundary); the reference's greedy
 * tokens are reproduced exactly. */
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

/* ---- embedding row (tlm_dequantize_row, src/lib/tlm_quant.c:629-660) -------- */
/* The step's position and token live in device memory (st[0] = pos, seq[pos]
 * = the token), so one captured graph serves every position. */
__device__ __forceinline__ float embed_at(const uint8_t *row, int dt, int i) {
    if (dt == DT_F32) return ((const float *)row)[i];
    const uint8_t *b = row + (size_t)(i >> 5) * 34;   /* Q8_0: y = f16(d) * (float)q */
    const float dd = f16_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    return dd * (float)(int8_t)b[2 + (i & 31)];
}
__global__ __launch_bounds__(NT) void k_embed(const uint8_t *__restrict__ embd, size_t row_bytes, int dt,
                                              const int32_t *__restrict__ seq, const int32_t *__restrict__ st, int D,
                                              float *__restrict__ h) {
    const uint8_t *row = embd + (size_t)seq[st[0]] * row_bytes;
    for (int i = threadIdx.x + blockIdx.x * NT; i < D; i += NT * gridDim.x) h[i] = embed_at(row, dt, i);
}
/* prefill: the rows of tokens seq[0 .. gridDim.y) into h[t * D ..] */
__global__ __launch_bounds__(NT) void k_pf_embed(const uint8_t *__restrict__ embd, size_t row_bytes, int dt,
                                                 const int32_t *__restrict__ seq, int D, float *__restrict__ h) {
    const uint8_t *row = embd + (size_t)seq[blockIdx.y] * row_bytes;
    float *ht = h + (size_t)blockIdx.y * D;
    for (int i = threadIdx.x + blockIdx.x * NT; i < D; i += NT * gridDim.x) ht[i] = embed_at(row, dt, i);
}
/* prefill: h += y (the o projection's accumulation, tlm_model.c:762) */
__global__ __launch_bounds__(NT) void k_pf_add(float *__restrict__ h, const float *__restrict__ y, int64_t n) {
    for (int64_t i = threadIdx.x + (int64_t)blockIdx.x * NT; i < n; i += (int64_t)NT * gridDim.x) h[i] = h[i] + y[i];
}

/* ---- attention: attention() (src/lib/tlm_model.c:743-756) and attn_heads
 * (:683-719), the reference's bits, in two launches -------------------------
 * Both kernels issue every load that does not depend on the position before
 * the position itself arrives (it lives in device memory, so one captured
 * graph serves every step), clamped to the cache's capacity where the
 * context would bound them; what lies past the context is masked.
 * k_attn_scores: one group per (key head, slice of positions).  It
 * normalises and rotates the query heads that share the key head (q-norm,
 * RoPE) and the new key (k-norm, RoPE) - 16 lanes per vector, every vector
 * at once - then walks its slice in chunks of ATT_CH positions staged in LDS
 * and stores every (query head, position) score: the dot in ascending i,
 * scaled after the dot.  The group whose slice holds the new position appends
 * its key and value to the cache.
 * k_attn_pv: a group per (query head, PV_EW = 16 output elements), so a
 * head of width 128 spreads over 8 groups and 32 heads cover the chip's 256
 * CUs.  All four waves run the softmax in the reference's order - the
 * maximum over the context, e_t = e^(s_t - max) (kept in LDS), their sum in
 * double, inv = 1 / sum, p_t = e_t * inv (formed by the producers as they
 * read e_t), e^x with its table held in the lanes - then the P.V sums out +=
 * p_t * v_t[i] over ascending t:
 * wave 0 holds the chains (lane i mod 16 runs element i's) and only adds,
 * one dependent add per position (about 6.5 clocks); waves 1-3, 12 lanes per
 * element, form the products p_t v_t[i] (the reference's rounded products)
 * into a ring of three LDS blocks of 48 value tiles, two blocks ahead of the
 * chains, with their value tiles PV_VPF blocks ahead in registers (the first
 * ones loaded at entry); one barrier per block.  A group streams 64 bytes of
 * values per position: with 64 elements per group (256 bytes) the value
 * stream of one CU and the few groups in flight held the ring to ~5 ns per
 * position, the chain's own rate being under 2.  The value cache is kept in
 * tiles of 4 positions, element-major inside (V[t][i] at ((t / 4) * HD + i) *
 * 4 + t % 4), where one 16-byte lane load is positions 4j..4j+3 of element i
 * and 16 lanes load 256 contiguous bytes.
 *
 * Numerics: the scores, maximum, products and chains are the reference's
 * operations in its order; the double sums (squares of the norms, softmax
 * terms) are trees instead of sequences (a float rounding of such a sum can
 * differ only when it lies within a double ulp or so of a rounding
 * boundary); e^x is libm's expf (expf_ref).
 *
 * Cache layout (per layer and key head): K[t][i] at t * HD + i (the
 * reference's), values in the 4-position tiles above (att_vstride floats per
 * key head).  Slices: G per key head (fixed for the captured graph),
 * att_slice_len(T, G) positions at context T; groups past the context return
 * at once. */
constexpr int ATT_CH = 32;       /* positions per LDS chunk of the scores */
constexpr int ATT_LMIN = 32;     /* shortest slice */
constexpr int ATT_QMAX = 4096;   /* query values per key head (query heads per key head x HD) */
constexpr int ATT_GMAX = 128;    /* slices per key head */
constexpr int ATT_PSEG = 4096;   /* probabilities per LDS segment of k_attn_pv */
constexpr int PV_EW = 16;        /* output elements per k_attn_pv group */
constexpr int PV_TPL = 4;        /* value tiles (4 positions each) per producer lane per block of the ring */
constexpr int PV_VPF = 3;        /* blocks of value tiles a producer lane holds in flight (a multiple of 3) */

/* floats of value cache per key head: whole 4-position tiles */
__host__ __device__ inline size_t att_vstride(int max_ctx, int hd) { return (size_t)((max_ctx + 3) & ~3) * hd; }
/* V[t][i] in the tiled layout */
__host__ __device__ inline size_t att_vidx(int t, int i, int hd) {
    return ((size_t)(t >> 2) * hd + i) * 4 + (t & 3);
}

__host__ __device__ inline int att_slice_len(int T, int G) {
    int L = (T + G - 1) / G;
    L = (L + 15) & ~15;
    return L < ATT_LMIN ? ATT_LMIN : L;
}

/* LDS of k_attn_scores, offsets in floats: query heads, new key and value,
 * a chunk of K (rows padded by 4 floats) */
struct AttLds {
    int q, kn, vn, k, total;
};
__host__ __device__ inline AttLds att_lds(int hd, int R) {
    AttLds o;
    o.q = 0;
    o.kn = R * hd;
    o.vn = o.kn + hd;
    o.k = o.vn + hd;
    o.total = o.k + ATT_CH * (hd + 4);
    return o;
}

/* max over the aligned 32 lanes of a half wave, uniform in it (no NaN
 * inputs wins: a NaN never compares greater) */
__device__ __forceinline__ float half_max_f32(float v) {
    float o;
    o = dpp_f32<DPP_XOR1>(v);        v = o > v ? o : v;
    o = dpp_f32<DPP_XOR2>(v);        v = o > v ? o : v;
    o = dpp_f32<DPP_HALF_MIRROR>(v); v = o > v ? o : v;
    o = dpp_f32<DPP_MIRROR>(v);      v = o > v ? o : v;
    o = __shfl_xor(v, 16, 64);       v = o > v ? o : v;
    return v;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* One head vector x (LDS, HD floats) by 16 lanes (lane sub holds elements
 * sub + 16 e): rmsnorm when norm (tlm_model.c:743-746: double sum of squares -
 * the lane's elements in order, then a 16-lane tree -, x * r * w), then RoPE
 * (rope(), :721-728: the pair (j, j + HD/2) is elements e and e + EL/2 of one
 * lane).  w, cv, sv: the lane's norm weights and RoPE factors.  Shared by the
 * decode and prefill attention, so both rotate with the same bits. */
template <int HD>
__device__ __forceinline__ void norm_rope16(float *x, bool norm, const float (&w)[HD / 16],
                                            const float (&cv)[HD / 32], const float (&sv)[HD / 32], float eps,
                                            int sub) {
    constexpr int EL = HD / 16;
    float e[EL];
#pragma unroll
    for (int k = 0; k < EL; k++) e[k] = x[sub + 16 * k];
    if (norm) {
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < EL; k++) ss += (double)e[k] * (double)e[k];
        ss += dpp_f64<DPP_XOR1>(ss);
        ss += dpp_f64<DPP_XOR2>(ss);
        ss += dpp_f64<DPP_HALF_MIRROR>(ss);
        ss += dpp_f64<DPP_MIRROR>(ss);
        const float r = 1.0f / sqrtf((float)(ss / (double)HD) + eps);
#pragma unroll
        for (int k = 0; k < EL; k++) e[k] = e[k] * r * w[k];
    }
#pragma unroll
    for (int k = 0; k < EL / 2; k++) {
        const float a = e[k], c = e[k + EL / 2];
        e[k] = a * cv[k] - c * sv[k];
        e[k + EL / 2] = c * cv[k] + a * sv[k];
    }
#pragma unroll
    for (int k = 0; k < EL; k++) x[sub + 16 * k] = e[k];
}

template <int HD>
__global__ __launch_bounds__(NT) void k_attn_scores(const float *__restrict__ q, const float *__restrict__ kx,
                                                    const float *__restrict__ vx, const float *__restrict__ q_norm,
                                                    const float *__restrict__ k_norm, int has_qn, int has_kn,
                                                    const float *__restrict__ cs_all, const float *__restrict__ sn_all,
                                                    float *__restrict__ kc, float *__restrict__ vc,
                                                    float *__restrict__ scores, int H, int KV, int max_ctx, int G,
                                                    const int32_t *__restrict__ st, float eps) {
    /* the arguments the first loads need, in the launch's first scalar round
     * trip (the compiler otherwise fetches them in batches where they are
     * first used; eps is needed only after the first loads land) */
    asm volatile("" : "+s"(has_qn), "+s"(has_kn), "+s"(H), "+s"(KV), "+s"(max_ctx), "+s"(G)
                 : "s"(q), "s"(kx), "s"(vx), "s"(q_norm), "s"(k_norm), "s"(cs_all), "s"(sn_all), "s"(kc), "s"(vc),
                   "s"(scores), "s"(st));
    constexpr int H4 = HD / 4, HALF = HD / 2, KS = HD + 4;
    constexpr int CF = ATT_CH * H4 / NT;            /* float4 of a chunk's K per thread */
    constexpr int QF = ATT_QMAX / 4 / NT;           /* float4 of the query heads per thread, at most */
    constexpr int SU = ATT_QMAX / HD * ATT_CH / NT; /* (query head, position) items per thread per chunk, at most */
    constexpr int EL = HD / 16;                     /* elements per lane of a vector's 16 lanes */
    extern __shared__ __align__(16) float s_dyn[];
    const int R = H / KV, kvh = blockIdx.x, tid = threadIdx.x, sub = tid & 15;
    const AttLds lo = att_lds(HD, R);
    float *s_q = s_dyn + lo.q, *s_kn = s_dyn + lo.kn, *s_vn = s_dyn + lo.vn, *s_k = s_dyn + lo.k;
    float *K = kc + (size_t)kvh * max_ctx * HD, *V = vc + (size_t)kvh * att_vstride(max_ctx, HD);

    /* what does not depend on the position is loaded while the position is
     * read: the query heads (consecutive heads h = kvh * R + j), the new key
     * and value, the norm weights of the lane's elements sub + 16 e */
    const int nq4 = R * H4;
    const f32x4 *q4 = (const f32x4 *)(q + (size_t)kvh * R * HD);
    f32x4 qv[QF];
#pragma unroll
    for (int k = 0; k < QF; k++) qv[k] = q4[min(tid + NT * k, nq4 - 1)];
    const f32x4 knv = ((const f32x4 *)kx)[(size_t)kvh * H4 + min(tid, H4 - 1)];
    const f32x4 vnv = ((const f32x4 *)vx)[(size_t)kvh * H4 + min(tid, H4 - 1)];
    float qn[EL], kn[EL];
#pragma unroll
    for (int e = 0; e < EL; e++) {
        qn[e] = q_norm[sub + 16 * e];
        kn[e] = k_norm[sub + 16 * e];
    }
    /* those loads stay above the position's read and the slice test that
     * follows it (the compiler would otherwise sink them below the branch) */
    asm volatile("" ::: "memory");
    const int pos = st[0], T = pos + 1;
    const int L = att_slice_len(T, G), t0 = (int)blockIdx.y * L;
    if (t0 >= T) return;
    const int tn = min(L, T - t0);
    /* RoPE factors of the lane's pairs (sub + 16 e, sub + 16 e + HD/2), then
     * the first chunk's key rows (clamped to the context; rows past the
     * slice are never used) */
    float cv[EL / 2], sv[EL / 2];
#pragma unroll
    for (int e = 0; e < EL / 2; e++) {
        cv[e] = cs_all[(size_t)pos * HALF + sub + 16 * e];
        sv[e] = sn_all[(size_t)pos * HALF + sub + 16 * e];
    }
    const int nch = (tn + ATT_CH - 1) / ATT_CH;
    f32x4 kr[CF];
    auto kload = [&](int c) {
        const int tc = t0 + c * ATT_CH;
#pragma unroll
        for (int k = 0; k < CF; k++) {
            const int e = tid + NT * k, t = min(tc + e / H4, T - 1);
            kr[k] = ((const f32x4 *)(K + (size_t)t * HD))[e % H4];
        }
    };
    kload(0);
    /* the value rows of this slice and of its sibling (slice ^ 1) towards this
     * XCD's L2 for the P.V launch: direct-to-LDS loads into one 1 KB sink, never
     * read, so they hold no registers (k_attn_pv puts a key head's P.V groups
     * on the XCDs its slices run on; block b runs on XCD b mod 8 and slice
     * parity alternates the two) */
    __shared__ __align__(16) float s_sink[256];
    for (int sl = (int)blockIdx.y & ~1; sl <= ((int)blockIdx.y | 1); sl++) {
        const int a0 = sl * L;   /* a multiple of 16: whole tiles, one contiguous run */
        if (a0 >= T) break;
        const int nc = (min(L, T - a0) + 3) / 4 * HD;   /* 16-byte pieces: a tile's element i each */
        for (int c = tid; c < nc; c += NT)
            __builtin_amdgcn_global_load_lds((const void *)(V + att_vidx(a0, 0, HD) + 4 * (size_t)c),
                                             (__attribute__((address_space(3))) void *)s_sink, 16, 0, 0);
    }

#pragma unroll
    for (int k = 0; k < QF; k++)
        if (tid + NT * k < nq4) ((f32x4 *)s_q)[tid + NT * k] = qv[k];
    if (tid < H4) {
        ((f32x4 *)s_kn)[tid] = knv;
        ((f32x4 *)s_vn)[tid] = vnv;
    }
    __syncthreads();

    /* rmsnorm of each query head and of the new key, then RoPE (norm_rope16);
     * 16 lanes per vector, all vectors at once, vector R being the key */
    for (int v = tid >> 4; v <= R; v += NT / 16)   /* uniform over each 16 lanes */
        norm_rope16<HD>(v < R ? s_q + v * HD : s_kn, v < R ? has_qn : has_kn, v < R ? qn : kn, cv, sv, eps, sub);
    __syncthreads();

    const float scale = 1.0f / sqrtf((float)HD);
    const int nsc = R * ATT_CH;
    for (int c = 0; c < nch; c++) {   /* uniform over the group */
        const int tc = t0 + c * ATT_CH, tnc = min(ATT_CH, tn - c * ATT_CH);
        /* stage the chunk's keys; row pos from this group's copy */
#pragma unroll
        for (int k = 0; k < CF; k++) {
            const int e = tid + NT * k, t = e / H4, i4 = e % H4;
            ((f32x4 *)(s_k + t * KS))[i4] = tc + t == pos ? ((const f32x4 *)s_kn)[i4] : kr[k];
        }
        __syncthreads();
        if (c + 1 < nch) kload(c + 1);   /* the next chunk flies while this one is scored */
        /* item (j, t), positions fastest: a query head's ATT_CH positions are
         * one half wave */
#pragma unroll
        for (int u = 0; u < SU; u++) {
            const int idx = tid + NT * u;
            if (idx < nsc) {
                const int j = idx / ATT_CH, t = idx % ATT_CH;
                const f32x4 *qq = (const f32x4 *)(s_q + j * HD), *kk = (const f32x4 *)(s_k + t * KS);
                float d = 0.0f;
#pragma unroll 8
                for (int i4 = 0; i4 < H4; i4++) {
                    const f32x4 a = qq[i4], b = kk[i4];
                    d += a.x * b.x;
                    d += a.y * b.y;
                    d += a.z * b.z;
                    d += a.w * b.w;
                }
                d *= scale;   /* after the dot, before the maximum (tlm_model.c:699-702) */
                if (t < tnc) scores[(size_t)(kvh * R + j) * max_ctx + tc + t] = d;
            }
        }
        __syncthreads();   /* before the next chunk overwrites the keys */
    }
    if (t0 + tn == T)   /* the KV append (tlm_model.c:748-752), after the last read */
        for (int i4 = tid; i4 < H4; i4 += NT) {
            ((f32x4 *)K)[(size_t)pos * H4 + i4] = ((const f32x4 *)s_kn)[i4];
            const f32x4 v4 = ((const f32x4 *)s_vn)[i4];
            V[att_vidx(pos, 4 * i4, HD)] = v4.x;
            V[att_vidx(pos, 4 * i4 + 1, HD)] = v4.y;
            V[att_vidx(pos, 4 * i4 + 2, HD)] = v4.z;
            V[att_vidx(pos, 4 * i4 + 3, HD)] = v4.w;
        }
    __builtin_amdgcn_s_waitcnt(0);   /* the prefetches land before the group's LDS is released */
}

template <int HD>
__global__ __launch_bounds__(NT) void k_attn_pv(const float *__restrict__ scores, const float *__restrict__ vc,
                                                float *__restrict__ att, int H, int KV, int max_ctx,
                                                const int32_t *__restrict__ st) {
    constexpr int EW = PV_EW;             /* output elements per group */
    constexpr int NWC = HD / EW;          /* element slabs per query head, a group each */
    constexpr int PB = 8;                 /* score loads per thread per round */
    constexpr int PL = NT - 64;           /* producer lanes (waves 1..3) */
    constexpr int TL = PL / EW;           /* producer lanes per element: tile columns of a block */
    constexpr int TPL = PV_TPL;           /* tiles per producer lane per block */
    constexpr int BT = TL * TPL;          /* tiles per block */
    constexpr int VPF = PV_VPF;
    static_assert(HD % EW == 0 && PL % EW == 0 && VPF % 3 == 0 && BT % 3 == 0, "ring shape");
    __shared__ __align__(16) float s_p[ATT_PSEG];
    __shared__ __align__(16) f32x4 s_prod[3][BT][EW];   /* three blocks of products, tile-major */
    __shared__ double s_sum[NT / 64];
    __shared__ float s_max[NT / 64];
    const int R = H / KV;
    /* block b: key head b mod KV (so b runs on an XCD of that key head's
     * slices, where k_attn_scores left its values), then (query head of the key
     * head, slab) */
    const int kvg = (int)blockIdx.x % KV, rest = (int)blockIdx.x / KV;
    if (rest >= R * NWC) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = kvg * R + rest / NWC;
    /* a producer lane's element and tile column; the chain wave's lane l runs
     * element l mod EW (lanes past EW repeat a chain and store nothing) */
    const int pl = wave > 0 ? tid - 64 : lane;
    const int e = pl % EW, tc = pl / EW;
    const int ic = EW * (rest % NWC) + e;
    const float *S = scores + (size_t)h * max_ctx;
    const char *vbase = (const char *)(vc + (size_t)kvg * att_vstride(max_ctx, HD));
    const uint32_t lane_off = (uint32_t)ic * 16u;   /* element ic's 16 bytes of a tile */
    /* a producer lane forms tiles tc + TL u (u < TPL) of each block; the chain
     * wave issues the same first loads (and drops them), so that every wave
     * runs the same loads up to the role split and the compiler's wait for the
     * scores is the same count on every path */
    auto vload = [&](int q0, int blk, int lastq, f32x4 (&r)[TPL]) {
#pragma unroll
        for (int u = 0; u < TPL; u++) {
            const int tq = min(q0 + blk * BT + tc + TL * u, lastq);
            r[u] = *(const f32x4 *)(vbase + (size_t)tq * (HD * 16) + lane_off);
        }
    };

    /* entry loads, none waiting for the position: the first scores and the
     * first blocks' value tiles (both clamped to the capacity: what lies past
     * the context is masked below), the exp table */
    float sv[PB];
#pragma unroll
    for (int k = 0; k < PB; k++) sv[k] = S[min(tid + NT * k, max_ctx - 1)];
    ExpTabLanes tab;
    tab.load();
    f32x4 vq[VPF][TPL];   /* producers: value tiles of VPF blocks */
#pragma unroll
    for (int k = 0; k < VPF; k++) vload(0, k, (max_ctx - 1) >> 2, vq[k]);
    const int pos = st[0], T = pos + 1, lastq = (T - 1) >> 2;

    /* the maximum over the context (tlm_model.c:698-703; NaN never compares
     * greater, and a maximum is the same in any order), then e_t = e^(s_t -
     * max) and their sum (:704-709, the double sum as a tree) */
    const int nround = (T + PB * NT - 1) / (PB * NT);
    float m = -INFINITY;
    for (int r = 0; r < nround; r++) {
        if (r > 0) {
#pragma unroll
            for (int k = 0; k < PB; k++) sv[k] = S[min(r * PB * NT + tid + NT * k, T - 1)];
        }
#pragma unroll
        for (int k = 0; k < PB; k++) {
            const int t = r * PB * NT + tid + NT * k;
            m = t < T && sv[k] > m ? sv[k] : m;
        }
    }
    m = wave_max_f32(m);
    if (lane == 0) s_max[wave] = m;
    __syncthreads();
    float mx = s_max[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) mx = s_max[w] > mx ? s_max[w] : mx;
    const int nseg = (T + ATT_PSEG - 1) / ATT_PSEG;
    double sum = 0.0;
    for (int r = 0; r < nround; r++) {
        if (nround > 1) {
#pragma unroll
            for (int k = 0; k < PB; k++) sv[k] = S[min(r * PB * NT + tid + NT * k, T - 1)];
        }
#pragma unroll
        for (int k = 0; k < PB; k++) {   /* every lane computes; past the context it adds 0, stores nothing */
            const int t = r * PB * NT + tid + NT * k;
            const float ex = expf_ref_with(sv[k] - mx, tab);
            sum += t < T ? (double)ex : 0.0;
            if (nseg == 1 && t < T) s_p[t] = ex;
        }
    }
    sum = wave_sum_f64(sum);
    if (lane == 0) s_sum[wave] = sum;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) tot += s_sum[w];
    const float inv_s = (float)(1.0 / tot);

    /* P.V: wave 0 runs the chains out += p_t v_t[i] (ascending t); waves
     * 1..3 form the products p_t v_t[i] - the reference's rounded products -
     * into a ring of three LDS blocks of BT tiles, two blocks ahead of the
     * chains, with their value tiles VPF blocks ahead in registers.  Products
     * past the segment are +0, and adding +0 leaves the chain unchanged (it
     * starts at +0 and never holds -0), so the chains run whole blocks. */
    float acc = 0.0f;
    for (int sb = 0; sb < T; sb += ATT_PSEG) {   /* uniform over the group */
        const int se = min(T, sb + ATT_PSEG);
        /* s_p holds the segment's terms e_t; the producers form p_t = e_t *
         * inv as they read them.  One segment: the exp pass stored them */
        if (nseg > 1) {   /* every lane through every pass: e^x reads its table from the other lanes */
            for (int t0 = sb; t0 < se; t0 += NT) {
                const int t = t0 + tid;
                const float ex = expf_ref_with(S[min(t, se - 1)] - mx, tab);
                if (t < se) s_p[t - sb] = ex;
            }
        }
        const int nbk = (se - sb + BT * 4 - 1) / (BT * 4);   /* blocks of the segment */
        const int q0 = sb >> 2;   /* the segment's first tile */
        /* the probabilities p_t = e_t * inv (tlm_model.c:710, 715) of a
         * producer lane's tiles of block blk (LDS reads shared by the lanes of
         * a tile column), read a block ahead of their use */
        auto pread = [&](int blk, f32x4 (&p)[TPL]) {
            const f32x4 *p4 = (const f32x4 *)s_p;
#pragma unroll
            for (int u = 0; u < TPL; u++) {
                const f32x4 ev = p4[min(blk * BT + tc + TL * u, ATT_PSEG / 4 - 1)];
                p[u].x = ev.x * inv_s;
                p[u].y = ev.y * inv_s;
                p[u].z = ev.z * inv_s;
                p[u].w = ev.w * inv_s;
            }
        };
        auto produce = [&](int blk, const f32x4 (&p)[TPL], const f32x4 (&r)[TPL], int buf) {
            const int tl0 = blk * BT;   /* the block's first tile in the segment */
            if (sb + 4 * (tl0 + BT) <= se) {   /* uniform: the block lies inside the segment */
#pragma unroll
                for (int u = 0; u < TPL; u++) {
                    f32x4 o;
                    o.x = p[u].x * r[u].x;
                    o.y = p[u].y * r[u].y;
                    o.z = p[u].z * r[u].z;
                    o.w = p[u].w * r[u].w;
                    s_prod[buf][tc + TL * u][e] = o;
                }
            } else {
#pragma unroll
                for (int u = 0; u < TPL; u++) {
                    const int t = sb + 4 * (tl0 + tc + TL * u);
                    f32x4 o;
                    o.x = t < se ? p[u].x * r[u].x : 0.0f;
                    o.y = t + 1 < se ? p[u].y * r[u].y : 0.0f;
                    o.z = t + 2 < se ? p[u].z * r[u].z : 0.0f;
                    o.w = t + 3 < se ? p[u].w * r[u].w : 0.0f;
                    s_prod[buf][tc + TL * u][e] = o;
                }
            }
        };
        /* the two roles run separate loops with the same barriers, so that
         * neither's memory counters are merged with the other's path */
        if (wave > 0) {
            if (sb > 0) {   /* later segments: their first blocks' tiles now */
#pragma unroll
                for (int k = 0; k < VPF; k++) vload(q0, k, lastq, vq[k]);
            }
            f32x4 pc[TPL];
            if (nseg > 1) __syncthreads();   /* the segment's terms (one segment: stored before the sum's barrier) */
            pread(0, pc);
            produce(0, pc, vq[0], 0);
            vload(q0, VPF, lastq, vq[0]);
            pread(1, pc);
            produce(1, pc, vq[1], 1);
            vload(q0, VPF + 1, lastq, vq[1]);
            pread(2, pc);
            __syncthreads();
            /* one step (and barrier) per block of the segment; step s of a
             * round produces block b + s + 2 into buffer (s + 2) mod 3.  The
             * loop runs the rounds whose blocks all lie in the segment, with
             * the full prefetch in flight at its head (so the compiler's wait
             * counts there keep it); the steps after it produce only blocks
             * of the segment, so none waits for a tile past the context */
            auto step = [&](int b, int k) {
                produce(b + k + 2, pc, vq[(k + 2) % VPF], (k + 2) % 3);
                vload(q0, b + k + 2 + VPF, lastq, vq[(k + 2) % VPF]);
                pread(b + k + 3, pc);
                __syncthreads();
            };
            int b = 0;
            for (; b + VPF + 2 <= nbk; b += VPF) {
#pragma unroll
                for (int k = 0; k < VPF; k++) step(b, k);
            }
#pragma unroll
            for (int k = 0; k < VPF + 1; k++) {   /* uniform: the chain wave runs the same blocks */
                if (b + k >= nbk) break;
                if (b + k + 2 < nbk) produce(b + k + 2, pc, vq[(k + 2) % VPF], (k + 2) % 3);
                pread(b + k + 3, pc);
                __syncthreads();
            }
        } else {
            /* the chain reads a block in parts of 8 tiles, each one part ahead
             * of its adds (the next block's first part during this block's last) */
            constexpr int SUB = 8, NPART = BT / SUB;
            static_assert(BT % SUB == 0, "whole parts");
            if (nseg > 1) __syncthreads();   /* the segment's terms */
            __syncthreads();
            f32x4 cur[SUB];
            const bool chain = lane < EW;   /* lanes past EW stay out of the LDS reads and adds */
            if (chain)
#pragma unroll
                for (int u = 0; u < SUB; u++) cur[u] = s_prod[0][u][e];
            auto block = [&](int k) {   /* block b + k from buffer (b + k) mod 3 */
                if (chain)
#pragma unroll
                for (int c = 0; c < NPART; c++) {
                    f32x4 nx[SUB];
#pragma unroll
                    for (int u = 0; u < SUB; u++)
                        nx[u] = c < NPART - 1 ? s_prod[k % 3][SUB * (c + 1) + u][e] : s_prod[(k + 1) % 3][u][e];
                    /* the reads stay ahead of the adds (the scheduler would
                     * otherwise sink them to their use) */
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int u = 0; u < SUB; u++) {
                        acc += cur[u].x;
                        acc += cur[u].y;
                        acc += cur[u].z;
                        acc += cur[u].w;
                    }
#pragma unroll
                    for (int u = 0; u < SUB; u++) cur[u] = nx[u];
                }
                /* the chain wave writes no LDS, and its reads in flight are
                 * of the next block's buffer, which the next step does not
                 * overwrite: a bare barrier, without draining them */
                __builtin_amdgcn_s_barrier();
            };
            int b = 0;
            for (; b + VPF <= nbk; b += VPF) {
#pragma unroll
                for (int k = 0; k < VPF; k++) block(k);
            }
#pragma unroll
            for (int k = 0; k < VPF - 1; k++)
                if (b + k < nbk) block(k);
        }
    }
    if (wave == 0 && lane < EW) att[(size_t)h * HD + ic] = acc;
}

/* ---- split attention (attn_split): a partial softmax and P.V per (key
 * head, slice of positions), merged per query head ---------------------------
 * k_attn_split: one group per (key head, slice), as k_attn_scores: the query
 * heads and the new key normalised and rotated, the slice's keys staged in
 * LDS a chunk at a time, the scores (each dot as four interleaved partial
 * sums) kept in LDS; then per query head j the slice maximum m_j, e_t =
 * e^(s_t - m_j), l_j = sum_t e_t, and o_j[i] = sum_t e_t v_t[i] (thread (i,
 * js) runs the heads j = js (mod NT / HD) of element i, fma chains over the
 * slice's positions with the value tiles one chunk ahead in registers),
 * stored as the slice's partials; the group holding the new position also
 * appends its key and value.
 * k_attn_merge: one group per query head: M = max_s m_s, w_s = e^(m_s - M),
 * out[i] = (sum_s w_s o_s[i]) / (sum_s w_s l_s).
 * The same quantity as attn_heads (src/lib/tlm_model.c:683-719) in another
 * order of operations: within 1e-5 relative of the reference's outputs, not
 * its bits (the exact order is k_attn_scores + k_attn_pv). */
struct AttSplitLds {
    int q, kn, vn, k, e, m, total;
};
__host__ __device__ inline AttSplitLds att_split_lds(int hd, int R, int lmax) {
    AttSplitLds o;
    o.q = 0;
    o.kn = R * hd;
    o.vn = o.kn + hd;
    o.k = o.vn + hd;
    o.e = o.k + ATT_CH * (hd + 4);
    o.m = o.e + R * lmax;   /* lmax: a multiple of 16 */
    o.total = o.m + R;
    return o;
}

/* sum over the aligned 32 lanes of a half wave, uniform in it */
__device__ __forceinline__ float half_sum_f32(float v) {
    v += dpp_f32<DPP_XOR1>(v);
    v += dpp_f32<DPP_XOR2>(v);
    v += dpp_f32<DPP_HALF_MIRROR>(v);
    v += dpp_f32<DPP_MIRROR>(v);
    v += __shfl_xor(v, 16, 64);
    return v;
}

template <int HD>
__global__ __launch_bounds__(NT) void k_attn_split(const float *__restrict__ q, const float *__restrict__ kx,
                                                   const float *__restrict__ vx, const float *__restrict__ q_norm,
                                                   const float *__restrict__ k_norm, int has_qn, int has_kn,
                                                   const float *__restrict__ cs_all, const float *__restrict__ sn_all,
                                                   float *__restrict__ kc, float *__restrict__ vc,
                                                   float *__restrict__ part_o, float *__restrict__ part_ml, int H,
                                                   int KV, int max_ctx, int G, int lmax,
                                                   const int32_t *__restrict__ st, float eps) {
    constexpr int H4 = HD / 4, HALF = HD / 2, KS = HD + 4;
    constexpr int CF = ATT_CH * H4 / NT;            /* float4 of a chunk's K per thread */
    constexpr int QF = ATT_QMAX / 4 / NT;           /* float4 of the query heads per thread, at most */
    constexpr int SU = ATT_QMAX / HD * ATT_CH / NT; /* (query head, position) items per thread per chunk, at most */
    constexpr int KE = (HD + 63) / 64, KH = (HALF + 63) / 64;   /* elements / pairs per lane */
    constexpr int JS = NT / HD;                     /* threads per output element in the P.V */
    constexpr int JK = ATT_QMAX / HD / JS;          /* query heads per P.V thread, at most */
    constexpr int VQ = ATT_CH / 4;                  /* value tiles per chunk */
    extern __shared__ __align__(16) float s_dyn[];
    const int pos = st[0], T = pos + 1, R = H / KV;
    const int L = att_slice_len(T, G), t0 = (int)blockIdx.y * L;
    if (t0 >= T) return;
    const int tn = min(L, T - t0), kvh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const AttSplitLds lo = att_split_lds(HD, R, lmax);
    float *s_q = s_dyn + lo.q, *s_kn = s_dyn + lo.kn, *s_vn = s_dyn + lo.vn, *s_k = s_dyn + lo.k;
    float *s_e = s_dyn + lo.e, *s_m = s_dyn + lo.m;
    float *K = kc + (size_t)kvh * max_ctx * HD, *V = vc + (size_t)kvh * att_vstride(max_ctx, HD);

    /* entry loads in the order of use: query heads, new key and value, norm
     * weights and RoPE factors, the first chunk's keys, the first chunk's
     * value tiles */
    const int nq4 = R * H4;
    const f32x4 *q4 = (const f32x4 *)(q + (size_t)kvh * R * HD);
    f32x4 qv[QF];
#pragma unroll
    for (int k = 0; k < QF; k++) qv[k] = q4[min(tid + NT * k, nq4 - 1)];
    const f32x4 knv = ((const f32x4 *)kx)[(size_t)kvh * H4 + min(tid, H4 - 1)];
    const f32x4 vnv = ((const f32x4 *)vx)[(size_t)kvh * H4 + min(tid, H4 - 1)];
    float qn[KE], kn[KE], cv[KH], sv[KH];
#pragma unroll
    for (int k = 0; k < KE; k++) qn[k] = q_norm[min(lane + 64 * k, HD - 1)];
#pragma unroll
    for (int k = 0; k < KE; k++) kn[k] = k_norm[min(lane + 64 * k, HD - 1)];
#pragma unroll
    for (int k = 0; k < KH; k++) {
        cv[k] = cs_all[(size_t)pos * HALF + min(lane + 64 * k, HALF - 1)];
        sv[k] = sn_all[(size_t)pos * HALF + min(lane + 64 * k, HALF - 1)];
    }
    const int nch = (tn + ATT_CH - 1) / ATT_CH;
    f32x4 kr[CF];
    auto kload = [&](int c) {
        const int tc = t0 + c * ATT_CH;
#pragma unroll
        for (int k = 0; k < CF; k++) {
            const int e = tid + NT * k, t = min(tc + e / H4, T - 1);
            kr[k] = ((const f32x4 *)(K + (size_t)t * HD))[e % H4];
        }
    };
    kload(0);
    const int vi = tid % HD, js = tid / HD, lastq = (T - 1) >> 2;
    f32x4 vr[VQ];
    auto vload = [&](int c) {   /* chunk c's tiles of element vi, clamped to the context */
        const int q0 = (t0 + c * ATT_CH) >> 2;
#pragma unroll
        for (int u = 0; u < VQ; u++) vr[u] = ((const f32x4 *)V)[(size_t)min(q0 + u, lastq) * HD + vi];
    };
    vload(0);

#pragma unroll
    for (int k = 0; k < QF; k++)
        if (tid + NT * k < nq4) ((f32x4 *)s_q)[tid + NT * k] = qv[k];
    if (tid < H4) {
        ((f32x4 *)s_kn)[tid] = knv;
        ((f32x4 *)s_vn)[tid] = vnv;
    }
    __syncthreads();

    /* q-norm / k-norm and RoPE as in k_attn_scores (tlm_model.c:743-746,
     * 721-728) */
    for (int v = wave; v <= R; v += NT / 64) {
        float *x = v < R ? s_q + v * HD : s_kn;
        if (v < R ? has_qn : has_kn) {
            float e[KE];
#pragma unroll
            for (int k = 0; k < KE; k++) e[k] = x[min(lane + 64 * k, HD - 1)];
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < KE; k++)
                if (lane + 64 * k < HD) ss += (double)e[k] * (double)e[k];
            ss = wave_sum_f64(ss);
            const float r = 1.0f / sqrtf((float)(ss / (double)HD) + eps);
#pragma unroll
            for (int k = 0; k < KE; k++)
                if (lane + 64 * k < HD) x[lane + 64 * k] = e[k] * r * (v < R ? qn[k] : kn[k]);
            wave_lds_sync();
        }
#pragma unroll
        for (int k = 0; k < KH; k++) {
            const int j = lane + 64 * k;
            if (j < HALF) {
                const float a = x[j], c = x[j + HALF];
                x[j] = a * cv[k] - c * sv[k];
                x[j + HALF] = c * cv[k] + a * sv[k];
            }
        }
    }
    __syncthreads();

    /* scores of the slice into LDS (row j of s_e: query head j's positions),
     * with each thread's running maximum over its items */
    const float scale = 1.0f / sqrtf((float)HD);
    const int nsc = R * ATT_CH;
    float rmx[SU];
#pragma unroll
    for (int u = 0; u < SU; u++) rmx[u] = -INFINITY;
    for (int c = 0; c < nch; c++) {   /* uniform over the group */
        const int tc = t0 + c * ATT_CH, tnc = min(ATT_CH, tn - c * ATT_CH);
#pragma unroll
        for (int k = 0; k < CF; k++) {
            const int e = tid + NT * k, t = e / H4, i4 = e % H4;
            ((f32x4 *)(s_k + t * KS))[i4] = tc + t == pos ? ((const f32x4 *)s_kn)[i4] : kr[k];
        }
        __syncthreads();
        if (c + 1 < nch) kload(c + 1);
#pragma unroll
        for (int u = 0; u < SU; u++) {
            const int idx = tid + NT * u;
            if (idx < nsc) {
                const int j = idx / ATT_CH, t = idx % ATT_CH;
                const f32x4 *qq = (const f32x4 *)(s_q + j * HD), *kk = (const f32x4 *)(s_k + t * KS);
                float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll 8
                for (int i4 = 0; i4 < H4; i4++) {
                    const f32x4 a = qq[i4], b = kk[i4];
                    d0 = fmaf(a.x, b.x, d0);
                    d1 = fmaf(a.y, b.y, d1);
                    d2 = fmaf(a.z, b.z, d2);
                    d3 = fmaf(a.w, b.w, d3);
                }
                const float d = ((d0 + d1) + (d2 + d3)) * scale;
                if (t < tnc) {
                    s_e[j * lmax + c * ATT_CH + t] = d;
                    rmx[u] = d > rmx[u] ? d : rmx[u];
                }
            }
        }
        __syncthreads();   /* before the next chunk overwrites the keys */
    }
    /* the slice maximum per query head (a half wave holds one head's items) */
#pragma unroll
    for (int u = 0; u < SU; u++) {
        const int idx = tid + NT * u;
        if (idx < nsc) {
            const float m = half_max_f32(rmx[u]);
            if (idx % ATT_CH == 0) s_m[idx / ATT_CH] = m;
        }
    }
    __syncthreads();
    /* e_t = e^(s_t - m_j) in place; l_j */
    float rl[SU];
#pragma unroll
    for (int u = 0; u < SU; u++) rl[u] = 0.0f;
    for (int c = 0; c < nch; c++) {
#pragma unroll
        for (int u = 0; u < SU; u++) {
            const int idx = tid + NT * u, t = c * ATT_CH + idx % ATT_CH;
            if (idx < nsc && t < tn) {
                float *e = s_e + (idx / ATT_CH) * lmax + t;
                const float v = expf_ref(*e - s_m[idx / ATT_CH]);
                *e = v;
                rl[u] += v;
            }
        }
    }
    const size_t slot = (size_t)kvh * R * G + blockIdx.y;   /* (head kvh * R + j, slice) at slot + j * G */
#pragma unroll
    for (int u = 0; u < SU; u++) {
        const int idx = tid + NT * u;
        if (idx < nsc) {
            const float l = half_sum_f32(rl[u]);
            if (idx % ATT_CH == 0) {
                const int j = idx / ATT_CH;
                part_ml[(slot + (size_t)j * G) * 2] = s_m[j];
                part_ml[(slot + (size_t)j * G) * 2 + 1] = l;
            }
        }
    }
    __syncthreads();

    /* o_j[i] = sum_t e_t v_t[i] over the slice; the new position's value from
     * this group's copy */
    const int jk = js < JS ? (R - js + JS - 1) / JS : 0;
    float acc[JK];
#pragma unroll
    for (int k = 0; k < JK; k++) acc[k] = 0.0f;
    const float vnew = s_vn[vi];
    for (int c = 0; c < nch; c++) {
        f32x4 vcur[VQ];
#pragma unroll
        for (int u = 0; u < VQ; u++) vcur[u] = vr[u];
        if (c + 1 < nch) vload(c + 1);
        const int tb = c * ATT_CH, tnc = min(ATT_CH, tn - tb);
        if (t0 + tb <= pos && pos < t0 + tb + ATT_CH) vcur[(pos - t0 - tb) >> 2][pos & 3] = vnew;
        if (tnc == ATT_CH) {
#pragma unroll
            for (int u = 0; u < VQ; u++) {
#pragma unroll
                for (int k = 0; k < JK; k++) {
                    if (k < jk) {
                        const f32x4 e4 = *(const f32x4 *)(s_e + (js + JS * k) * lmax + tb + 4 * u);
                        acc[k] = fmaf(e4.x, vcur[u].x, acc[k]);
                        acc[k] = fmaf(e4.y, vcur[u].y, acc[k]);
                        acc[k] = fmaf(e4.z, vcur[u].z, acc[k]);
                        acc[k] = fmaf(e4.w, vcur[u].w, acc[k]);
                    }
                }
            }
        } else {   /* the slice's last, partial chunk: positions past it skipped */
#pragma unroll
            for (int u = 0; u < VQ; u++) {
#pragma unroll
                for (int k = 0; k < JK; k++) {
                    if (k < jk) {
                        const f32x4 e4 = *(const f32x4 *)(s_e + (js + JS * k) * lmax + tb + 4 * u);
#pragma unroll
                        for (int w = 0; w < 4; w++)
                            if (4 * u + w < tnc) acc[k] = fmaf(e4[w], vcur[u][w], acc[k]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < JK; k++)
        if (k < jk) part_o[(slot + (size_t)(js + JS * k) * G) * HD + vi] = acc[k];
    if (t0 + tn == T) {   /* the KV append (tlm_model.c:748-752), after the group's reads */
        __syncthreads();
        for (int i4 = tid; i4 < H4; i4 += NT) {
            ((f32x4 *)K)[(size_t)pos * H4 + i4] = ((const f32x4 *)s_kn)[i4];
            const f32x4 v4 = ((const f32x4 *)s_vn)[i4];
            V[att_vidx(pos, 4 * i4, HD)] = v4.x;
            V[att_vidx(pos, 4 * i4 + 1, HD)] = v4.y;
            V[att_vidx(pos, 4 * i4 + 2, HD)] = v4.z;
            V[att_vidx(pos, 4 * i4 + 3, HD)] = v4.w;
        }
    }
}

template <int HD>
__global__ __launch_bounds__(NT) void k_attn_merge(const float *__restrict__ part_o,
                                                   const float *__restrict__ part_ml, float *__restrict__ att,
                                                   int G, const int32_t *__restrict__ st) {
    constexpr int JS = NT / HD;               /* threads per element: slices s = js (mod JS) each */
    constexpr int SP = ATT_GMAX / JS;         /* slices per thread, at most */
    __shared__ float s_w[ATT_GMAX];
    __shared__ float s_part[NT];
    __shared__ float s_mx[NT / 64];
    __shared__ double s_l[NT / 64];
    const int pos = st[0], T = pos + 1, L = att_slice_len(T, G), ns = (T + L - 1) / L;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int vi = tid % HD, js = tid / HD;
    const float *po = part_o + (size_t)h * G * HD, *ml = part_ml + (size_t)h * G * 2;
    /* every load at entry: the slice's maximum and sum (thread s), the
     * thread's partial outputs */
    const float m = tid < ns ? ml[2 * tid] : -INFINITY;
    const float l = tid < ns ? ml[2 * tid + 1] : 0.0f;
    float o[SP];
#pragma unroll
    for (int k = 0; k < SP; k++) {
        const int sl = js + JS * k;
        o[k] = js < JS && sl < ns ? po[(size_t)sl * HD + vi] : 0.0f;
    }
    float mx = wave_max_f32(m);
    if (lane == 0) s_mx[wave] = mx;
    __syncthreads();
    mx = s_mx[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) mx = s_mx[w] > mx ? s_mx[w] : mx;
    const float w = tid < ns ? expf_ref(m - mx) : 0.0f;
    if (tid < ATT_GMAX) s_w[tid] = w;
    const double wl = wave_sum_f64((double)w * (double)l);
    if (lane == 0) s_l[wave] = wl;
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < SP; k++) {
        const int sl = js + JS * k;
        if (sl < ns) acc = fmaf(s_w[sl], o[k], acc);
    }
    s_part[tid] = acc;
    __syncthreads();
    if (tid < HD) {
        double tot = 0.0;
#pragma unroll
        for (int v = 0; v < NT / 64; v++) tot += s_l[v];
        float out = 0.0f;
#pragma unroll
        for (int k = 0; k < JS; k++) out += s_part[tid + HD * k];
        att[(size_t)h * HD + tid] = out * (float)(1.0 / tot);
    }
}

/* ---- prefill attention: the step's attention for a chunk of ntok prompt
 * tokens at positions p0 .. p0 + ntok - 1 (tlm_model_prefill, src/lib/
 * tlm_model.c:1105-1113, steps each token in turn: token t attends to
 * positions 0 .. p0 + t), the step's operations in the step's order per
 * token, in four launches:
 * k_pf_prep: a group per token: q-norm + RoPE of every query head in place,
 *   k-norm + RoPE of every key head (norm_rope16, the decode's code), the key
 *   and value appended to the cache at the token's position.
 * k_pf_scores: a group per (key head, PF_TOK tokens, 64 positions): lane =
 *   position with its key row in registers, wave = token, HB query heads of
 *   the key head at a time from LDS; each score is the dot in ascending i,
 *   scaled after the dot (the decode's expression).
 * k_pf_softmax: a group per (token, query head): the decode P.V launch's
 *   softmax with its thread mapping and reduction trees (the maximum, e_t,
 *   their double sum, inv); p_t = e_t * inv replaces the score.
 * k_pf_pv: a group per (key head, 64-element slab, PF_TOK tokens): lane =
 *   element, wave = token, one chain per query head (HB at a time), out +=
 *   p_t * v_t[i] over ascending t up to the token's position (the rounded
 *   product, then the add), the probabilities staged in LDS PF_PCH positions
 *   at a time.  Products past the position are never added (adding +0 would
 *   leave the chain unchanged, as in the decode ring).
 * Score rows: [token][query head][SL] floats, SL the capacity rounded up to 4. */
constexpr int PF_TOK = 4;     /* tokens per group, a wave each */
constexpr int PF_PCH = 256;   /* positions per staged chunk of probabilities */

template <int HD>
__global__ __launch_bounds__(NT) void k_pf_prep(float *__restrict__ q, const float *__restrict__ kx,
                                                const float *__restrict__ vx, const float *__restrict__ q_norm,
                                                const float *__restrict__ k_norm, int has_qn, int has_kn,
                                                const float *__restrict__ cs_all, const float *__restrict__ sn_all,
                                                float *__restrict__ kc, float *__restrict__ vc, int H, int KV,
                                                int max_ctx, int p0, float eps) {
    constexpr int EL = HD / 16, HALF = HD / 2;
    const int t = blockIdx.x, pos = p0 + t, tid = threadIdx.x, sub = tid & 15;
    float qn[EL], kn[EL], cv[EL / 2], sv[EL / 2];
#pragma unroll
    for (int e = 0; e < EL; e++) {
        qn[e] = q_norm[sub + 16 * e];
        kn[e] = k_norm[sub + 16 * e];
    }
#pragma unroll
    for (int e = 0; e < EL / 2; e++) {
        cv[e] = cs_all[(size_t)pos * HALF + sub + 16 * e];
        sv[e] = sn_all[(size_t)pos * HALF + sub + 16 * e];
    }
    for (int v = tid >> 4; v < H + KV; v += NT / 16) {   /* uniform over each 16 lanes */
        if (v < H) {
            norm_rope16<HD>(q + ((size_t)t * H + v) * HD, has_qn, qn, cv, sv, eps, sub);
        } else {   /* the KV append (tlm_model.c:748-752): the rotated key, the value in its tile */
            const int kvh = v - H;
            float *K = kc + ((size_t)kvh * max_ctx + pos) * HD, *V = vc + (size_t)kvh * att_vstride(max_ctx, HD);
            const float *kr = kx + ((size_t)t * KV + kvh) * HD, *vr = vx + ((size_t)t * KV + kvh) * HD;
#pragma unroll
            for (int e = 0; e < EL; e++) {
                K[sub + 16 * e] = kr[sub + 16 * e];
                V[att_vidx(pos, sub + 16 * e, HD)] = vr[sub + 16 * e];
            }
            norm_rope16<HD>(K, has_kn, kn, cv, sv, eps, sub);   /* the lane's own elements, in place */
        }
    }
}

template <int HD, int HB>
__global__ __launch_bounds__(NT) void k_pf_scores(const float *__restrict__ q, const float *__restrict__ kc,
                                                  float *__restrict__ scores, int H, int KV, int max_ctx, int p0,
                                                  int ntok, int SL) {
    constexpr int H4 = HD / 4;
    __shared__ __align__(16) f32x4 s_q[PF_TOK][HB][H4];
    const int R = H / KV, kvh = blockIdx.z, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = (int)blockIdx.y * PF_TOK, u0 = (int)blockIdx.x * 64;
    const int tlast = min(t0 + PF_TOK, ntok) - 1;
    if (u0 > p0 + tlast) return;   /* uniform: no token of the group reaches these positions */
    const int t = t0 + wave, P = t < ntok ? p0 + t : -1, u = u0 + lane;
    /* the lane's key row (positions past the group's last are clamped, never stored) */
    const f32x4 *K4 = (const f32x4 *)(kc + ((size_t)kvh * max_ctx + min(u, p0 + tlast)) * HD);
    f32x4 kr[H4];
#pragma unroll
    for (int i4 = 0; i4 < H4; i4++) kr[i4] = K4[i4];
    const float scale = 1.0f / sqrtf((float)HD);
    for (int hb = 0; hb < R; hb += HB) {   /* uniform */
        if (hb > 0) __syncthreads();       /* the previous heads are read */
        for (int idx = tid; idx < PF_TOK * HB * H4; idx += NT) {
            const int tk = idx / (HB * H4), j = (idx / H4) % HB, i4 = idx % H4;
            const int tt = min(t0 + tk, ntok - 1);
            s_q[tk][j][i4] = ((const f32x4 *)(q + ((size_t)tt * H + kvh * R + hb + j) * HD))[i4];
        }
        __syncthreads();
        float acc[HB];
#pragma unroll
        for (int j = 0; j < HB; j++) acc[j] = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < H4; i4++) {   /* whole: the key row stays in registers */
            const f32x4 b = kr[i4];
#pragma unroll
            for (int j = 0; j < HB; j++) {
                const f32x4 a = s_q[wave][j][i4];
                acc[j] += a.x * b.x;
                acc[j] += a.y * b.y;
                acc[j] += a.z * b.z;
                acc[j] += a.w * b.w;
            }
        }
        if (u <= P) {
#pragma unroll
            for (int j = 0; j < HB; j++) scores[((size_t)t * H + kvh * R + hb + j) * SL + u] = acc[j] * scale;
        }
    }
}

__global__ __launch_bounds__(NT) void k_pf_softmax(float *__restrict__ scores, int H, int p0, int SL) {
    constexpr int PB = 8;   /* k_attn_pv's scores per thread per round */
    __shared__ double s_sum[NT / 64];
    __shared__ float s_max[NT / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *S = scores + ((size_t)blockIdx.y * H + blockIdx.x) * SL;
    const int T = p0 + (int)blockIdx.y + 1;
    ExpTabLanes tab;
    tab.load();
    const int nround = (T + PB * NT - 1) / (PB * NT);
    float sv[PB];
    float m = -INFINITY;
    for (int r = 0; r < nround; r++) {
#pragma unroll
        for (int k = 0; k < PB; k++) sv[k] = S[min(r * PB * NT + tid + NT * k, T - 1)];
#pragma unroll
        for (int k = 0; k < PB; k++) {
            const int t = r * PB * NT + tid + NT * k;
            m = t < T && sv[k] > m ? sv[k] : m;
        }
    }
    m = wave_max_f32(m);
    if (lane == 0) s_max[wave] = m;
    __syncthreads();
    float mx = s_max[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) mx = s_max[w] > mx ? s_max[w] : mx;
    double sum = 0.0;
    float e[PB];
    for (int r = 0; r < nround; r++) {
        if (nround > 1) {
#pragma unroll
            for (int k = 0; k < PB; k++) sv[k] = S[min(r * PB * NT + tid + NT * k, T - 1)];
        }
#pragma unroll
        for (int k = 0; k < PB; k++) {
            const int t = r * PB * NT + tid + NT * k;
            e[k] = expf_ref_with(sv[k] - mx, tab);
            sum += t < T ? (double)e[k] : 0.0;
        }
    }
    sum = wave_sum_f64(sum);
    if (lane == 0) s_sum[wave] = sum;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) tot += s_sum[w];
    const float inv_s = (float)(1.0 / tot);
    if (nround == 1) {
#pragma unroll
        for (int k = 0; k < PB; k++)
            if (tid + NT * k < T) S[tid + NT * k] = e[k] * inv_s;
    } else {   /* every lane through every pass: e^x reads its table from the other lanes */
        for (int t0 = 0; t0 < T; t0 += NT) {
            const int t = t0 + tid;
            const float p = expf_ref_with(S[min(t, T - 1)] - mx, tab) * inv_s;
            if (t < T) S[t] = p;
        }
    }
}

template <int HD, int HB>
__global__ __launch_bounds__(NT) void k_pf_pv(const float *__restrict__ scores, const float *__restrict__ vc,
                                              float *__restrict__ att, int H, int KV, int max_ctx, int p0, int ntok,
                                              int SL) {
    constexpr int NWC = (HD + 63) / 64, PQ = PF_PCH / 4;
    __shared__ __align__(16) f32x4 s_p[PF_TOK][HB][PQ];
    const int R = H / KV, kvh = (int)blockIdx.x / NWC, slab = (int)blockIdx.x % NWC;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = (int)blockIdx.y * PF_TOK, tlast = min(t0 + PF_TOK, ntok) - 1, pmax = p0 + tlast;
    const int t = t0 + wave, P = t < ntok ? p0 + t : -1, ic = 64 * slab + lane;
    const char *vbase = (const char *)(vc + (size_t)kvh * att_vstride(max_ctx, HD));
    const uint32_t lane_off = (uint32_t)min(ic, HD - 1) * 16u;   /* element ic's 16 bytes of a tile */
    auto vtile = [&](int tq) { return *(const f32x4 *)(vbase + (size_t)tq * (HD * 16) + lane_off); };
    for (int hb = 0; hb < R; hb += HB) {   /* uniform */
        float acc[HB];
#pragma unroll
        for (int j = 0; j < HB; j++) acc[j] = 0.0f;
        for (int c0 = 0; c0 <= pmax; c0 += PF_PCH) {   /* uniform */
            __syncthreads();   /* the previous chunk is read */
            for (int idx = tid; idx < PF_TOK * HB * PQ; idx += NT) {
                const int tk = idx / (HB * PQ), j = (idx / PQ) % HB, u4 = idx % PQ;
                const int tt = t0 + tk, uu = c0 + 4 * u4;
                f32x4 pv = {0.0f, 0.0f, 0.0f, 0.0f};
                if (tt <= tlast && uu <= p0 + tt)   /* row tt holds positions 0 .. p0 + tt (within SL) */
                    pv = *(const f32x4 *)(scores + ((size_t)tt * H + kvh * R + hb + j) * SL + uu);
                s_p[tk][j][u4] = pv;
            }
            __syncthreads();
            const int ue = min(P, c0 + PF_PCH - 1);   /* the wave's last position in the chunk */
            int u = c0;
            for (; u + 15 <= ue; u += 16) {
                f32x4 vt[4];
#pragma unroll
                for (int k = 0; k < 4; k++) vt[k] = vtile((u >> 2) + k);
#pragma unroll
                for (int k = 0; k < 4; k++) {
#pragma unroll
                    for (int j = 0; j < HB; j++) {
                        const f32x4 pp = s_p[wave][j][((u - c0) >> 2) + k];
                        acc[j] += pp.x * vt[k].x;
                        acc[j] += pp.y * vt[k].y;
                        acc[j] += pp.z * vt[k].z;
                        acc[j] += pp.w * vt[k].w;
                    }
                }
            }
            for (; u <= ue; u += 4) {   /* the last positions, up to ue */
                const f32x4 vt = vtile(u >> 2);
#pragma unroll
                for (int j = 0; j < HB; j++) {
                    const f32x4 pp = s_p[wave][j][(u - c0) >> 2];
                    acc[j] += pp.x * vt.x;
                    if (u + 1 <= ue) acc[j] += pp.y * vt.y;
                    if (u + 2 <= ue) acc[j] += pp.z * vt.z;
                    if (u + 3 <= ue) acc[j] += pp.w * vt.w;
                }
            }
        }
        if (t < ntok && ic < HD) {
#pragma unroll
            for (int j = 0; j < HB; j++) att[((size_t)t * H + kvh * R + hb + j) * HD + ic] = acc[j];
        }
    }
}

/* prefill: whether the attention launches take this geometry (the key row in
 * registers: head width at most 128) */
bool pf_att_supported(int hd, int H, int KV) {
    return (hd == 32 || hd == 64 || hd == 96 || hd == 128) && KV > 0 && H % KV == 0;
}

/* the four prefill attention launches for ntok tokens at p0 (q rotated in
 * place, K/V appended, att [ntok][H][hd]) */
int launch_pf_attn(int hd, int H, int KV, int max_ctx, int p0, int ntok, float *q, const float *kx, const float *vx,
                   const float *q_norm, const float *k_norm, const float *cs, const float *sn, float *kc, float *vc,
                   float *scores, int SL, float *att, float eps, hipStream_t s) {
    const int has_qn = q_norm != nullptr, has_kn = k_norm != nullptr;
    if (!q_norm) q_norm = q;   /* read and dropped */
    if (!k_norm) k_norm = q;
    const int R = H / KV, HB = R % 8 == 0 ? 8 : R % 4 == 0 ? 4 : R % 2 == 0 ? 2 : 1;
    const dim3 gsc((unsigned)((p0 + ntok + 63) / 64), (unsigned)((ntok + PF_TOK - 1) / PF_TOK), (unsigned)KV);
    const dim3 gpv((unsigned)(KV * ((hd + 63) / 64)), (unsigned)((ntok + PF_TOK - 1) / PF_TOK));
#define TLM_PF_HB(W, B)                                                                                         \
    case B:                                                                                                     \
        hipLaunchKernelGGL((k_pf_scores<W, B>), gsc, dim3(NT), 0, s, (const float *)q, (const float *)kc,      \
                           scores, H, KV, max_ctx, p0, ntok, SL);                                               \
        hipLaunchKernelGGL(k_pf_softmax, dim3((unsigned)H, (unsigned)ntok), dim3(NT), 0, s, scores, H, p0, SL); \
        hipLaunchKernelGGL((k_pf_pv<W, B>), gpv, dim3(NT), 0, s, (const float *)scores, (const float *)vc, att, \
                           H, KV, max_ctx, p0, ntok, SL);                                                       \
        break;
#define TLM_PF(W)                                                                                                \
    case W:                                                                                                      \
        hipLaunchKernelGGL((k_pf_prep<W>), dim3((unsigned)ntok), dim3(NT), 0, s, q, kx, vx, q_norm, k_norm,     \
                           has_qn, has_kn, cs, sn, kc, vc, H, KV, max_ctx, p0, eps);                            \
        switch (HB) { TLM_PF_HB(W, 8) TLM_PF_HB(W, 4) TLM_PF_HB(W, 2) TLM_PF_HB(W, 1) }                          \
        break;
    switch (hd) {
        TLM_PF(32) TLM_PF(64) TLM_PF(96) TLM_PF(128)
    default: return tlmh_seterr(TLM_HIP_EUNSUP, "model prefill: head width %d", hd);
    }
#undef TLM_PF
#undef TLM_PF_HB
    return tlmh_check(hipGetLastError(), "model: prefill attention");
}

/* slices per key head: enough groups to cover the chip at long contexts
 * (about 256 with every key head), a slice at least ATT_LMIN positions long;
 * req > 0 asks for that many (a test hook: several chunks per slice) */
int att_groups(int max_ctx, int KV, int req) {
    if (req > 0) return req < ATT_GMAX ? req : ATT_GMAX;
    int cap = 256 / KV;
    cap = cap < 1 ? 1 : cap > ATT_GMAX ? ATT_GMAX : cap;
    const int want = (max_ctx + ATT_LMIN - 1) / ATT_LMIN;
    return want < cap ? want : cap;
}

/* whether the attention kernels take this geometry (query heads per key
 * head x head width within the scores launch's share and LDS) */
bool att_supported(int hd, int H, int KV) {
    const int R = H / KV;
    return hd % 32 == 0 && hd <= 256 && R * hd <= ATT_QMAX && (size_t)att_lds(hd, R).total * 4 <= 65536;
}
/* LDS bytes of the split launch at a context capacity of max_ctx positions */
size_t att_split_bytes(int hd, int H, int KV, int max_ctx, int G) {
    return (size_t)att_split_lds(hd, H / KV, att_slice_len(max_ctx, G)).total * 4;
}

/* host: launch for the model's head width (a multiple of 32, at most 256);
 * split: k_attn_split + k_attn_merge (partials in part_o / part_ml), else the
 * reference's order k_attn_scores + k_attn_pv */
int launch_attn(int hd, int H, int KV, int max_ctx, int G, bool split, const float *q, const float *kx,
                const float *vx, const float *q_norm, const float *k_norm, const float *cs, const float *sn,
                float *kc, float *vc, float *scores, float *part_o, float *part_ml, float *att,
                const int32_t *st, float eps, hipStream_t s) {
    const int has_qn = q_norm != nullptr, has_kn = k_norm != nullptr;
    if (!q_norm) q_norm = q;   /* read (clamped) and dropped */
    if (!k_norm) k_norm = q;
    const size_t dyn = (size_t)att_lds(hd, H / KV).total * 4;
    const int lmax = att_slice_len(max_ctx, G);
    const size_t dyn_split = att_split_bytes(hd, H, KV, max_ctx, G);
    const unsigned npv = (unsigned)(H * (hd / PV_EW));   /* k_attn_pv: a group per (query head, 16 elements) */
#define TLM_ATT(W)                                                                                                \
    case W:                                                                                                       \
        if (split) {                                                                                              \
            hipLaunchKernelGGL((k_attn_split<W>), dim3(KV, G), dim3(NT), dyn_split, s, q, kx, vx, q_norm, k_norm, \
                               has_qn, has_kn, cs, sn, kc, vc, part_o, part_ml, H, KV, max_ctx, G, lmax, st, eps); \
            hipLaunchKernelGGL((k_attn_merge<W>), dim3(H), dim3(NT), 0, s, part_o, part_ml, att, G, st);          \
        } else {                                                                                                  \
            hipLaunchKernelGGL((k_attn_scores<W>), dim3(KV, G), dim3(NT), dyn, s, q, kx, vx, q_norm, k_norm,      \
                               has_qn, has_kn, cs, sn, kc, vc, scores, H, KV, max_ctx, G, st, eps);               \
            hipLaunchKernelGGL((k_attn_pv<W>), dim3(npv), dim3(NT), 0, s, scores, vc, att, H, KV, max_ctx, st);    \
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

/* the context position (the next step's), as a rollback sets it */
__global__ void k_set_pos(int32_t *st, int pos) { st[0] = pos; }

/* tlm_hip_model_opts.stats: stamps of the device clock (s_memrealtime, a
 * fixed 100 MHz count shared by the chip).  A step stamps S before its
 * embedding, A_l / M_l where layer l's attention and MoE block begin and T
 * before its tail (at st[0], st[1 + 2l], st[2 + 2l], st[1 + 2L]); k_stamp_acc
 * reads the end itself and adds the split, in ns, to st[2L + 2 ..]: attention
 * = sum (M_l - A_l), MoE = sum (A_l+1 - M_l) with A_L = T, other = (A_0 - S)
 * + (end - T). */
__global__ void k_stamp(uint64_t *dst) {
    if (threadIdx.x == 0) dst[0] = __builtin_amdgcn_s_memrealtime();
}
__global__ void k_stamp_acc(uint64_t *st, int L) {
    if (threadIdx.x != 0) return;
    const uint64_t end = __builtin_amdgcn_s_memrealtime();
    const uint64_t S = st[0], T = st[1 + 2 * L];
    uint64_t attn = 0, moe = 0;
    for (int l = 0; l < L; l++) {
        const uint64_t A = st[1 + 2 * l], Mb = st[2 + 2 * l], An = l + 1 < L ? st[3 + 2 * l] : T;
        attn += Mb - A;
        moe += An - Mb;
    }
    uint64_t *acc = st + 2 * L + 2;
    acc[0] += attn * 10;
    acc[1] += moe * 10;
    acc[2] += ((st[1] - S) + (end - T)) * 10;
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
    /* a dense-FFN layer (first_k_dense_replace / mlp_only_layers): gate, up
     * [dffn x D], down [D x dffn]; no router, no experts */
    bool dense = false;
    DevMat dg, du, dd;
    int64_t dffn = 0;
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
    float *kc = nullptr, *vc = nullptr, *cs = nullptr, *sn = nullptr;
    int att_g = 1;                                     /* attention slices per key head */
    bool att_split = false;                            /* split attention; false: the reference's order */
    float *scores = nullptr;                           /* [H][max_ctx] scores */
    float *part_o = nullptr, *part_ml = nullptr;       /* split partials: [H][att_g][hd]; [H][att_g] (m, l) */
    float *h = nullptr, *q = nullptr, *kx = nullptr, *vx = nullptr, *att = nullptr;
    float *logits = nullptr;
    uint8_t *lm_act = nullptr;   /* the final norm's quantised activation, once per step for every lm_head group */
    uint8_t *moe_ws = nullptr;
    float *dffn_buf = nullptr;   /* dense FFN layers: gate | up | silu(gate) * up, dffn_max each */
    float *pf_ffn = nullptr;     /* the same for a prefill chunk, [cap][dffn_max] each */
    int64_t dffn_max = 0;
    uint32_t dense_prefix = 0;   /* leading dense-FFN layers */
    bool any_dense = false;
    int32_t *st = nullptr, *seq = nullptr, *ids = nullptr;   /* st[0] = position; seq[max_ctx + 1] tokens */
    unsigned long long *keys = nullptr;                      /* greedy key per lm_head tile */
    float *w = nullptr;
    int32_t *host_tok = nullptr;   /* pinned */
    hipGraphExec_t graph[2] = {nullptr, nullptr};   /* step without / with logits, captured at first use */
    /* tlm_hip_model_opts.stats: device stamps of the step, then the
     * accumulated attention / MoE / other ns (k_stamp_acc); host counts */
    bool stats = false;
    uint64_t *stamps = nullptr;
    uint64_t st_tokens = 0, st_wait0 = 0;
    bool graph_failed[2] = {false, false};
    /* experts through the slot cache (expert_cache_bytes > 0) */
    uint64_t xs_budget = 0;
    double xs_pin = 0.0;
    bool xs_prefetch = true;
    tlm_hip_store *xs = nullptr;
    void *xs_payload = nullptr;                  /* page-locked expert payloads */
    std::vector<tlm_hip_expert_src> xs_src;
    uint8_t *stack_ws = nullptr;
    tlm_hip_stack_opts xopts{};
    std::vector<double> instinct;                /* tlm_model's per-layer instinct (tlm_model.c:974-980) */
    std::vector<uint32_t> instinct_seen;
    std::vector<tlm_hip_moe_desc> descs;
    std::vector<float> layer_heat;               /* mean manifest heat of a layer's experts (tlm_model.c:546-560) */
    std::vector<int32_t> route_ids;              /* the last step's routing, n_layers x top_k (host) */
    std::vector<float> route_w;
    /* batched prefill: chunk option, then its buffers (allocated at first use,
     * pf_cap tokens each; score rows of pf_sl floats) */
    int pf_chunk = 0, pf_cap = 0, pf_sl = 0;
    bool pf_nomem = false;                       /* the buffers did not fit: prompts step token by token */
    float *pf_h = nullptr, *pf_q = nullptr, *pf_kx = nullptr, *pf_vx = nullptr, *pf_att = nullptr, *pf_y = nullptr;
    float *pf_scores = nullptr, *pf_w = nullptr;
    uint8_t *pf_act = nullptr, *pf_ws = nullptr;
    int32_t *pf_ids = nullptr;
    /* batched prefill with the experts in the slot cache: the chunk's routing
     * on the host (page-locked) and one expert table per pass (page-locked
     * staging, device copies) */
    int32_t *pf_host_ids = nullptr;
    const void **pf_host_tab = nullptr;
    const void **pf_dev_tab = nullptr;

    void *dalloc(size_t n) {
        void *p = nullptr;
        if (hipMalloc(&p, n ? n : 16) != hipSuccess) return nullptr;
        allocs.push_back(p);
        return p;
    }
    /* frees an allocation of dalloc now (nullptr: nothing) */
    void dfree(void *p) {
        if (!p) return;
        for (size_t i = 0; i < allocs.size(); i++)
            if (allocs[i] == p) {
                (void)hipFree(p);
                allocs[i] = allocs.back();
                allocs.pop_back();
                return;
            }
    }
    ~tlm_hip_model() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (xs) tlm_hip_store_close(xs);   /* waits for its loads, which read the payloads */
        for (hipGraphExec_t g : graph)
            if (g) (void)hipGraphExecDestroy(g);
        for (void *p : allocs) (void)hipFree(p);
        if (host_tok) (void)hipHostFree(host_tok);
        if (pf_host_ids) (void)hipHostFree(pf_host_ids);
        if (pf_host_tab) (void)hipHostFree(pf_host_tab);
        if (xs_payload) (void)hipHostFree(xs_payload);
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
    M->xs_budget = o ? o->expert_cache_bytes : 0;
    M->xs_pin = !o || o->pin_frac == 0.0 ? 0.30 : o->pin_frac < 0.0 ? 0.0 : o->pin_frac;
    M->xs_prefetch = !(o && o->prefetch_off);
    M->xopts.lookahead = M->xs_prefetch ? 1 : 0;   /* src/bin/tierlm.c:307-309 */
    M->xopts.lookahead_k = o ? o->lookahead_k : 0;
    M->xopts.interest = o ? o->interest : 0.0;
    M->pf_chunk = o ? o->prefill_chunk : 0;
    M->stats = o && o->stats;
    M->xopts.host_routes = o && o->host_routes ? 1 : 0;
    if (M->xopts.lookahead_k < 0 || M->xopts.lookahead_k > 32)
        return tlmh_seterr(TLM_HIP_EINVAL, "model: lookahead_k %d (0..32)", M->xopts.lookahead_k);
    /* a step through the cache waits on the host between layers: never a graph */
    M->graph_failed[0] = M->graph_failed[1] = (o && o->eager) || M->xs_budget > 0;
    if (!att_supported((int)g.head_dim, (int)g.n_heads, (int)g.n_kv_heads))
        return tlmh_seterr(TLM_HIP_EUNSUP, "model: %u query heads per key head of width %u exceed the attention "
                           "kernel's share", g.n_heads / g.n_kv_heads, g.head_dim);
    M->att_g = att_groups(max_ctx, (int)g.n_kv_heads, o ? o->attn_slices : 0);
    M->att_split = o && o->attn_split;
    if (M->att_split &&
        att_split_bytes((int)g.head_dim, (int)g.n_heads, (int)g.n_kv_heads, max_ctx, M->att_g) > 65536)
        return tlmh_seterr(TLM_HIP_EUNSUP, "model: a context of %d positions in %d slices exceeds the split "
                           "attention's LDS (more attn_slices, or attn_split 0)", max_ctx, M->att_g);
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
    M->vc = (float *)M->dalloc((size_t)g.n_layers * KV * att_vstride(max_ctx, (int)hd) * 4);
    M->scores = (float *)M->dalloc((size_t)H * max_ctx * 4);
    M->part_o = (float *)M->dalloc((size_t)H * M->att_g * hd * 4);
    M->part_ml = (float *)M->dalloc((size_t)H * M->att_g * 2 * 4);
    M->h = (float *)M->dalloc((size_t)D * 4);
    M->q = (float *)M->dalloc((size_t)H * hd * 4);
    M->kx = (float *)M->dalloc((size_t)KV * hd * 4);
    M->vx = (float *)M->dalloc((size_t)KV * hd * 4);
    M->att = (float *)M->dalloc((size_t)H * hd * 4);
    M->logits = (float *)M->dalloc((size_t)g.vocab * 4);
    M->lm_act = (uint8_t *)M->dalloc(act_bytes(DT_Q8_K, D) + act_bytes(DT_Q8_0, D));
    size_t ws = 0;
    for (const Layer &Ly : M->L)
        if (!Ly.dense) ws = std::max(ws, tlm_hip_moe_workspace_bytes(&Ly.moe));
    M->moe_ws = (uint8_t *)M->dalloc(ws + 256);
    if (M->any_dense) {
        M->dffn_buf = (float *)M->dalloc((size_t)M->dffn_max * 3 * 4);
        if (!M->dffn_buf) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory for the dense FFN");
    }
    M->st = (int32_t *)M->dalloc(16);
    if (M->stats) {
        const size_t nst = (2 * (size_t)g.n_layers + 5) * 8;
        M->stamps = (uint64_t *)M->dalloc(nst);
        if (M->stamps && hipMemset(M->stamps, 0, nst) != hipSuccess) M->stamps = nullptr;
        if (!M->stamps) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory (stats)");
    }
    M->seq = (int32_t *)M->dalloc(((size_t)max_ctx + 1) * 4);
    M->ids = (int32_t *)M->dalloc((size_t)g.n_layers * 32 * 4);   /* the step's routing, per layer */
    M->w = (float *)M->dalloc((size_t)g.n_layers * 32 * 4);
    M->keys = (unsigned long long *)M->dalloc(((size_t)g.vocab + TILE_ROWS - 1) / TILE_ROWS * 8);
    for (void *p : {(void *)M->kc, (void *)M->vc, (void *)M->scores, (void *)M->part_o,
                    (void *)M->part_ml, (void *)M->h,
                    (void *)M->q, (void *)M->kx, (void *)M->vx, (void *)M->att, (void *)M->logits,
                    (void *)M->moe_ws, (void *)M->st, (void *)M->seq, (void *)M->ids,
                    (void *)M->w, (void *)M->keys, (void *)M->lm_act})
        if (!p) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory for the KV cache / scratch");
    if ((rc = tlmh_check(hipHostMalloc((void **)&M->host_tok, 64, hipHostMallocDefault), "model: pinned scratch")))
        return rc;
    if ((rc = tlmh_check(hipMemset(M->st, 0, 16), "model: position"))) return rc;
    /* dense-FFN layers route nothing: their routing reads back as zeros */
    if ((rc = tlmh_check(hipMemset(M->ids, 0, (size_t)g.n_layers * 32 * 4), "model: routing"))) return rc;
    if ((rc = tlmh_check(hipMemset(M->w, 0, (size_t)g.n_layers * 32 * 4), "model: routing"))) return rc;
    return tlmh_check(hipStreamSynchronize(M->stream), "model: load");
}

/* The experts' slot cache over M->xs_src (payloads already in M->xs_payload):
 * the budget raised to top_k slots and the pin share capped so that pins
 * leave top_k slots (src/bin/tierlm.c:273-294), tlm_store_open +
 * tlm_store_warm (:295-305); the step's stack workspace and state. */
int open_expert_store(tlm_hip_model *M) {
    const tlm_hip_model_geom &g = M->g;
    const int64_t D = g.d_model, de = g.d_expert;
    size_t slot = 0;
    for (const tlm_hip_expert_src &x : M->xs_src) {
        if (x.flags & 2u) continue;
        size_t at = 0;
        const int64_t rows[3] = {de, de, D}, n[3] = {D, D, de};
        for (int k = 0; k < 3; k++) at += (packed_bytes(x.dtype, rows[k], n[k]) + 255) & ~(size_t)255;
        slot = std::max(slot, at);
    }
    if (slot == 0) return tlmh_seterr(TLM_HIP_EFORMAT, "model: no experts for the slot cache");
    for (uint32_t l = M->dense_prefix; l < g.n_layers; l++)
        if (M->L[l].dense)
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: with the slot cache, dense-FFN layers must come first (layer %u)",
                               l);
    uint64_t budget = std::max<uint64_t>(M->xs_budget, (uint64_t)g.top_k * slot);
    uint64_t ns = budget / slot;
    ns = std::min<uint64_t>(ns, M->xs_src.size());
    double pin = M->xs_pin;
    if (ns > 0 && pin > 0.0) {
        const double maxf = (double)(ns > g.top_k ? ns - g.top_k : 0) / (double)ns;
        pin = std::min(pin, maxf);
    }
    tlm_hip_store_opts so{};
    so.d_model = D;
    so.d_expert = de;
    so.top_k = (int32_t)g.top_k;
    so.prefetch = M->xs_prefetch ? 1 : 0;
    so.pin_frac = pin;
    so.budget_bytes = budget;
    int rc = tlm_hip_store_open(M->xs_src.data(), (int)M->xs_src.size(), &so, &M->xs);
    if (!rc) rc = tlm_hip_store_warm(M->xs);
    if (rc) return rc;
    M->descs.clear();
    for (const Layer &Ly : M->L) M->descs.push_back(Ly.moe);
    M->instinct.assign(g.n_layers, 0.0);
    M->instinct_seen.assign(g.n_layers, 0);
    if (M->layer_heat.size() == g.n_layers) M->xopts.layer_heat = M->layer_heat.data();
    M->xopts.instinct = M->instinct.data();
    M->xopts.instinct_seen = M->instinct_seen.data();
    M->route_ids.assign((size_t)g.n_layers * g.top_k, 0);
    M->route_w.assign((size_t)g.n_layers * g.top_k, 0.0f);
    /* the stack runs the MoE layers after the dense prefix */
    const uint32_t K = M->dense_prefix;
    const size_t ws = tlm_hip_moe_stack_workspace_bytes(M->descs.data() + K, (int)(g.n_layers - K), &M->xopts);
    M->stack_ws = (uint8_t *)M->dalloc(ws + 256);
    if (!M->stack_ws) return tlmh_seterr(TLM_HIP_ENOMEM, "model: out of device memory for the stack workspace");
    return TLM_HIP_OK;
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
        if ((rc = dev_vec(M, pk, "attn_norm", D, true, &Ly.attn_norm)) ||
            (rc = dev_vec(M, pk, "ffn_norm", D, true, &Ly.ffn_norm)) ||
            (rc = dev_vec(M, pk, "q_norm", hd, false, &Ly.q_norm)) ||
            (rc = dev_vec(M, pk, "k_norm", hd, false, &Ly.k_norm)) ||
            (rc = dir_mat(M, pk, "attn_q", H * hd, D, &Ly.q)) || (rc = dir_mat(M, pk, "attn_k", KV * hd, D, &Ly.k)) ||
            (rc = dir_mat(M, pk, "attn_v", KV * hd, D, &Ly.v)) || (rc = dir_mat(M, pk, "attn_o", D, H * hd, &Ly.o)))
            return rc;
        if (dt_act_kind(Ly.q.dt) != dt_act_kind(Ly.k.dt) || dt_act_kind(Ly.q.dt) != dt_act_kind(Ly.v.dt))
            return tlmh_seterr(TLM_HIP_EUNSUP, "model: q / k / v of layer %u take different activation kinds", l);
        if (tlm_hip_dir_find(pk.payload(), pk.len, "ffn_gate", &t) == TLM_HIP_OK) {
            /* a dense FFN (tlm_model.c:312-324): one SwiGLU block on ffn_norm's output */
            const int64_t dffn = (int64_t)t.shape[0];
            if (t.shape[1] != (uint64_t)D || dffn <= 0)
                return tlmh_seterr(TLM_HIP_EFORMAT, "model: layer %u ffn_gate shape [%llu x %llu]", l,
                                   (unsigned long long)t.shape[0], (unsigned long long)t.shape[1]);
            if ((rc = dir_mat(M, pk, "ffn_gate", dffn, D, &Ly.dg)) || (rc = dir_mat(M, pk, "ffn_up", dffn, D, &Ly.du)) ||
                (rc = dir_mat(M, pk, "ffn_down", D, dffn, &Ly.dd)))
                return rc;
            if (dt_act_kind(Ly.dg.dt) != dt_act_kind(Ly.du.dt))
                return tlmh_seterr(TLM_HIP_EUNSUP, "model: gate / up of layer %u take different activation kinds", l);
            Ly.dense = true;
            Ly.dffn = dffn;
            M->dffn_max = std::max(M->dffn_max, dffn);
            if (M->dense_prefix == l) M->dense_prefix = l + 1;
            M->any_dense = true;
            continue;
        }
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
    /* experts (load_experts, tlm_model.c:343-392): every one resident, packed;
     * or, with the slot cache, every payload kept in page-locked host memory */
    const bool cached = M->xs_budget > 0;
    std::vector<std::vector<const void *>> tables(g.n_layers, std::vector<const void *>(3 * E, nullptr));
    std::vector<std::vector<uint8_t>> masks(g.n_layers, std::vector<uint8_t>(E, 1));
    std::vector<int> edt(g.n_layers, -1);
    std::vector<std::vector<uint8_t>> payloads;
    std::vector<double> heat_sum(g.n_layers, 0.0);
    std::vector<int> heat_cnt(g.n_layers, 0);
    for (int i = 0; i < tlm_hip_manifest_n_packets(m); i++) {
        const tlm_hip_packet_loc *loc = tlm_hip_manifest_packet(m, i);
        if (loc->type != TLM_HIP_PK_EXPERT) continue;
        if (loc->layer >= g.n_layers || loc->id >= E || M->L[loc->layer].dense)
            return tlmh_seterr(TLM_HIP_EFORMAT, "model: EXPERT packet %u:%u out of range", loc->layer, loc->id);
        heat_sum[loc->layer] += loc->heat;
        heat_cnt[loc->layer]++;
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
            if (cached) continue;
            DevMat dm;
            if ((rc = dev_matrix(M, dt, pk.payload() + off[k], shapes[k][0], shapes[k][1], &dm))) return rc;
            tables[loc->layer][3 * loc->id + k] = dm.p;
        }
        masks[loc->layer][loc->id] = 0;
        if (cached) {   /* the store's source: layer, flags, id, dtype, heat, item offsets, payload */
            tlm_hip_expert_src x{};
            x.layer = (uint16_t)loc->layer;
            x.flags = (uint16_t)(loc->flags & 1u);
            x.id = loc->id;
            x.dtype = dt;
            x.heat = loc->heat;
            for (int k = 0; k < 3; k++) x.item_off[k] = off[k];
            x.payload_len = pk.len;
            M->xs_src.push_back(x);
            payloads.emplace_back(pk.payload(), pk.payload() + pk.len);
        }
    }
    M->layer_heat.assign(g.n_layers, 0.0f);
    for (uint32_t l = 0; l < g.n_layers; l++)
        M->layer_heat[l] = heat_cnt[l] ? (float)(heat_sum[l] / (double)heat_cnt[l]) : 0.0f;
    if (cached) {   /* one page-locked block for every payload */
        size_t total = 0;
        for (const auto &pl : payloads) total += (pl.size() + 255) & ~(size_t)255;
        if ((rc = tlmh_check(hipHostMalloc(&M->xs_payload, total ? total : 256, hipHostMallocDefault),
                             "model: page-locked expert payloads")))
            return rc;
        size_t at = 0;
        for (size_t i = 0; i < payloads.size(); i++) {
            memcpy((uint8_t *)M->xs_payload + at, payloads[i].data(), payloads[i].size());
            M->xs_src[i].payload = (uint8_t *)M->xs_payload + at;
            at += (payloads[i].size() + 255) & ~(size_t)255;
        }
    }
    for (uint32_t l = 0; l < g.n_layers; l++) {
        if (M->L[l].dense) continue;   /* no experts to route (tlm_model.c:406, 621) */
        int live = 0;
        for (int64_t e = 0; e < E; e++) live += !masks[l][e];
        if (live < (int)g.top_k)   /* tlm_model.c:597-600 */
            return tlmh_seterr(TLM_HIP_EFORMAT, "model: layer %u has %d routable experts, needs top_k=%u", l, live,
                               g.top_k);
        if (cached) {   /* the block reads the slots the store hands out; no table */
            void *mp;
            if ((rc = dev_upload(M, masks[l].data(), masks[l].size(), &mp))) return rc;
            M->L[l].moe.experts = nullptr;
            M->L[l].moe.mask = (const uint8_t *)mp;
            M->L[l].moe.expert_dt = edt[l];
            continue;
        }
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
    if (M->xs_budget > 0 && (rc = open_expert_store(M))) return rc;
    return finish(M);
}

/* tlm_model_step, src/lib/tlm_model.c:1058-1103, enqueued: the token is
 * seq[pos], pos = st[0]; with logits, the greedy next token goes to
 * seq[pos + 1]; st[0] advances.  Every argument is the same at every position
 * (the step is captured once as a graph). */
/* layer l's attention (attention(), tlm_model.c:730-763): q | k | v in one
 * launch whose groups each normalise and quantise h themselves, the two
 * attention kernels, o added into h */
int enqueue_attention(tlm_hip_model *M, uint32_t l) {
    const tlm_hip_model_geom &g = M->g;
    const int D = (int)g.d_model, hd = (int)g.head_dim, H = (int)g.n_heads, KV = (int)g.n_kv_heads;
    hipStream_t s = M->stream;
    const Layer &Ly = M->L[l];
    const MvNorm an{M->h, Ly.attn_norm, g.norm_eps};
    const void *W3[3] = {Ly.q.p, Ly.k.p, Ly.v.p};
    const int64_t R3[3] = {Ly.q.rows, Ly.k.rows, Ly.v.rows};
    float *const Y3[3] = {M->q, M->kx, M->vx};
    int rc = TLM_HIP_OK;
    if (Ly.q.dt == Ly.k.dt && Ly.q.dt == Ly.v.dt) {
        rc = launch_mv_segs(Ly.q.dt, D, W3, R3, Y3, 3, 0, nullptr, s, &an);
    } else {
        for (int m = 0; m < 3 && !rc; m++) {
            const DevMat &Wm = m == 0 ? Ly.q : m == 1 ? Ly.k : Ly.v;
            rc = launch_mv_segs(Wm.dt, D, &W3[m], &R3[m], &Y3[m], 1, 0, nullptr, s, &an);
        }
    }
    if (rc) return rc;
    const size_t kbase = (size_t)l * KV * M->max_ctx * hd, vbase = (size_t)l * KV * att_vstride(M->max_ctx, hd);
    rc = launch_attn(hd, H, KV, M->max_ctx, M->att_g, M->att_split, M->q, M->kx, M->vx, Ly.q_norm, Ly.k_norm,
                     M->cs, M->sn, M->kc + kbase, M->vc + vbase, M->scores, M->part_o, M->part_ml,
                     M->att, (const int32_t *)M->st, g.norm_eps, s);
    /* o: every group quantises the attention output itself */
    const MvNorm ao{M->att, nullptr, 0.0f};
    const void *Wo = Ly.o.p;
    const int64_t Ro = Ly.o.rows;
    float *const Yo = M->h;
    if (!rc) rc = launch_mv_segs(Ly.o.dt, (int64_t)H * hd, &Wo, &Ro, &Yo, 1, 1, nullptr, s, &ao);
    return rc;
}

/* silu(g) * u of a dense FFN (tlm_model.c:171, 955-956) */
__global__ __launch_bounds__(256) void k_dense_swiglu(const float *__restrict__ g, const float *__restrict__ u,
                                                      float *__restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float gv = g[i];
        out[i] = gv / (1.0f + expf_ref(-gv)) * u[i];
    }
}

/* layer l's dense FFN (moe()'s dense branch, tlm_model.c:946-964): gate | up
 * in one launch whose groups each normalise and quantise h themselves (ffn_norm,
 * as q | k | v do with attn_norm), silu(gate) * up, then down with the
 * activation quantised in each group's prologue, added into h */
int enqueue_dense_ffn(tlm_hip_model *M, uint32_t l) {
    const tlm_hip_model_geom &g = M->g;
    const int64_t D = g.d_model;
    hipStream_t s = M->stream;
    const Layer &Ly = M->L[l];
    const int64_t F = Ly.dffn;
    float *gb = M->dffn_buf, *ub = gb + M->dffn_max, *hb = ub + M->dffn_max;
    const MvNorm fn{M->h, Ly.ffn_norm, g.norm_eps};
    const void *W2[2] = {Ly.dg.p, Ly.du.p};
    const int64_t R2[2] = {F, F};
    float *const Y2[2] = {gb, ub};
    int rc = TLM_HIP_OK;
    if (Ly.dg.dt == Ly.du.dt) {
        rc = launch_mv_segs(Ly.dg.dt, D, W2, R2, Y2, 2, 0, nullptr, s, &fn);
    } else {
        rc = launch_mv_segs(Ly.dg.dt, D, &W2[0], &R2[0], &Y2[0], 1, 0, nullptr, s, &fn);
        if (!rc) rc = launch_mv_segs(Ly.du.dt, D, &W2[1], &R2[1], &Y2[1], 1, 0, nullptr, s, &fn);
    }
    if (rc) return rc;
    hipLaunchKernelGGL(k_dense_swiglu, dim3((unsigned)((F + 255) / 256)), dim3(256), 0, s, gb, ub, hb, F);
    if ((rc = tlmh_check(hipGetLastError(), "model: dense swiglu"))) return rc;
    const MvNorm dn{hb, nullptr, 0.0f};
    const void *Wd = Ly.dd.p;
    const int64_t Rd = Ly.dd.rows;
    float *const Yd = M->h;
    return launch_mv_segs(Ly.dd.dt, F, &Wd, &Rd, &Yd, 1, 1, nullptr, s, &dn);
}

/* the step's end: final norm + lm_head with the greedy keys (tlm_model.c:
 * 1087-1095), then the argmax and the position's advance */
int enqueue_tail(tlm_hip_model *M, bool want_logits) {
    const tlm_hip_model_geom &g = M->g;
    const int D = (int)g.d_model;
    hipStream_t s = M->stream;
    const int nkeys = (int)((g.vocab + TILE_ROWS - 1) / TILE_ROWS);
    if (want_logits) {
        /* the final norm and its activation once (the GEMV prologue's code,
         * so the same bytes), not in each of the vocab / 16 groups */
        const int kind = dt_act_kind(M->lm_head.dt);
        int rc = launch_tok_norm_act(kind, M->h, D, M->out_norm, g.norm_eps, D, 1, M->lm_act,
                                     (int64_t)act_bytes(kind, D), s);
        const void *Wl = M->lm_head.p;
        const int64_t Rl = M->lm_head.rows;
        float *const Yl = M->logits;
        if (!rc) rc = launch_mv_segs(M->lm_head.dt, D, &Wl, &Rl, &Yl, 1, 0, M->lm_act, s, nullptr, M->keys);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(want_logits ? 1024 : 64), 0, s, M->st, M->seq,
                       want_logits ? (const unsigned long long *)M->keys : nullptr, nkeys);
    return tlmh_check(hipGetLastError(), "model: step");
}

void enqueue_embed(tlm_hip_model *M) {
    const int D = (int)M->g.d_model;
    hipLaunchKernelGGL(k_embed, dim3((D + NT - 1) / NT), dim3(NT), 0, M->stream, M->embd, M->embd_row, M->embd_dt,
                       (const int32_t *)M->seq, (const int32_t *)M->st, D, M->h);
}

/* tlm_model_step, src/lib/tlm_model.c:1058-1103, enqueued: the token is
 * seq[pos], pos = st[0]; with logits, the greedy next token goes to
 * seq[pos + 1]; st[0] advances.  Every argument is the same at every position
 * (the step is captured once as a graph). */
/* stats stamp i (no-op without tlm_hip_model_opts.stats) */
void stamp(tlm_hip_model *M, size_t i) {
    if (M->stats) hipLaunchKernelGGL(k_stamp, dim3(1), dim3(64), 0, M->stream, M->stamps + i);
}
void stamp_acc(tlm_hip_model *M) {
    if (M->stats) hipLaunchKernelGGL(k_stamp_acc, dim3(1), dim3(64), 0, M->stream, M->stamps, (int)M->g.n_layers);
}

int enqueue_step(tlm_hip_model *M, bool want_logits) {
    const size_t L = M->g.n_layers;
    stamp(M, 0);
    enqueue_embed(M);
    int rc = tlmh_check(hipGetLastError(), "model: embed");
    for (uint32_t l = 0; l < L && !rc; l++) {
        const Layer &Ly = M->L[l];
        stamp(M, 1 + 2 * (size_t)l);
        rc = enqueue_attention(M, l);
        stamp(M, 2 + 2 * (size_t)l);
        /* moe(), tlm_model.c:940-1055 */
        if (!rc)
            rc = Ly.dense ? enqueue_dense_ffn(M, l)
                          : launch_moe_layer(&Ly.moe, M->h, M->ids + (size_t)l * 32, M->w + (size_t)l * 32, M->moe_ws,
                                             M->stream);
    }
    if (rc) return rc;
    stamp(M, 1 + 2 * L);
    rc = enqueue_tail(M, want_logits);
    stamp_acc(M);
    return rc ? rc : tlmh_check(hipGetLastError(), "model: stats");
}

/* The same step with the experts in the slot cache: tlm_model_step's layer
 * loop with moe() through the store (tlm_model.c:960-1055) and the router
 * lookahead, one tick per token (:1097): each layer's attention is queued
 * right before its router; the device resolves the routed experts' slots
 * while the host replays the store operations behind it, or, with
 * host_routes, the host acquires layer l + 1's experts while the device runs
 * layer l's block (moe_stack_run). */
int step_cached(tlm_hip_model *M, bool want_logits) {
    const size_t L = M->g.n_layers;
    stamp(M, 0);
    enqueue_embed(M);
    int rc = tlmh_check(hipGetLastError(), "model: embed");
    /* the leading dense-FFN layers, then the MoE layers through the store
     * (its layer numbers stay the model's; the per-layer state starts at K) */
    const uint32_t K = M->dense_prefix;
    for (uint32_t l = 0; l < K && !rc; l++) {
        stamp(M, 1 + 2 * (size_t)l);
        rc = enqueue_attention(M, l);
        stamp(M, 2 + 2 * (size_t)l);
        if (!rc) rc = enqueue_dense_ffn(M, l);
    }
    tlm_hip_stack_opts so = M->xopts;
    if (so.layer_heat) so.layer_heat += K;
    so.instinct += K;
    so.instinct_seen += K;
    if (!rc)
        rc = moe_stack_run(M->descs.data() + K, (int)(L - K), M->xs, M->h, &so,
                           M->route_ids.data() + (size_t)K * M->g.top_k, M->route_w.data() + (size_t)K * M->g.top_k,
                           M->stack_ws, M->stream,
                           [M, K](int l) {
                               const uint32_t ml = K + (uint32_t)l;
                               stamp(M, 1 + 2 * (size_t)ml);
                               const int r = enqueue_attention(M, ml);
                               stamp(M, 2 + 2 * (size_t)ml);
                               return r;
                           },
                           (int)K);
    if (rc) return rc;
    stamp(M, 1 + 2 * L);
    rc = enqueue_tail(M, want_logits);
    stamp_acc(M);
    return rc ? rc : tlmh_check(hipGetLastError(), "model: stats");
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
    int rc = M->xs ? step_cached(M, want_logits)
             : M->graph[k] ? tlmh_check(hipGraphLaunch(M->graph[k], M->stream), "model: step graph")
                           : enqueue_step(M, want_logits);
    if (!rc) {
        M->kv_len++;
        M->st_tokens++;
    }
    return rc;
}

/* ---- batched prefill --------------------------------------------------------
 * tlm_model_prefill steps each prompt token in turn (src/lib/tlm_model.c:
 * 1105-1113).  Per chunk of tokens each layer runs once for all of them:
 * rmsnorm + the activation quantiser per token (the decode GEMV prologue's
 * code), q / k / v as int8 MFMA token matmuls (bit-equal to the decode GEMV
 * per token), the causal attention launches (the step's order per token),
 * o the same way plus the residual add, and the batched MoE block (the
 * decode block's result per token); the chunk's last token then takes the
 * step's final norm, lm_head and argmax.  Every token's values are the
 * step's bits, so the cache, the logits and the greedy token are those of n
 * steps. */
bool pf_dense_ok(const DevMat &m) {
    return m.dt == DT_Q4_K || m.dt == DT_Q5_K || m.dt == DT_Q6_K || m.dt == DT_Q8_0;
}
bool pf_supported(const tlm_hip_model *M) {
    const tlm_hip_model_geom &g = M->g;
    if (M->pf_chunk < 0 || M->att_split || M->pf_nomem) return false;
    if (!pf_att_supported((int)g.head_dim, (int)g.n_heads, (int)g.n_kv_heads)) return false;
    if (g.d_model % 256 || ((int64_t)g.n_heads * g.head_dim) % 256 || g.d_model > 8192 ||
        (int64_t)g.n_heads * g.head_dim > 8192)
        return false;
    for (const Layer &Ly : M->L) {
        if (!pf_dense_ok(Ly.q) || !pf_dense_ok(Ly.k) || !pf_dense_ok(Ly.v) || !pf_dense_ok(Ly.o)) return false;
        if (Ly.dense) {   /* gate / up / down as token matmuls */
            if (!pf_dense_ok(Ly.dg) || !pf_dense_ok(Ly.du) || !pf_dense_ok(Ly.dd) || Ly.dffn % 256 || Ly.dffn > 65536)
                return false;
            continue;
        }
        const int edt = Ly.moe.expert_dt;
        if ((edt != DT_Q4_K && edt != DT_Q5_K && edt != DT_Q6_K) || (!Ly.moe.experts && !M->xs)) return false;
        const int sdt = Ly.moe.shared_dt;
        if (Ly.moe.ds > 0 && ((sdt != DT_Q4_K && sdt != DT_Q5_K && sdt != DT_Q6_K && sdt != DT_Q8_0) || Ly.moe.ds % 256))
            return false;
    }
    return true;
}

/* the chunk's buffers: pf_cap tokens, score rows for the whole capacity
 * (at most 256 MB of scores, no more tokens than the context holds, the
 * chunk a multiple of 4, by default at most 1024: 2047 tokens in 122 ms
 * against 130 in chunks of 512).  On a failed allocation the buffers this
 * call did get are freed again. */
int pf_alloc(tlm_hip_model *M) {
    if (M->pf_cap) return TLM_HIP_OK;
    const tlm_hip_model_geom &g = M->g;
    const int64_t D = g.d_model, HQ = (int64_t)g.n_heads * g.head_dim, KVD = (int64_t)g.n_kv_heads * g.head_dim;
    const int sl = (M->max_ctx + 3) & ~3;
    int64_t cap = ((int64_t)256 << 20) / ((int64_t)g.n_heads * sl * 4);
    const int64_t want = M->pf_chunk > 0 ? M->pf_chunk : 1024;
    cap = cap > want ? want : cap;
    cap = cap > sl ? sl : cap;   /* a chunk never holds more tokens than the capacity */
    cap = cap >= 4 ? cap & ~3 : cap < 1 ? 1 : cap;
    size_t ws = 0;
    for (const Layer &Ly : M->L) {
        if (Ly.dense) continue;
        const size_t b = moe_prefill_workspace_bytes(&Ly.moe, cap);
        ws = b > ws ? b : ws;
    }
    int64_t wmax = D > HQ ? D : HQ;
    wmax = wmax > M->dffn_max ? wmax : M->dffn_max;
    M->pf_h = (float *)M->dalloc((size_t)cap * D * 4);
    M->pf_q = (float *)M->dalloc((size_t)cap * HQ * 4);
    M->pf_kx = (float *)M->dalloc((size_t)cap * KVD * 4);
    M->pf_vx = (float *)M->dalloc((size_t)cap * KVD * 4);
    M->pf_att = (float *)M->dalloc((size_t)cap * HQ * 4);
    M->pf_y = (float *)M->dalloc((size_t)cap * D * 4);
    M->pf_scores = (float *)M->dalloc((size_t)cap * g.n_heads * sl * 4);
    M->pf_act = (uint8_t *)M->dalloc((size_t)cap * (wmax / 256) * 292);   /* Q8_K or a8 rows of the widest input */
    M->pf_ws = (uint8_t *)M->dalloc(ws);
    M->pf_ids = (int32_t *)M->dalloc((size_t)cap * g.top_k * 4);
    M->pf_w = (float *)M->dalloc((size_t)cap * g.top_k * 4);
    if (M->any_dense) M->pf_ffn = (float *)M->dalloc((size_t)cap * M->dffn_max * 3 * 4);
    bool host_ok = true;
    if (M->xs) {   /* the routing back on the host; an expert table per pass, at most one pass per expert */
        const size_t tab = (size_t)g.n_experts * 3 * g.n_experts * sizeof(void *);
        host_ok = hipHostMalloc((void **)&M->pf_host_ids, (size_t)cap * g.top_k * 4, hipHostMallocDefault) ==
                      hipSuccess &&
                  hipHostMalloc((void **)&M->pf_host_tab, tab, hipHostMallocDefault) == hipSuccess;
        M->pf_dev_tab = (const void **)M->dalloc(tab);
        host_ok = host_ok && M->pf_dev_tab;
    }
    if (!M->pf_h || !M->pf_q || !M->pf_kx || !M->pf_vx || !M->pf_att || !M->pf_y || !M->pf_scores || !M->pf_act ||
        !M->pf_ws || !M->pf_ids || !M->pf_w || !host_ok || (M->any_dense && !M->pf_ffn)) {
        (void)hipGetLastError();
        for (void **p : {(void **)&M->pf_h, (void **)&M->pf_q, (void **)&M->pf_kx, (void **)&M->pf_vx,
                         (void **)&M->pf_att, (void **)&M->pf_y, (void **)&M->pf_scores, (void **)&M->pf_act,
                         (void **)&M->pf_ws, (void **)&M->pf_ids, (void **)&M->pf_w, (void **)&M->pf_dev_tab,
                         (void **)&M->pf_ffn}) {
            M->dfree(*p);
            *p = nullptr;
        }
        if (M->pf_host_ids) (void)hipHostFree(M->pf_host_ids);
        if (M->pf_host_tab) (void)hipHostFree(M->pf_host_tab);
        M->pf_host_ids = nullptr;
        M->pf_host_tab = nullptr;
        M->pf_nomem = true;
        return tlmh_seterr(TLM_HIP_ENOMEM, "model prefill: out of device memory (%lld-token chunks)", (long long)cap);
    }
    M->pf_sl = sl;
    M->pf_cap = (int)cap;
    return TLM_HIP_OK;
}

/* rmsnorm (w given) + the activation quantiser of dt's kind on nt rows of x
 * (width n), then the token matmul into y [nt][W.rows] */
int pf_matmul(tlm_hip_model *M, const DevMat &W, const float *x, int64_t n, const float *w, int nt, float *y,
              int *act_kind) {
    const int kind = dt_act_kind(W.dt);
    const int64_t astride = (int64_t)act_bytes(kind, n);
    int rc = TLM_HIP_OK;
    if (*act_kind != kind) {
        rc = launch_tok_norm_act(kind, x, n, w, M->g.norm_eps, n, nt, M->pf_act, astride, M->stream);
        *act_kind = rc ? -1 : kind;
    }
    if (!rc) rc = launch_tokmm(W.dt, W.p, W.rows, n, M->pf_act, nt, y, M->stream);
    return rc;
}

/* Layer l's dense FFN for the chunk's nt tokens: the step's launches as
 * token matmuls (each token's values the step's bits) */
int pf_dense_ffn(tlm_hip_model *M, uint32_t l, int nt) {
    const Layer &Ly = M->L[l];
    const int64_t D = M->g.d_model, F = Ly.dffn;
    float *gb = M->pf_ffn, *ub = gb + (size_t)nt * F, *hb = ub + (size_t)nt * F;
    int ak = -1;
    int rc = pf_matmul(M, Ly.dg, M->pf_h, D, Ly.ffn_norm, nt, gb, &ak);
    if (!rc) rc = pf_matmul(M, Ly.du, M->pf_h, D, Ly.ffn_norm, nt, ub, &ak);
    if (rc) return rc;
    const int64_t cnt = (int64_t)nt * F;
    hipLaunchKernelGGL(k_dense_swiglu, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, M->stream, gb, ub, hb, cnt);
    if ((rc = tlmh_check(hipGetLastError(), "model prefill: dense swiglu"))) return rc;
    ak = -1;
    rc = pf_matmul(M, Ly.dd, hb, F, nullptr, nt, M->pf_y, &ak);
    if (!rc) {
        const int64_t c2 = (int64_t)nt * D;
        hipLaunchKernelGGL(k_pf_add, dim3((unsigned)((c2 + NT * 4 - 1) / (NT * 4))), dim3(NT), 0, M->stream, M->pf_h,
                           (const float *)M->pf_y, c2);
        rc = tlmh_check(hipGetLastError(), "model prefill: dense residual");
    }
    return rc;
}

/* Layer l's MoE block for the chunk's nt tokens with the experts in the slot
 * cache: the routing stage, the (token, rank) expert ids back on the host, the
 * union of the chunk's experts in the order the steps would first select them
 * (token by token, rank order), acquired in passes of as many experts as the
 * unpinned slots hold (each pass's loads waited for on the stream, its expert
 * table - the pass's matrices, null for every other expert - copied up, the
 * grouped expert work for its experts, its slots released behind that work),
 * then the rank-order combine.  The (token, rank) results are the resident
 * block's bits whatever the pass split. */
int pf_moe_cached(tlm_hip_model *M, uint32_t l, int nt) {
    const tlm_hip_model_geom &g = M->g;
    hipStream_t s = M->stream;
    const int k = (int)g.top_k, E = (int)g.n_experts;
    tlm_hip_moe_desc d = M->descs[l];
    int rc = launch_moe_prefill_route(&d, M->pf_h, nt, M->pf_ids, M->pf_w, M->pf_ws, s);
    if (!rc)
        rc = tlmh_check(hipMemcpyAsync(M->pf_host_ids, M->pf_ids, (size_t)nt * k * 4, hipMemcpyDeviceToHost, s),
                        "model prefill: routes");
    if (!rc) rc = tlmh_check(hipStreamSynchronize(s), "model prefill: routes");
    if (rc) return rc;
    std::vector<int> order;
    std::vector<char> seen(E, 0);
    for (int i = 0; i < nt * k; i++) {
        const int e = M->pf_host_ids[i];
        if (e < 0 || e >= E) return tlmh_seterr(TLM_HIP_EIO, "model prefill: routing produced expert %d of %d", e, E);
        if (!seen[e]) {
            seen[e] = 1;
            order.push_back(e);
        }
    }
    tlm_hip_store_stats ss;
    tlm_hip_store_get_stats(M->xs, &ss);
    const int per = std::max(1, ss.slots - ss.pinned);
    const size_t tabn = (size_t)3 * E;
    std::vector<tlm_hip_expert_ref> refs;
    for (int p0 = 0, pass = 0; p0 < (int)order.size() && !rc; p0 += per, pass++) {
        const int np = std::min(per, (int)order.size() - p0);
        refs.assign(np, tlm_hip_expert_ref{});
        rc = tlm_hip_store_acquire(M->xs, (int)l, order.data() + p0, np, refs.data());
        for (int i = 0; i < np && !rc; i++) rc = tlm_hip_store_stream_wait(M->xs, &refs[i], s);
        const void **ht = M->pf_host_tab + (size_t)pass * tabn;
        const void **dt = M->pf_dev_tab + (size_t)pass * tabn;
        if (!rc) {
            for (size_t i = 0; i < tabn; i++) ht[i] = nullptr;
            for (int i = 0; i < np; i++)
                for (int m = 0; m < 3; m++) ht[3 * (size_t)order[p0 + i] + m] = refs[i].mats[m];
            rc = tlmh_check(hipMemcpyAsync(dt, ht, tabn * sizeof(void *), hipMemcpyHostToDevice, s),
                            "model prefill: expert table");
        }
        if (!rc) {
            d.experts = dt;
            rc = launch_moe_prefill_experts(&d, nt, M->pf_ws, s);
        }
        for (int i = 0; i < np; i++)
            if (refs[i].slot >= 0) tlm_hip_store_release(M->xs, &refs[i], s);
    }
    if (!rc) rc = launch_moe_prefill_combine(&d, M->pf_h, nt, M->pf_ws, s);
    return rc;
}

/* tokens seq[p0 .. p0 + n) (already on the device) through the model, from
 * position p0; the step's tail on the last one */
int prefill_batched(tlm_hip_model *M, int p0, int n, bool want_logits) {
    if (int rc = pf_alloc(M)) return rc;
    const tlm_hip_model_geom &g = M->g;
    const int D = (int)g.d_model, hd = (int)g.head_dim, H = (int)g.n_heads, KV = (int)g.n_kv_heads;
    const int k = (int)g.top_k;
    hipStream_t s = M->stream;
    int rc = TLM_HIP_OK;
    int nt = 0;
    /* chunks of equal length (a multiple of 4 up to the buffers' pf_cap): a
     * short last chunk would run its long causal chains on a few groups */
    const int nch = (n + M->pf_cap - 1) / M->pf_cap;
    int per = (n + nch - 1) / nch;
    per = (per + 3) & ~3;
    per = per > M->pf_cap ? M->pf_cap : per;
    const size_t L = g.n_layers;
    for (int c0 = 0; c0 < n && !rc; c0 += per) {
        nt = n - c0 < per ? n - c0 : per;
        const int pc = p0 + c0;
        stamp(M, 0);
        hipLaunchKernelGGL(k_pf_embed, dim3((D + NT - 1) / NT, nt), dim3(NT), 0, s, M->embd, M->embd_row, M->embd_dt,
                           (const int32_t *)M->seq + pc, D, M->pf_h);
        rc = tlmh_check(hipGetLastError(), "model prefill: embed");
        for (uint32_t l = 0; l < g.n_layers && !rc; l++) {
            const Layer &Ly = M->L[l];
            int ak = -1;
            stamp(M, 1 + 2 * (size_t)l);
            if (Ly.q.dt == Ly.k.dt && Ly.q.dt == Ly.v.dt) {   /* q | k | v in one launch */
                const int kind = dt_act_kind(Ly.q.dt);
                rc = launch_tok_norm_act(kind, M->pf_h, D, Ly.attn_norm, g.norm_eps, D, nt, M->pf_act,
                                         (int64_t)act_bytes(kind, D), s);
                const void *W3[3] = {Ly.q.p, Ly.k.p, Ly.v.p};
                const int64_t R3[3] = {Ly.q.rows, Ly.k.rows, Ly.v.rows};
                float *const Y3[3] = {M->pf_q, M->pf_kx, M->pf_vx};
                if (!rc) rc = launch_tokmm_segs(Ly.q.dt, 3, W3, R3, D, M->pf_act, nt, Y3, s);
            } else {
                rc = pf_matmul(M, Ly.q, M->pf_h, D, Ly.attn_norm, nt, M->pf_q, &ak);
                if (!rc) rc = pf_matmul(M, Ly.k, M->pf_h, D, Ly.attn_norm, nt, M->pf_kx, &ak);
                if (!rc) rc = pf_matmul(M, Ly.v, M->pf_h, D, Ly.attn_norm, nt, M->pf_vx, &ak);
            }
            const size_t kbase = (size_t)l * KV * M->max_ctx * hd, vbase = (size_t)l * KV * att_vstride(M->max_ctx, hd);
            if (!rc)
                rc = launch_pf_attn(hd, H, KV, M->max_ctx, pc, nt, M->pf_q, M->pf_kx, M->pf_vx, Ly.q_norm, Ly.k_norm,
                                    M->cs, M->sn, M->kc + kbase, M->vc + vbase, M->pf_scores, M->pf_sl, M->pf_att,
                                    g.norm_eps, s);
            ak = -1;
            if (!rc) rc = pf_matmul(M, Ly.o, M->pf_att, (int64_t)H * hd, nullptr, nt, M->pf_y, &ak);
            if (!rc) {
                const int64_t cnt = (int64_t)nt * D;
                hipLaunchKernelGGL(k_pf_add, dim3((unsigned)((cnt + NT * 4 - 1) / (NT * 4))), dim3(NT), 0, s, M->pf_h,
                                   (const float *)M->pf_y, cnt);
                rc = tlmh_check(hipGetLastError(), "model prefill: residual");
            }
            stamp(M, 2 + 2 * (size_t)l);
            if (Ly.dense) {   /* the dense FFN, token by token's bits: gate, up, silu(gate) * up, down, + h */
                if (!rc) rc = pf_dense_ffn(M, l, nt);
                continue;
            }
            if (!rc)
                rc = M->xs ? pf_moe_cached(M, l, nt)
                           : launch_moe_prefill(&Ly.moe, M->pf_h, nt, M->pf_ids, M->pf_w, M->pf_ws, s);
            if (!rc && c0 + nt == n && M->xs) {   /* the last token's routing, on the host as the cached step keeps it */
                for (int r = 0; r < k; r++)
                    M->route_ids[(size_t)l * k + r] = M->pf_host_ids[(size_t)(nt - 1) * k + r];
                rc = tlmh_check(hipMemcpyAsync(M->route_w.data() + (size_t)l * k, M->pf_w + (size_t)(nt - 1) * k,
                                               (size_t)k * 4, hipMemcpyDeviceToHost, s), "model prefill: routes");
            } else if (!rc && c0 + nt == n) {   /* the last token's routing, as the step leaves it */
                rc = tlmh_check(hipMemcpyAsync(M->ids + (size_t)l * 32, M->pf_ids + (size_t)(nt - 1) * k, (size_t)k * 4,
                                               hipMemcpyDeviceToDevice, s), "model prefill: routes");
                if (!rc)
                    rc = tlmh_check(hipMemcpyAsync(M->w + (size_t)l * 32, M->pf_w + (size_t)(nt - 1) * k,
                                                   (size_t)k * 4, hipMemcpyDeviceToDevice, s), "model prefill: routes");
            }
        }
        stamp(M, 1 + 2 * L);
        if (c0 + nt < n) stamp_acc(M);   /* the last chunk's split takes the tail */
    }
    if (rc) return rc;
    rc = tlmh_check(hipMemcpyAsync(M->h, M->pf_h + (size_t)(nt - 1) * D, (size_t)D * 4, hipMemcpyDeviceToDevice, s),
                    "model prefill: h");
    if (rc) return rc;
    hipLaunchKernelGGL(k_set_pos, dim3(1), dim3(1), 0, s, M->st, p0 + n - 1);
    rc = enqueue_tail(M, want_logits);
    stamp_acc(M);
    if (!rc) rc = tlmh_check(hipGetLastError(), "model prefill: stats");
    if (!rc) {
        M->kv_len = p0 + n;
        M->st_tokens += (uint64_t)n;
        if (M->xs)   /* the steps' store ticks (tlm_model.c:1097), one per token */
            for (int i = 0; i < n; i++) tlm_hip_store_tick(M->xs);
    }
    return rc;
}

/* the n tokens at seq[kv_len ..]: batched where supported (and its chunk
 * buffers fit), else one step each */
int run_prompt(tlm_hip_model *M, int n, bool want_logits) {
    if (pf_supported(M)) {
        const int rc = pf_alloc(M);
        if (!rc) return prefill_batched(M, M->kv_len, n, want_logits);
        if (rc != TLM_HIP_ENOMEM) return rc;
        (void)hipGetLastError();   /* no room for the chunk buffers: step token by token */
    }
    int rc = TLM_HIP_OK;
    for (int i = 0; i < n && !rc; i++) rc = step(M, want_logits && i == n - 1);
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
    /* experts: one arena, 256-byte aligned matrices; or, with the slot cache,
     * payloads in the reference's row layout (gate | up | down) in page-locked
     * host memory, expert (l, e) reading payload (l E + e) mod pool - the same
     * bytes as the resident arena's when every expert has its own */
    const bool cached = M->xs_budget > 0;
    const size_t pg = (packed_bytes(edt, de, D) + 255) & ~(size_t)255, pd = (packed_bytes(edt, D, de) + 255) & ~(size_t)255;
    uint8_t *arena = nullptr;
    if (!cached) {
        arena = (uint8_t *)M->dalloc((size_t)g.n_layers * E * (2 * pg + pd));
        if (!arena) return tlmh_seterr(TLM_HIP_ENOMEM, "model synth: out of device memory for the experts");
    }
    const int ebv = dt_block_values(edt);
    const size_t rg = (size_t)(D / ebv) * dt_block_bytes(edt), rd = (size_t)(de / ebv) * dt_block_bytes(edt);
    const size_t plen = 2 * (size_t)de * rg + (size_t)D * rd, pst = (plen + 255) & ~(size_t)255;
    const int64_t nexp = (int64_t)g.n_layers * E;
    const int64_t pool = cached ? (so->expert_pool > 0 ? std::min<int64_t>(so->expert_pool, nexp) : nexp) : 0;
    if (cached) {
        if ((rc = tlmh_check(hipHostMalloc(&M->xs_payload, (size_t)pool * pst, hipHostMallocDefault),
                             "model synth: page-locked expert payloads")))
            return rc;
        M->xs_src.reserve((size_t)nexp);
    }
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
        if (so->heat_gamma > 0.0 && g.router == 2) {   /* bias -gamma ln(rank + 1), ranks a seeded permutation */
            std::vector<int> perm(E);
            for (int64_t e = 0; e < E; e++) perm[e] = (int)e;
            uint64_t r = next();
            for (int64_t e = E - 1; e > 0; e--) {   /* Fisher-Yates on the splitmix64 stream */
                r = mix64(r);
                std::swap(perm[e], perm[(int64_t)(r % (uint64_t)(e + 1))]);
            }
            std::vector<float> bias(E);
            for (int64_t e = 0; e < E; e++) bias[e] = (float)(-so->heat_gamma * log((double)perm[e] + 1.0));
            void *bp;
            if ((rc = dev_upload(M, bias.data(), bias.size() * 4, &bp))) return rc;
            d.router_bias = (const float *)bp;
        }
        d.expert_dt = edt;
        for (int64_t e = 0; e < E && !rc; e++) {
            const uint64_t s1 = next(), s2 = next(), s3 = next();
            if (cached) {
                const int64_t slot = ((int64_t)l * E + e) % pool;
                uint8_t *hp = (uint8_t *)M->xs_payload + (size_t)slot * pst;
                if ((int64_t)l * E + e < pool) {   /* this payload's bytes, as the arena would hold them */
                    const uint64_t seeds[3] = {s1, s2, s3};
                    const int64_t rows[3] = {de, de, D}, n[3] = {D, D, de};
                    const size_t off[3] = {0, (size_t)de * rg, 2 * (size_t)de * rg};
                    const size_t bytes[3] = {(size_t)de * rg, (size_t)de * rg, (size_t)D * rd};
                    for (int k = 0; k < 3 && !rc; k++) {
                        rc = synth_rows(M->stream, edt, tmp, rows[k], n[k], seeds[k]);
                        if (!rc) rc = tlmh_check(hipMemcpyAsync(hp + off[k], tmp, bytes[k], hipMemcpyDeviceToHost,
                                                                M->stream), "model synth: payload");
                        if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model synth: payload");
                    }
                    if (rc) return rc;
                }
                tlm_hip_expert_src x{};
                x.layer = (uint16_t)l;
                x.id = (uint32_t)e;
                x.dtype = edt;
                x.item_off[0] = 0;
                x.item_off[1] = (uint32_t)((size_t)de * rg);
                x.item_off[2] = (uint32_t)(2 * (size_t)de * rg);
                x.payload_len = plen;
                x.payload = hp;
                M->xs_src.push_back(x);
                continue;
            }
            uint8_t *base = arena + ((size_t)l * E + e) * (2 * pg + pd);
            DevMat dm;
            if ((rc = synth_matrix(M, edt, de, D, s1, tmp, base, &dm)) ||
                (rc = synth_matrix(M, edt, de, D, s2, tmp, base + pg, &dm)) ||
                (rc = synth_matrix(M, edt, D, de, s3, tmp, base + 2 * pg, &dm)))
                return rc;
            table[3 * e] = base;
            table[3 * e + 1] = base + pg;
            table[3 * e + 2] = base + 2 * pg;
        }
        if (!cached) {
            void *tp;
            if ((rc = dev_upload(M, table.data(), table.size() * sizeof(void *), &tp))) return rc;
            d.experts = (const void *const *)tp;
        }
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
    if (cached && (rc = open_expert_store(M))) return rc;
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

int tlm_hip_model_routes(tlm_hip_model *M, int32_t *ids, float *w) {
    if (!M || !ids || !w) return tlmh_seterr(TLM_HIP_EINVAL, "model routes: NULL argument");
    const int L = (int)M->g.n_layers, k = (int)M->g.top_k;
    if (M->xs) {   /* the cached step read them on the host */
        int rc = tlmh_check(hipStreamSynchronize(M->stream), "model routes");
        if (rc) return rc;
        memcpy(ids, M->route_ids.data(), (size_t)L * k * 4);
        memcpy(w, M->route_w.data(), (size_t)L * k * 4);
        return TLM_HIP_OK;
    }
    std::vector<int32_t> di((size_t)L * 32);
    std::vector<float> dw((size_t)L * 32);
    int rc = tlmh_check(hipStreamSynchronize(M->stream), "model routes");
    if (!rc) rc = tlmh_check(hipMemcpy(di.data(), M->ids, di.size() * 4, hipMemcpyDeviceToHost), "model routes");
    if (!rc) rc = tlmh_check(hipMemcpy(dw.data(), M->w, dw.size() * 4, hipMemcpyDeviceToHost), "model routes");
    if (rc) return rc;
    for (int l = 0; l < L; l++)
        for (int r = 0; r < k; r++) {
            ids[(size_t)l * k + r] = di[(size_t)l * 32 + r];
            w[(size_t)l * k + r] = dw[(size_t)l * 32 + r];
        }
    return TLM_HIP_OK;
}
int tlm_hip_model_rewind(tlm_hip_model *M, int len) {
    if (!M) return tlmh_seterr(TLM_HIP_EINVAL, "model rewind: NULL");
    if (len < 0 || len > M->kv_len)
        return tlmh_seterr(TLM_HIP_ERANGE, "model rewind: %d positions, the context holds %d", len, M->kv_len);
    if (len == M->kv_len) return TLM_HIP_OK;
    hipLaunchKernelGGL(k_set_pos, dim3(1), dim3(1), 0, M->stream, M->st, len);
    int rc = tlmh_check(hipGetLastError(), "model rewind");
    if (!rc) M->kv_len = len;
    return rc;
}

int tlm_hip_model_decode(tlm_hip_model *M, int n) {
    if (!M || n < 0) return tlmh_seterr(TLM_HIP_EINVAL, "model decode: bad arguments");
    if (M->kv_len == 0) return tlmh_seterr(TLM_HIP_EINVAL, "model decode: no token yet (prefill first)");
    if ((int64_t)M->kv_len + n > M->max_ctx)
        return tlmh_seterr(TLM_HIP_ERANGE, "model decode: %d + %d tokens exceed the context (%d)", M->kv_len, n,
                           M->max_ctx);
    int rc = TLM_HIP_OK;
    for (int i = 0; i < n && !rc; i++) rc = step(M, true);
    return rc;
}

int tlm_hip_model_sync(tlm_hip_model *M) {
    return M ? tlmh_check(hipStreamSynchronize(M->stream), "model sync") : TLM_HIP_OK;
}

void *tlm_hip_model_stream(const tlm_hip_model *M) { return M ? (void *)M->stream : nullptr; }
tlm_hip_store *tlm_hip_model_expert_store(const tlm_hip_model *M) { return M ? M->xs : nullptr; }

int tlm_hip_model_get_stats(tlm_hip_model *M, tlm_hip_model_stats *out) {
    if (!M || !out) return tlmh_seterr(TLM_HIP_EINVAL, "model stats: NULL argument");
    memset(out, 0, sizeof *out);
    int rc = tlmh_check(hipStreamSynchronize(M->stream), "model stats");
    if (rc) return rc;
    out->tokens = M->st_tokens;
    if (M->stats) {
        uint64_t acc[3];
        rc = tlmh_check(hipMemcpy(acc, M->stamps + 2 * (size_t)M->g.n_layers + 2, sizeof acc, hipMemcpyDeviceToHost),
                        "model stats");
        if (rc) return rc;
        out->attn_ns = acc[0];
        out->moe_ns = acc[1];
        out->other_ns = acc[2];
    }
    if (M->xs) {
        tlm_hip_store_stats ss;
        tlm_hip_store_get_stats(M->xs, &ss);
        out->expert_wait_ns = ss.wait_ns - M->st_wait0;
    }
    return TLM_HIP_OK;
}

void tlm_hip_model_reset_stats(tlm_hip_model *M) {
    if (!M) return;
    (void)hipStreamSynchronize(M->stream);
    M->st_tokens = 0;
    if (M->stats) {
        const uint64_t z[3] = {0, 0, 0};
        (void)hipMemcpy(M->stamps + 2 * (size_t)M->g.n_layers + 2, z, sizeof z, hipMemcpyHostToDevice);
    }
    if (M->xs) {
        tlm_hip_store_stats ss;
        tlm_hip_store_get_stats(M->xs, &ss);
        M->st_wait0 = ss.wait_ns;
    }
}

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

int tlm_hip_model_prefill_batched(const tlm_hip_model *M) { return M && pf_supported(M) ? 1 : 0; }

int tlm_hip_model_prefill(tlm_hip_model *M, const int32_t *tokens, int n, float *logits) {
    if (!M || !tokens || n <= 0) return tlmh_seterr(TLM_HIP_EINVAL, "prefill: no tokens");
    const int pos0 = M->kv_len;
    if ((int64_t)pos0 + n > M->max_ctx)
        return tlmh_seterr(TLM_HIP_ERANGE, "model prefill: %d + %d tokens exceed the context (%d)", pos0, n,
                           M->max_ctx);
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= M->g.vocab)
            return tlmh_seterr(TLM_HIP_EINVAL, "token %d out of range", tokens[i]);
    int rc = tlmh_check(hipMemcpy(M->seq + pos0, tokens, (size_t)n * 4, hipMemcpyHostToDevice), "model: prompt");
    if (!rc) rc = run_prompt(M, n, logits != nullptr);
    if (!rc && logits)
        rc = tlmh_check(hipMemcpyAsync(logits, M->logits, (size_t)M->g.vocab * 4, hipMemcpyDeviceToHost, M->stream),
                        "model: logits");
    if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model: prefill");
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
    if (!rc) rc = run_prompt(M, n_prompt, n_gen > 0);
    for (int gi = 1; gi < n_gen && !rc; gi++) rc = step(M, true);
    if (!rc && n_gen > 0)
        rc = tlmh_check(hipMemcpyAsync(out, M->seq + pos0 + n_prompt, (size_t)n_gen * 4, hipMemcpyDeviceToHost,
                                       M->stream), "model: out");
    if (!rc) rc = tlmh_check(hipStreamSynchronize(M->stream), "model: generate");
    return rc;
}

}  // extern "C"
