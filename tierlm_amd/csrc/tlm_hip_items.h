/* tlm_hip_items.h - device-side building blocks shared by the GEMV and MoE
 * kernels: the activation staged in LDS, and the per-item integer kernels of
 * the packed layout.  An item is one (row, block) of one matrix, handled by
 * LPI lanes; each format splits into load() (global -> registers, 16-byte
 * vector loads) and compute() (registers + LDS -> exact int32 sums and the
 * float factors of the reference's chain), so a lane can put every item's
 * loads in flight before it waits on any of them.  Included by .hip files. */
#ifndef TLM_HIP_ITEMS_H
#define TLM_HIP_ITEMS_H

#include "tlm_hip_internal.h"

/* ---- activation block staged in LDS ---------------------------------------
 * Q8_K: codes [nb][256] bytes, bsums [nb][16] int16, d [nb] float.
 * a8:   codes [nb][32] bytes, d [nb] float. */
struct XLds {
    const LAS int8_t  *q;
    const LAS int16_t *bs;
    const LAS float   *d;
};

__host__ __device__ static inline size_t stage_bytes(int kind, int nb) {
    return kind == DT_Q8_K ? (size_t)nb * (256 + 32 + 4) : (size_t)nb * (32 + 4);
}

__device__ __forceinline__ static XLds xlds_at(int kind, int nb, uint8_t *lds_generic) {
    XLds X;
    LAS uint8_t *lds = (LAS uint8_t *)lds_generic;
    if (kind == DT_Q8_K) {
        X.q = (const LAS int8_t *)lds;
        X.bs = (const LAS int16_t *)(lds + nb * 256);
        X.d = (const LAS float *)(lds + nb * 256 + nb * 32);
    } else {
        X.q = (const LAS int8_t *)lds;
        X.bs = nullptr;
        X.d = (const LAS float *)(lds + nb * 32);
    }
    return X;
}

/* Copy nb activation blocks (global, reference layout) into the LDS layout;
 * every thread of the group takes part; the caller synchronises. */
static __device__ __forceinline__ XLds stage_act(int kind, const uint8_t *__restrict__ act, int nb, uint8_t *lds_g) {
    const int tid = threadIdx.x, nt = GROUP_THREADS;
    const GAS uint32_t *a = (const GAS uint32_t *)act;
    LAS uint8_t *lds = (LAS uint8_t *)lds_g;
    if (kind == DT_Q8_K) {
        LAS uint32_t *q = (LAS uint32_t *)lds;
        LAS uint32_t *bs = (LAS uint32_t *)(lds + nb * 256);
        LAS float *d = (LAS float *)(lds + nb * 256 + nb * 32);
        for (int k = tid; k < nb * 73; k += nt) {
            int b = k / 73, j = k - b * 73;
            uint32_t v = a[k];
            if (j == 0) d[b] = __uint_as_float(v);
            else if (j <= 64) q[b * 64 + (j - 1)] = v;
            else bs[b * 8 + (j - 65)] = v;
        }
    } else {
        LAS uint32_t *q = (LAS uint32_t *)lds;
        LAS float *d = (LAS float *)(lds + nb * 32);
        for (int k = tid; k < nb * 9; k += nt) {
            int b = k / 9, j = k - b * 9;
            uint32_t v = a[k];
            if (j == 0) d[b] = __uint_as_float(v);
            else q[b * 8 + (j - 1)] = v;
        }
    }
    return xlds_at(kind, nb, lds_g);
}

/* ---- per-item kernels on the packed layout ---------------------------------
 * Packed<DT>::load(Wp, units, u, q) reads lane q's share of unit u;
 * Packed<DT>::compute(raw, X, b, q, ...) returns, identically in the LPI
 * lanes of the item, the block's isum (and msum) and d_w * d_a (dmin_w * d_a). */
template <int DT> struct Packed;

template <> struct Packed<DT_Q6_K> {
    static constexpr int LPI = 4, BV = 256;
    struct Raw { u32x4 A, B, C; u32x2 S; uint32_t dw; };
    __device__ static __forceinline__ Raw load(const uint8_t *__restrict__ Wp, int64_t units, int64_t u, int q) {
        Raw r;
        const GAS uint8_t *W = (const GAS uint8_t *)Wp;
        const GAS uint8_t *unit = W + u * 208;
        const int h = q >> 1, p = q & 1;
        r.A = *(const GAS u32x4 *)(unit + 64 * h + 16 * p);
        r.B = *(const GAS u32x4 *)(unit + 64 * h + 32 + 16 * p);
        r.C = *(const GAS u32x4 *)(unit + 128 + 32 * h + 16 * p);
        r.S = *(const GAS u32x2 *)(unit + 192 + 8 * h);
        r.dw = *(const GAS uint16_t *)(W + units * 208 + u * 2);
        return r;
    }
    __device__ static __forceinline__ void compute(const Raw &r, const XLds &X, int b, int q, int32_t &is,
                                                   int32_t &ms, float &dA, float &dM) {
        const int h = q >> 1, p = q & 1;
        const LAS int8_t *xq = X.q + b * 256 + 128 * h + 16 * p;
        const u32x4 X0 = *(const LAS u32x4 *)(xq), X1 = *(const LAS u32x4 *)(xq + 32);
        const u32x4 X2 = *(const LAS u32x4 *)(xq + 64), X3 = *(const LAS u32x4 *)(xq + 96);
        const uint32_t a[4] = {r.A.x, r.A.y, r.A.z, r.A.w}, bq[4] = {r.B.x, r.B.y, r.B.z, r.B.w};
        const uint32_t c[4] = {r.C.x, r.C.y, r.C.z, r.C.w};
        const uint32_t x0[4] = {X0.x, X0.y, X0.z, X0.w}, x1[4] = {X1.x, X1.y, X1.z, X1.w};
        const uint32_t x2[4] = {X2.x, X2.y, X2.z, X2.w}, x3[4] = {X3.x, X3.y, X3.z, X3.w};
        int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            /* element 128h+16p+4j+k: low nibble of A (+0), of B (+32), high
             * nibble of A (+64), of B (+96), with 2-bit fields of C on top */
            uint32_t u0 = (a[j] & 0x0F0F0F0Fu) | ((c[j] << 4) & 0x30303030u);
            uint32_t u1 = (bq[j] & 0x0F0F0F0Fu) | ((c[j] << 2) & 0x30303030u);
            uint32_t u2 = ((a[j] >> 4) & 0x0F0F0F0Fu) | (c[j] & 0x30303030u);
            uint32_t u3 = ((bq[j] >> 4) & 0x0F0F0F0Fu) | ((c[j] >> 2) & 0x30303030u);
            s0 = dot4((int)u0, (int)x0[j], s0);
            s1 = dot4((int)u1, (int)x1[j], s1);
            s2 = dot4((int)u2, (int)x2[j], s2);
            s3 = dot4((int)u3, (int)x3[j], s3);
        }
        /* groups 8h+p, 8h+2+p, 8h+4+p, 8h+6+p: scale bytes p, p+2, p+4, p+6 of S */
        const LAS int16_t *bs = X.bs + b * 16 + 8 * h + p;
        const uint32_t sw0 = r.S.x >> (8 * p), sw1 = r.S.y >> (8 * p);
        const int sc0 = (int8_t)(sw0 & 0xFF), sc1 = (int8_t)((sw0 >> 16) & 0xFF);
        const int sc2 = (int8_t)(sw1 & 0xFF), sc3 = (int8_t)((sw1 >> 16) & 0xFF);
        int part = sc0 * (s0 - 32 * (int)bs[0]) + sc1 * (s1 - 32 * (int)bs[2]) +
                   sc2 * (s2 - 32 * (int)bs[4]) + sc3 * (s3 - 32 * (int)bs[6]);
        part += (int)dpp_u32<DPP_XOR1>((uint32_t)part);
        part += (int)dpp_u32<DPP_XOR2>((uint32_t)part);
        is = part;
        ms = 0;
        dA = f16_to_f32(r.dw) * X.d[b];
        dM = 0.0f;
    }
};

template <> struct Packed<DT_Q8_0> {
    static constexpr int LPI = 2, BV = 32;
    struct Raw { u32x4 W; uint32_t dw; };
    __device__ static __forceinline__ Raw load(const uint8_t *__restrict__ Wp, int64_t units, int64_t u, int q) {
        Raw r;
        const GAS uint8_t *W = (const GAS uint8_t *)Wp;
        r.W = *(const GAS u32x4 *)(W + u * 32 + 16 * q);
        r.dw = *(const GAS uint16_t *)(W + units * 32 + u * 2);
        return r;
    }
    __device__ static __forceinline__ void compute(const Raw &r, const XLds &X, int b, int q, int32_t &is,
                                                   int32_t &ms, float &dA, float &dM) {
        const u32x4 Xv = *(const LAS u32x4 *)(X.q + b * 32 + 16 * q);
        int s = dot4((int)r.W.x, (int)Xv.x, 0);
        s = dot4((int)r.W.y, (int)Xv.y, s);
        s = dot4((int)r.W.z, (int)Xv.z, s);
        s = dot4((int)r.W.w, (int)Xv.w, s);
        s += (int)dpp_u32<DPP_XOR1>((uint32_t)s);
        is = s;
        ms = 0;
        dA = f16_to_f32(r.dw) * X.d[b];
        dM = 0.0f;
    }
};

/* Q4_K / Q5_K: lane c takes 64-element chunk c (sub-blocks 2c, 2c+1). */
template <int DT> struct PackedKQ {
    static constexpr int LPI = 4, BV = 256;
    static constexpr bool Q5 = DT == DT_Q5_K;
    static constexpr int BB = Q5 ? 176 : 144, QS = Q5 ? 48 : 16;
    struct Raw { u32x4 H, Q0, Q1, P0, P1; };
    __device__ static __forceinline__ Raw load(const uint8_t *__restrict__ Wp, int64_t units, int64_t u, int c) {
        Raw r;
        const GAS uint8_t *blk = (const GAS uint8_t *)Wp + u * BB;
        r.H = *(const GAS u32x4 *)blk;
        r.Q0 = *(const GAS u32x4 *)(blk + QS + 32 * c);
        r.Q1 = *(const GAS u32x4 *)(blk + QS + 32 * c + 16);
        if (Q5) {
            r.P0 = *(const GAS u32x4 *)(blk + 16);
            r.P1 = *(const GAS u32x4 *)(blk + 32);
        } else {
            r.P0 = u32x4{0, 0, 0, 0};
            r.P1 = r.P0;
        }
        return r;
    }
    __device__ static __forceinline__ void compute(const Raw &r, const XLds &X, int b, int c, int32_t &is,
                                                   int32_t &ms, float &dA, float &dM) {
        const uint32_t qw[8] = {r.Q0.x, r.Q0.y, r.Q0.z, r.Q0.w, r.Q1.x, r.Q1.y, r.Q1.z, r.Q1.w};
        const uint32_t qh[8] = {r.P0.x, r.P0.y, r.P0.z, r.P0.w, r.P1.x, r.P1.y, r.P1.z, r.P1.w};
        const LAS int8_t *xq = X.q + b * 256 + 64 * c;
        const u32x4 XL0 = *(const LAS u32x4 *)(xq), XL1 = *(const LAS u32x4 *)(xq + 16);
        const u32x4 XH0 = *(const LAS u32x4 *)(xq + 32), XH1 = *(const LAS u32x4 *)(xq + 48);
        const uint32_t xl[8] = {XL0.x, XL0.y, XL0.z, XL0.w, XL1.x, XL1.y, XL1.z, XL1.w};
        const uint32_t xh[8] = {XH0.x, XH0.y, XH0.z, XH0.w, XH1.x, XH1.y, XH1.z, XH1.w};
        int slo = 0, shi = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t lo = qw[j] & 0x0F0F0F0Fu, hi = (qw[j] >> 4) & 0x0F0F0F0Fu;
            if (Q5) {
                lo |= ((qh[j] >> (2 * c)) & 0x01010101u) << 4;
                hi |= ((qh[j] >> (2 * c + 1)) & 0x01010101u) << 4;
            }
            slo = dot4((int)lo, (int)xl[j], slo);
            shi = dot4((int)hi, (int)xh[j], shi);
        }
        /* 6-bit scales/mins of sub-blocks 2c, 2c+1 (src/lib/tlm_quant.c:253-261) */
        const uint32_t w1 = r.H.y, w2 = r.H.z, w3 = r.H.w;    /* s12 bytes 0..3, 4..7, 8..11 */
        int sc[2], mn[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int sb = 2 * c + k;
            if (sb < 4) {
                sc[k] = (w1 >> (8 * sb)) & 63;
                mn[k] = (w2 >> (8 * sb)) & 63;
            } else {
                const int j = sb - 4;
                sc[k] = ((w3 >> (8 * j)) & 15) | (((w1 >> (8 * j + 6)) & 3) << 4);
                mn[k] = ((w3 >> (8 * j + 4)) & 15) | (((w2 >> (8 * j + 6)) & 3) << 4);
            }
        }
        const LAS int16_t *bs = X.bs + b * 16 + 4 * c;
        int part = sc[0] * slo + sc[1] * shi;
        int mpart = mn[0] * ((int)bs[0] + (int)bs[1]) + mn[1] * ((int)bs[2] + (int)bs[3]);
        part += (int)dpp_u32<DPP_XOR1>((uint32_t)part);
        part += (int)dpp_u32<DPP_XOR2>((uint32_t)part);
        mpart += (int)dpp_u32<DPP_XOR1>((uint32_t)mpart);
        mpart += (int)dpp_u32<DPP_XOR2>((uint32_t)mpart);
        is = part;
        ms = mpart;
        const float da = X.d[b];
        dA = f16_to_f32(r.H.x & 0xFFFFu) * da;
        dM = f16_to_f32(r.H.x >> 16) * da;
    }
};
template <> struct Packed<DT_Q4_K> : PackedKQ<DT_Q4_K> {};
template <> struct Packed<DT_Q5_K> : PackedKQ<DT_Q5_K> {};

/* Q8_K weights (4-byte aligned 292-byte blocks): lane q takes codes 64q..64q+63. */
template <> struct Packed<DT_Q8_K> {
    static constexpr int LPI = 4, BV = 256;
    struct Raw { uint32_t w[16]; uint32_t d; };
    __device__ static __forceinline__ Raw load(const uint8_t *__restrict__ Wp, int64_t units, int64_t u, int q) {
        Raw r;
        const GAS uint32_t *blk = (const GAS uint32_t *)(Wp + u * 292);
#pragma unroll
        for (int j = 0; j < 16; j++) r.w[j] = blk[1 + 16 * q + j];
        r.d = blk[0];
        return r;
    }
    __device__ static __forceinline__ void compute(const Raw &r, const XLds &X, int b, int q, int32_t &is,
                                                   int32_t &ms, float &dA, float &dM) {
        const LAS uint32_t *xq = (const LAS uint32_t *)(X.q + b * 256 + 64 * q);
        int s = 0;
#pragma unroll
        for (int j = 0; j < 16; j++) s = dot4((int)r.w[j], (int)xq[j], s);
        s += (int)dpp_u32<DPP_XOR1>((uint32_t)s);
        s += (int)dpp_u32<DPP_XOR2>((uint32_t)s);
        is = s;
        ms = 0;
        dA = __uint_as_float(r.d) * X.d[b];
        dM = 0.0f;
    }
};

/* ---- parked item results in LDS: [item] for one matrix tile ---------------- */
struct Park {
    LAS int32_t *is, *ms;
    LAS float *da, *dm;
};
__host__ __device__ static inline size_t park_bytes(int nitems) { return (size_t)nitems * 16; }
__device__ __forceinline__ static Park park_at(uint8_t *p, int nitems) {
    Park k;
    k.is = (LAS int32_t *)p;
    k.ms = k.is + nitems;
    k.da = (LAS float *)(k.ms + nitems);
    k.dm = k.da + nitems;
    return k;
}

/* Items it = slot + SLOTS*j (j < IPL) of a list of nitems (>= 1).  map(it,
 * W, units, u, b, pk) names the item's packed matrix, its unit, its
 * activation block and its park slot.  Every load is issued first; then
 * stage() runs (it fills the LDS activation while the loads are in flight
 * and returns it); then every compute.  Lanes of an item share `it`, so
 * shuffles stay in-item.  Items past the end are skipped, or with CLAMP
 * load the last item's bytes and are dropped: with many items per lane the
 * compiler keeps branch-free loads in flight together, where a branch per
 * item made it wait between them.  Returns the XLds that stage() produced. */
template <int DT, int IPL, bool CLAMP = false, class Map, class Stage>
__device__ __forceinline__ XLds run_items(int nitems, Map map, Stage stage, Park park) {
    using F = Packed<DT>;
    constexpr bool AFF = DT == DT_Q4_K || DT == DT_Q5_K;
    const int slots = GROUP_THREADS / F::LPI;
    const int q = threadIdx.x % F::LPI, slot = threadIdx.x / F::LPI;
    typename F::Raw raw[IPL];
    int bb[IPL], pk[IPL];
#pragma unroll
    for (int j = 0; j < IPL; j++) {
        const int it = slot + slots * j;
        const uint8_t *W;
        int64_t units, u;
        if constexpr (CLAMP) {
            map(it < nitems ? it : nitems - 1, W, units, u, bb[j], pk[j]);
            if (it >= nitems) pk[j] = -1;
            raw[j] = F::load(W, units, u, q);
        } else {
            pk[j] = -1;
            bb[j] = 0;
            if (it < nitems) {
                map(it, W, units, u, bb[j], pk[j]);
                raw[j] = F::load(W, units, u, q);
            }
        }
    }
    const XLds X = stage();
#pragma unroll
    for (int j = 0; j < IPL; j++) {
        if (pk[j] >= 0) {
            int32_t is, ms;
            float dA, dM;
            F::compute(raw[j], X, bb[j], q, is, ms, dA, dM);
            if (q == 0) {
                park.is[pk[j]] = is;
                park.da[pk[j]] = dA;
                if (AFF) { park.ms[pk[j]] = ms; park.dm[pk[j]] = dM; }
            }
        }
    }
    return X;
}

/* Row i's float chain continued over nb parked blocks in ascending order:
 * the reference's per-row fma sequence (acc = fmaf(d_w d_a, isum, acc), then
 * for Q4_K / Q5_K acc = fmaf(-dmin_w d_a, msum, acc)); park index
 * o + b * stride + i.  Eight blocks' values are read before their fmas so
 * the LDS reads overlap; the fma order is unchanged. */
template <bool AFF>
__device__ __forceinline__ float chain_park(const Park &k, int nb, int o, int stride, int i, float acc) {
    int b = 0;
    for (; b + 8 <= nb; b += 8) {
        float da[8], dm[8];
        int32_t is[8], ms[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int p = o + (b + u) * stride + i;
            da[u] = k.da[p];
            is[u] = k.is[p];
            if (AFF) {
                dm[u] = k.dm[p];
                ms[u] = k.ms[p];
            }
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            acc = fmaf(da[u], (float)is[u], acc);
            if (AFF) acc = fmaf(-dm[u], (float)ms[u], acc);
        }
    }
    for (; b < nb; b++) {
        const int p = o + b * stride + i;
        acc = fmaf(k.da[p], (float)k.is[p], acc);
        if (AFF) acc = fmaf(-k.dm[p], (float)k.ms[p], acc);
    }
    return acc;
}

#endif
