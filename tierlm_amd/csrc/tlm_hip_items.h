/* tlm_hip_items.h - device-side building blocks shared by the GEMV and MoE
 * kernels: the staged activation block in LDS and the per-item integer
 * kernels of the packed layout (one (row, block) item per LPI lanes).
 * Included by .hip files only. */
#ifndef TLM_HIP_ITEMS_H
#define TLM_HIP_ITEMS_H

#include "tlm_hip_internal.h"

/* ---- activation block staged in LDS -------------------------------------
 * Q8_K: codes [nb][256] bytes, bsums [nb][16] int16, d [nb] float.
 * a8:   codes [nb][32] bytes, d [nb] float. */
struct XLds {
    const int8_t  *q;
    const int16_t *bs;
    const float   *d;
};

static __device__ __forceinline__ XLds stage_act(int kind, const uint8_t *__restrict__ act, int nb, uint8_t *lds) {
    XLds X;
    const int tid = threadIdx.x, nt = blockDim.x;
    if (kind == DT_Q8_K) {
        uint32_t *q = (uint32_t *)lds;
        uint32_t *bs = (uint32_t *)(lds + nb * 256);
        float *d = (float *)(lds + nb * 256 + nb * 32);
        const uint32_t *a = (const uint32_t *)act;
        for (int k = tid; k < nb * 73; k += nt) {
            int b = k / 73, j = k - b * 73;
            uint32_t v = a[k];
            if (j == 0) d[b] = __uint_as_float(v);
            else if (j <= 64) q[b * 64 + (j - 1)] = v;
            else bs[b * 8 + (j - 65)] = v;
        }
        X.q = (const int8_t *)q;
        X.bs = (const int16_t *)bs;
        X.d = d;
    } else {
        uint32_t *q = (uint32_t *)lds;
        float *d = (float *)(lds + nb * 32);
        const uint32_t *a = (const uint32_t *)act;
        for (int k = tid; k < nb * 9; k += nt) {
            int b = k / 9, j = k - b * 9;
            uint32_t v = a[k];
            if (j == 0) d[b] = __uint_as_float(v);
            else q[b * 8 + (j - 1)] = v;
        }
        X.q = (const int8_t *)q;
        X.bs = nullptr;
        X.d = d;
    }
    return X;
}

__host__ __device__ static inline size_t stage_bytes(int kind, int nb) {
    return kind == DT_Q8_K ? (size_t)nb * (256 + 32 + 4) : (size_t)nb * (32 + 4);
}

/* ---- per-item integer kernels on the packed layout ----------------------
 * An item is (tile t, block b, row i) for one matrix.  LPI lanes cooperate
 * on an item; `q` is the lane's index within the item.  Outputs (identical
 * in all LPI lanes after the reduction): isum, msum, and the float factors. */
template <int DT> struct Packed;

template <> struct Packed<DT_Q6_K> {
    static constexpr int LPI = 4, BV = 256;
    __device__ static __forceinline__ void item(const uint8_t *__restrict__ Wp, int64_t units, int64_t u, int b,
                                                int q, const XLds &X, int32_t &is, int32_t &ms, float &dA,
                                                float &dM) {
        const uint8_t *unit = Wp + u * 208;
        const int h = q >> 1, p = q & 1;
        const uint4 A = *(const uint4 *)(unit + 64 * h + 16 * p);
        const uint4 B = *(const uint4 *)(unit + 64 * h + 32 + 16 * p);
        const uint4 C = *(const uint4 *)(unit + 128 + 32 * h + 16 * p);
        const uint2 S = *(const uint2 *)(unit + 192 + 8 * h);
        const uint32_t dw = *(const uint16_t *)(Wp + units * 208 + u * 2);
        const int8_t *xq = X.q + b * 256 + 128 * h + 16 * p;
        const uint4 X0 = *(const uint4 *)(xq), X1 = *(const uint4 *)(xq + 32);
        const uint4 X2 = *(const uint4 *)(xq + 64), X3 = *(const uint4 *)(xq + 96);
        const uint32_t a[4] = {A.x, A.y, A.z, A.w}, bq[4] = {B.x, B.y, B.z, B.w}, c[4] = {C.x, C.y, C.z, C.w};
        const uint32_t x0[4] = {X0.x, X0.y, X0.z, X0.w}, x1[4] = {X1.x, X1.y, X1.z, X1.w};
        const uint32_t x2[4] = {X2.x, X2.y, X2.z, X2.w}, x3[4] = {X3.x, X3.y, X3.z, X3.w};
        int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t u0 = (a[j] & 0x0F0F0F0Fu) | ((c[j] << 4) & 0x30303030u);
            uint32_t u1 = (bq[j] & 0x0F0F0F0Fu) | ((c[j] << 2) & 0x30303030u);
            uint32_t u2 = ((a[j] >> 4) & 0x0F0F0F0Fu) | (c[j] & 0x30303030u);
            uint32_t u3 = ((bq[j] >> 4) & 0x0F0F0F0Fu) | ((c[j] >> 2) & 0x30303030u);
            s0 = dot4((int)u0, (int)x0[j], s0);
            s1 = dot4((int)u1, (int)x1[j], s1);
            s2 = dot4((int)u2, (int)x2[j], s2);
            s3 = dot4((int)u3, (int)x3[j], s3);
        }
        /* groups 8h+p, 8h+2+p, 8h+4+p, 8h+6+p; sc bytes p, p+2, p+4, p+6 of S */
        const int16_t *bs = X.bs + b * 16 + 8 * h + p;
        const uint32_t sw0 = S.x >> (8 * p), sw1 = S.y >> (8 * p);
        int sc0 = (int8_t)(sw0 & 0xFF), sc1 = (int8_t)((sw0 >> 16) & 0xFF);
        int sc2 = (int8_t)(sw1 & 0xFF), sc3 = (int8_t)((sw1 >> 16) & 0xFF);
        int part = sc0 * (s0 - 32 * (int)bs[0]) + sc1 * (s1 - 32 * (int)bs[2]) +
                   sc2 * (s2 - 32 * (int)bs[4]) + sc3 * (s3 - 32 * (int)bs[6]);
        part += __shfl_xor(part, 1, 64);
        part += __shfl_xor(part, 2, 64);
        is = part;
        ms = 0;
        dA = f16_to_f32(dw) * X.d[b];
        dM = 0.0f;
    }
};

template <> struct Packed<DT_Q8_0> {
    static constexpr int LPI = 2, BV = 32;
    __device__ static __forceinline__ void item(const uint8_t *__restrict__ Wp, int64_t units, int64_t u, int b,
                                                int q, const XLds &X, int32_t &is, int32_t &ms, float &dA,
                                                float &dM) {
        const uint4 Wv = *(const uint4 *)(Wp + u * 32 + 16 * q);
        const uint32_t dw = *(const uint16_t *)(Wp + units * 32 + u * 2);
        const uint4 Xv = *(const uint4 *)(X.q + b * 32 + 16 * q);
        int s = dot4((int)Wv.x, (int)Xv.x, 0);
        s = dot4((int)Wv.y, (int)Xv.y, s);
        s = dot4((int)Wv.z, (int)Xv.z, s);
        s = dot4((int)Wv.w, (int)Xv.w, s);
        s += __shfl_xor(s, 1, 64);
        is = s;
        ms = 0;
        dA = f16_to_f32(dw) * X.d[b];
        dM = 0.0f;
    }
};

template <int DT> struct PackedKQ {
    static constexpr int LPI = 4, BV = 256;
    static constexpr bool Q5 = DT == DT_Q5_K;
    static constexpr int BB = Q5 ? 176 : 144, QS = Q5 ? 48 : 16;
    __device__ static __forceinline__ void item(const uint8_t *__restrict__ Wp, int64_t units, int64_t u, int b,
                                                int c, const XLds &X, int32_t &is, int32_t &ms, float &dA,
                                                float &dM) {
        const uint8_t *blk = Wp + u * BB;
        const uint4 H = *(const uint4 *)blk;
        const uint4 Q0 = *(const uint4 *)(blk + QS + 32 * c), Q1 = *(const uint4 *)(blk + QS + 32 * c + 16);
        uint32_t qh[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (Q5) {
            const uint4 P0 = *(const uint4 *)(blk + 16), P1 = *(const uint4 *)(blk + 32);
            qh[0] = P0.x; qh[1] = P0.y; qh[2] = P0.z; qh[3] = P0.w;
            qh[4] = P1.x; qh[5] = P1.y; qh[6] = P1.z; qh[7] = P1.w;
        }
        const uint32_t qw[8] = {Q0.x, Q0.y, Q0.z, Q0.w, Q1.x, Q1.y, Q1.z, Q1.w};
        const int8_t *xq = X.q + b * 256 + 64 * c;
        const uint4 XL0 = *(const uint4 *)(xq), XL1 = *(const uint4 *)(xq + 16);
        const uint4 XH0 = *(const uint4 *)(xq + 32), XH1 = *(const uint4 *)(xq + 48);
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
        /* 6-bit scales/mins of sub-blocks 2c and 2c+1 (src/lib/tlm_quant.c:253-261) */
        const uint8_t s12[12] = {(uint8_t)H.y, (uint8_t)(H.y >> 8), (uint8_t)(H.y >> 16), (uint8_t)(H.y >> 24),
                                 (uint8_t)H.z, (uint8_t)(H.z >> 8), (uint8_t)(H.z >> 16), (uint8_t)(H.z >> 24),
                                 (uint8_t)H.w, (uint8_t)(H.w >> 8), (uint8_t)(H.w >> 16), (uint8_t)(H.w >> 24)};
        int sc[2], mn[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            int sb = 2 * c + k;
            if (sb < 4) { sc[k] = s12[sb] & 63; mn[k] = s12[4 + sb] & 63; }
            else {
                sc[k] = (s12[sb + 4] & 15) | ((s12[sb - 4] >> 6) << 4);
                mn[k] = (s12[sb + 4] >> 4) | ((s12[sb] >> 6) << 4);
            }
        }
        const int16_t *bs = X.bs + b * 16 + 4 * c;
        int part = sc[0] * slo + sc[1] * shi;
        int mpart = mn[0] * ((int)bs[0] + (int)bs[1]) + mn[1] * ((int)bs[2] + (int)bs[3]);
        part += __shfl_xor(part, 1, 64);
        part += __shfl_xor(part, 2, 64);
        mpart += __shfl_xor(mpart, 1, 64);
        mpart += __shfl_xor(mpart, 2, 64);
        is = part;
        ms = mpart;
        const float da = X.d[b];
        dA = f16_to_f32(H.x & 0xFFFFu) * da;
        dM = f16_to_f32(H.x >> 16) * da;
    }
};
template <> struct Packed<DT_Q4_K> : PackedKQ<DT_Q4_K> {};
template <> struct Packed<DT_Q5_K> : PackedKQ<DT_Q5_K> {};

template <> struct Packed<DT_Q8_K> {
    static constexpr int LPI = 4, BV = 256;
    __device__ static __forceinline__ void item(const uint8_t *__restrict__ Wp, int64_t units, int64_t u, int b,
                                                int q, const XLds &X, int32_t &is, int32_t &ms, float &dA,
                                                float &dM) {
        const uint32_t *blk = (const uint32_t *)(Wp + u * 292);
        const uint32_t *xq = (const uint32_t *)(X.q + b * 256 + 64 * q);
        int s = 0;
#pragma unroll
        for (int j = 0; j < 16; j++) s = dot4((int)blk[1 + 16 * q + j], (int)xq[j], s);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        is = s;
        ms = 0;
        dA = __uint_as_float(blk[0]) * X.d[b];
        dM = 0.0f;
    }
};

#endif
