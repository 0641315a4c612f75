/* hip_gemv.hip - quantised GEMV (decode matvec) kernels for gfx950.
 *
 * Numerics (src/lib/tlm_quant.h:113-128): per (row, block) an exact int32
 * isum (and msum for Q4_K/Q5_K); per row the float chain
 *     acc = fmaf(d_w * d_a, (float)isum, acc)  [; acc = fmaf(-(dmin_w * d_a), (float)msum, acc)]
 * over blocks in ascending order from +0, run by one thread.  Integer sums are
 * order-free, so they are split over lanes freely; the float chain never is.
 * F32 rows: lane i mod 32 accumulates with fmaf in element order, then the
 * fixed reduce32 tree (src/lib/tlm_quant.c:721-738).
 *
 * Two layouts:
 *   plain  - the reference's row-major bytes, any stride / base offset
 *            (the drop-in tlm_matvec_rows path).  One lane per block,
 *            byte-granular weight reads.
 *   packed - tile layout produced on device by launch_pack (see
 *            packed_bytes): rows grouped in tiles of 16; the tile's rows are
 *            contiguous per block column, and the f16 scale of Q6_K / Q8_0
 *            blocks moves to a side region so every remaining weight read is
 *            a 16-byte aligned vector load.  This is the HBM-bandwidth path.
 */
#include "tlm_hip_internal.h"
#include <type_traits>
#include "tlm_hip_items.h"
#include "tlm_hip_act.h"

#include <math.h>

namespace {

/* ======================================================================
 * plain layout
 * ==================================================================== */
__device__ __forceinline__ uint32_t ld_u8(const uint8_t *p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16u(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

/* Integer sums of one plain block (any alignment) against a 4-byte aligned
 * activation block - the per-element rules of src/lib/tlm_quant.c:778-902. */
template <int DT>
__device__ void plain_block(const uint8_t *w, const uint8_t *a, int32_t &is, int32_t &ms) {
    is = 0;
    ms = 0;
    const int8_t *x = (const int8_t *)(a + 4);
    if constexpr (DT == DT_Q8_0) {
        for (int i = 0; i < 32; i++) is += (int32_t)(int8_t)w[2 + i] * x[i];
    } else if constexpr (DT == DT_Q8_K) {
        for (int i = 0; i < 256; i++) is += (int32_t)(int8_t)w[4 + i] * x[i];
    } else if constexpr (DT == DT_Q6_K) {
        const int16_t *bs = (const int16_t *)(a + 260);
        for (int g = 0; g < 16; g++) {
            int32_t gs = 0;
            for (int k = 0; k < 16; k++) {
                int e = 16 * g + k, h = e >> 7, q = (e >> 5) & 3, l = e & 31;
                uint32_t nib = w[64 * h + 32 * (q & 1) + l];
                nib = (q & 2) ? (nib >> 4) : (nib & 15u);
                uint32_t hi = (w[128 + 32 * h + l] >> (2 * q)) & 3u;
                gs += (int32_t)(nib | (hi << 4)) * x[e];
            }
            is += (int32_t)(int8_t)w[192 + g] * (gs - 32 * (int32_t)bs[g]);
        }
    } else {   /* Q4_K / Q5_K */
        constexpr bool Q5 = DT == DT_Q5_K;
        const uint8_t *qs = w + (Q5 ? 48 : 16), *s12 = w + 4;
        const int16_t *bs = (const int16_t *)(a + 260);
        for (int sb = 0; sb < 8; sb++) {
            int c = sb >> 1, hb = sb & 1;
            uint32_t sc, mn;
            if (sb < 4) { sc = s12[sb] & 63u; mn = s12[4 + sb] & 63u; }
            else {
                sc = (s12[sb + 4] & 15u) | ((uint32_t)(s12[sb - 4] >> 6) << 4);
                mn = ((uint32_t)s12[sb + 4] >> 4) | ((uint32_t)(s12[sb] >> 6) << 4);
            }
            int32_t s = 0;
            for (int l = 0; l < 32; l++) {
                uint32_t code = hb ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 15u);
                if (Q5) code |= ((w[16 + l] >> (2 * c + hb)) & 1u) << 4;
                s += (int32_t)code * x[32 * sb + l];
            }
            is += (int32_t)sc * s;
            ms += (int32_t)mn * ((int32_t)bs[2 * sb] + (int32_t)bs[2 * sb + 1]);
        }
    }
}

template <int DT>
__device__ __forceinline__ void plain_scales(const uint8_t *w, const uint8_t *a, float &dA, float &dM) {
    float da = *(const float *)a;
    if constexpr (DT == DT_Q6_K) { dA = f16_to_f32(ld_u16u(w + 208)) * da; dM = 0.0f; }
    else if constexpr (DT == DT_Q8_0) { dA = f16_to_f32(ld_u16u(w)) * da; dM = 0.0f; }
    else if constexpr (DT == DT_Q8_K) {
        uint32_t u = ld_u16u(w) | (ld_u16u(w + 2) << 16);
        dA = __uint_as_float(u) * da;
        dM = 0.0f;
    } else { dA = f16_to_f32(ld_u16u(w)) * da; dM = f16_to_f32(ld_u16u(w + 2)) * da; }
}

/* One wave per row, 4 rows per work-group.  Lanes take blocks lane, lane+64,
 * ...; the chain runs in every lane (same values) over shuffled block results
 * in ascending order. */
template <int DT>
__device__ __forceinline__ void mv_plain_rows(const uint8_t *__restrict__ W, size_t row_bytes,
                                              const uint8_t *__restrict__ act, float *__restrict__ y, int64_t n,
                                              int64_t r0, int64_t r1, int64_t bid) {
    constexpr int BV = DT == DT_Q8_0 ? 32 : 256;
    constexpr int AB = DT == DT_Q8_0 ? 36 : 292;
    constexpr int WB = DT == DT_Q8_0 ? 34 : DT == DT_Q4_K ? 144 : DT == DT_Q5_K ? 176 : DT == DT_Q6_K ? 210 : 292;
    constexpr bool AFF = DT == DT_Q4_K || DT == DT_Q5_K;
    const int lane = threadIdx.x & 63;
    const int64_t row = r0 + bid * 4 + (threadIdx.x >> 6);
    if (row >= r1) return;
    const uint8_t *w = W + (size_t)row * row_bytes;
    const int64_t nb = n / BV;
    float acc = 0.0f;
    for (int64_t base = 0; base < nb; base += 64) {
        int64_t b = base + lane;
        int32_t is = 0, ms = 0;
        float dA = 0.0f, dM = 0.0f;
        if (b < nb) {
            plain_block<DT>(w + (size_t)b * WB, act + (size_t)b * AB, is, ms);
            plain_scales<DT>(w + (size_t)b * WB, act + (size_t)b * AB, dA, dM);
        }
        float fis = (float)is, fms = (float)ms;
        int cnt = (int)(nb - base < 64 ? nb - base : 64);
        for (int j = 0; j < cnt; j++) {
            acc = fmaf(__shfl(dA, j, 64), __shfl(fis, j, 64), acc);
            if (AFF) acc = fmaf(-__shfl(dM, j, 64), __shfl(fms, j, 64), acc);
        }
    }
    if (lane == 0) y[row] = acc;
}
template <int DT>
__global__ __launch_bounds__(256) void k_mv_plain_int(const uint8_t *__restrict__ W, size_t row_bytes,
                                                      const uint8_t *__restrict__ act, float *__restrict__ y,
                                                      int64_t n, int64_t r0, int64_t r1) {
    mv_plain_rows<DT>(W, row_bytes, act, y, n, r0, r1, blockIdx.x);
}

/* F32 row dot with the reference lane order: lanes 0..31 of a half-wave own
 * elements i = lane mod 32; two rows per wave, 8 rows per work-group. */
template <bool ALIGNED>
__device__ __forceinline__ void mv_f32_rows(const uint8_t *__restrict__ W, size_t row_bytes,
                                            const float *__restrict__ x, float *__restrict__ y, int64_t n,
                                            int64_t r0, int64_t r1, int64_t bid) {
    const int lane = threadIdx.x & 31;
    const int64_t row = r0 + bid * 8 + (threadIdx.x >> 5);
    const bool live = row < r1;
    float r = 0.0f;
    if (live) {
        const uint8_t *w = W + (size_t)row * row_bytes;
        for (int64_t i = lane; i < n; i += 32) {
            float wv;
            if (ALIGNED) wv = ((const float *)w)[i];
            else {
                const uint8_t *p = w + 4 * i;
                wv = __uint_as_float(ld_u16u(p) | (ld_u16u(p + 2) << 16));
            }
            r = fmaf(wv, x[i], r);
        }
    }
    /* reduce32: s16[l] = r[l] + r[l+16]; s8; s4; (s4[0]+s4[2]) + (s4[1]+s4[3]) */
    float s = r + __shfl_down(r, 16, 32);
    s = s + __shfl_down(s, 8, 32);
    s = s + __shfl_down(s, 4, 32);
    float a = s + __shfl_down(s, 2, 32);           /* lane 0: s4[0] + s4[2]; lane 1: s4[1] + s4[3] */
    float res = a + __shfl_down(a, 1, 32);
    if (live && lane == 0) y[row] = res;
}
template <bool ALIGNED>
__global__ __launch_bounds__(256) void k_mv_f32(const uint8_t *__restrict__ W, size_t row_bytes,
                                                const float *__restrict__ x, float *__restrict__ y,
                                                int64_t n, int64_t r0, int64_t r1) {
    mv_f32_rows<ALIGNED>(W, row_bytes, x, y, n, r0, r1, blockIdx.x);
}

__global__ void k_nan_fill(float *y, int64_t count) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) y[i] = __uint_as_float(0x7FC00000u);
}

/* ======================================================================
 * packed layout
 *
 *   T  = ceil(rows / 16) tiles, nb blocks per row, unit index
 *        u(t, b, i) = (t * nb + b) * 16 + i    (i = row within the tile)
 *   Q6_K: 208-byte unit ql|qh|sc at u*208; f16 d at T*nb*16*208 + u*2
 *   Q8_0: 32-byte codes at u*32;            f16 d at T*nb*16*32  + u*2
 *   Q4_K / Q5_K / Q8_K: whole block at u*block_bytes
 *   F32: plain rows of n floats
 * Rows past `rows` in the last tile are zero.
 * ==================================================================== */
/* One work-group per (16-row tile, chunk of cb block columns).  The tile's
 * source - 16 row pieces of cb * block_bytes contiguous bytes - is loaded into
 * LDS with aligned dword loads (the dwords holding the piece: never outside
 * the piece's pages), so the reads stream whether src is device memory or
 * page-locked host memory read over PCIe; then the chunk's units (contiguous
 * in the packed layout) and d values are written with coalesced dword stores.
 * Unit u = (t*nb + b)*16 + i holds row t*16 + i, block b: Q6_K bytes 0..207,
 * Q8_0 codes 2..33, other formats the whole block; Q6_K and Q8_0 keep their
 * f16 d in a plane after the units.  Rows past the matrix pack as zeros. */
__global__ __launch_bounds__(256) void k_pack(int dt, const uint8_t *__restrict__ src, size_t row_bytes, int64_t rows,
                                             int nb, int cb, int rstride, uint8_t *__restrict__ dst) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int64_t t = blockIdx.x, T = gridDim.x;
    const int b0 = (int)blockIdx.y * cb;
    const int ncb = nb - b0 < cb ? nb - b0 : cb;
    const int bb = dt_block_bytes(dt);
    const int U = dt == DT_Q6_K ? 208 : dt == DT_Q8_0 ? 32 : bb;   /* unit bytes, a multiple of 4 */
    const int skip = dt == DT_Q8_0 ? 2 : 0;                          /* f16 d leads a Q8_0 block */
    const int dpos = dt == DT_Q6_K ? 208 : 0;                        /* where d sits in the block */
    const bool plane = dt == DT_Q6_K || dt == DT_Q8_0;
    const int piece = ncb * bb, dmax = (piece + 6) / 4 + 1;
    const int tid = threadIdx.x;
    auto head_of = [&](int i) -> int {
        return (int)(((uintptr_t)src + (size_t)(t * TILE_ROWS + i) * row_bytes + (size_t)b0 * bb) & 3u);
    };
    /* eight loads in flight per thread before any is stored: over PCIe each
     * is a round trip of microseconds */
    constexpr int BATCH = 8;
    for (int base = tid; base < TILE_ROWS * dmax; base += 256 * BATCH) {
        uint32_t v[BATCH];
        int at[BATCH];
#pragma unroll
        for (int q = 0; q < BATCH; q++) {
            const int idx = base + 256 * q;
            at[q] = -1;
            const int i = idx / dmax, w = idx - i * dmax;
            const int64_t r = t * TILE_ROWS + i;
            if (idx < TILE_ROWS * dmax && r < rows) {
                const uint8_t *p = src + (size_t)r * row_bytes + (size_t)b0 * bb;
                const int head = (int)((uintptr_t)p & 3u);
                if (4 * w < head + piece) {
                    v[q] = *(const uint32_t *)(p - head + 4 * w);
                    at[q] = i * rstride + 4 * w;
                }
            }
        }
#pragma unroll
        for (int q = 0; q < BATCH; q++)
            if (at[q] >= 0) *(uint32_t *)(lds + at[q]) = v[q];
    }
    __syncthreads();
    const int64_t units = T * nb * TILE_ROWS, u0 = (t * nb + b0) * TILE_ROWS;
    const int n1 = ncb * TILE_ROWS * (U / 4), n2 = plane ? ncb * TILE_ROWS / 2 : 0;
    for (int o = tid; o < n1 + n2; o += 256) {
        if (o < n1) {
            const int lu = o / (U / 4), k = (o - lu * (U / 4)) * 4;
            const int i = lu % TILE_ROWS, bl = lu / TILE_ROWS;
            uint32_t v = 0;
            if (t * TILE_ROWS + i < rows) {
                const uint8_t *q = lds + i * rstride + head_of(i) + bl * bb + skip + k;
                v = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
            }
            *(uint32_t *)(dst + (u0 + lu) * U + k) = v;
        } else {
            const int lu = 2 * (o - n1), i = lu % TILE_ROWS, bl = lu / TILE_ROWS;
            uint32_t v = 0;
            for (int h = 0; h < 2; h++)
                if (t * TILE_ROWS + i + h < rows) {
                    const uint8_t *q = lds + (i + h) * rstride + head_of(i + h) + bl * bb + dpos;
                    v |= ((uint32_t)q[0] | ((uint32_t)q[1] << 8)) << (16 * h);
                }
            *(uint32_t *)(dst + units * U + 2 * (u0 + lu)) = v;
        }
    }
}

__global__ void k_pack_f32(const uint8_t *__restrict__ src, size_t row_bytes, int64_t rows, int64_t n,
                           float *__restrict__ dst) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= rows * n) return;
    int64_t r = e / n, c = e % n;
    const uint8_t *p = src + (size_t)r * row_bytes + 4 * c;
    dst[e] = __uint_as_float(ld_u16u(p) | (ld_u16u(p + 2) << 16));
}

}  // namespace

/* ---- packed GEMV kernel --------------------------------------------------
 * Work-group = 4 waves, one 16-row tile; block columns are chunked by NBC so
 * LDS stays bounded for long rows.  Per chunk every wave computes items
 * (b, i) with LPI lanes each and parks (isum, msum, dA, dM) in LDS; then 16
 * threads extend their row's float chain over the chunk in block order.
 * The activation is staged once per work-group (all blocks).  Items in
 * flight per lane (IPL) and blocks per chunk (NBC): a round of loads costs
 * one memory latency, so for wide Q8_0 rows (DEEP: at least 128 blocks, in
 * groups of part of a tile) a lane (5 registers per item) keeps 16 in
 * flight, branch-free, and a chunk of 128 blocks is one round - a 16-row
 * tile of up to 4096 columns streams in a single latency; rows of 64 to 127
 * blocks and whole-tile groups (MID) keep 8 per lane, a chunk of 64 blocks
 * in one round; narrower rows keep 4 per lane (a deep round would be mostly
 * dropped items).  A group of RPG rows of a tile scales the items per lane by
 * RPG / 16. */
enum { MV_SHALLOW = 0, MV_DEEP = 1, MV_MID = 2 };
constexpr int MV_EARLY_WORDS = 5;   /* a8 words per thread of an activation loaded early */
template <int DT, int V> struct MvCfg {
    static constexpr int IPL = 4, NBC = 64;
    static constexpr bool CLAMP = false;
};
template <> struct MvCfg<DT_Q8_0, MV_DEEP> {
    static constexpr int IPL = 16, NBC = 128;
    static constexpr bool CLAMP = true;
};
/* rows of 64 blocks in one round: a chunk of 64 blocks is exactly one round
 * (the deep tile's round of 128 would load every second item in vain) */
template <> struct MvCfg<DT_Q8_0, MV_MID> {
    static constexpr int IPL = 8, NBC = 64;
    static constexpr bool CLAMP = true;
};
static bool mv_deep(int dt, int nb) { return dt == DT_Q8_0 && nb >= 64; }
static int mv_nbc(int dt, int nb) { return mv_deep(dt, nb) ? MvCfg<DT_Q8_0, MV_DEEP>::NBC : MvCfg<DT_Q6_K, MV_SHALLOW>::NBC; }

/* rmsnorm of x (when w is given) then the activation quantiser of kind,
 * written straight into the LDS layout that stage_act fills from a quantised
 * vector: r = 1 / sqrtf(mean(x^2) + eps) with the sum of squares in double
 * (per thread, then a fixed tree), values x * r * w (rmsnorm,
 * src/lib/tlm_model.c:164-169, then the quantiser of
 * src/lib/tlm_quant.c:458-506); without w, x itself is quantised.  Each lane
 * takes 16 contiguous values (quant16_to): a Q8_K block spans 16 lanes, an a8
 * block 2, so one pass of 256 threads covers 4096 values.  The first pass's
 * x and w are loaded by norm_act_load before the tile's weight loads (loads
 * retire in issue order: the norm must not wait for the weights), with no
 * branch around them (lanes past the last block read the last block); later
 * passes reload.  Every thread takes part; the caller synchronises. */
struct NormIn {
    f32x4 xv[4], wv[4];
};
struct NormMap {
    int bv, per, myb, sub;
    __device__ NormMap(int kind) {
        const bool k8 = kind == DT_Q8_K;
        const int lpb = k8 ? 16 : 2;   /* lanes per block */
        bv = k8 ? 256 : 32;
        per = GROUP_THREADS / lpb;
        myb = (int)threadIdx.x / lpb;
        sub = (int)threadIdx.x % lpb;
    }
};

static __device__ __forceinline__ void norm_act_load(int kind, const float *__restrict__ x,
                                                     const float *__restrict__ w, int nb, NormIn &in) {
    const NormMap m(kind);
    const int b = min(m.myb, nb - 1);
    const GAS f32x4 *x4 = (const GAS f32x4 *)x + (b * m.bv + 16 * m.sub) / 4;
    const GAS f32x4 *w4 = (const GAS f32x4 *)(w ? w : x) + (b * m.bv + 16 * m.sub) / 4;
#pragma unroll
    for (int u = 0; u < 4; u++) in.xv[u] = x4[u];
#pragma unroll
    for (int u = 0; u < 4; u++) in.wv[u] = w4[u];
}

static __device__ __forceinline__ XLds stage_norm_act(int kind, const float *__restrict__ x,
                                                      const float *__restrict__ w, float eps, int nb, uint8_t *lds_g,
                                                      const NormIn &in) {
    __shared__ double red[16];
    const NormMap m(kind);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = GROUP_THREADS >> 6;
    const int n = nb * m.bv, nit = (nb + m.per - 1) / m.per;
    const bool plain = w == nullptr;
    auto ld = [&](const float *p, int b, f32x4 (&v)[4]) {
        const GAS f32x4 *p4 = (const GAS f32x4 *)p + (b * m.bv + 16 * m.sub) / 4;
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = p4[u];
    };
    float r = 1.0f;
    if (!plain) {
        double ss = 0.0;
        if (m.myb < nb)
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int j = 0; j < 4; j++) ss += (double)in.xv[u][j] * (double)in.xv[u][j];
        for (int it = 1; it < nit; it++) {
            const int b = it * m.per + m.myb;
            if (b < nb) {
                f32x4 a[4];
                ld(x, b, a);
                for (int u = 0; u < 4; u++)
                    for (int j = 0; j < 4; j++) ss += (double)a[u][j] * (double)a[u][j];
            }
        }
        ss = wave_sum_f64(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        ss = 0.0;
        for (int i = 0; i < nw; i++) ss += red[i];
        r = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    }
    LAS uint8_t *lds = (LAS uint8_t *)lds_g;
    const bool k8 = kind == DT_Q8_K;
    LAS int16_t *bs16 = (LAS int16_t *)(lds + nb * 256);
    LAS float *dl = (LAS float *)(lds + (k8 ? nb * 288 : nb * 32));
    auto quant = [&](int b, const f32x4 (&a)[4], const f32x4 (&ww)[4]) {
        f32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int j = 0; j < 4; j++) v[u][j] = plain ? a[u][j] : a[u][j] * r * ww[u][j];
        quant16_to(kind, v, b < nb, m.sub, lds, bs16, dl, b);
    };
    quant(m.myb, in.xv, in.wv);
    for (int it = 1; it < nit; it++) {   /* uniform over the group */
        const int b = it * m.per + m.myb, bc = min(b, nb - 1);
        f32x4 a[4], ww[4];
        ld(x, bc, a);
        ld(plain ? x : w, bc, ww);
        quant(b, a, ww);
    }
    return xlds_at(kind, nb, lds_g);
}

/* Per token: rmsnorm (w given) or the plain vector, then the activation
 * quantiser of kind, with the decode GEMV prologue's code (norm_act_load +
 * stage_norm_act, the same thread mapping and reduction tree, so the same
 * codes and scales), written in the reference layout (a8: 36-byte blocks;
 * Q8_K: 292-byte blocks) at out + t * ostride.  One group per token. */
__global__ __launch_bounds__(256) void k_tok_norm_act(int kind, const float *__restrict__ x, int64_t xstride,
                                                      const float *__restrict__ w, float eps, int nb,
                                                      uint8_t *__restrict__ out, int64_t ostride) {
    extern __shared__ __align__(16) uint8_t lds[];
    const float *xt = x + (int64_t)blockIdx.x * xstride;
    NormIn nin;
    norm_act_load(kind, xt, w, nb, nin);
    stage_norm_act(kind, xt, w, eps, nb, lds, nin);
    __syncthreads();
    const bool k8 = kind == DT_Q8_K;
    const int words = k8 ? 73 : 9;   /* 4-byte words per block: d, codes (, bsums) */
    const LAS uint8_t *l = (const LAS uint8_t *)lds;
    const LAS float *dl = (const LAS float *)(l + (k8 ? nb * 288 : nb * 32));
    GAS uint32_t *o = (GAS uint32_t *)(out + (int64_t)blockIdx.x * ostride);
    for (int i = threadIdx.x; i < nb * words; i += GROUP_THREADS) {
        const int b = i / words, wd = i - b * words;
        uint32_t v;
        if (wd == 0) v = __float_as_uint(dl[b]);
        else if (wd <= (k8 ? 64 : 8)) v = *(const LAS uint32_t *)(l + (size_t)b * (k8 ? 256 : 32) + 4 * (wd - 1));
        else v = *(const LAS uint32_t *)(l + (size_t)nb * 256 + (size_t)b * 32 + 4 * (wd - 65));
        o[i] = v;
    }
}

int launch_tok_norm_act(int kind, const float *x, int64_t xstride, const float *w, float eps, int64_t n,
                        int64_t ntok, void *out, int64_t ostride, hipStream_t s) {
    if (kind != DT_Q8_0 && kind != DT_Q8_K) return tlmh_seterr(TLM_HIP_EINVAL, "tok_norm_act: kind %d", kind);
    const int bv = kind == DT_Q8_K ? 256 : 32;
    if (n <= 0 || n % bv || ntok <= 0 || ((uintptr_t)x & 15u) || (xstride & 3) || (ostride & 3) ||
        ((uintptr_t)out & 3u))
        return tlmh_seterr(TLM_HIP_EINVAL, "tok_norm_act: n=%lld ntok=%lld", (long long)n, (long long)ntok);
    const int nb = (int)(n / bv);
    const size_t lds = stage_bytes(kind, nb);
    if (lds > 64 * 1024) return tlmh_seterr(TLM_HIP_EUNSUP, "tok_norm_act: n=%lld exceeds LDS", (long long)n);
    hipLaunchKernelGGL(k_tok_norm_act, dim3((unsigned)ntok), dim3(256), lds, s, kind, x, xstride, w, eps, nb,
                       (uint8_t *)out, ostride);
    return tlmh_check(hipGetLastError(), "tok_norm_act launch");
}

/* The same tile for up to MV_SEGS matrices of one dtype and width in one
 * launch (segment s owns tiles [tile_end[s-1], tile_end[s])), all taking the
 * same activation; accum: y[r] += acc instead of y[r] = acc (the reference's
 * residual update h += W x, tlm_model.c:762, adds the finished product). */
struct MvTile {
    const uint8_t *Wp;   /* packed matrix */
    int64_t rows, t;     /* its rows; the tile this group computes */
    int i0;              /* the first of the group's RPG rows inside the tile */
    float *y;
    const float *nx, *nw;
    float eps;
    int accum;
    unsigned long long *keys;
};
/* RPG rows of a 16-row tile per group (16, 8 or 4): a compute unit streams
 * only some tens of GB/s, so a matrix of few tiles (the o projection's 128)
 * spreads its rows over more groups than tiles, each with fewer items in
 * flight per lane */
template <int DT, int DEEP, int RPG, bool EARLY = false>
__device__ __forceinline__ void mv_packed_tile(const MvTile &sg, int nb, const uint8_t *__restrict__ act,
                                               bool have_x = false) {
    using F = Packed<DT>;
    constexpr bool AFF = DT == DT_Q4_K || DT == DT_Q5_K;
    constexpr int IPL0 = MvCfg<DT, DEEP>::IPL * RPG / TILE_ROWS;
    constexpr int IPL = IPL0 > 0 ? IPL0 : 1;
    static_assert(RPG == 16 || RPG == 8 || RPG == 4, "rows per group");
    extern __shared__ __align__(16) uint8_t lds[];
    const uint8_t *Wp = sg.Wp;
    const int64_t rows = sg.rows, t = sg.t;
    float *y = sg.y;
    const int kind = dt_act_kind(DT);
    XLds X = xlds_at(kind, nb, lds);
    NormIn nin;
    /* EARLY (a given a8 activation of at most AWN words per thread, no
     * norm): the activation goes into registers ahead of the weight loads
     * and into LDS once they are out (loads retire in issue order: one round
     * trip for both instead of the staging's own before the weights) */
    constexpr int AWN = MV_EARLY_WORDS;
    constexpr bool EARLY_OK = EARLY && DT == DT_Q8_0;
    uint32_t aw[AWN];
    if (have_x) {
        /* the activation is in LDS from the group's previous tile */
    } else if constexpr (EARLY_OK) {
        const GAS uint32_t *ag = (const GAS uint32_t *)act;
#pragma unroll
        for (int j = 0; j < AWN; j++) {
            const int k = (int)threadIdx.x + GROUP_THREADS * j;
            aw[j] = ag[k < nb * 9 ? k : 0];
        }
    } else if (!sg.nx) {
        stage_act(kind, act, nb, lds);
        /* its loads are all consumed; a wait the compiler can see keeps its
         * count from holding back the other path's first weight loads */
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    } else {
        norm_act_load(kind, sg.nx, sg.nw, nb, nin);
    }
    const int cap = nb < MvCfg<DT, DEEP>::NBC ? nb : MvCfg<DT, DEEP>::NBC;
    const Park park = park_at(lds + ((stage_bytes(kind, nb) + 15) & ~(size_t)15), cap * RPG);
    bool staged = EARLY_OK ? have_x : !sg.nx || have_x;
    /* the activation from rmsnorm once the first weight loads are out: the
     * empty asm keeps the norm's arithmetic (and so its wait for x) below
     * the weight loads, where the compiler would otherwise hoist it */
    auto stage = [&]() {
        if constexpr (EARLY_OK) {
            if (staged) return X;
            LAS uint32_t *q = (LAS uint32_t *)lds;
            LAS float *d = (LAS float *)((LAS uint8_t *)lds + nb * 32);
#pragma unroll
            for (int j = 0; j < AWN; j++) {
                const int k = (int)threadIdx.x + GROUP_THREADS * j, b = k / 9, w = k - b * 9;
                if (k < nb * 9) {
                    if (w == 0) d[b] = __uint_as_float(aw[j]);
                    else q[b * 8 + (w - 1)] = aw[j];
                }
            }
            __syncthreads();
            staged = true;
        } else if (!staged) {
#pragma unroll
            for (int u = 0; u < 4; u++) asm volatile("" : "+v"(nin.xv[u]), "+v"(nin.wv[u])::"memory");
            stage_norm_act(kind, sg.nx, sg.nw, sg.eps, nb, lds, nin);
            __syncthreads();
            staged = true;
        }
        return X;
    };
    const int64_t T = (rows + TILE_ROWS - 1) / TILE_ROWS;
    const int64_t units = T * nb * TILE_ROWS;
    const int round_items = (GROUP_THREADS / F::LPI) * IPL;
    float acc = 0.0f;
    const int i0 = sg.i0;
    for (int b0 = 0; b0 < nb; b0 += cap) {
        const int nbc = nb - b0 < cap ? nb - b0 : cap;
        const int nitems = nbc * RPG;
        for (int base = 0; base < nitems; base += round_items) {
            auto map = [&](int it, const uint8_t *&W, int64_t &un, int64_t &u, int &b, int &pk) {
                const int g = base + it, bl = g / RPG, i = g % RPG;
                W = Wp;
                un = units;
                b = b0 + bl;
                u = ((int64_t)t * nb + b) * TILE_ROWS + i0 + i;
                pk = g;
            };
            run_items<DT, IPL, MvCfg<DT, DEEP>::CLAMP>(nitems - base, map, stage, park);
        }
        __syncthreads();
        if (threadIdx.x < RPG) acc = chain_park<AFF>(park, nbc, 0, RPG, threadIdx.x, acc);
        __syncthreads();
        /* nothing is in flight here (a dropped item's load aside); a wait
         * the compiler can see keeps the loop head's counts from holding the
         * first pass's weight loads back behind the norm's x and w */
        __builtin_amdgcn_s_waitcnt(0);
    }
    const int64_t r = t * TILE_ROWS + i0 + threadIdx.x;
    if (threadIdx.x < RPG && r < rows) ((GAS float *)y)[r] = sg.accum ? ((GAS float *)y)[r] + acc : acc;
    if (RPG == TILE_ROWS && sg.keys && threadIdx.x < 64) {   /* lanes 0..15 hold the tile's rows */
        unsigned long long key = threadIdx.x < TILE_ROWS && r < rows ? argmax_key(acc, (uint32_t)r) : 0ull;
        for (int o = 8; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(key, o, 64);
            key = other > key ? other : key;
        }
        if (threadIdx.x == 0) ((GAS unsigned long long *)sg.keys)[t] = key;
    }
}
/* group g -> (tile, part): work-groups go to the 8 XCDs round-robin by id,
 * so in each run of 8 SPT ids the parts of 8 tiles go to one XCD each (ids g,
 * g + 8, ... share the XCD, and its L2, whose lines hold neighbouring rows of
 * a tile); ids of a last incomplete run map straight */
template <int RPG>
__device__ __forceinline__ void mv_group_tile(int64_t g, int64_t ngroups, int64_t &tile, int &part) {
    constexpr int SPT = TILE_ROWS / RPG;
    const int64_t run = g / (8 * SPT);
    if ((run + 1) * 8 * SPT <= ngroups) {
        tile = run * 8 + g % 8;
        part = (int)((g / 8) % SPT);
    } else {
        tile = g / SPT;
        part = (int)(g % SPT);
    }
}
template <int DT, int DEEP, int RPG, int TPG = 1>
__global__ __launch_bounds__(256) void k_mv_packed_seg(MvSegs sg, int nb, const uint8_t *__restrict__ act) {
    static_assert(TPG == 1 || RPG == TILE_ROWS, "several tiles per group take whole tiles");
    int64_t tile;
    int part;
    /* every per-segment field is read at entry, in the launch's first
     * scalar round trip, and passed through an empty asm so that the
     * compiler cannot turn the select below back into a read at a
     * computed offset (a second, dependent round trip) */
    static_assert(MV_SEGS == 4, "segment select");
    const uint8_t *Wv[MV_SEGS];
    int64_t rv[MV_SEGS], te[MV_SEGS];
    float *yv[MV_SEGS];
#pragma unroll
    for (int i = 0; i < MV_SEGS; i++) {
        Wv[i] = sg.W[i];
        rv[i] = sg.rows[i];
        te[i] = sg.tile_end[i];
        yv[i] = sg.y[i];
    }
    const float *nx = sg.nx, *nw = sg.nw;
    unsigned long long *keys = sg.keys;
    float eps = sg.eps;
    int nseg = sg.n, accum = sg.accum, nbv = nb;
    const uint8_t *actv = act;
    unsigned ngrid = gridDim.x;
    asm volatile("" : "+s"(Wv[0]), "+s"(Wv[1]), "+s"(Wv[2]), "+s"(Wv[3]), "+s"(rv[0]), "+s"(rv[1]), "+s"(rv[2]),
                 "+s"(rv[3]), "+s"(te[0]), "+s"(te[1]), "+s"(te[2]), "+s"(te[3]), "+s"(yv[0]), "+s"(yv[1]),
                 "+s"(yv[2]), "+s"(yv[3]), "+s"(nx), "+s"(nw), "+s"(keys), "+s"(eps), "+s"(nseg), "+s"(accum),
                 "+s"(nbv), "+s"(actv), "+s"(ngrid));
    /* TPG > 1: whole tiles, TPG neighbouring tiles per group (the
     * activation staged once): fewer groups, each with less of its life
     * spent on its start and the staging */
    int64_t end = te[0];
#pragma unroll
    for (int i = 1; i < MV_SEGS; i++) end = te[i] > end ? te[i] : end;
#pragma unroll
    for (int k = 0; k < TPG; k++) {
        if constexpr (TPG > 1) {
            tile = (int64_t)blockIdx.x * TPG + k;
            part = 0;
            if (tile >= end) break;
        } else {
            mv_group_tile<RPG>(blockIdx.x, ngrid, tile, part);
        }
        /* the group's segment: the count of segment ends at or below its tile */
        int s = 0;
#pragma unroll
        for (int i = 0; i + 1 < MV_SEGS; i++) s += i + 1 < nseg && tile >= te[i] ? 1 : 0;
        const uint8_t *W = Wv[0];
        int64_t rows = rv[0], first = 0;
        float *y = yv[0];
#pragma unroll
        for (int i = 1; i < MV_SEGS; i++)
            if (s == i) {
                W = Wv[i];
                rows = rv[i];
                first = te[i - 1];
                y = yv[i];
            }
        const MvTile tl{W, rows, tile - first, part * RPG, y, nx, nw, eps, accum, keys};
        mv_packed_tile<DT, DEEP, RPG, (TPG > 1)>(tl, nbv, actv, k > 0);
    }
}

/* One launch for a whole job of matrices (mv_job / mv_exec,
 * src/lib/tlm_model.c:175-222): JOB_SEGS segments of any dtype, width,
 * layout and activation; segment s owns groups [first[s], first[s + 1]) and
 * every group runs its segment's body (a uniform switch): a 16-row tile of a
 * packed matrix, 4 plain rows of an integer format or 8 f32 rows. */
enum { JK_PACKED = 0, JK_PACKED_MID = 1, JK_PLAIN = 2, JK_F32 = 3, JK_F32_UNALIGNED = 4 };
struct JobSeg {
    const uint8_t *W, *act;
    float *y;
    uint64_t row_bytes;
    int64_t n, rows, first;
    int dt, kind;
};
#define JOB_SEGS 24
struct MvJob {
    JobSeg s[JOB_SEGS];
    int n;
};
__global__ __launch_bounds__(256) void k_mv_job(MvJob j) {
    int s = 0;
    while (s + 1 < j.n && (int64_t)blockIdx.x >= j.s[s + 1].first) s++;
    const JobSeg &g = j.s[s];
    const int64_t bid = (int64_t)blockIdx.x - g.first;
    if (g.kind == JK_PACKED || g.kind == JK_PACKED_MID) {
        const int nb = (int)(g.n / dt_block_values(g.dt));
        const MvTile tl{g.W, g.rows, bid, 0, g.y, nullptr, nullptr, 0.0f, 0, nullptr};
        switch (g.dt) {
        case DT_Q8_0:
            if (g.kind == JK_PACKED_MID) mv_packed_tile<DT_Q8_0, MV_MID, TILE_ROWS>(tl, nb, g.act);
            else mv_packed_tile<DT_Q8_0, MV_SHALLOW, TILE_ROWS>(tl, nb, g.act);
            break;
        case DT_Q4_K: mv_packed_tile<DT_Q4_K, MV_SHALLOW, TILE_ROWS>(tl, nb, g.act); break;
        case DT_Q5_K: mv_packed_tile<DT_Q5_K, MV_SHALLOW, TILE_ROWS>(tl, nb, g.act); break;
        case DT_Q6_K: mv_packed_tile<DT_Q6_K, MV_SHALLOW, TILE_ROWS>(tl, nb, g.act); break;
        case DT_Q8_K: mv_packed_tile<DT_Q8_K, MV_SHALLOW, TILE_ROWS>(tl, nb, g.act); break;
        }
    } else if (g.kind == JK_PLAIN) {
        switch (g.dt) {
        case DT_Q8_0: mv_plain_rows<DT_Q8_0>(g.W, g.row_bytes, g.act, g.y, g.n, 0, g.rows, bid); break;
        case DT_Q4_K: mv_plain_rows<DT_Q4_K>(g.W, g.row_bytes, g.act, g.y, g.n, 0, g.rows, bid); break;
        case DT_Q5_K: mv_plain_rows<DT_Q5_K>(g.W, g.row_bytes, g.act, g.y, g.n, 0, g.rows, bid); break;
        case DT_Q6_K: mv_plain_rows<DT_Q6_K>(g.W, g.row_bytes, g.act, g.y, g.n, 0, g.rows, bid); break;
        case DT_Q8_K: mv_plain_rows<DT_Q8_K>(g.W, g.row_bytes, g.act, g.y, g.n, 0, g.rows, bid); break;
        }
    } else if (g.kind == JK_F32) {
        mv_f32_rows<true>(g.W, g.row_bytes, (const float *)g.act, g.y, g.n, 0, g.rows, bid);
    } else {
        mv_f32_rows<false>(g.W, g.row_bytes, (const float *)g.act, g.y, g.n, 0, g.rows, bid);
    }
}

static size_t packed_lds_bytes(int dt, int nb) {
    const int cap = nb < mv_nbc(dt, nb) ? nb : mv_nbc(dt, nb);
    return ((stage_bytes(dt_act_kind(dt), nb) + 15) & ~(size_t)15) + (size_t)cap * TILE_ROWS * 16;
}

/* ======================================================================
 * host launchers
 * ==================================================================== */
int launch_nan_fill(float *y, int64_t count, hipStream_t s) {
    if (count <= 0) return TLM_HIP_OK;
    hipLaunchKernelGGL(k_nan_fill, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, y, count);
    return tlmh_check(hipGetLastError(), "nan_fill launch");
}

int launch_matvec_plain(int dt, const void *W, size_t row_bytes, const void *act, float *y, int64_t n,
                        int64_t r0, int64_t r1, hipStream_t s) {
    int bv = dt_block_values(dt);
    if (bv == 0 || n < 0 || n % bv || (dt != DT_F32 && !dt_int_ok(dt))) {
        if (y && r1 > r0) launch_nan_fill(y + r0, r1 - r0, s);
        return tlmh_seterr(TLM_HIP_EINVAL, "matvec_rows: bad dtype %d or n=%lld", dt, (long long)n);
    }
    if (r1 <= r0) return TLM_HIP_OK;
    if (!W || !act || !y) return tlmh_seterr(TLM_HIP_EINVAL, "matvec_rows: NULL pointer");
    if ((uintptr_t)act & 3u) return tlmh_seterr(TLM_HIP_EINVAL, "matvec_rows: activation must be 4-byte aligned");
    const uint8_t *w = (const uint8_t *)W;
    const uint8_t *a = (const uint8_t *)act;
    int64_t rows = r1 - r0;
    if (dt == DT_F32) {
        bool al = ((uintptr_t)W % 4 == 0) && (row_bytes % 4 == 0);
        dim3 g((unsigned)((rows + 7) / 8));
        if (al) hipLaunchKernelGGL(k_mv_f32<true>, g, dim3(256), 0, s, w, row_bytes, (const float *)a, y, n, r0, r1);
        else hipLaunchKernelGGL(k_mv_f32<false>, g, dim3(256), 0, s, w, row_bytes, (const float *)a, y, n, r0, r1);
        return tlmh_check(hipGetLastError(), "matvec f32 launch");
    }
    dim3 g((unsigned)((rows + 3) / 4)), blk(256);
    switch (dt) {
    case DT_Q8_0: hipLaunchKernelGGL(k_mv_plain_int<DT_Q8_0>, g, blk, 0, s, w, row_bytes, a, y, n, r0, r1); break;
    case DT_Q4_K: hipLaunchKernelGGL(k_mv_plain_int<DT_Q4_K>, g, blk, 0, s, w, row_bytes, a, y, n, r0, r1); break;
    case DT_Q5_K: hipLaunchKernelGGL(k_mv_plain_int<DT_Q5_K>, g, blk, 0, s, w, row_bytes, a, y, n, r0, r1); break;
    case DT_Q6_K: hipLaunchKernelGGL(k_mv_plain_int<DT_Q6_K>, g, blk, 0, s, w, row_bytes, a, y, n, r0, r1); break;
    case DT_Q8_K: hipLaunchKernelGGL(k_mv_plain_int<DT_Q8_K>, g, blk, 0, s, w, row_bytes, a, y, n, r0, r1); break;
    }
    return tlmh_check(hipGetLastError(), "matvec launch");
}

size_t packed_bytes(int dt, int64_t rows, int64_t n) {
    int bv = dt_block_values(dt);
    if (bv == 0 || rows < 0 || n < 0 || n % bv) return 0;
    if (dt == DT_F32) return (size_t)rows * (size_t)n * 4;
    if (!dt_int_ok(dt)) return 0;
    int64_t T = (rows + TILE_ROWS - 1) / TILE_ROWS;
    return (size_t)T * (size_t)(n / bv) * TILE_ROWS * (size_t)dt_block_bytes(dt);
}

int launch_pack(int dt, const void *src, size_t row_bytes, int64_t rows, int64_t n, void *dst, hipStream_t s) {
    size_t pb = packed_bytes(dt, rows, n);
    if (pb == 0 && rows > 0 && n > 0) return tlmh_seterr(TLM_HIP_EINVAL, "pack: bad dtype %d or n=%lld", dt, (long long)n);
    if (pb == 0) return TLM_HIP_OK;
    if (!src || !dst) return tlmh_seterr(TLM_HIP_EINVAL, "pack: NULL pointer");
    if ((uintptr_t)dst & 15u) return tlmh_seterr(TLM_HIP_EINVAL, "pack: destination must be 16-byte aligned");
    if (dt == DT_F32) {
        int64_t e = rows * n;
        hipLaunchKernelGGL(k_pack_f32, dim3((unsigned)((e + 255) / 256)), dim3(256), 0, s, (const uint8_t *)src,
                           row_bytes, rows, n, (float *)dst);
    } else {
        const int nb = (int)(n / dt_block_values(dt)), bb = dt_block_bytes(dt);
        const int64_t T = (rows + TILE_ROWS - 1) / TILE_ROWS;
        const int cb = 2040 / bb < nb ? 2040 / bb : nb;                 /* <= 2040 source bytes per row piece */
        const int rstride = (cb * bb + 8 + 3) & ~3;                    /* piece + alignment head + tail */
        if (T > 0x7FFFFFFF) return tlmh_seterr(TLM_HIP_EINVAL, "pack: %lld rows", (long long)rows);
        hipLaunchKernelGGL(k_pack, dim3((unsigned)T, (unsigned)((nb + cb - 1) / cb)), dim3(256),
                           (size_t)TILE_ROWS * rstride, s, dt, (const uint8_t *)src, row_bytes, rows, nb, cb, rstride,
                           (uint8_t *)dst);
    }
    return tlmh_check(hipGetLastError(), "pack launch");
}

int launch_matvec_packed(int dt, const void *Wp, int64_t rows, int64_t n, const void *act, float *y, hipStream_t s) {
    if (packed_bytes(dt, rows, n) == 0 && rows > 0 && n > 0)
        return tlmh_seterr(TLM_HIP_EINVAL, "matvec_packed: bad dtype %d or n=%lld", dt, (long long)n);
    if (rows <= 0) return TLM_HIP_OK;
    if (!Wp || !act || !y) return tlmh_seterr(TLM_HIP_EINVAL, "matvec_packed: NULL pointer");
    if ((uintptr_t)act & 3u) return tlmh_seterr(TLM_HIP_EINVAL, "matvec_packed: activation must be 4-byte aligned");
    if (dt == DT_F32) return launch_matvec_plain(dt, Wp, (size_t)n * 4, act, y, n, 0, rows, s);
    if ((uintptr_t)Wp & 15u) return tlmh_seterr(TLM_HIP_EINVAL, "matvec_packed: weights must be 16-byte aligned");
    int nb = (int)(n / dt_block_values(dt));
    if (packed_lds_bytes(dt, nb) > 64 * 1024)
        return tlmh_seterr(TLM_HIP_EUNSUP, "matvec_packed: n=%lld exceeds the staged-activation limit", (long long)n);
    if (n == 0) return launch_matvec_plain(dt, Wp, 0, act, y, 0, 0, rows, s);
    /* the model's segmented launch with one segment: the same kernel, the
     * same rows-per-group rule */
    float *ys[1] = {y};
    const void *Ws[1] = {Wp};
    const int64_t rs[1] = {rows};
    return launch_mv_segs(dt, n, Ws, rs, ys, 1, 0, act, s, nullptr, nullptr);
}

int launch_mv_segs(int dt, int64_t n, const void *const *W, const int64_t *rows, float *const *y, int nseg, int accum,
                   const void *act, hipStream_t s, const MvNorm *norm, unsigned long long *keys) {
    if (nseg < 1 || nseg > MV_SEGS) return tlmh_seterr(TLM_HIP_EINVAL, "mv_segs: %d segments", nseg);
    if (packed_bytes(dt, 1, n) == 0 || dt == DT_F32 || n <= 0 || n % dt_block_values(dt))
        return tlmh_seterr(TLM_HIP_EINVAL, "mv_segs: dtype %d, n=%lld", dt, (long long)n);
    if (norm ? (!norm->x || ((uintptr_t)norm->x & 15u) || ((uintptr_t)norm->w & 15u))
             : (!act || ((uintptr_t)act & 3u)))
        return tlmh_seterr(TLM_HIP_EINVAL, "mv_segs: activation");
    if (keys && (nseg != 1 || ((uintptr_t)keys & 7u) || rows[0] > 0x7FFFFFFF))
        return tlmh_seterr(TLM_HIP_EINVAL, "mv_segs: greedy key needs one segment");
    const int nb = (int)(n / dt_block_values(dt));
    if (packed_lds_bytes(dt, nb) > 64 * 1024)
        return tlmh_seterr(TLM_HIP_EUNSUP, "mv_segs: n=%lld exceeds the staged-activation limit", (long long)n);
    MvSegs sg{};
    sg.n = nseg;
    sg.accum = accum;
    sg.nx = norm ? norm->x : nullptr;
    sg.nw = norm ? norm->w : nullptr;
    sg.eps = norm ? norm->eps : 0.0f;
    sg.keys = keys;
    int64_t end = 0;
    for (int i = 0; i < nseg; i++) {
        if (!W[i] || !y[i] || rows[i] <= 0 || ((uintptr_t)W[i] & 15u))
            return tlmh_seterr(TLM_HIP_EINVAL, "mv_segs: segment %d", i);
        sg.W[i] = (const uint8_t *)W[i];
        sg.rows[i] = rows[i];
        sg.y[i] = y[i];
        end += (rows[i] + TILE_ROWS - 1) / TILE_ROWS;
        sg.tile_end[i] = end;
    }
    const size_t lds = packed_lds_bytes(dt, nb);
    /* rows per group: whole tiles for matrices of many tiles (and for the
     * greedy keys, one per tile), else halves or quarters of tiles so that
     * the launch spreads over the chip (at the Qwen3-235B-A22B shape's
     * 4352- and 8704-byte rows quarter or whole tiles were both slower than
     * halves) */
    const int rpg = keys || end >= 1024 ? 16 : end >= 256 ? 8 : 4;
    /* Q8_0 rows of 64 blocks or more: the mid tile (one round per 64-block
     * chunk) for rows under 128 blocks and for whole-tile launches (lm_head),
     * else the deep tile (one round per 128-block chunk).  For lm_head the
     * deep tile holds 16 items per lane (234 VGPRs, one group per compute
     * unit); the shallow tile (4 per lane, two rounds per chunk, four groups
     * per compute unit) took 151936 x 2048 from 103 to 80 us and the mid
     * tile to 71 us (Qwen3-30B-A3B-shape decode 381.9 -> 383.4 tok/s), and
     * 151936 x 4096 from 150 us in the shallow tile to 127 us (5.2 TB/s) */
    const int var = !mv_deep(dt, nb) ? MV_SHALLOW : nb < 128 || rpg == TILE_ROWS ? MV_MID : MV_DEEP;
    const dim3 blk(256);
    const uint8_t *a = (const uint8_t *)act;
    auto go = [&](auto rpg_c) -> int {
        constexpr int R = decltype(rpg_c)::value;
        const dim3 g((unsigned)(end * (TILE_ROWS / R)));
        switch (dt) {
        case DT_Q8_0:
            if (var == MV_DEEP) hipLaunchKernelGGL((k_mv_packed_seg<DT_Q8_0, MV_DEEP, R>), g, blk, lds, s, sg, nb, a);
            else if (var == MV_MID && R == TILE_ROWS && nb < 128 && !norm && nb * 9 <= MV_EARLY_WORDS * 256)
                /* two tiles per group, the given activation loaded early */
                hipLaunchKernelGGL((k_mv_packed_seg<DT_Q8_0, MV_MID, R, (R == TILE_ROWS ? 2 : 1)>),
                                   dim3((unsigned)((end + 1) / 2)), blk, lds, s, sg, nb, a);
            else if (var == MV_MID) hipLaunchKernelGGL((k_mv_packed_seg<DT_Q8_0, MV_MID, R>), g, blk, lds, s, sg, nb, a);
            else hipLaunchKernelGGL((k_mv_packed_seg<DT_Q8_0, MV_SHALLOW, R>), g, blk, lds, s, sg, nb, a);
            break;
        case DT_Q4_K: hipLaunchKernelGGL((k_mv_packed_seg<DT_Q4_K, MV_SHALLOW, R>), g, blk, lds, s, sg, nb, a); break;
        case DT_Q5_K: hipLaunchKernelGGL((k_mv_packed_seg<DT_Q5_K, MV_SHALLOW, R>), g, blk, lds, s, sg, nb, a); break;
        case DT_Q6_K: hipLaunchKernelGGL((k_mv_packed_seg<DT_Q6_K, MV_SHALLOW, R>), g, blk, lds, s, sg, nb, a); break;
        case DT_Q8_K: hipLaunchKernelGGL((k_mv_packed_seg<DT_Q8_K, MV_SHALLOW, R>), g, blk, lds, s, sg, nb, a); break;
        default: return tlmh_seterr(TLM_HIP_EINVAL, "mv_segs: dtype %d", dt);
        }
        return tlmh_check(hipGetLastError(), "mv_segs launch");
    };
    return rpg == 16 ? go(std::integral_constant<int, 16>{})
           : rpg == 8 ? go(std::integral_constant<int, 8>{}) : go(std::integral_constant<int, 4>{});
}

int launch_mv_job(const tlm_hip_seg *segs, int nseg, hipStream_t s) {
    if (nseg < 0 || nseg > TLM_HIP_MAX_SEGS || (nseg > 0 && !segs))
        return tlmh_seterr(TLM_HIP_EINVAL, "mv_job: bad segment count %d", nseg);
    /* every segment checked as tlm_hip_matvec_rows / _packed check theirs; an
     * invalid one is NaN-filled (its rows, as tlm_matvec_rows does) and
     * reported, the others still run */
    int rc = TLM_HIP_OK;
    MvJob j{};
    size_t lds = 0;
    int64_t groups = 0;
    auto flush = [&]() -> int {
        if (j.n == 0) return TLM_HIP_OK;
        hipLaunchKernelGGL(k_mv_job, dim3((unsigned)groups), dim3(256), lds, s, j);
        j.n = 0;
        groups = 0;
        lds = 0;
        return tlmh_check(hipGetLastError(), "mv_job launch");
    };
    for (int i = 0; i < nseg; i++) {
        const tlm_hip_seg *g = &segs[i];
        const int bv = dt_block_values(g->dt);
        const bool fmt = bv > 0 && g->n > 0 && g->n % bv == 0 && (g->dt == DT_F32 || dt_int_ok(g->dt));
        const bool ptrs = g->W && g->act && g->y && !((uintptr_t)g->act & 3u);
        if (g->rows <= 0) continue;
        int kind = -1;
        size_t need = 0;
        int64_t ng = 0;
        if (fmt && ptrs && g->packed && g->dt != DT_F32 && !((uintptr_t)g->W & 15u)) {
            const int nb = (int)(g->n / bv);
            need = packed_lds_bytes(g->dt, nb);
            if (need <= 64 * 1024) {
                kind = mv_deep(g->dt, nb) ? JK_PACKED_MID : JK_PACKED;
                ng = (g->rows + TILE_ROWS - 1) / TILE_ROWS;
            }
        } else if (fmt && ptrs && !g->packed &&
                   g->row_bytes >= (uint64_t)(g->n / bv) * (uint64_t)dt_block_bytes(g->dt)) {
            if (g->dt == DT_F32) {
                kind = ((uintptr_t)g->W % 4 == 0 && g->row_bytes % 4 == 0) ? JK_F32 : JK_F32_UNALIGNED;
                ng = (g->rows + 7) / 8;
            } else {
                kind = JK_PLAIN;
                ng = (g->rows + 3) / 4;
            }
        }
        if (kind < 0) {
            if (g->y) launch_nan_fill(g->y, g->rows, s);
            rc = tlmh_seterr(TLM_HIP_EINVAL, "mv_job: segment %d (dtype %d, n=%lld, %s layout) is invalid", i, g->dt,
                             (long long)g->n, g->packed ? "packed" : "plain");
            continue;
        }
        if (j.n == JOB_SEGS) {
            const int r2 = flush();
            if (r2) return r2;
        }
        JobSeg &d = j.s[j.n++];
        d.W = (const uint8_t *)g->W;
        d.act = (const uint8_t *)g->act;
        d.y = g->y;
        d.row_bytes = g->row_bytes;
        d.n = g->n;
        d.rows = g->rows;
        d.first = groups;
        d.dt = g->dt;
        d.kind = kind;
        groups += ng;
        lds = need > lds ? need : lds;
    }
    const int r2 = flush();
    return r2 ? r2 : rc;
}
