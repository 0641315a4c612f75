/* tlm_hip_mfma.h - token-batched K-quant tiles on int8 MFMA, shared by the
 * public token matmul and the prefill MoE kernels.  Included by .hip files.
 *
 * The reference's prefill runs the decode step once per token
 * (src/lib/tlm_model.c:1105-1113), so every (token, row) output must carry
 * the decode dot's bits: per super-block an exact int32 sum, then the row's
 * fma chain in ascending block order (src/lib/tlm_quant.c:812-882).
 *
 * A group of 4 waves streams its weight rows once for 32 tokens.  The
 * tokens' Q8_K block is staged once in LDS for all 4 waves (two buffers, one
 * barrier per block); each wave streams 32 rows, with the weights and
 * activations of block b+1 in flight while block b computes.
 *
 * Integer sums per block (exact in int32):
 *   Q6_K:  isum = sum_g sc_g * (sum_{k in g} u_k x_k - 32 S_g), 16 groups of
 *          16, u in [0,63], S_g = bsums[g]: one v_mfma_i32_32x32x16_i8 per
 *          group (u is a non-negative int8), then sc_g * P_g
 *          (src/lib/tlm_quant.c:856-882);
 *   Q4_K / Q5_K: isum = sum_s sc_s * sum_{k in s} q_k x_k over 8 sub-blocks
 *          of 32, one v_mfma_i32_32x32x32_i8 each; msum = sum_s mn_s *
 *          (bsums[2s] + bsums[2s+1]) (src/lib/tlm_quant.c:812-843).
 *   Q8_0:  isum = sum_k w_k x_k over each 32-value block (a8 activations),
 *          one v_mfma_i32_32x32x32_i8 per block, eight blocks per staged
 *          256 values (src/lib/tlm_quant.c:778-792).
 * The group-sum terms sum_i c_i S_i (c = sc or mn) take two MFMAs per block:
 * S = 64 hi + lo with lo in [0,63] and hi in [-64,63] (the range of a
 * well-formed Q8_K block, whose bsums are sums of 16 int8 codes) is staged as
 * bytes, and sum c S = (sum c hi) << 6 + sum c lo.
 *
 * MFMA roles: srcA = activations (lane l: token l%32), srcB = weights (lane l:
 * weight row l%32); lanes l and l+32 hold the two halves of the K range, byte
 * j of A and byte j of B naming the same k.  D[token][row] in lane l,
 * element v: token 8*(v/4) + 4*(l/32) + v%4, row l%32. */
#ifndef TLM_HIP_MFMA_H
#define TLM_HIP_MFMA_H

#include "tlm_hip_internal.h"

namespace tokmm {

constexpr int TM_ROWS = 32;      /* weight rows per wave */
constexpr int TM_TOK = 32;       /* tokens per tile */
constexpr int TM_WAVES = 4;      /* waves per group */

typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr bool tile_dt(int dt) {
    return dt == DT_Q4_K || dt == DT_Q5_K || dt == DT_Q6_K || dt == DT_Q8_0;
}

/* bytes of one (row, block) unit of the packed layout: the Q6_K block
 * without its d (which sits in a plane after the units), whole Q4_K / Q5_K
 * blocks */
template <int DT> constexpr int unit_bytes() {
    return DT == DT_Q6_K ? 208 : DT == DT_Q5_K ? 176 : DT == DT_Q8_0 ? 32 : 144;
}
/* packed (row, block) units per staged 256 values: one K-quant block, eight Q8_0 blocks */
template <int DT> constexpr int blocks_per_stage() { return DT == DT_Q8_0 ? 8 : 1; }

/* One staged Q8_K block of the tile's 32 tokens in LDS.  Code rows are 8
 * (Q6_K: 8-byte reads) or 16 (16-byte reads) bytes past a multiple of 256 so
 * that the lanes of one LDS cycle fall on distinct banks; group-sum rows are
 * 48 bytes for the same reason. */
template <int DT> struct Stage {
    static constexpr int CS = DT == DT_Q6_K ? 264 : 272;
    static constexpr int SS = 48;
    static constexpr int D = TM_TOK * CS;           /* f32 d per token */
    static constexpr int S = D + TM_TOK * 4;        /* group sums: lo bytes [0,16), hi bytes [16,32) */
    static constexpr int BYTES = S + TM_TOK * SS;
};
/* Q8_0: the eight a8 blocks' codes of a token in a row, their d block-major
 * ([block][token], so four consecutive tokens are one 16-byte read) */
template <> struct Stage<DT_Q8_0> {
    static constexpr int CS = 272;
    static constexpr int D = TM_TOK * CS;
    static constexpr int BYTES = D + 8 * TM_TOK * 4;
};
template <int DT> constexpr int tile_lds_bytes() { return 2 * Stage<DT>::BYTES; }

/* ---- weights: one block of one row, this lane's half --------------------- */
template <int DT> struct WRaw;
template <> struct WRaw<DT_Q6_K> {   /* ql pieces [h][qq&1][g&1], qh pieces [h][g&1], scales, d */
    u32x2 ql[8], qh[4];
    u32x4 sc;
    uint32_t d;
};
template <> struct WRaw<DT_Q5_K> {   /* d | dmin, scales[12]; qs bytes 32c + 16 half ..; qh bytes 16 half .. */
    u32x4 hdr, qs[4], qh;
};
template <> struct WRaw<DT_Q4_K> {
    u32x4 hdr, qs[4];
};
template <> struct WRaw<DT_Q8_0> {   /* eight blocks: this lane's 16 code bytes of each, and each block's d */
    u32x4 q[8];
    uint32_t d[8];
};

/* block 0 of a chain's row: its unit, and (Q6_K) its d in the d plane */
struct Chain {
    const GAS uint8_t *unit;
    const GAS uint16_t *dp;
};

template <int DT>
__device__ __forceinline__ Chain chain_at(const uint8_t *Wp, int64_t units, int64_t ubase) {
    Chain c;
    c.unit = (const GAS uint8_t *)Wp + ubase * unit_bytes<DT>();
    /* the f16 d plane after the units (Q6_K, Q8_0; unused for Q4_K / Q5_K) */
    c.dp = (const GAS uint16_t *)((const GAS uint8_t *)Wp + units * unit_bytes<DT>()) + ubase;
    return c;
}

template <int DT>
__device__ __forceinline__ WRaw<DT> wload(const Chain &ch, int b, int half) {
    WRaw<DT> r;
    const GAS uint8_t *u = ch.unit + (size_t)b * (TILE_ROWS * unit_bytes<DT>());
    if constexpr (DT == DT_Q6_K) {
#pragma unroll
        for (int p = 0; p < 8; p++) {      /* p = 4h + 2(qq&1) + gl */
            const int h = p >> 2, q1 = (p >> 1) & 1, gl = p & 1;
            r.ql[p] = *(const GAS u32x2 *)(u + 64 * h + 32 * q1 + 16 * gl + 8 * half);
        }
#pragma unroll
        for (int p = 0; p < 4; p++)        /* p = 2h + gl */
            r.qh[p] = *(const GAS u32x2 *)(u + 128 + 32 * (p >> 1) + 16 * (p & 1) + 8 * half);
        r.sc = *(const GAS u32x4 *)(u + 192);
        r.d = ch.dp[b * TILE_ROWS];
    } else if constexpr (DT == DT_Q8_0) {   /* b counts staged 256-value groups: blocks 8b .. 8b + 7 */
#pragma unroll
        for (int i = 0; i < 8; i++) {
            r.q[i] = *(const GAS u32x4 *)(ch.unit + (size_t)(8 * b + i) * (TILE_ROWS * 32) + 16 * half);
            r.d[i] = ch.dp[(8 * b + i) * TILE_ROWS];
        }
    } else {
        constexpr int QS = DT == DT_Q5_K ? 48 : 16;
        r.hdr = *(const GAS u32x4 *)u;
#pragma unroll
        for (int c = 0; c < 4; c++) r.qs[c] = *(const GAS u32x4 *)(u + QS + 32 * c + 16 * half);
        if constexpr (DT == DT_Q5_K) r.qh = *(const GAS u32x4 *)(u + 16 + 16 * half);
    }
    return r;
}

/* ---- activations: thread (token j = tid/8, part p = tid%8) stages 32 code
 * bytes, one bsum pair and the token's d of each block ------------------- */
struct StageRegs {
    u32x4 c0, c1;
    uint32_t bs;
    float d;
};

/* x: the token's activation, Q8_K blocks in the split layout of the MoE
 * kernels (all codes, then all bsums, then all d; 16-byte aligned) or the
 * reference layout (292-byte blocks: d, codes, bsums; 4-byte aligned). */
template <bool SPLIT>
__device__ __forceinline__ StageRegs stage_load(const GAS uint8_t *x, int nb, int b, int p) {
    StageRegs r;
    if constexpr (SPLIT) {
        const GAS uint8_t *c = x + (size_t)b * 256;
        r.c0 = *(const GAS u32x4 *)(c + 16 * p);
        r.c1 = *(const GAS u32x4 *)(c + 128 + 16 * p);
        r.bs = *(const GAS uint32_t *)(x + (size_t)nb * 256 + 32 * b + 4 * p);
        r.d = *(const GAS float *)(x + (size_t)nb * 288 + 4 * b);
    } else {
        const GAS uint8_t *blk = x + (size_t)b * 292;
        const GAS uint32_t *c = (const GAS uint32_t *)(blk + 4);
        r.c0 = u32x4{c[4 * p], c[4 * p + 1], c[4 * p + 2], c[4 * p + 3]};
        r.c1 = u32x4{c[32 + 4 * p], c[33 + 4 * p], c[34 + 4 * p], c[35 + 4 * p]};
        r.bs = *(const GAS uint32_t *)(blk + 260 + 4 * p);
        r.d = *(const GAS float *)blk;
    }
    return r;
}

/* a8 activations (reference layout, 36-byte blocks: d, 32 codes; 4-byte
 * aligned): part p of staged group b is block 8b + p */
__device__ __forceinline__ StageRegs stage_load_a8(const GAS uint8_t *x, int b, int p) {
    StageRegs r;
    const GAS uint32_t *blk = (const GAS uint32_t *)(x + (size_t)(8 * b + p) * 36);
    r.d = __uint_as_float(blk[0]);
    r.c0 = u32x4{blk[1], blk[2], blk[3], blk[4]};
    r.c1 = u32x4{blk[5], blk[6], blk[7], blk[8]};
    r.bs = 0;
    return r;
}

template <int DT, bool SPLIT>
__device__ __forceinline__ StageRegs stage_in(const GAS uint8_t *x, int nb, int b, int p) {
    if constexpr (DT == DT_Q8_0) return stage_load_a8(x, b, p);
    else return stage_load<SPLIT>(x, nb, b, p);
}

template <int DT>
__device__ __forceinline__ void stage_store(LAS uint8_t *buf, const StageRegs &r, int j, int p) {
    using S = Stage<DT>;
    if constexpr (DT == DT_Q8_0) {   /* block p of token j: codes at 32 p of the row, d block-major */
        *(LAS u32x4 *)(buf + j * S::CS + 32 * p) = r.c0;
        *(LAS u32x4 *)(buf + j * S::CS + 32 * p + 16) = r.c1;
        *(LAS float *)(buf + S::D + 4 * (32 * p + j)) = r.d;
        return;
    } else {
    LAS uint8_t *c = buf + j * S::CS + 16 * p;
    if constexpr (S::CS % 16 == 0) {
        *(LAS u32x4 *)c = r.c0;
        *(LAS u32x4 *)(c + 128) = r.c1;
    } else {
        *(LAS u32x2 *)c = r.c0.xy;
        *(LAS u32x2 *)(c + 8) = r.c0.zw;
        *(LAS u32x2 *)(c + 128) = r.c1.xy;
        *(LAS u32x2 *)(c + 136) = r.c1.zw;
    }
    if (p == 0) *(LAS float *)(buf + S::D + 4 * j) = r.d;
    const int s0 = (int)(int16_t)(r.bs & 0xFFFFu), s1 = (int)(int16_t)(r.bs >> 16);
    LAS uint8_t *sv = buf + S::S + j * S::SS;
    if constexpr (DT == DT_Q6_K) {           /* groups 2p, 2p+1 */
        *(LAS uint16_t *)(sv + 2 * p) = (uint16_t)((s0 & 63) | ((s1 & 63) << 8));
        *(LAS uint16_t *)(sv + 16 + 2 * p) = (uint16_t)(((s0 >> 6) & 0xFF) | (((s1 >> 6) & 0xFF) << 8));
    } else {                                 /* sub-block p; bytes 8..15 and 24..31 stay zero */
        const int s = s0 + s1;
        sv[p] = (uint8_t)(s & 63);
        sv[16 + p] = (uint8_t)((s >> 6) & 0xFF);
    }
    }
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return (long)(((unsigned long long)hi << 32) | lo);
}

/* sum_i c_i S_i for this lane's row (c: 16 int8 in B layout, lane half 0 the
 * lo part, half 1 the hi part) */
__device__ __forceinline__ v16i group_sum_term(v4i sa, v4i c, int half) {
    const v4i z = {0, 0, 0, 0};
    v16i m = __builtin_amdgcn_mfma_i32_32x32x32_i8(sa, half ? c : z, v16i{}, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 16; v++) m[v] <<= 6;
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(sa, half ? z : c, m, 0, 0, 0);
}

/* ---- one block of one chain --------------------------------------------- */
__device__ __forceinline__ void block_chain(const WRaw<DT_Q6_K> &w, const LAS uint8_t *buf, int t, int half,
                                            float (&acc)[16]) {
    using S = Stage<DT_Q6_K>;
    const LAS uint8_t *cod = buf + t * S::CS + 8 * half;
    int isum[16];
#pragma unroll
    for (int v = 0; v < 16; v++) isum[v] = 0;
#pragma unroll
    for (int g = 0; g < 16; g++) {
        const int h = g >> 3, qq = (g >> 1) & 3, gl = g & 1;
        const long aw = *(const LAS long *)(cod + 16 * g);
        const u32x2 qlp = w.ql[4 * h + 2 * (qq & 1) + gl], qhp = w.qh[2 * h + gl];
        const int nib = qq >> 1, sh = 2 * qq;
        const uint32_t lo = ((qlp.x >> (4 * nib)) & 0x0F0F0F0Fu) | (((qhp.x >> sh) & 0x03030303u) << 4);
        const uint32_t hi = ((qlp.y >> (4 * nib)) & 0x0F0F0F0Fu) | (((qhp.y >> sh) & 0x03030303u) << 4);
        const v16i p = __builtin_amdgcn_mfma_i32_32x32x16_i8(aw, pack2(lo, hi), v16i{}, 0, 0, 0);
        const uint32_t scw = g < 4 ? w.sc.x : g < 8 ? w.sc.y : g < 12 ? w.sc.z : w.sc.w;
        const int sg = (int)(int8_t)((scw >> (8 * (g & 3))) & 0xFF);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            isum[v] = __mul24(sg, p[v]) + isum[v];   /* |p| <= 129024, |sg| <= 128 */
            /* materialise the running sum here: otherwise the integer sums
             * are reassociated across groups and every MFMA result stays live */
            asm volatile("" : "+v"(isum[v]));
        }
    }
    const v4i sa = *(const LAS v4i *)(buf + S::S + t * S::SS + 16 * half);
    const v4i scv = {(int)w.sc.x, (int)w.sc.y, (int)w.sc.z, (int)w.sc.w};
    const v16i m = group_sum_term(sa, scv, half);       /* sum_g sc_g S_g, |.| <= 2^22 */
    const LAS float *dd = (const LAS float *)(buf + S::D) + 4 * half;
    const float dwf = f16_to_f32(w.d);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const f32x4 da = *(const LAS f32x4 *)(dd + 8 * q);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int v = 4 * q + k;
            const int is = __mul24(m[v], -32) + isum[v];
            acc[v] = fmaf(dwf * da[k], (float)is, acc[v]);
        }
    }
}

/* eight Q8_0 blocks: per block the exact int32 sum, then the row's fma
 * (d_w d_a, isum) in ascending block order, as the decode dot */
__device__ __forceinline__ void block_chain(const WRaw<DT_Q8_0> &w, const LAS uint8_t *buf, int t, int half,
                                            float (&acc)[16]) {
    using S = Stage<DT_Q8_0>;
    const LAS uint8_t *cod = buf + t * S::CS + 16 * half;
    auto mm = [&](int i) {
        v4i ax = *(const LAS v4i *)(cod + 32 * i);
        /* ordered after the previous block's chain (the volatile statements
         * below keep their order): at most two products live - hoisting all
         * eight 16-register results spills */
        asm volatile("" : "+v"(ax));
        const v4i bw = {(int)w.q[i].x, (int)w.q[i].y, (int)w.q[i].z, (int)w.q[i].w};
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(ax, bw, v16i{}, 0, 0, 0);
    };
    /* block i + 1's product is issued before block i's chain */
    v16i pn = mm(0);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const v16i p = pn;
        if (i < 7) pn = mm(i + 1);
        const LAS float *dd = (const LAS float *)(buf + S::D) + 32 * i + 4 * half;
        const float dw = f16_to_f32(w.d[i]);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const f32x4 da = *(const LAS f32x4 *)(dd + 8 * q);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int v = 4 * q + k;
                acc[v] = fmaf(dw * da[k], (float)p[v], acc[v]);
            }
        }
#pragma unroll
        for (int v = 0; v < 16; v++) asm volatile("" : "+v"(acc[v]));
    }
}

template <int DT>
__device__ __forceinline__ void block_chain(const WRaw<DT> &w, const LAS uint8_t *buf, int t, int half,
                                            float (&acc)[16]) {
    using S = Stage<DT>;
    const LAS uint8_t *cod = buf + t * S::CS + 16 * half;
    /* 6-bit scales and mins of the 8 sub-blocks (src/lib/tlm_quant.c:253-261) */
    const uint32_t a0 = w.hdr.y, a1 = w.hdr.z, a2 = w.hdr.w;
    const uint32_t scw[2] = {a0 & 0x3F3F3F3Fu, (a2 & 0x0F0F0F0Fu) | (((a0 >> 6) & 0x03030303u) << 4)};
    const uint32_t mn0 = a1 & 0x3F3F3F3Fu, mn1 = ((a2 >> 4) & 0x0F0F0F0Fu) | (((a1 >> 6) & 0x03030303u) << 4);
    int isum[16];
#pragma unroll
    for (int v = 0; v < 16; v++) isum[v] = 0;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int c4 = s >> 1, nib = s & 1;
        const v4i ax = *(const LAS v4i *)(cod + 32 * s);
        v4i bw;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t q = (w.qs[c4][k] >> (4 * nib)) & 0x0F0F0F0Fu;
            if constexpr (DT == DT_Q5_K) q |= ((w.qh[k] >> s) & 0x01010101u) << 4;
            bw[k] = (int)q;
        }
        const v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(ax, bw, v16i{}, 0, 0, 0);
        const int sc = (int)((scw[s >> 2] >> (8 * (s & 3))) & 0xFF);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            isum[v] = __mul24(sc, p[v]) + isum[v];    /* |p| <= 126976, sc <= 63 */
            asm volatile("" : "+v"(isum[v]));
        }
    }
    const v4i sa = *(const LAS v4i *)(buf + S::S + t * S::SS + 16 * half);
    const v4i mnv = {(int)mn0, (int)mn1, 0, 0};
    const v16i ms = group_sum_term(sa, mnv, half);      /* msum */
    const LAS float *dd = (const LAS float *)(buf + S::D) + 4 * half;
    const float dw = f16_to_f32(w.hdr.x & 0xFFFFu), dmw = f16_to_f32(w.hdr.x >> 16);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const f32x4 da = *(const LAS f32x4 *)(dd + 8 * q);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int v = 4 * q + k;
            const float dA = dw * da[k], dM = dmw * da[k];
            acc[v] = fmaf(dA, (float)isum[v], acc[v]);
            acc[v] = fmaf(-dM, (float)ms[v], acc[v]);
        }
    }
}

/* The group's tile.  Every thread of the (256-thread) group calls this with
 * the same nb; ch: this lane's chain (row l%32 of its wave's 32 rows); x: the
 * activation of token tid/8 of the tile (threads past the tile's last token
 * pass the last one's); lds: tile_lds_bytes<DT>() bytes, 16-byte aligned.
 * acc[v] = the row . token (8*(v/4) + 4*(l/32) + v%4).  Block b+1's weights
 * and activations are in flight while block b computes. */
template <int DT, bool SPLIT>
__device__ __forceinline__ void tile_run(const Chain &ch, int nb, const GAS uint8_t *x, LAS uint8_t *lds,
                                         float (&acc)[16]) {
    using S = Stage<DT>;
    const int tid = threadIdx.x, j = tid >> 3, p = tid & 7, lane = tid & 63, t = lane & 31, half = lane >> 5;
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;
    if constexpr (DT == DT_Q4_K || DT == DT_Q5_K) {   /* the unused bytes of the group-sum rows, both buffers */
        if (tid < 128)
            *(LAS uint64_t *)(lds + (tid >> 6) * S::BYTES + S::S + ((tid >> 1) & 31) * S::SS + 8 + 16 * (tid & 1)) = 0;
    }
    LAS uint8_t *buf0 = lds, *buf1 = lds + S::BYTES;
    StageRegs r = stage_in<DT, SPLIT>(x, nb, 0, p);
    WRaw<DT> w0 = wload<DT>(ch, 0, half), w1;
    stage_store<DT>(buf0, r, j, p);
    __syncthreads();
    for (int b = 0; b < nb; b += 2) {
        const bool n1 = b + 1 < nb;
        if (n1) {
            r = stage_in<DT, SPLIT>(x, nb, b + 1, p);
            w1 = wload<DT>(ch, b + 1, half);
        }
        block_chain(w0, buf0, t, half, acc);
        if (n1) stage_store<DT>(buf1, r, j, p);
        __syncthreads();
        if (!n1) break;
        const bool n2 = b + 2 < nb;
        if (n2) {
            r = stage_in<DT, SPLIT>(x, nb, b + 2, p);
            w0 = wload<DT>(ch, b + 2, half);
        }
        block_chain(w1, buf1, t, half, acc);
        if (n2) stage_store<DT>(buf0, r, j, p);
        __syncthreads();
    }
}

}  // namespace tokmm

#endif
